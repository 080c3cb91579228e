"""The GeGLU's tanh (huggingfaceeacp_amd/csrc/gq8_tanh.hpp, built for the host
with g++) against libm's tanh, which the oracle's GeGLU uses (Gelu.h:27-46 in
double): within 4 ulps over [-10, 10], and fp32 GeGLU outputs identical on
two million seeded (gate, up) pairs and on every fp32 gate whose tanh
argument lies in [-10, -3] (where 1 + tanh cancels and a tanh error is
magnified most), against seven up values from 1e-3 to 65504."""
import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "huggingfaceeacp_amd", "csrc")


def test_tanh_from_exp_against_libm(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no g++")
    exe = tmp_path / "tanh_check"
    subprocess.run([gxx, "-O2", "-ffp-contract=off", "-I", CSRC, "-o", str(exe),
                    os.path.join(HERE, "native", "tanh_check.cpp"), "-lm"], check=True)
    out = subprocess.run([str(exe), "2000000"], check=True, capture_output=True, text=True).stdout
    print(out)
    worst = int(re.search(r"worst (\d+) ulp", out).group(1))
    differ = int(re.search(r"differing from libm: (\d+)", out).group(1))
    sweep = re.search(r"dense sweep .* differing from libm: (\d+) of (\d+)", out)
    assert worst <= 4
    assert differ == 0
    assert int(sweep.group(2)) > 20_000_000
    assert int(sweep.group(1)) == 0
