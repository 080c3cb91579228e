"""The block-scale quotient without a division (gq8_numerics.hpp
scale_bits_from_amax): amax / 127 rounded to fp32, as Int8Blocks.cpp:25-36
computes it, equals the double product amax * (1 / 127) rounded to fp32 for
every non-negative finite fp32 amax.  The argument in the source (the exact
quotient stays at least 2^-32 from any fp32 rounding midpoint, the double
product within 2^-52 of it) is checked here exhaustively: all 2^31 - 2^23
values, subnormals and zero included."""
import numpy as np


def test_double_product_rounds_to_the_fp32_quotient_everywhere():
    inverse = np.float64(1.0) / np.float64(127.0)
    step = 1 << 24
    mismatched = 0
    for start in range(0, 0x7F800000, step):
        bits = np.arange(start, min(start + step, 0x7F800000), dtype=np.uint32)
        amax = bits.view(np.float32)
        want = amax / np.float32(127.0)
        got = (amax.astype(np.float64) * inverse).astype(np.float32)
        mismatched += int(np.count_nonzero(want.view(np.uint32) != got.view(np.uint32)))
    assert mismatched == 0


def test_infinity_and_nan_carry_through():
    inverse = np.float64(1.0) / np.float64(127.0)
    for value in (np.float32(np.inf), np.float32(np.nan)):
        want = value / np.float32(127.0)
        got = np.float32(np.float64(value) * inverse)
        assert (np.isnan(want) and np.isnan(got)) or want == got
