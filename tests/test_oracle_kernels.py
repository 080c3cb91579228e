"""Pins of the oracle's per-operation arithmetic (CPU only).

Every operation is checked against what the mathematics fixes, computed
independently here in numpy float64 or exact rationals: the reference's test
cases where it has them (RoPETests, RMSNormTests, GeluTests / GeGLUTests,
ArgmaxTests, MultiQueryAttentionTests), closed forms (position 0 is the
identity, the unit pair at position 1, the unit row), invariants (a rotation
keeps the norm and depends only on the position difference), and brute force
on small inputs (exact products of the Q8 dot, the double softmax).
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

BLOCK = 32


def f32(x):
    return np.asarray(x, dtype=np.float32)


# ---- rotary table and RoPE (RoPE.cpp:7-34, RoPE.h:59-81) ------------------------
def test_rotary_table_is_the_definition():
    head_dim, positions = 256, 8192
    cos, sin = O.rotary_table(positions, head_dim)
    half = head_dim // 2
    for p in (0, 1, 2, 17, 511, 4096, 8191):
        i = np.arange(half, dtype=np.float64)
        angle = p / np.power(10000.0, 2.0 * i / head_dim)
        assert np.array_equal(cos[p], f32(np.cos(angle))), p
        assert np.array_equal(sin[p], f32(np.sin(angle))), p


def rope(x, heads, head_dim, position, cos, sin):
    out = np.ascontiguousarray(x, dtype=np.float32).copy()
    O.lib().gor_rope_row(O.ptr(out), heads * head_dim, heads, head_dim, position,
                         O.ptr(cos), O.ptr(sin))
    return out


def test_rope_position_zero_is_the_identity_and_the_unit_pair_turns_by_one():
    # RoPETests.cpp:134 (position 0) and :155-172 (unit pair at position 1)
    heads, head_dim = 2, 16
    cos, sin = O.rotary_table(16, head_dim)
    x = np.random.default_rng(1).standard_normal(heads * head_dim).astype(np.float32)
    assert np.array_equal(rope(x, heads, head_dim, 0, cos, sin), x)
    unit = np.zeros(head_dim, np.float32)
    unit[0] = 1.0  # the pair (0, half) = (1, 0)
    turned = rope(unit, 1, head_dim, 1, cos, sin)
    assert turned[0] == np.float32(np.cos(1.0)) and turned[head_dim // 2] == np.float32(np.sin(1.0))


def test_rope_keeps_the_norm_and_depends_on_the_position_difference():
    # RoPETests.cpp:191-220 and :271-292
    heads, head_dim = 1, 64
    cos, sin = O.rotary_table(64, head_dim)
    rng = np.random.default_rng(2)
    q = rng.standard_normal(head_dim).astype(np.float32)
    k = rng.standard_normal(head_dim).astype(np.float32)
    for p in (0, 5, 33):
        r = rope(q, heads, head_dim, p, cos, sin).astype(np.float64)
        assert abs(np.linalg.norm(r) / np.linalg.norm(q.astype(np.float64)) - 1) < 1e-6
    d = 7
    base = np.dot(rope(q, 1, head_dim, 0, cos, sin).astype(np.float64),
                  rope(k, 1, head_dim, d, cos, sin).astype(np.float64))
    for p in (3, 20, 50):
        moved = np.dot(rope(q, 1, head_dim, p, cos, sin).astype(np.float64),
                       rope(k, 1, head_dim, p + d, cos, sin).astype(np.float64))
        assert abs(moved - base) < 1e-5 * (1 + abs(base))


def test_rope_is_rotate_half_in_double():
    heads, head_dim, position = 3, 32, 11
    cos, sin = O.rotary_table(16, head_dim)
    x = np.random.default_rng(3).standard_normal(heads * head_dim).astype(np.float32)
    got = rope(x, heads, head_dim, position, cos, sin).reshape(heads, head_dim)
    h = head_dim // 2
    xs = x.reshape(heads, head_dim).astype(np.float64)
    c, s = cos[position].astype(np.float64), sin[position].astype(np.float64)
    want = np.concatenate([xs[:, :h] * c - xs[:, h:] * s, xs[:, h:] * c + xs[:, :h] * s], axis=1)
    assert np.array_equal(got, f32(want))


# ---- RMSNorm with (1 + w) (RMSNorm.h:44-56) ---------------------------------------
def test_rmsnorm_unit_row_zero_row_and_the_offset_by_one():
    # RMSNormTests.cpp:167-185 (unit row), :146 (zero row), :111-129 (1 + w)
    n, eps = 2048, 1e-6
    w = np.random.default_rng(4).standard_normal(n).astype(np.float32) * np.float32(0.1)
    unit = O.rmsnorm_row(np.ones(n, np.float32), w, eps)
    want = f32((1.0 + w.astype(np.float64)) / np.sqrt(1.0 + float(np.float32(eps))))
    assert np.array_equal(unit, want)
    zero = O.rmsnorm_row(np.zeros(n, np.float32), w, eps)
    assert np.all(np.isfinite(zero)) and np.all(zero == 0)
    plain = O.rmsnorm_row(np.full(n, 3.0, np.float32), np.zeros(n, np.float32), eps)
    assert np.allclose(plain, 1.0, atol=1e-6)


def test_rmsnorm_is_the_double_formula():
    n, eps = 2048, 1e-6
    rng = np.random.default_rng(5)
    x = rng.standard_normal(n).astype(np.float32)
    w = (rng.standard_normal(n) * 0.1).astype(np.float32)
    xd = x.astype(np.float64)
    scale = 1.0 / np.sqrt(np.sum(xd * xd) / n + float(np.float32(eps)))
    assert np.array_equal(O.rmsnorm_row(x, w, eps), f32(xd * scale * (1.0 + w.astype(np.float64))))


# ---- tanh GELU and GeGLU (Gelu.h:38-46, GeGLU.h:50-73) ----------------------------
def test_gelu_closed_form_and_saturated_tails():
    # Gelu.h:38-46: 0.5 x (1 + tanh(inner)) with eacp's saturatingTanh, which
    # answers |inner| >= 10 with +-1; within 1e-8 of the reference tests' own
    # non-saturating double form (Tests/Kernels/Common.h:170-175) everywhere
    gelu = O.lib().gor_tanh_gelu
    for x in np.linspace(-8, 8, 161).tolist():
        inner = 0.7978845608028654 * (x + 0.044715 * x * x * x)
        t = math.tanh(inner) if abs(inner) < 10 else math.copysign(1.0, inner)
        assert gelu(float(x)) == 0.5 * x * (1.0 + t)  # libm's tanh on both sides
        assert abs(gelu(float(x)) - 0.5 * x * (1.0 + math.tanh(inner))) <= 1e-8 * (1 + abs(x))
    # GeluTests.cpp:115-138: the tails are finite and equal the saturated form
    for x in (30.0, 1000.0):
        assert gelu(x) == x
        assert gelu(-x) == 0.0
    assert gelu(0.0) == 0.0


def test_geglu_zero_up_and_gate_only():
    # GeGLUTests.cpp:114-155
    geglu = O.lib().gor_geglu
    for g in (-3.0, -0.5, 0.0, 0.25, 2.0):
        assert geglu(g, 0.0) == 0.0
        assert geglu(g, 1.0) == np.float32(O.lib().gor_tanh_gelu(float(np.float32(g))))


# ---- the Q8 product (the exact int8 dot per block) --------------------------------
def exact_product(xq, xs, wbytes, rows, inner):
    wq = wbytes[:rows * inner].view(np.int8).reshape(rows, inner).astype(np.int64)
    ws = wbytes[rows * inner:].view(np.uint16).reshape(rows, inner // BLOCK)
    xsf = [Fraction(float(v)) for v in xs.view(np.float16).astype(np.float64)]
    out = []
    for r in range(rows):
        total = Fraction(0)
        wsf = ws[r].view(np.float16).astype(np.float64)
        for b in range(inner // BLOCK):
            dot = int(np.dot(wq[r, b * BLOCK:(b + 1) * BLOCK], xq[b * BLOCK:(b + 1) * BLOCK].astype(np.int64)))
            total += dot * Fraction(float(wsf[b])) * xsf[b]
        out.append(float(np.float32(float(total))))
    return np.array(out, np.float32)


def test_q8_product_is_the_exact_sum_rounded_once():
    rows, inner = 24, 256
    rng = np.random.default_rng(6)
    w = (rng.standard_normal(rows * inner) * 0.05).astype(np.float32)
    x = rng.standard_normal(inner).astype(np.float32)
    wbytes = O.quantize_int8_blocks(w)
    xq, xs = O.quantize_row(x)
    assert np.array_equal(O.q8_matvec(xq, xs, wbytes, rows, inner),
                          exact_product(xq, xs, wbytes, rows, inner))


def test_q8_product_of_a_one_hot_row_is_a_weight_column():
    # LinearTests.cpp:164-185 (identity input -> the transposed weight)
    rows, inner, column = 16, 128, 37
    w = np.random.default_rng(7).standard_normal(rows * inner).astype(np.float32)
    wbytes = O.quantize_int8_blocks(w)
    x = np.zeros(inner, np.float32)
    x[column] = 1.0
    xq, xs = O.quantize_row(x)
    assert xq[column] == 127
    recovered = O.dequantize_int8_blocks(wbytes, rows * inner).reshape(rows, inner)
    sx = np.float64(np.float16(xs[column // BLOCK].view(np.float16)))
    want = f32(recovered[:, column].astype(np.float64) * 127 * sx)
    assert np.array_equal(O.q8_matvec(xq, xs, wbytes, rows, inner), want)


# ---- argmax (Argmax.h, ArgmaxTests.cpp:207-245) -----------------------------------
def test_argmax_planted_winner_mask_ties_and_empty():
    logits = (np.random.default_rng(8).standard_normal(256000) * 0.1).astype(np.float32)
    logits[137425] = 9.0
    logits[318] = 8.0
    assert O.argmax(logits) == 137425
    mask = np.zeros(256000, np.float32)
    mask[137425] = 1.0
    assert O.argmax(logits, mask) == 318
    last = logits.copy()
    last[-1] = 10.0
    assert O.argmax(last) == 255999
    ties = np.zeros(64, np.float32)
    ties[[9, 3, 40]] = 2.0
    assert O.argmax(ties) == 3
    assert O.argmax(np.ones(8, np.float32), np.ones(8, np.float32)) == 0


# ---- MQA over an fp16 cache (MultiQueryAttention.h:138-260) -----------------------
def mqa_double(q, k16, v16, heads, kv_heads, head_dim, count, scale):
    k = k16.view(np.float16).astype(np.float64).reshape(-1, kv_heads, head_dim)[:count]
    v = v16.view(np.float16).astype(np.float64).reshape(-1, kv_heads, head_dim)[:count]
    out = np.empty((heads, head_dim))
    for h in range(heads):
        g = h // (heads // kv_heads)
        s = float(np.float32(scale)) * (k[:, g, :] @ q.reshape(heads, head_dim)[h].astype(np.float64))
        w = np.exp(s - s.max())
        out[h] = (w @ v[:, g, :]) / w.sum()
    return out.ravel()


@pytest.mark.parametrize("count", [1, 5, 64, 300])
def test_mqa_is_the_double_softmax(count):
    heads, kv_heads, head_dim = 4, 2, 32
    rng = np.random.default_rng(count)
    q = rng.standard_normal(heads * head_dim).astype(np.float32)
    k = rng.standard_normal(count * kv_heads * head_dim).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(count * kv_heads * head_dim).astype(np.float16).view(np.uint16)
    scale = 1.0 / np.sqrt(head_dim)
    got = O.mqa_row_f16(q, k, v, heads, kv_heads, head_dim, count, scale)
    want = mqa_double(q, k, v, heads, kv_heads, head_dim, count, scale)
    # the same double computation summed in another order: equal after rounding
    # to fp32 but for a last-place tie-break
    assert np.max(np.abs(got.astype(np.float64) - want) / (np.abs(want) + 1e-30)) < 2 ** -23


def test_mqa_uniform_scores_average_the_values():
    # SoftmaxTests.cpp:109-187 (a uniform row): a zero query weighs every key alike
    heads, head_dim, count = 2, 16, 10
    q = np.zeros(heads * head_dim, np.float32)
    rng = np.random.default_rng(9)
    k = rng.standard_normal(count * head_dim).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(count * head_dim).astype(np.float16)
    got = O.mqa_row_f16(q, k, v.view(np.uint16), heads, 1, head_dim, count, 0.25)
    mean = v.astype(np.float64).reshape(count, head_dim).mean(axis=0)
    assert np.allclose(got.reshape(heads, head_dim), mean, rtol=1e-6, atol=1e-7)
