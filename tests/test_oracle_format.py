"""Pins of the oracle's number formats and generators (CPU only).

Each check is chosen so that a plausible mistake in the oracle fails it:
the reference's own Int8Blocks test cases (Tests/Kernels/Int8BlocksTests.cpp)
restated on the same inputs, IEEE binary16 conversion against two independent
implementations (the CPU's F16C instruction over all 2^32 inputs, and numpy),
the quantized byte against exact rational arithmetic (a float instead of a
double quotient fails it), and the C++ standard's known answers for the
Mersenne Twister engines the reference seeds its data with.
"""
import ctypes
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

BLOCK = 32


def spread_values(count, seed, value_range):
    """Tests/Kernels/Common.h:90-99: range * ((engine() % 2001) / 1000 - 1)
    in fp32, engine = std::mt19937{seed} (numpy's legacy seeding is the
    standard's init_genrand)."""
    bits = np.random.MT19937(0)
    bits._legacy_seeding(seed)
    raw = bits.random_raw(count).astype(np.uint64)
    steps = (raw % np.uint64(2001)).astype(np.float32)
    return np.float32(value_range) * (steps / np.float32(1000.0) - np.float32(1.0))


def half_bits_numpy(x):
    with np.errstate(over="ignore"):  # beyond the fp16 range is infinity, as intended
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def expected_scale(block):
    """Int8BlocksTests.cpp:28-38: halfToFloat(halfFromFloat(amax / 127.f))."""
    amax = np.max(np.abs(block)).astype(np.float32)
    return float(np.float32(amax / np.float32(127.0)).astype(np.float16).astype(np.float32))


# ---- generators ---------------------------------------------------------------
def test_mt19937_known_answer():
    # [rand.predef]: the 10000th output of a default-constructed mt19937
    bits = np.random.MT19937(0)
    bits._legacy_seeding(5489)
    assert int(bits.random_raw(10000)[-1]) == 4123659995


def test_mt19937_64_known_answer(oracle_lib):
    # [rand.predef]: the 10000th output of a default-constructed mt19937_64
    engine = (ctypes.c_uint64 * 313)()
    oracle_lib.lib().gor_mt64_seed(engine, 5489)
    value = 0
    for _ in range(10000):
        value = oracle_lib.lib().gor_mt64_next(engine)
    assert value == 9981545732273789042


def test_prompt_ids_follow_the_engine(oracle_lib):
    # id = engine() % vocab with engine = mt19937_64(seed)
    engine = (ctypes.c_uint64 * 313)()
    oracle_lib.lib().gor_mt64_seed(engine, 0xC0FFEE + 2)
    expected = [oracle_lib.lib().gor_mt64_next(engine) % 256000 for _ in range(64)]
    assert list(O.prompt_ids(0xC0FFEE + 2, 256000, 64)) == expected


def test_normal_fill_statistics(oracle_lib):
    values = O.normal_fill(O.lib().gor_tensor_seed(3), 0.02, 1 << 21)
    assert values.dtype == np.float32
    assert abs(float(values.mean())) < 0.02 * 5 / np.sqrt(values.size)
    assert abs(float(values.std()) / 0.02 - 1.0) < 5e-3
    # chunks are seeded by position: a prefix is the same whatever the length
    assert np.array_equal(O.normal_fill(O.lib().gor_tensor_seed(3), 0.02, 1000), values[:1000])


# ---- IEEE binary16 --------------------------------------------------------------
@pytest.mark.slow
def test_half_from_float_matches_f16c_for_every_fp32(oracle_lib):
    assert oracle_lib.lib().gor_check_half_exhaustive() == 0


def test_half_round_trip_every_half(oracle_lib):
    assert oracle_lib.lib().gor_check_half_roundtrip() == 0


def test_half_from_float_matches_numpy(oracle_lib):
    rng = np.random.default_rng(11)
    patterns = rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32)
    values = patterns.view(np.float32)
    values = values[np.isfinite(values)]
    ours = np.array([O.half_from_float(float(v)) for v in values[:20000]], dtype=np.uint16)
    theirs = half_bits_numpy(values[:20000])
    assert np.array_equal(ours, theirs)
    # ties to even at the subnormal and normal boundaries
    edges = np.array([2.0 ** -25, 3 * 2.0 ** -25, 2.0 ** -24 * 1.5, 65519.996, 65520.0,
                      1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], dtype=np.float32)
    assert [O.half_from_float(float(v)) for v in edges] == list(half_bits_numpy(edges))


# ---- Int8Blocks (Int8BlocksTests.cpp) ------------------------------------------
def test_round_trip_of_the_reference_case():
    # tInt8BlocksRoundTrip (Int8BlocksTests.cpp:92-126): spreadValues(1280, 8181, 3)
    elements = BLOCK * 40
    values = spread_values(elements, 8181, 3.0)
    stored = O.quantize_int8_blocks(values)
    recovered = O.dequantize_int8_blocks(stored, elements)
    assert stored.size == elements + 2 * (elements // BLOCK)
    for b in range(elements // BLOCK):
        block = values[b * BLOCK:(b + 1) * BLOCK]
        scale = np.float32(expected_scale(block))
        assert scale > 0
        stored_scale = int(stored[elements + 2 * b]) | (int(stored[elements + 2 * b + 1]) << 8)
        assert stored_scale == half_bits_numpy(scale)
        got = recovered[b * BLOCK:(b + 1) * BLOCK]
        steps = np.rint(got / scale)
        assert np.all(np.abs(steps) <= 127)
        assert np.array_equal(got, scale * steps.astype(np.float32))
        assert np.all(np.abs(got - block) <= np.float32(0.5) * scale)


def test_blocks_follow_their_own_magnitude():
    # tInt8BlocksFollowTheBlockMagnitude (Int8BlocksTests.cpp:133-187)
    magnitudes = np.array([1.0e-2, 1.0e3, 0.0, 1.0, 6.0e-8, 1.0e4], dtype=np.float32)
    values = spread_values(6 * BLOCK, 1717, 1.0)
    for b, m in enumerate(magnitudes):
        values[b * BLOCK:(b + 1) * BLOCK] *= m
    recovered = O.dequantize_int8_blocks(O.quantize_int8_blocks(values), values.size)
    for b, m in enumerate(magnitudes):
        got = recovered[b * BLOCK:(b + 1) * BLOCK]
        if m == 0 or m < 1e-7:  # the zero block and the block no fp16 scale can hold
            assert np.all(got == 0)
            continue
        assert np.all(np.abs(got - values[b * BLOCK:(b + 1) * BLOCK])
                      <= np.float32(0.5) * m / np.float32(127.0))


def test_shapes_and_byte_counts():
    # tInt8BlocksShapes (Int8BlocksTests.cpp:196-216)
    accepts = O.lib().gor_quantizes_as_int8_blocks
    assert accepts(2048, 2048 * 2048)
    assert accepts(16384, 2048 * 16384)
    assert accepts(2048, 256000 * 2048)
    assert accepts(32, 64)
    assert not accepts(48, 32 * 48)
    assert not accepts(32, 32 * 3)
    assert not accepts(0, 0)
    assert O.lib().gor_int8_blocks_byte_count(64) == 68
    assert O.lib().gor_int8_blocks_byte_count(2048 * 2048) == 2048 * 2048 + 2048 * 2048 // 16


def test_quantize_in_pieces_is_the_whole():
    # tInt8BlocksQuantizeInPieces (Int8BlocksTests.cpp:222-243)
    elements = BLOCK * 20
    values = spread_values(elements, 5150, 2.0)
    whole = O.quantize_int8_blocks(values)
    pieces = np.zeros_like(whole)
    for first in range(0, elements, 4 * BLOCK):
        piece = np.ascontiguousarray(values[first:first + 4 * BLOCK])
        O.lib().gor_quantize_int8_blocks(O.ptr(piece), piece.size, first, elements, O.ptr(pieces))
    assert np.array_equal(pieces, whole)


def test_block_scale_rule_including_unrepresentable_scales():
    # blockScaleBits (Int8Blocks.cpp:25-36): fp16(amax / 127.f), zero when the
    # fp16 scale is zero or not finite
    rng = np.random.default_rng(5)
    cases = [rng.standard_normal(BLOCK).astype(np.float32) * np.float32(10.0 ** e)
             for e in range(-9, 8)]
    cases.append(np.zeros(BLOCK, np.float32))
    cases.append(np.full(BLOCK, 65504.0 * 127 * 2, np.float32))  # scale overflows fp16
    for block in cases:
        bits = O.lib().gor_block_scale_bits(O.ptr(np.ascontiguousarray(block)))
        with np.errstate(over="ignore"):
            scale = np.float32(np.max(np.abs(block)) / np.float32(127.0)).astype(np.float16)
        want = 0 if (scale == 0 or not np.isfinite(scale)) else int(scale.view(np.uint16))
        assert bits == want


def exact_byte(value, scale):
    """nearbyint of the exact quotient, ties to even, clamped to +-127."""
    q = Fraction(float(value)) / Fraction(float(scale))
    floor = q.numerator // q.denominator
    rest = q - floor
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and floor % 2 == 1):
        floor += 1
    return max(-127, min(127, floor))


def test_quantized_byte_is_the_exact_rounded_quotient():
    # Int8Blocks.cpp:41-47 divides in double; for fp32 operands that quotient
    # rounds like the exact one.  A float division would not: the near-ties
    # below (k + 1/2 +- one fp32 ulp of the value) separate the two.
    rng = np.random.default_rng(7)
    byte = O.lib().gor_quantized_byte
    scales = np.float32(2.0) ** rng.integers(-24, 10, 300).astype(np.float32)
    scales *= (1 + rng.integers(0, 1024, 300) / 1024).astype(np.float32)
    for scale in scales:
        scale = np.float32(np.float16(scale))
        if scale == 0:
            continue
        for k in rng.integers(-128, 128, 6):
            tie = np.float32((k + 0.5) * scale)
            for v in (tie, np.nextafter(tie, np.float32(np.inf)), np.nextafter(tie, np.float32(-np.inf)),
                      np.float32(k * scale), np.float32(rng.uniform(-130, 130) * scale)):
                assert byte(float(v), float(scale)) == exact_byte(v, scale)


def test_quantize_row_is_the_weight_rule(oracle_lib):
    # activations use the same block rule as the weights (the Q8 path's rule)
    values = spread_values(BLOCK * 16, 99, 5.0)
    q, s = O.quantize_row(values)
    stored = O.quantize_int8_blocks(values)
    assert np.array_equal(q.view(np.uint8), stored[:values.size])
    assert np.array_equal(s, stored[values.size:].view(np.uint16))
