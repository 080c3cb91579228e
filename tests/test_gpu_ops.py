"""Parity of every op-level entry point of libgemma_q8 against the CPU oracle.

The GPU path computes in double and rounds to fp32 where the oracle does, so
most outputs are expected to be bit-identical; where a summation order differs
(parallel reductions) the tests allow the rare last-bit difference and bound
the error at the reference's own tolerances.
"""
import math

import numpy as np
import pytest

import oracle as O
from gpu_helpers import empty, exact_fraction, q8_bytes, split_q8, spread, to_device, worst_error
from huggingfaceeacp_amd import gemma_q8 as G

pytestmark = pytest.mark.gpu

# Device copies of the inputs stay referenced until the test ends: a tensor
# whose only use is an inline data_ptr() would go back to torch's caching
# allocator before the kernel reads it.
_alive = []


@pytest.fixture(autouse=True)
def _keep_device_inputs():
    _alive.clear()
    yield
    _alive.clear()


def dev(array) -> int:
    import torch
    tensor = to_device(torch, np.ascontiguousarray(array))
    _alive.append(tensor)
    return tensor.data_ptr()


def special_blocks() -> np.ndarray:
    """Blocks chosen to exercise every branch of the Int8Blocks rule."""
    blocks = []
    rng = np.random.default_rng(11)
    # exact ties at every k: scale 2^-7, values (k + 0.5) * s, the amax 127 s
    s = np.float32(2.0 ** -7)
    ks = np.arange(-127, 127, dtype=np.float32)
    ties = ((ks + np.float32(0.5)) * s).astype(np.float32)
    for start in range(0, ties.size, 31):
        block = np.zeros(32, np.float32)
        part = ties[start:start + 31]
        block[:part.size] = part
        block[31] = np.float32(127) * s
        blocks.append(block)
    # ties one ulp either side
    for direction in (np.inf, -np.inf):
        for start in range(0, ties.size, 31):
            block = np.zeros(32, np.float32)
            part = np.nextafter(ties[start:start + 31], np.float32(direction))
            block[:part.size] = part
            block[31] = np.float32(127) * s
            blocks.append(block)
    # magnitudes across the fp16 range, subnormal scales, and the zero rule
    for magnitude in [1e-2, 1e3, 0.0, 1.0, 6e-8, 1e4, 1e-5, 3e-6, 9.9e-4, 7.8e-3, 2e6, 8.3e6, 1e7]:
        blocks.append((rng.uniform(-1, 1, 32) * magnitude).astype(np.float32))
    # non-finite elements
    b = rng.standard_normal(32).astype(np.float32)
    b[3] = np.inf
    blocks.append(b)
    b = rng.standard_normal(32).astype(np.float32)
    b[7] = np.nan
    blocks.append(b)
    b = np.full(32, np.nan, np.float32)
    blocks.append(b)
    return np.concatenate(blocks)


def test_quantize_rows_bit_exact(torch_cuda):
    torch = torch_cuda
    special = special_blocks()
    normal = spread(64 * 2048, 3, 0.7)
    x = np.concatenate([special, normal])
    x = x[: (x.size // 64) * 64]
    inner = 64
    rows = x.size // inner
    out = empty(torch, q8_bytes(rows, inner), torch.uint8)
    G.quantize_rows(dev(x), rows, inner, out.data_ptr())
    torch.cuda.synchronize()
    q_gpu, s_gpu = split_q8(out.cpu().numpy(), rows, inner)
    q_ref, s_ref = O.quantize_row(x)
    assert np.array_equal(s_gpu.ravel(), s_ref)
    assert np.array_equal(q_gpu.ravel(), q_ref)
    # and the bytes are the reference's tensor layout exactly
    assert np.array_equal(out.cpu().numpy(), O.quantize_int8_blocks(x))


def test_scale_rule_over_amax_sweep(torch_cuda):
    """Every block's scale is fp16(amax / 127) or zero: a dense sweep of amax
    values across the whole fp16 range, each as the largest element of a block."""
    torch = torch_cuda
    amax = np.geomspace(1e-9, 9e6, 1 << 16).astype(np.float32)
    amax = np.concatenate([amax, np.nextafter(amax, np.float32(0)), np.nextafter(amax, np.float32(np.inf))])
    x = np.zeros((amax.size, 32), np.float32)
    x[:, 5] = amax
    x[:, 9] = -amax * np.float32(0.5)
    x = x.ravel()
    out = empty(torch, q8_bytes(amax.size, 32), torch.uint8)
    G.quantize_rows(dev(x), amax.size, 32, out.data_ptr())
    torch.cuda.synchronize()
    q_gpu, s_gpu = split_q8(out.cpu().numpy(), amax.size, 32)
    q_ref, s_ref = O.quantize_row(x)
    assert np.array_equal(s_gpu.ravel(), s_ref)
    assert np.array_equal(q_gpu.ravel(), q_ref)


def test_embed_bit_exact(torch_cuda):
    torch = torch_cuda
    vocab, width = 1000, 2048
    table_f = spread(vocab * width, 5, 0.02)
    table = O.quantize_int8_blocks(table_f)
    tokens = np.array([0, 999, 17, 500, 17], dtype=np.uint32)
    out = empty(torch, tokens.size * width, torch.float32)
    scale = float(np.sqrt(np.float32(2048), dtype=np.float32))
    G.embed(dev(tokens), tokens.size, dev(table),
            vocab, width, scale, out.data_ptr())
    torch.cuda.synchronize()
    deq = O.dequantize_int8_blocks(table, vocab * width).reshape(vocab, width)
    expected = (np.float32(scale) * deq[tokens.astype(np.int64)]).astype(np.float32)
    assert np.array_equal(out.cpu().numpy().reshape(tokens.size, width), expected)


# (rows past 64 take a workgroup a row; 1056 leaves part of its last 256-element
# stretch past the row)
@pytest.mark.parametrize("width,rows", [(2048, 1), (2048, 5), (32, 3), (16384, 2), (2048, 80),
                                        (1056, 70)])
def test_rmsnorm_and_q8(torch_cuda, width, rows):
    torch = torch_cuda
    x = spread(rows * width, 7 + width, 3.0)
    w = spread(width, 8, 0.1)
    y = empty(torch, rows * width, torch.float32)
    q8 = empty(torch, q8_bytes(rows, width), torch.uint8)
    G.rmsnorm(dev(x), dev(w), rows, width, 1e-6,
              y.data_ptr(), q8.data_ptr())
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(rows, width)
    q_gpu, s_gpu = split_q8(q8.cpu().numpy(), rows, width)
    for r in range(rows):
        ref = O.rmsnorm_row(x[r * width:(r + 1) * width], w)
        assert worst_error(got[r], ref) <= 1e-6
        assert exact_fraction(got[r], ref) >= 0.999
        # the quantization of the GPU's own rows is exact
        q_ref, s_ref = O.quantize_row(got[r])
        assert np.array_equal(q_gpu[r], q_ref) and np.array_equal(s_gpu[r], s_ref)


def test_rope_matches_oracle(torch_cuda):
    torch = torch_cuda
    heads, head_dim, rows, first = 8, 256, 3, 8189
    cos, sin = O.rotary_table(8192, head_dim)
    x = spread(rows * heads * head_dim, 9, 2.0)
    xd = to_device(torch, x)
    G.rope(xd.data_ptr(), heads * head_dim, heads, head_dim, first, rows,
           dev(cos), dev(sin))
    torch.cuda.synchronize()
    got = xd.cpu().numpy().reshape(rows, heads * head_dim)
    for r in range(rows):
        ref = x[r * heads * head_dim:(r + 1) * heads * head_dim].copy()
        O.lib().gor_rope_row(O.ptr(ref), heads * head_dim, heads, head_dim, first + r,
                             O.ptr(cos), O.ptr(sin))
        assert np.array_equal(got[r], ref)


SHAPES = [(2048, 2560), (2048, 32768), (16384, 2048), (2048, 2048), (2048, 256000)]


@pytest.mark.parametrize("inner,outputs", SHAPES)
def test_q8_product_real_shapes(torch_cuda, inner, outputs):
    torch = torch_cuda
    w = O.quantize_int8_blocks(spread(inner * outputs, inner + outputs, 0.02))
    x = spread(inner, 1, 1.5)
    xq, xs = O.quantize_row(x)
    x8 = np.concatenate([xq.view(np.uint8), xs.view(np.uint8)])
    y = empty(torch, outputs, torch.float32)
    G.q8_product(dev(x8), dev(w), 1, inner,
                 outputs, y.data_ptr(), outputs)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = O.q8_matvec(xq, xs, w, outputs, inner)
    assert worst_error(got, ref) <= 1e-6
    assert exact_fraction(got, ref) >= 0.999


@pytest.mark.parametrize("rows", [2, 3, 8, 17])
def test_q8_product_rows_and_residual(torch_cuda, rows):
    torch = torch_cuda
    inner, outputs = 2048, 2048
    w = O.quantize_int8_blocks(spread(inner * outputs, 77, 0.02))
    x = spread(rows * inner, 78, 1.0)
    q_all, s_all = O.quantize_row(x)
    x8 = np.concatenate([q_all.view(np.uint8), s_all.view(np.uint8)])
    base = spread(rows * outputs, 79, 1.0)
    y = to_device(torch, base)
    G.q8_product(dev(x8), dev(w), rows, inner,
                 outputs, y.data_ptr(), outputs, residual=True)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(rows, outputs)
    for r in range(rows):
        ref = O.q8_matvec(q_all[r * inner:(r + 1) * inner], s_all[r * 64:(r + 1) * 64], w,
                          outputs, inner).astype(np.float64) + base[r * outputs:(r + 1) * outputs]
        assert worst_error(got[r], ref) <= 1e-6


@pytest.mark.parametrize("rows,inner,outputs", [(32, 2048, 2560), (64, 2048, 2048),
                                                 (100, 16384, 2048), (130, 64, 96),
                                                 (33, 2048, 32768), (300, 512, 200)])
def test_q8_gemm_rows_are_the_one_row_products(torch_cuda, rows, inner, outputs):
    """Steps of 32 rows or more run on the int8 MFMA GEMM (an inner size of
    64 takes the row kernel); each row is the exact block dot scaled and
    summed in double in block order, as the oracle does, so the rows are
    bit-identical to the one-row products.  Shapes cover whole and partial
    128 x 64 tiles and one to 64 K chunks."""
    torch = torch_cuda
    w = O.quantize_int8_blocks(spread(inner * outputs, 81, 0.02))
    x = spread(rows * inner, 82, 1.0)
    q_all, s_all = O.quantize_row(x)
    x8 = np.concatenate([q_all.view(np.uint8), s_all.view(np.uint8)])
    y = empty(torch, rows * outputs, torch.float32)
    G.q8_product(dev(x8), dev(w), rows, inner, outputs, y.data_ptr(), outputs)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(rows, outputs)
    nb = inner // 32
    for r in range(rows):
        ref = O.q8_matvec(q_all[r * inner:(r + 1) * inner], s_all[r * nb:(r + 1) * nb], w,
                          outputs, inner)
        assert np.array_equal(got[r], ref), f"row {r}"


def test_q8_gemm_residual(torch_cuda):
    torch = torch_cuda
    rows, inner, outputs = 48, 2048, 2048
    w = O.quantize_int8_blocks(spread(inner * outputs, 83, 0.02))
    x = spread(rows * inner, 84, 1.0)
    q_all, s_all = O.quantize_row(x)
    x8 = np.concatenate([q_all.view(np.uint8), s_all.view(np.uint8)])
    base = spread(rows * outputs, 85, 1.0)
    y = to_device(torch, base)
    G.q8_product(dev(x8), dev(w), rows, inner, outputs, y.data_ptr(), outputs, residual=True)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(rows, outputs)
    for r in range(rows):
        ref = O.q8_matvec(q_all[r * inner:(r + 1) * inner], s_all[r * 64:(r + 1) * 64], w,
                          outputs, inner).astype(np.float64) + base[r * outputs:(r + 1) * outputs]
        assert worst_error(got[r], ref) <= 1e-6


def test_kv_store_f16(torch_cuda):
    torch = torch_cuda
    rows, kv, pos, maxpos = 3, 256, 5, 16
    k = spread(rows * 512, 21, 3.0)
    v = spread(rows * 512, 22, 3.0)
    kc = torch.zeros(maxpos * kv, dtype=torch.int16, device="cuda")
    vc = torch.zeros(maxpos * kv, dtype=torch.int16, device="cuda")
    G.kv_store_f16(dev(k), dev(v), 512, rows, kv,
                   kc.data_ptr(), vc.data_ptr(), pos)
    torch.cuda.synchronize()
    kh = kc.cpu().numpy().view(np.uint16).reshape(maxpos, kv)
    vh = vc.cpu().numpy().view(np.uint16).reshape(maxpos, kv)
    for r in range(rows):
        assert np.array_equal(kh[pos + r], k[r * 512:r * 512 + kv].astype(np.float16).view(np.uint16))
        assert np.array_equal(vh[pos + r], v[r * 512:r * 512 + kv].astype(np.float16).view(np.uint16))
    assert not kh[:pos].any() and not kh[pos + rows:].any()


def _cache(count, kv, seed):
    return spread(count * kv, seed, 1.5).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("keys", [1, 63, 64, 65, 640, 8192])
def test_mqa_decode(torch_cuda, keys):
    torch = torch_cuda
    heads, kvh, hd = 8, 1, 256
    q = spread(heads * hd, 31, 1.0)
    kc, vc = _cache(keys, hd, 32), _cache(keys, hd, 33)
    ws_bytes = G.mqa_workspace_bytes(1, heads, hd, keys)
    ws = empty(torch, ws_bytes, torch.uint8)
    out = empty(torch, heads * hd, torch.float32)
    G.mqa_decode(dev(q), dev(kc),
                 dev(vc), heads, kvh, hd, keys, 0.0625, out.data_ptr(),
                 ws.data_ptr(), ws_bytes)
    torch.cuda.synchronize()
    ref = O.mqa_row_f16(q, kc, vc, heads, kvh, hd, keys, 0.0625)
    got = out.cpu().numpy()
    assert worst_error(got, ref) <= 2e-6
    assert exact_fraction(got, ref) >= 0.99


def test_mqa_prefill_equals_rows_of_decodes(torch_cuda):
    """MultiQueryAttentionTests.cpp:217-256: prefill row r == a decode over
    offset + r + 1 keys."""
    torch = torch_cuda
    heads, kvh, hd, rows, offset = 8, 1, 256, 70, 3
    total = offset + rows
    q = spread(rows * heads * hd, 41, 1.0)
    kc, vc = _cache(total, hd, 42), _cache(total, hd, 43)
    ws_bytes = G.mqa_workspace_bytes(rows, heads, hd, total)
    ws = empty(torch, ws_bytes, torch.uint8)
    out = empty(torch, rows * heads * hd, torch.float32)
    G.mqa_prefill(dev(q), dev(kc),
                  dev(vc), heads, kvh, hd, rows, offset, 0.0625,
                  out.data_ptr(), ws.data_ptr(), ws_bytes)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(rows, heads * hd)
    for r in range(rows):
        ref = O.mqa_row_f16(q[r * heads * hd:(r + 1) * heads * hd], kc, vc, heads, kvh, hd,
                            offset + r + 1, 0.0625)
        assert worst_error(got[r], ref) <= 2e-6


@pytest.mark.parametrize("rows,offset,hd", [(32, 0, 256), (45, 100, 256), (16, 7, 128),
                                            (20, 0, 64)])
def test_prefill_attention_blocks(torch_cuda, rows, offset, hd):
    """Blocks of 16+ rows take the fp64-MFMA prefill kernel: every row equals
    a decode over its own keys (MultiQueryAttentionTests.cpp:217-256), and keys
    past the block's last position (poisoned here) are never read."""
    torch = torch_cuda
    heads, kvh = 8, 2 if hd == 64 else 1
    total = offset + rows
    q = spread(rows * heads * hd, 61 + rows, 1.0)
    kc, vc = _cache(total + 8, kvh * hd, 62), _cache(total + 8, kvh * hd, 63)
    kw = kvh * hd
    kp, vp = kc.copy().reshape(total + 8, kw), vc.copy().reshape(total + 8, kw)
    kp[total:] = np.float16(3e4).view(np.uint16)
    vp[total:] = np.float16(-3e4).view(np.uint16)
    ws_bytes = G.mqa_workspace_bytes(rows, heads, hd, total)
    ws = empty(torch, ws_bytes, torch.uint8)
    out = empty(torch, rows * heads * hd, torch.float32)
    G.mqa_prefill(dev(q), dev(kp), dev(vp), heads, kvh, hd, rows, offset, 1.0 / math.sqrt(hd),
                  out.data_ptr(), ws.data_ptr(), ws_bytes)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(rows, heads * hd)
    exact = []
    for r in range(rows):
        ref = O.mqa_row_f16(q[r * heads * hd:(r + 1) * heads * hd], kc, vc, heads, kvh, hd,
                            offset + r + 1, 1.0 / math.sqrt(hd))
        assert worst_error(got[r], ref) <= 2e-6, f"row {r}"
        exact.append(exact_fraction(got[r], ref))
    print(f"prefill attention rows={rows} hd={hd}: bit-identical {np.mean(exact):.4f}")


def test_mqa_causal_never_reads_later_keys(torch_cuda):
    """MultiQueryAttentionTests.cpp:165-190: poison past each row's position."""
    torch = torch_cuda
    heads, kvh, hd, rows = 2, 1, 16, 5
    q = spread(rows * heads * hd, 51, 1.0)
    kc, vc = _cache(rows, hd, 52), _cache(rows, hd, 53)
    poisoned_k, poisoned_v = kc.copy().reshape(rows, hd), vc.copy().reshape(rows, hd)
    outs = []
    for variant in range(2):
        k = kc if variant == 0 else poisoned_k
        v = vc if variant == 0 else poisoned_v
        ws_bytes = G.mqa_workspace_bytes(1, heads, hd, rows)
        ws = empty(torch, ws_bytes, torch.uint8)
        out = empty(torch, heads * hd, torch.float32)
        # the query at position 1 attends keys 0..1
        if variant == 1:
            k[2:] = np.float16(1e4).view(np.uint16)
            v[2:] = np.float16(-1e4).view(np.uint16)
        G.mqa_prefill(dev(q[heads * hd:2 * heads * hd]),
                      dev(np.ascontiguousarray(k)),
                      dev(np.ascontiguousarray(v)), heads, kvh, hd, 1, 1,
                      0.25, out.data_ptr(), ws.data_ptr(), ws_bytes)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("rows", [1, 4])
def test_geglu_and_q8(torch_cuda, rows):
    torch = torch_cuda
    inter = 16384
    fused = spread(rows * 2 * inter, 61, 2.0)
    fused[:8] = [30, -30, 1000, -1000, 0, 5, -5, 9]  # saturated tails (GeluTests.cpp:115-138)
    out = empty(torch, rows * inter, torch.float32)
    q8 = empty(torch, q8_bytes(rows, inter), torch.uint8)
    G.geglu(dev(fused), rows, inter, out.data_ptr(), q8.data_ptr())
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(rows, inter)
    q_gpu, s_gpu = split_q8(q8.cpu().numpy(), rows, inter)
    f = fused.reshape(rows, 2 * inter)
    for r in range(rows):
        ref = np.array([O.lib().gor_geglu(float(g), float(u))
                        for g, u in zip(f[r, :inter], f[r, inter:])], dtype=np.float32)
        assert worst_error(got[r], ref) <= 1e-6
        assert exact_fraction(got[r], ref) >= 0.999
        q_ref, s_ref = O.quantize_row(got[r])
        assert np.array_equal(q_gpu[r], q_ref) and np.array_equal(s_gpu[r], s_ref)
    assert np.isfinite(got).all()


def _argmax_gpu(torch, logits, mask=None, rows=1):
    length = logits.size // rows
    ws_bytes = G.argmax_workspace_bytes(rows, length)
    ws = empty(torch, ws_bytes, torch.uint8)
    out = torch.zeros(rows, dtype=torch.int32, device="cuda")
    G.argmax_rows(dev(logits),
                  dev(mask) if mask is not None else None, rows, length,
                  out.data_ptr(), ws.data_ptr(), ws_bytes)
    torch.cuda.synchronize()
    return out.cpu().numpy().astype(np.int64)


def test_argmax_over_the_vocabulary(torch_cuda):
    """ArgmaxTests.cpp:207-245: planted winner, suppressed winner, last token."""
    torch = torch_cuda
    vocab = 256000
    logits = spread(vocab, 256, 4.0)
    logits[137425] = 900.0
    logits[318] = 800.0
    assert _argmax_gpu(torch, logits)[0] == 137425
    mask = np.zeros(vocab, np.float32)
    mask[137425] = 1.0
    assert _argmax_gpu(torch, logits, mask)[0] == 318
    last = spread(vocab, 4242, 4.0)
    last[-1] = 900.0
    assert _argmax_gpu(torch, last)[0] == vocab - 1


def test_argmax_ties_and_masks(torch_cuda):
    torch = torch_cuda
    n = 5000
    logits = np.zeros(n, np.float32)
    logits[[4000, 77, 2500]] = 3.0
    assert _argmax_gpu(torch, logits)[0] == 77  # lowest index among equal maxima
    assert _argmax_gpu(torch, logits, np.ones(n, np.float32))[0] == 0  # all suppressed
    rows = np.stack([spread(n, s, 1.0) for s in range(4)])
    got = _argmax_gpu(torch, rows.ravel(), rows=4)
    assert [int(v) for v in got] == [O.argmax(r) for r in rows]
