"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.  The
product never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

MODE_Q8 = 0
MODE_REFERENCE = 1
MODE_Q8_PATH_F32 = 2  # the Q8 path with fp32 product inputs and an fp32 KV cache

T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN, T_INPUT_NORM, T_POST_NORM = range(9)
PER_LAYER = 9
DBG_NORMALISED, DBG_ATTENDED, DBG_ACTIVATED, DBG_HIDDEN = range(4)


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


class Shape(ctypes.Structure):
    _fields_ = [
        ("width", ctypes.c_int), ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int), ("layers", ctypes.c_int), ("intermediate", ctypes.c_int),
        ("vocab", ctypes.c_int), ("max_positions", ctypes.c_int),
        ("rms_epsilon", ctypes.c_float), ("rope_theta", ctypes.c_double),
        ("embedding_scale", ctypes.c_float),
    ]


def make_shape(width, heads, kv_heads, head_dim, layers, intermediate, vocab, max_positions,
               rms_epsilon=1e-6, rope_theta=10000.0, embedding_scale=None) -> Shape:
    if embedding_scale is None:
        embedding_scale = float(np.sqrt(np.float32(width), dtype=np.float32))
    return Shape(width, heads, kv_heads, head_dim, layers, intermediate, vocab, max_positions,
                 rms_epsilon, rope_theta, embedding_scale)


def gemma_2b_shape(layers=18, max_positions=8192) -> Shape:
    return make_shape(2048, 8, 1, 256, layers, 16384, 256000, max_positions)


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    i64, i32, u16, u64 = ctypes.c_int64, ctypes.c_int, ctypes.c_uint16, ctypes.c_uint64
    sig = {
        "gor_half_from_float": (u16, [ctypes.c_float]),
        "gor_half_to_float": (ctypes.c_float, [u16]),
        "gor_int8_block_count": (i64, [i64]),
        "gor_int8_blocks_byte_count": (i64, [i64]),
        "gor_quantizes_as_int8_blocks": (i32, [i64, i64]),
        "gor_block_scale_bits": (u16, [P]),
        "gor_quantized_byte": (ctypes.c_int8, [ctypes.c_float, ctypes.c_float]),
        "gor_quantize_int8_blocks": (None, [P, i64, i64, i64, P]),
        "gor_dequantize_int8_blocks": (None, [P, i64, P]),
        "gor_quantize_row": (None, [P, i64, P, P]),
        "gor_mt64_seed": (None, [P, u64]),
        "gor_mt64_next": (u64, [P]),
        "gor_normal_fill": (None, [u64, ctypes.c_double, P, i64]),
        "gor_prompt_ids": (None, [u64, i32, i32, P]),
        "gor_rotary_table": (None, [i32, i32, ctypes.c_double, P, P]),
        "gor_rmsnorm_row": (None, [P, P, i32, ctypes.c_float, P]),
        "gor_tanh_gelu": (ctypes.c_double, [ctypes.c_double]),
        "gor_geglu": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
        "gor_rope_row": (None, [P, i32, i32, i32, i32, P, P]),
        "gor_q8_matvec": (None, [P, P, P, i64, i64, P]),
        "gor_argmax": (i32, [P, P, i32]),
        "gor_sample": (i32, [P, P, i32, ctypes.c_float, i32, ctypes.c_float, ctypes.c_double]),
        "gor_mt64_uniform": (ctypes.c_double, [P]),
        "gor_mqa_row_f16": (None, [P, P, P, i32, i32, i32, i32, ctypes.c_float, P]),
        "gor_tensor_count": (i32, [P]),
        "gor_tensor_elements": (i64, [P, i32]),
        "gor_tensor_is_norm": (i32, [P, i32]),
        "gor_tensor_seed": (u64, [i32]),
        "gor_tensor_sigma": (ctypes.c_double, [P, i32]),
        "gor_model_create": (P, [P, i32]),
        "gor_model_destroy": (None, [P]),
        "gor_model_set_tensor": (i32, [P, i32, P]),
        "gor_model_fill_synthetic": (i32, [P]),
        "gor_model_tensor_bytes": (P, [P, i32]),
        "gor_model_begin": (None, [P]),
        "gor_model_position": (i32, [P]),
        "gor_model_step": (i32, [P, P, i32, P, P]),
        "gor_model_step_block": (i32, [P, P, i32, P, i32]),
        "gor_model_debug": (P, [P, i32, i32]),
        "gor_model_debug_q": (P, [P, i32, i32]),
        "gor_model_debug_s": (P, [P, i32, i32]),
        "gor_generate": (i32, [P, P, i32, i32, i32, P, P]),
        "gor_check_half_exhaustive": (i64, []),
        "gor_check_half_roundtrip": (i64, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


# ---- format ------------------------------------------------------------------
def half_from_float(x: float) -> int:
    return int(lib().gor_half_from_float(ctypes.c_float(x)))


def half_to_float(h: int) -> float:
    return float(lib().gor_half_to_float(h))


def quantize_int8_blocks(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32).ravel()
    n = values.size
    out = np.zeros(int(lib().gor_int8_blocks_byte_count(n)), dtype=np.uint8)
    lib().gor_quantize_int8_blocks(ptr(values), n, 0, n, ptr(out))
    return out


def dequantize_int8_blocks(stored: np.ndarray, element_count: int) -> np.ndarray:
    stored = np.ascontiguousarray(stored, dtype=np.uint8)
    out = np.zeros(element_count, dtype=np.float32)
    lib().gor_dequantize_int8_blocks(ptr(stored), element_count, ptr(out))
    return out


def quantize_row(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    q = np.zeros(x.size, dtype=np.int8)
    s = np.zeros(x.size // 32, dtype=np.uint16)
    lib().gor_quantize_row(ptr(x), x.size, ptr(q), ptr(s))
    return q, s


def normal_fill(seed: int, sigma: float, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib().gor_normal_fill(seed, sigma, ptr(out), count)
    return out


def prompt_ids(seed: int, vocab: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.int32)
    lib().gor_prompt_ids(seed, vocab, count, ptr(out))
    return out


def rotary_table(max_positions: int, head_dim: int, theta: float = 10000.0):
    half = head_dim // 2
    c = np.empty(max_positions * half, dtype=np.float32)
    s = np.empty(max_positions * half, dtype=np.float32)
    lib().gor_rotary_table(max_positions, head_dim, theta, ptr(c), ptr(s))
    return c.reshape(max_positions, half), s.reshape(max_positions, half)


def rmsnorm_row(x, w, eps=1e-6):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    lib().gor_rmsnorm_row(ptr(x), ptr(w), x.size, eps, ptr(out))
    return out


def q8_matvec(xq, xs, weight_bytes, rows, inner):
    out = np.empty(rows, dtype=np.float32)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xs = np.ascontiguousarray(xs, dtype=np.uint16)
    wb = np.ascontiguousarray(weight_bytes, dtype=np.uint8)
    lib().gor_q8_matvec(ptr(xq), ptr(xs), ptr(wb), rows, inner, ptr(out))
    return out


def mqa_row_f16(query, keys_f16, values_f16, heads, kv_heads, head_dim, key_count, scale):
    query = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(keys_f16, dtype=np.uint16)
    v = np.ascontiguousarray(values_f16, dtype=np.uint16)
    out = np.empty(heads * head_dim, dtype=np.float32)
    lib().gor_mqa_row_f16(ptr(query), ptr(k), ptr(v), heads, kv_heads, head_dim, key_count,
                          scale, ptr(out))
    return out


def argmax(logits, mask=None):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32)
    return int(lib().gor_argmax(ptr(logits), ptr(m) if m is not None else None, logits.size))


class Sampler:
    """Sampler (Sampler.h:52-109): options, a seeded std::mt19937_64, one draw
    a sample (Sampler::uniform), the sample restated in C (gor_sample)."""

    def __init__(self, temperature=0.0, top_k=0, top_p=1.0, seed=0):
        self.temperature, self.top_k, self.top_p = temperature, top_k, top_p
        self.engine = (ctypes.c_uint64 * 313)()
        lib().gor_mt64_seed(self.engine, seed)

    def uniform(self) -> float:
        return float(lib().gor_mt64_uniform(self.engine))

    def sample(self, logits, mask=None) -> int:
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32)
        if self.temperature == 0.0:
            return argmax(logits, m)
        return int(lib().gor_sample(ptr(logits), ptr(m) if m is not None else None, logits.size,
                                    self.temperature, self.top_k, self.top_p, self.uniform()))


def uniform_draws(seed: int, count: int) -> np.ndarray:
    """The first `count` Sampler::uniform draws of a seed."""
    engine = (ctypes.c_uint64 * 313)()
    lib().gor_mt64_seed(engine, seed)
    return np.array([lib().gor_mt64_uniform(engine) for _ in range(count)], dtype=np.float64)


# ---- the model ---------------------------------------------------------------
class Model:
    """The oracle decoder (Q8 path or the reference's double path)."""

    def __init__(self, shape: Shape, mode: int = MODE_Q8):
        self.shape = shape
        self._shape_ref = shape
        self.mode = mode
        self.handle = lib().gor_model_create(ctypes.byref(shape), mode)

    def close(self):
        if self.handle:
            lib().gor_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def tensor_count(self) -> int:
        return int(lib().gor_tensor_count(ctypes.byref(self.shape)))

    def tensor_elements(self, index: int) -> int:
        return int(lib().gor_tensor_elements(ctypes.byref(self.shape), index))

    def is_norm(self, index: int) -> bool:
        return bool(lib().gor_tensor_is_norm(ctypes.byref(self.shape), index))

    def set_tensor(self, index: int, values: np.ndarray) -> int:
        values = np.ascontiguousarray(values, dtype=np.float32).ravel()
        return int(lib().gor_model_set_tensor(self.handle, index, ptr(values)))

    def fill_synthetic(self) -> int:
        return int(lib().gor_model_fill_synthetic(self.handle))

    def tensor_bytes(self, index: int) -> np.ndarray:
        p = lib().gor_model_tensor_bytes(self.handle, index)
        n = int(lib().gor_int8_blocks_byte_count(self.tensor_elements(index)))
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint8)), (n,)).copy()

    def begin(self):
        lib().gor_model_begin(self.handle)

    @property
    def position(self) -> int:
        return int(lib().gor_model_position(self.handle))

    def step(self, tokens, want_logits=True, want_hidden=False):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        n = tokens.size
        logits = np.empty((n, self.shape.vocab), dtype=np.float32) if want_logits else None
        hidden = np.empty((n, self.shape.width), dtype=np.float32) if want_hidden else None
        status = int(lib().gor_model_step(self.handle, ptr(tokens), n,
                                          ptr(logits) if logits is not None else None,
                                          ptr(hidden) if hidden is not None else None))
        return status, logits, hidden

    def step_block(self, tokens, logits_rows=1):
        """The Q8 path's step over a block of tokens with the products taken
        over all rows at once: bit-identical to step(), much faster for long
        prompts; (status, logits of the last logits_rows rows or None)."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        logits = (np.empty((logits_rows, self.shape.vocab), dtype=np.float32)
                  if logits_rows > 0 else None)
        status = int(lib().gor_model_step_block(self.handle, ptr(tokens), tokens.size,
                                                ptr(logits) if logits is not None else None,
                                                logits_rows))
        return status, logits

    def debug(self, which: int, layer: int) -> np.ndarray:
        sizes = {DBG_NORMALISED: self.shape.width,
                 DBG_ATTENDED: self.shape.heads * self.shape.head_dim,
                 DBG_ACTIVATED: self.shape.intermediate, DBG_HIDDEN: self.shape.width}
        p = lib().gor_model_debug(self.handle, which, layer)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)),
                                     (sizes[which],)).copy()

    def debug_q(self, which: int, layer: int):
        sizes = {DBG_NORMALISED: self.shape.width,
                 DBG_ATTENDED: self.shape.heads * self.shape.head_dim,
                 DBG_ACTIVATED: self.shape.intermediate, DBG_HIDDEN: self.shape.width}
        n = sizes[which]
        pq = lib().gor_model_debug_q(self.handle, which, layer)
        ps = lib().gor_model_debug_s(self.handle, which, layer)
        q = np.ctypeslib.as_array(ctypes.cast(pq, ctypes.POINTER(ctypes.c_int8)), (n,)).copy()
        s = np.ctypeslib.as_array(ctypes.cast(ps, ctypes.POINTER(ctypes.c_uint16)),
                                  (n // 32,)).copy()
        return q, s

    def generate(self, prompt, max_tokens, eos=1):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        cap = max(1, max_tokens if max_tokens > 0 else self.shape.max_positions)
        out = np.zeros(cap, dtype=np.int32)
        margins = np.zeros(cap, dtype=np.float32)
        count = int(lib().gor_generate(self.handle, ptr(prompt), prompt.size, max_tokens, eos,
                                       ptr(out), ptr(margins)))
        if count < 0:
            return count, None, None
        return count, out[:count].copy(), margins[:count].copy()
