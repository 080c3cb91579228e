"""Python mirror of the reference's decoder interface over libgemma_q8.so.

The shipped compute path is the C ABI in include/gemma_q8.h (gfx950 HIP
kernels plus the C++ decoder runtime).  This module only binds it with ctypes,
with the reference's names: ``DecoderShape`` (Lib/HuggingFaceEACP/Decoder/
DecoderShape.h:42-110), ``Decoder`` (Decoder.h:69-319: prepare, beginSequence,
step, position, hiddenStates) and ``Gemma.generate`` (Generation/Gemma.h:
65-342, greedy).  Device buffers passed to the op-level functions are raw
pointers (torch tensors' ``data_ptr()`` in the tests).

There is no fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(HERE, "libgemma_q8.so")

OK = 0
ERR_ARGUMENT, ERR_SHAPE, ERR_CAPACITY, ERR_WINDOW, ERR_TOKEN = -1, -2, -3, -4, -5
ERR_UNQUANTIZABLE, ERR_NOT_PREPARED, ERR_EMPTY, ERR_DEVICE, ERR_MEMORY = -6, -7, -8, -9, -10
ERR_FORMAT = -11

# safetensors dtype tags (TensorType.h:12-27 order)
DTYPES = ["BOOL", "U8", "I8", "U16", "I16", "F16", "BF16", "U32", "I32", "F32", "U64", "I64",
          "F64"]

# GemmaTensors::all order (GemmaTensors.cpp:30-57)
T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN, T_INPUT_NORM, T_POST_NORM = range(9)
PER_LAYER = 9


# stage indices of gq8_decoder_timing
STAGES = ["embed", "norm", "qkv", "rope_kv", "attention", "o_proj", "gate_up", "geglu",
          "down", "lm_head", "argmax"]


class Gq8Error(RuntimeError):
    """A refusal or failure reported by libgemma_q8 (the reference's ModelError)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status


class _Shape(ctypes.Structure):
    _fields_ = [
        ("width", ctypes.c_int), ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int), ("layers", ctypes.c_int), ("intermediate", ctypes.c_int),
        ("vocab", ctypes.c_int), ("max_positions", ctypes.c_int),
        ("max_step_rows", ctypes.c_int), ("rms_epsilon", ctypes.c_float),
        ("rope_theta", ctypes.c_double), ("embedding_scale", ctypes.c_float),
    ]


class _TokenIds(ctypes.Structure):
    _fields_ = [("bos", ctypes.c_int), ("eos", ctypes.c_int), ("pad", ctypes.c_int)]


class _Sampling(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int),
                ("top_p", ctypes.c_float), ("seed", ctypes.c_uint64)]


@dataclass(frozen=True)
class SamplingOptions:
    """SamplingOptions (Sampling/Sampler.h:33-51): temperature 0 is the argmax,
    top_k 0 and top_p 1 switch their cut off."""
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    seed: int = 0

    @staticmethod
    def greedy() -> "SamplingOptions":
        return SamplingOptions(temperature=0.0)

    def as_c(self) -> _Sampling:
        return _Sampling(self.temperature, self.top_k, self.top_p, self.seed)


class _RunStats(ctypes.Structure):
    _fields_ = [("prefill_seconds", ctypes.c_double), ("decode_seconds", ctypes.c_double),
                ("step_count", ctypes.c_int), ("generated", ctypes.c_int)]


_lib = None

# gq8_token_callback: void (*)(int32_t token, void *user)
TOKEN_CALLBACK = ctypes.CFUNCTYPE(None, ctypes.c_int32, ctypes.c_void_p)


def library() -> ctypes.CDLL:
    """Load libgemma_q8.so (built in-tree); raise if it is not there."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY_PATH):
        raise RuntimeError(f"{LIBRARY_PATH} is not built: run `python -m huggingfaceeacp_amd.build`"
                           " (the HIP path has no fallback)")
    L = ctypes.CDLL(LIBRARY_PATH)
    P, i32, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    f32, f64 = ctypes.c_float, ctypes.c_double
    sig = {
        "gq8_status_string": (ctypes.c_char_p, [i32]),
        "gq8_last_error": (ctypes.c_char_p, []),
        "gq8_version": (ctypes.c_char_p, []),
        "gq8_int8_block_count": (i64, [i64]),
        "gq8_int8_blocks_byte_count": (i64, [i64]),
        "gq8_quantizes_as_int8_blocks": (i32, [i64, i64]),
        "gq8_quantize_int8_blocks_host": (i32, [P, i64, i64, i64, P]),
        "gq8_dequantize_int8_blocks_host": (i32, [P, i64, P]),
        "gq8_rotary_table_host": (i32, [i32, i32, f64, P, P]),
        "gq8_quantize_rows": (i32, [P, i64, i64, P, P]),
        "gq8_embed": (i32, [P, i32, P, i32, i32, f32, P, P]),
        "gq8_rmsnorm": (i32, [P, P, i32, i32, f32, P, P, P]),
        "gq8_rope": (i32, [P, i32, i32, i32, i32, i32, P, P, P]),
        "gq8_q8_product": (i32, [P, P, i32, i32, i32, P, i32, i32, P]),
        "gq8_kv_store_f16": (i32, [P, P, i32, i32, i32, P, P, i32, P]),
        "gq8_mqa_workspace_bytes": (sz, [i32, i32, i32, i32]),
        "gq8_mqa_decode": (i32, [P, P, P, i32, i32, i32, i32, f32, P, P, sz, P]),
        "gq8_mqa_decode_noalloc_limit_bytes": (sz, []),
        "gq8_mqa_decode_noalloc": (i32, [P, P, P, i32, i32, i32, i32, f32, P, P]),
        "gq8_mqa_prefill": (i32, [P, P, P, i32, i32, i32, i32, i32, f32, P, P, sz, P]),
        "gq8_geglu": (i32, [P, i32, i32, P, P, P]),
        "gq8_argmax_workspace_bytes": (sz, [i32, i32]),
        "gq8_argmax_rows": (i32, [P, P, i32, i32, P, P, sz, P]),
        "gq8_shape_validate": (i32, [P]),
        "gq8_gemma_2b_shape": (_Shape, [i32, i32, i32]),
        "gq8_decoder_create": (i32, [P, ctypes.POINTER(P)]),
        "gq8_decoder_destroy": (None, [P]),
        "gq8_tensor_count": (i32, [P]),
        "gq8_tensor_elements": (i64, [P, i32]),
        "gq8_tensor_is_norm": (i32, [P, i32]),
        "gq8_decoder_load_tensor": (i32, [P, i32, P]),
        "gq8_decoder_load_tensor_q8": (i32, [P, i32, P]),
        "gq8_decoder_fill_synthetic": (i32, [P, i32]),
        "gq8_decoder_read_tensor": (i32, [P, i32, P, sz]),
        "gq8_decoder_begin_sequence": (i32, [P]),
        "gq8_decoder_position": (i32, [P]),
        "gq8_decoder_device_position": (i32, [P]),
        "gq8_decoder_step": (i32, [P, P, i32, P, i32]),
        "gq8_decoder_hidden": (i32, [P, P, i32]),
        "gq8_decoder_set_debug": (i32, [P, i32]),
        "gq8_decoder_set_fused": (i32, [P, i32]),
        "gq8_decoder_attention_path": (i32, [P]),
        "gq8_decode_attention_fits": (i32, [P, i32]),
        "gq8_decoder_inject_wait_failure": (i32, [P]),
        "gq8_decoder_debug": (i32, [P, i32, i32, P, P]),
        "gq8_generate": (i32, [P, P, i32, i32, i32, i32, P, ctypes.POINTER(_RunStats)]),
        "gq8_decoder_decode": (i32, [P, i32, i32]),
        "gq8_prompt_ids": (i32, [ctypes.c_uint64, i32, i32, P]),
        "gq8_normal_fill_host": (i32, [ctypes.c_uint64, f64, P, i64]),
        "gq8_decoder_tokens": (i32, [P, i32, i32, P]),
        "gq8_decoder_set_timing": (i32, [P, i32]),
        "gq8_decoder_timing": (i32, [P, P, P]),
        "gq8_decoder_time_kernel": (i32, [P, i32, i32, ctypes.POINTER(f64), ctypes.POINTER(i32)]),
        "gq8_safetensors_open": (i32, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "gq8_safetensors_from_bytes": (i32, [P, ctypes.c_uint64, ctypes.POINTER(P)]),
        "gq8_safetensors_close": (None, [P]),
        "gq8_safetensors_count": (i32, [P]),
        "gq8_safetensors_find": (i32, [P, ctypes.c_char_p]),
        "gq8_safetensors_info": (i32, [P, i32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(i32),
                                       ctypes.POINTER(i32), P, i32, ctypes.POINTER(ctypes.c_uint64)]),
        "gq8_safetensors_read_floats": (i32, [P, i32, i64, i64, P]),
        "gq8_safetensors_raw": (ctypes.c_void_p, [P, i32]),
        "gq8_safetensors_metadata_count": (i32, [P]),
        "gq8_safetensors_metadata": (i32, [P, i32, ctypes.POINTER(ctypes.c_char_p),
                                           ctypes.POINTER(ctypes.c_char_p)]),
        "gq8_gemma_config_parse": (i32, [ctypes.c_char_p, sz, i32, i32, ctypes.POINTER(_Shape),
                                         ctypes.POINTER(_TokenIds)]),
        "gq8_decoder_load_safetensors": (i32, [P, P, i32]),
        "gq8_batch_create": (i32, [P, i32, ctypes.POINTER(P)]),
        "gq8_batch_destroy": (None, [P]),
        "gq8_batch_prefill": (i32, [P, i32, P, i32]),
        "gq8_batch_decode": (i32, [P, i32, i32]),
        "gq8_batch_sequences": (i32, [P]),
        "gq8_batch_position": (i32, [P, i32]),
        "gq8_batch_tokens": (i32, [P, i32, i32, i32, P]),
        "gq8_batch_logits": (i32, [P, P]),
        "gq8_sample_workspace_bytes": (sz, [i32]),
        "gq8_sample_row": (i32, [P, P, i32, P, f64, P, P, sz, P]),
        "gq8_decoder_set_sampling": (i32, [P, P]),
        "gq8_tokenizer_from_json": (i32, [ctypes.c_char_p, sz, ctypes.POINTER(P)]),
        "gq8_tokenizer_open": (i32, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "gq8_tokenizer_destroy": (None, [P]),
        "gq8_tokenizer_encode": (i32, [P, ctypes.c_char_p, sz, i32, P, i32]),
        "gq8_tokenizer_decode": (i32, [P, P, i32, i32, P, sz, ctypes.POINTER(sz)]),
        "gq8_tokenizer_vocabulary_size": (i32, [P]),
        "gq8_tokenizer_specials": (i32, [P, P]),
        "gq8_tokenizer_is_special": (i32, [P, i32]),
        "gq8_tokenizer_token_text": (i32, [P, i32, P, sz, ctypes.POINTER(sz)]),
        "gq8_tokenizer_token_for_text": (ctypes.c_int32, [P, ctypes.c_char_p, sz]),
        "gq8_tokenizer_metaspace": (i32, [P, P, sz, ctypes.POINTER(sz), ctypes.POINTER(i32),
                                          ctypes.POINTER(i32)]),
        "gq8_generate_streaming": (i32, [P, P, i32, i32, i32, i32, P, ctypes.POINTER(_RunStats),
                                         TOKEN_CALLBACK, P]),
        "gq8_gemma_create": (i32, [ctypes.POINTER(P)]),
        "gq8_gemma_destroy": (None, [P]),
        "gq8_gemma_load": (i32, [P, ctypes.c_char_p]),
        "gq8_gemma_directory_from_environment": (i32, [P, sz, ctypes.POINTER(sz)]),
        "gq8_gemma_is_loaded": (i32, [P]),
        "gq8_gemma_is_prepared": (i32, [P]),
        "gq8_gemma_file": (i32, [P, i32, i32, P, sz, ctypes.POINTER(sz)]),
        "gq8_gemma_shard_count": (i32, [P]),
        "gq8_gemma_config": (i32, [P, ctypes.POINTER(_Shape), ctypes.POINTER(_TokenIds)]),
        "gq8_gemma_set_maximum_tokens": (i32, [P, i32]),
        "gq8_gemma_maximum_tokens": (i32, [P]),
        "gq8_gemma_set_prompt_capacity": (i32, [P, i32]),
        "gq8_gemma_prompt_capacity": (i32, [P]),
        "gq8_gemma_set_sampling": (i32, [P, P]),
        "gq8_gemma_set_on_token": (i32, [P, TOKEN_CALLBACK, P]),
        "gq8_gemma_prepare": (i32, [P]),
        "gq8_gemma_decoder": (P, [P]),
        "gq8_gemma_tokenizer": (P, [P]),
        "gq8_gemma_generate": (i32, [P, P, i32, P, i32]),
        "gq8_gemma_generate_from_text": (i32, [P, ctypes.c_char_p, sz, P, i32]),
        "gq8_gemma_generate_text": (i32, [P, ctypes.c_char_p, sz, P, sz, ctypes.POINTER(sz)]),
        "gq8_gemma_text_for_tokens": (i32, [P, P, i32, P, sz, ctypes.POINTER(sz)]),
        "gq8_gemma_last_stats": (i32, [P, ctypes.POINTER(_RunStats)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(status: int) -> int:
    """Raise Gq8Error for a negative status, return it otherwise."""
    if status < 0:
        msg = library().gq8_last_error().decode(errors="replace")
        raise Gq8Error(status, msg or library().gq8_status_string(status).decode())
    return status


def _host(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


# ---- op-level entry points (device pointers as ints) --------------------------
def quantize_rows(x, rows, inner, q8, stream=0):
    return check(library().gq8_quantize_rows(x, rows, inner, q8, stream))


def embed(tokens, rows, table, vocab, width, scale, out, stream=0):
    return check(library().gq8_embed(tokens, rows, table, vocab, width, scale, out, stream))


def rmsnorm(x, weight, rows, width, epsilon, y, q8, stream=0):
    return check(library().gq8_rmsnorm(x, weight, rows, width, epsilon, y, q8, stream))


def rope(x, row_stride, heads, head_dim, first_position, rows, cosines, sines, stream=0):
    return check(library().gq8_rope(x, row_stride, heads, head_dim, first_position, rows,
                                    cosines, sines, stream))


def q8_product(x8, w8, rows, inner, outputs, y, y_stride, residual=False, stream=0):
    return check(library().gq8_q8_product(x8, w8, rows, inner, outputs, y, y_stride,
                                          int(residual), stream))


def kv_store_f16(k, v, src_stride, rows, kv_width, key_cache, value_cache, position, stream=0):
    return check(library().gq8_kv_store_f16(k, v, src_stride, rows, kv_width, key_cache,
                                            value_cache, position, stream))


def mqa_workspace_bytes(rows, heads, head_dim, max_keys):
    return int(library().gq8_mqa_workspace_bytes(rows, heads, head_dim, max_keys))


def mqa_decode(query, keys, values, heads, kv_heads, head_dim, key_count, scale, out,
               workspace, workspace_bytes, stream=0):
    return check(library().gq8_mqa_decode(query, keys, values, heads, kv_heads, head_dim,
                                          key_count, scale, out, workspace, workspace_bytes,
                                          stream))


def mqa_decode_noalloc_limit_bytes():
    return int(library().gq8_mqa_decode_noalloc_limit_bytes())


def mqa_decode_noalloc(query, keys, values, heads, kv_heads, head_dim, key_count, scale, out,
                       stream=0):
    """mqa_decode with its split partials in the library's static device
    array: no workspace argument, no allocation."""
    return check(library().gq8_mqa_decode_noalloc(query, keys, values, heads, kv_heads,
                                                  head_dim, key_count, scale, out, stream))


def mqa_prefill(queries, keys, values, heads, kv_heads, head_dim, rows, position_offset, scale,
                out, workspace, workspace_bytes, stream=0):
    return check(library().gq8_mqa_prefill(queries, keys, values, heads, kv_heads, head_dim,
                                           rows, position_offset, scale, out, workspace,
                                           workspace_bytes, stream))


def geglu(fused, rows, intermediate, out, q8, stream=0):
    return check(library().gq8_geglu(fused, rows, intermediate, out, q8, stream))


def argmax_workspace_bytes(rows, length):
    return int(library().gq8_argmax_workspace_bytes(rows, length))


def argmax_rows(logits, mask, rows, length, indices, workspace, workspace_bytes, stream=0):
    return check(library().gq8_argmax_rows(logits, mask, rows, length, indices, workspace,
                                           workspace_bytes, stream))


def sample_workspace_bytes(vocab):
    return int(library().gq8_sample_workspace_bytes(vocab))


def sample_row(logits, mask, vocab, options: SamplingOptions, uniform, token, workspace,
               workspace_bytes, stream=0):
    """Sampler::sample of one device row of logits; the id goes to *token."""
    c = options.as_c()
    return check(library().gq8_sample_row(logits, mask, vocab, ctypes.byref(c), float(uniform),
                                          token, workspace, workspace_bytes, stream))


# ---- host format helpers ---------------------------------------------------------
def quantize_int8_blocks_host(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32).ravel()
    n = values.size
    out = np.zeros(int(library().gq8_int8_blocks_byte_count(n)), dtype=np.uint8)
    check(library().gq8_quantize_int8_blocks_host(_host(values), n, 0, n, _host(out)))
    return out


def dequantize_int8_blocks_host(stored: np.ndarray, element_count: int) -> np.ndarray:
    stored = np.ascontiguousarray(stored, dtype=np.uint8)
    out = np.zeros(element_count, dtype=np.float32)
    check(library().gq8_dequantize_int8_blocks_host(_host(stored), element_count, _host(out)))
    return out


def rotary_table_host(max_positions: int, head_dim: int, theta: float = 10000.0):
    half = head_dim // 2
    c = np.empty(max_positions * half, dtype=np.float32)
    s = np.empty(max_positions * half, dtype=np.float32)
    check(library().gq8_rotary_table_host(max_positions, head_dim, theta, _host(c), _host(s)))
    return c.reshape(max_positions, half), s.reshape(max_positions, half)


# ---- the decoder ----------------------------------------------------------------------
@dataclass
class DecoderShape:
    """DecoderShape (DecoderShape.h:42-110)."""
    width: int
    heads: int
    kv_heads: int
    head_dim: int
    layers: int
    intermediate: int
    vocab: int
    max_positions: int
    max_step_rows: int = 0
    rms_epsilon: float = 1e-6
    rope_theta: float = 10000.0
    embedding_scale: float | None = None

    def __post_init__(self):
        if self.embedding_scale is None:  # sqrtf(hidden_size), GemmaConfig.cpp:123-126
            self.embedding_scale = float(np.sqrt(np.float32(self.width), dtype=np.float32))

    @staticmethod
    def gemma_2b(layers: int = 18, max_positions: int = 8192, max_step_rows: int = 512):
        return DecoderShape(2048, 8, 1, 256, layers, 16384, 256000, max_positions, max_step_rows)

    @property
    def query_width(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim

    def step_capacity(self) -> int:
        return self.max_step_rows if self.max_step_rows > 0 else self.max_positions

    def attention_scale(self) -> float:
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_dim), dtype=np.float32))

    def as_c(self) -> _Shape:
        return _Shape(self.width, self.heads, self.kv_heads, self.head_dim, self.layers,
                      self.intermediate, self.vocab, self.max_positions, self.max_step_rows,
                      self.rms_epsilon, self.rope_theta, self.embedding_scale)

    def validate(self) -> None:
        c = self.as_c()
        check(library().gq8_shape_validate(ctypes.byref(c)))

    def tensor_count(self) -> int:
        c = self.as_c()
        return int(library().gq8_tensor_count(ctypes.byref(c)))

    def tensor_elements(self, index: int) -> int:
        c = self.as_c()
        return int(library().gq8_tensor_elements(ctypes.byref(c), index))

    def tensor_is_norm(self, index: int) -> bool:
        c = self.as_c()
        return bool(library().gq8_tensor_is_norm(ctypes.byref(c), index))

    def attention_fits(self, resident_workgroups: int) -> bool:
        """Whether one-token steps of this shape take the split attention kernel
        when `resident_workgroups` of its workgroups fit on the device at once."""
        c = self.as_c()
        status = int(library().gq8_decode_attention_fits(ctypes.byref(c), resident_workgroups))
        if status < 0:
            check(status)
        return status == 1


@dataclass
class RunStats:
    prefill_seconds: float
    decode_seconds: float
    step_count: int
    generated: int


class Decoder:
    """HF::Decoder over libgemma_q8: one sequence, fp16 KV caches on the device."""

    def __init__(self, shape: DecoderShape):
        self.shape = shape
        self._c_shape = shape.as_c()
        handle = ctypes.c_void_p()
        check(library().gq8_decoder_create(ctypes.byref(self._c_shape), ctypes.byref(handle)))
        self.handle = handle

    def close(self) -> None:
        if self.handle:
            library().gq8_decoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # TensorLoader counterparts
    def load_tensor(self, index: int, values: np.ndarray) -> None:
        values = np.ascontiguousarray(values, dtype=np.float32).ravel()
        if values.size != self.shape.tensor_elements(index):
            raise ValueError("tensor size does not match the shape")
        check(library().gq8_decoder_load_tensor(self.handle, index, _host(values)))

    def load_tensor_q8(self, index: int, stored: np.ndarray) -> None:
        stored = np.ascontiguousarray(stored, dtype=np.uint8).ravel()
        check(library().gq8_decoder_load_tensor_q8(self.handle, index, _host(stored)))

    def fill_synthetic(self, threads: int = 0) -> None:
        check(library().gq8_decoder_fill_synthetic(self.handle, threads))

    def read_tensor(self, index: int) -> np.ndarray:
        n = self.shape.tensor_elements(index)
        if self.shape.tensor_is_norm(index):
            out = np.empty(n, dtype=np.float32)
        else:
            out = np.empty(int(library().gq8_int8_blocks_byte_count(n)), dtype=np.uint8)
        check(library().gq8_decoder_read_tensor(self.handle, index, _host(out), out.nbytes))
        return out

    # Decoder API
    def begin_sequence(self) -> None:
        check(library().gq8_decoder_begin_sequence(self.handle))

    @property
    def position(self) -> int:
        return int(library().gq8_decoder_position(self.handle))

    @property
    def device_position(self) -> int:
        """The position word on the device, once the decoder's stream is idle."""
        value = int(library().gq8_decoder_device_position(self.handle))
        if value < 0:
            check(value)
        return value

    def step(self, tokens_ptr: int, n: int, logits_ptr: int | None, logits_rows: int | None = None):
        rows = n if logits_rows is None else logits_rows
        check(library().gq8_decoder_step(self.handle, tokens_ptr, n, logits_ptr or None,
                                         rows if logits_ptr else 0))

    def hidden_states(self, rows: int) -> np.ndarray:
        out = np.empty((rows, self.shape.width), dtype=np.float32)
        check(library().gq8_decoder_hidden(self.handle, _host(out), rows))
        return out

    @property
    def attention_path(self) -> int:
        """1: the split attention kernel; 0: the partial/merge pair; -1: no fused step."""
        return int(library().gq8_decoder_attention_path(self.handle))

    def inject_wait_failure(self) -> None:
        """Sets the split attention's error word: the next step's bounded waits
        give up, and its check reports ERR_DEVICE and undoes the step."""
        check(library().gq8_decoder_inject_wait_failure(self.handle))

    def set_sampling(self, options: SamplingOptions) -> None:
        """Gemma::setSampling: how generate and decode choose each id (on the device)."""
        c = options.as_c()
        check(library().gq8_decoder_set_sampling(self.handle, ctypes.byref(c)))

    def set_fused(self, enabled: bool) -> None:
        """Choose the fused one-token kernels (default) or the unfused ones."""
        check(library().gq8_decoder_set_fused(self.handle, int(enabled)))

    def set_debug(self, enabled: bool) -> None:
        check(library().gq8_decoder_set_debug(self.handle, int(enabled)))

    def debug(self, which: int, layer: int):
        inner = {0: self.shape.width, 1: self.shape.query_width, 2: self.shape.intermediate,
                 3: self.shape.width}[which]
        values = np.empty(inner, dtype=np.float32)
        q8 = np.empty(inner + inner // 16, dtype=np.uint8)
        check(library().gq8_decoder_debug(self.handle, which, layer, _host(values), _host(q8)))
        return values, q8

    def load_safetensors(self, shards) -> None:
        """Every catalogue tensor from the checkpoint's shards, by its
        checkpoint name, checked against the shape before any upload
        (TensorLoader.cpp:186-347)."""
        handles = (ctypes.c_void_p * len(shards))(*[f.handle for f in shards])
        check(library().gq8_decoder_load_safetensors(self.handle, handles, len(shards)))

    def decode(self, steps: int, use_graph: bool = True) -> None:
        """Continue the greedy loop `steps` tokens (on-device token feedback)."""
        check(library().gq8_decoder_decode(self.handle, steps, int(use_graph)))

    def tokens(self, first: int, count: int) -> np.ndarray:
        """The sequence slots [first, first + count) (prompt ids, then chosen ids)."""
        out = np.empty(count, dtype=np.int32)
        check(library().gq8_decoder_tokens(self.handle, first, count, _host(out)))
        return out

    def set_timing(self, enabled, stages=None) -> None:
        """Bracket the launches of `stages` (names from STAGES; default all)
        with HIP events while enabled."""
        mask = 0
        if enabled:
            for name in (STAGES if stages is None else stages):
                mask |= 1 << STAGES.index(name)
        check(library().gq8_decoder_set_timing(self.handle, mask))

    def time_kernel(self, stage: str, repeats: int):
        """(milliseconds, launches) of one fused kernel ("gate_up", "down" or
        "lm_head") launched alone over every layer's weights, `repeats` rounds."""
        ms = ctypes.c_double(0.0)
        launches = ctypes.c_int(0)
        check(library().gq8_decoder_time_kernel(self.handle, STAGES.index(stage), int(repeats),
                                                ctypes.byref(ms), ctypes.byref(launches)))
        return ms.value, launches.value

    def timing(self) -> dict:
        """{stage: (total milliseconds, launches)} since the last call."""
        ms = np.zeros(len(STAGES), dtype=np.float64)
        launches = np.zeros(len(STAGES), dtype=np.int32)
        check(library().gq8_decoder_timing(self.handle, _host(ms), _host(launches)))
        return {name: (float(ms[i]), int(launches[i])) for i, name in enumerate(STAGES)}

    # Gemma::generate, greedy
    def generate(self, prompt, max_tokens: int, eos: int = 1, use_graph: bool = True):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        window = self.shape.max_positions - prompt.size
        cap = max(1, min(max_tokens, window) if max_tokens > 0 else window)
        out = np.zeros(cap, dtype=np.int32)
        stats = _RunStats()
        count = check(library().gq8_generate(self.handle, _host(prompt), prompt.size, max_tokens,
                                             eos, int(use_graph), _host(out),
                                             ctypes.byref(stats)))
        return out[:count].copy(), RunStats(stats.prefill_seconds, stats.decode_seconds,
                                            stats.step_count, stats.generated)


class SafeTensors:
    """SafeTensors (SafeTensors.h:78-183) over libgemma_q8: a mapped (open) or
    copied (from_bytes) safetensors file whose header was checked whole."""

    def __init__(self, handle):
        self.handle = handle

    @staticmethod
    def open(path) -> "SafeTensors":
        handle = ctypes.c_void_p()
        check(library().gq8_safetensors_open(os.fsencode(path), ctypes.byref(handle)))
        return SafeTensors(handle)

    @staticmethod
    def from_bytes(data: bytes) -> "SafeTensors":
        buf = np.frombuffer(bytes(data), dtype=np.uint8)
        handle = ctypes.c_void_p()
        check(library().gq8_safetensors_from_bytes(buf.ctypes.data if buf.size else None,
                                                    buf.size, ctypes.byref(handle)))
        return SafeTensors(handle)

    def close(self) -> None:
        if self.handle:
            library().gq8_safetensors_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _index(self, name: str) -> int:
        return check(library().gq8_safetensors_find(self.handle, name.encode()))

    def names(self) -> list[str]:
        return [self._info(i)[0] for i in range(check(library().gq8_safetensors_count(self.handle)))]

    def _info(self, index: int):
        name = ctypes.c_char_p()
        dtype, rank = ctypes.c_int(), ctypes.c_int()
        shape = np.zeros(16, dtype=np.int64)
        nbytes = ctypes.c_uint64()
        check(library().gq8_safetensors_info(self.handle, index, ctypes.byref(name),
                                             ctypes.byref(dtype), ctypes.byref(rank),
                                             shape.ctypes.data, shape.size, ctypes.byref(nbytes)))
        return (name.value.decode(), DTYPES[dtype.value], tuple(int(d) for d in shape[:rank.value]),
                int(nbytes.value))

    def contains(self, name: str) -> bool:
        return name in self.names()

    def info(self, name: str):
        """(dtype, shape, byte count) of a tensor; Gq8Error if there is none."""
        return self._info(self._index(name))[1:]

    def read_floats(self, name: str, first: int = 0, count: int | None = None) -> np.ndarray:
        index = self._index(name)
        elements = int(np.prod(self._info(index)[2], dtype=np.int64))
        count = elements - first if count is None else count
        out = np.empty(max(count, 0), dtype=np.float32)
        check(library().gq8_safetensors_read_floats(self.handle, index, first, count,
                                                    out.ctypes.data if out.size else None))
        return out

    def raw(self, name: str) -> bytes:
        index = self._index(name)
        nbytes = self._info(index)[3]
        ptr = library().gq8_safetensors_raw(self.handle, index)
        return ctypes.string_at(ptr, nbytes) if nbytes else b""

    def metadata(self) -> dict:
        out = {}
        for i in range(check(library().gq8_safetensors_metadata_count(self.handle))):
            k, v = ctypes.c_char_p(), ctypes.c_char_p()
            check(library().gq8_safetensors_metadata(self.handle, i, ctypes.byref(k),
                                                     ctypes.byref(v)))
            out[k.value.decode()] = v.value.decode()
        return out


def gemma_config(text: str, max_positions: int = 0, max_step_rows: int = 0):
    """GemmaConfig::fromJson + DecoderShape::fromConfig: (DecoderShape, (bos, eos, pad))."""
    raw = text.encode()
    c = _Shape()
    ids = _TokenIds()
    check(library().gq8_gemma_config_parse(raw, len(raw), max_positions, max_step_rows,
                                           ctypes.byref(c), ctypes.byref(ids)))
    shape = DecoderShape(c.width, c.heads, c.kv_heads, c.head_dim, c.layers, c.intermediate,
                         c.vocab, c.max_positions, c.max_step_rows, c.rms_epsilon, c.rope_theta,
                         c.embedding_scale)
    return shape, (ids.bos, ids.eos, ids.pad)


class Batch:
    """Up to 16 independent sequences decoded in lockstep over one Decoder's
    weights: S separate greedy loops (Gemma.cpp:459-543) in one step a token.
    The decoder must stay open while the batch is."""

    def __init__(self, decoder: Decoder, sequences: int):
        self.decoder = decoder
        handle = ctypes.c_void_p()
        check(library().gq8_batch_create(decoder.handle, sequences, ctypes.byref(handle)))
        self.handle = handle
        self.sequences = sequences

    def close(self) -> None:
        if self.handle:
            library().gq8_batch_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prefill(self, sequence: int, prompt) -> None:
        """Restart one sequence with `prompt`; its first chosen id fills slot len(prompt)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        check(library().gq8_batch_prefill(self.handle, sequence, _host(prompt), prompt.size))

    def decode(self, steps: int, use_graph: bool = True) -> None:
        """`steps` lockstep steps (every sequence one token a step, no EOS check)."""
        check(library().gq8_batch_decode(self.handle, steps, int(use_graph)))

    def position(self, sequence: int) -> int:
        return check(library().gq8_batch_position(self.handle, sequence))

    def tokens(self, sequence: int, first: int, count: int) -> np.ndarray:
        out = np.empty(count, dtype=np.int32)
        check(library().gq8_batch_tokens(self.handle, sequence, first, count, _host(out)))
        return out

    def logits(self) -> np.ndarray:
        """The last lockstep step's logits, [sequences, vocab]."""
        out = np.empty((self.sequences, self.decoder.shape.vocab), dtype=np.float32)
        check(library().gq8_batch_logits(self.handle, _host(out)))
        return out


def normal_fill_host(seed: int, sigma: float, count: int) -> np.ndarray:
    """The synthetic-weight generator for one tensor (host threads)."""
    out = np.empty(count, dtype=np.float32)
    check(library().gq8_normal_fill_host(seed, sigma, _host(out), count))
    return out


def prompt_ids(seed: int, vocab: int, count: int) -> np.ndarray:
    """Seeded uniform prompt ids (std::mt19937_64(seed), next() % vocab)."""
    out = np.empty(count, dtype=np.int32)
    check(library().gq8_prompt_ids(seed, vocab, count, _host(out)))
    return out


def version() -> str:
    return library().gq8_version().decode()


def exported_symbols() -> list[str]:
    """Every function include/gemma_q8.h declares (parsed from the header)."""
    import re
    header = os.path.join(os.path.dirname(HERE), "include", "gemma_q8.h")
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gq8_[a-z0-9_]+)\s*\(", text)))


def algorithmic_decode_bytes(shape: DecoderShape, attended_length: int) -> int:
    """Bytes one decode token must move: the Q8 weights (tied lm_head once),
    the fp32 norm vectors, one embedding row, the fp16 K+V read over
    attended_length positions and the token's own K+V write."""
    w = shape.width
    weights = shape.tensor_elements(0)
    for i in range(1, shape.tensor_count()):
        if not shape.tensor_is_norm(i):
            weights += shape.tensor_elements(i)
    q8 = weights + weights // 16
    norms = (2 * shape.layers + 1) * w * 4
    embed_row = w + w // 16
    kv_row = shape.layers * 2 * shape.kv_width * 2
    return q8 + norms + embed_row + kv_row * attended_length + kv_row


def algorithmic_batch_step_bytes(shape: DecoderShape, attended_lengths) -> int:
    """Bytes one lockstep step must move: the weights and norms once, and per
    sequence its embedding row, its K+V read over its attended length and
    its own K+V write."""
    w = shape.width
    embed_row = w + w // 16
    kv_row = shape.layers * 2 * shape.kv_width * 2
    shared = algorithmic_decode_bytes(shape, 0) - embed_row - kv_row
    return shared + sum(embed_row + kv_row * L + kv_row for L in attended_lengths)


def log2ceil(n: int) -> int:
    return int(math.ceil(math.log2(n))) if n > 1 else 0


# ---- the tokenizer ----------------------------------------------------------------
class _SpecialTokens(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int32) for name in
                ("pad", "eos", "bos", "unk", "start_of_turn", "end_of_turn")]


@dataclass(frozen=True)
class SpecialTokens:
    """SpecialTokens (Tokenizer/SpecialTokens.h:16-24); -1 where the file has none."""
    pad: int
    eos: int
    bos: int
    unk: int
    start_of_turn: int
    end_of_turn: int


@dataclass(frozen=True)
class Metaspace:
    replacement: str
    prepends_dummy_prefix: bool
    splits_before_replacement: bool


INVALID_TOKEN = -1


class Tokenizer:
    """HF::Tokenizer (Tokenizer/Tokenizer.h:35-124) over libgemma_q8: Gemma's
    SentencePiece BPE read from tokenizer.json.  Text is UTF-8 (str or bytes)."""

    def __init__(self, handle):
        self.handle = handle

    @staticmethod
    def from_json_text(text) -> "Tokenizer":
        raw = text.encode() if isinstance(text, str) else bytes(text)
        handle = ctypes.c_void_p()
        check(library().gq8_tokenizer_from_json(raw, len(raw), ctypes.byref(handle)))
        return Tokenizer(handle)

    @staticmethod
    def from_file(path) -> "Tokenizer":
        handle = ctypes.c_void_p()
        check(library().gq8_tokenizer_open(os.fsencode(path), ctypes.byref(handle)))
        return Tokenizer(handle)

    def close(self) -> None:
        if self.handle:
            library().gq8_tokenizer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _encode(self, text, with_bos) -> list[int]:
        raw = text.encode() if isinstance(text, str) else bytes(text)
        capacity = len(raw) + 2
        out = (ctypes.c_int32 * capacity)()
        count = check(library().gq8_tokenizer_encode(self.handle, raw, len(raw), int(with_bos),
                                                     out, capacity))
        if count > capacity:
            out = (ctypes.c_int32 * count)()
            check(library().gq8_tokenizer_encode(self.handle, raw, len(raw), int(with_bos), out,
                                                 count))
        return list(out[:count])

    def encode(self, text) -> list[int]:
        return self._encode(text, False)

    def encode_with_bos(self, text) -> list[int]:
        return self._encode(text, True)

    def _decode(self, tokens, keep_special) -> bytes:
        ids = (ctypes.c_int32 * max(1, len(tokens)))(*[int(t) for t in tokens])
        length = ctypes.c_size_t()
        check(library().gq8_tokenizer_decode(self.handle, ids, len(tokens), int(keep_special),
                                             None, 0, ctypes.byref(length)))
        out = ctypes.create_string_buffer(max(1, length.value))
        check(library().gq8_tokenizer_decode(self.handle, ids, len(tokens), int(keep_special), out,
                                             length.value, ctypes.byref(length)))
        return out.raw[:length.value]

    def decode_bytes(self, tokens) -> bytes:
        return self._decode(tokens, False)

    def decode(self, tokens) -> str:
        return self._decode(tokens, False).decode("utf-8")

    def decode_keeping_special_tokens(self, tokens) -> str:
        return self._decode(tokens, True).decode("utf-8")

    def vocabulary_size(self) -> int:
        return check(library().gq8_tokenizer_vocabulary_size(self.handle))

    def specials(self) -> SpecialTokens:
        s = _SpecialTokens()
        check(library().gq8_tokenizer_specials(self.handle, ctypes.byref(s)))
        return SpecialTokens(s.pad, s.eos, s.bos, s.unk, s.start_of_turn, s.end_of_turn)

    @property
    def bos(self) -> int:
        return self.specials().bos

    @property
    def eos(self) -> int:
        return self.specials().eos

    @property
    def pad(self) -> int:
        return self.specials().pad

    @property
    def unk(self) -> int:
        return self.specials().unk

    def is_special(self, token: int) -> bool:
        return bool(library().gq8_tokenizer_is_special(self.handle, int(token)))

    def text_for_token(self, token: int) -> str:
        length = ctypes.c_size_t()
        check(library().gq8_tokenizer_token_text(self.handle, int(token), None, 0,
                                                 ctypes.byref(length)))
        out = ctypes.create_string_buffer(max(1, length.value))
        check(library().gq8_tokenizer_token_text(self.handle, int(token), out, length.value,
                                                 ctypes.byref(length)))
        return out.raw[:length.value].decode("utf-8", errors="surrogateescape")

    def token_for_text(self, text) -> int:
        raw = text.encode() if isinstance(text, str) else bytes(text)
        return int(library().gq8_tokenizer_token_for_text(self.handle, raw, len(raw)))

    def metaspace(self) -> Metaspace:
        length, prepends, splits = ctypes.c_size_t(), ctypes.c_int(), ctypes.c_int()
        out = ctypes.create_string_buffer(64)
        check(library().gq8_tokenizer_metaspace(self.handle, out, 64, ctypes.byref(length),
                                                ctypes.byref(prepends), ctypes.byref(splits)))
        return Metaspace(out.raw[:length.value].decode("utf-8"), bool(prepends.value),
                         bool(splits.value))


# ModelFiles' files (Model/ModelFiles.h:13-27), in the C ABI's order
FILE_CONFIG, FILE_GENERATION_CONFIG, FILE_SHARD_INDEX, FILE_TOKENIZER_JSON, FILE_TOKENIZER_MODEL, \
    FILE_GGUF, FILE_SHARD = range(7)


def model_directory_from_environment() -> str:
    """ModelFiles::directoryFromEnvironment: GEMMA_MODEL_DIR, or "" when unset."""
    length = ctypes.c_size_t()
    check(library().gq8_gemma_directory_from_environment(None, 0, ctypes.byref(length)))
    out = ctypes.create_string_buffer(max(1, length.value))
    check(library().gq8_gemma_directory_from_environment(out, length.value, ctypes.byref(length)))
    return os.fsdecode(out.raw[:length.value])


class Gemma:
    """HF::Gemma (Generation/Gemma.h:65-251) over libgemma_q8: a Hugging Face
    Gemma directory loaded on the host, prepared on the device, and generated
    from by ids or by text.  ``on_token`` is called once per generated id."""

    def __init__(self):
        handle = ctypes.c_void_p()
        check(library().gq8_gemma_create(ctypes.byref(handle)))
        self.handle = handle
        self._callback = None
        self._on_token = None

    def close(self) -> None:
        if self.handle:
            library().gq8_gemma_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def load(self, model_directory) -> None:
        check(library().gq8_gemma_load(self.handle, os.fsencode(model_directory)))

    def is_loaded(self) -> bool:
        return bool(library().gq8_gemma_is_loaded(self.handle))

    def is_prepared(self) -> bool:
        return bool(library().gq8_gemma_is_prepared(self.handle))

    def file(self, which: int, index: int = 0) -> str:
        """A located file's path, "" when the directory does not hold it."""
        length = ctypes.c_size_t()
        check(library().gq8_gemma_file(self.handle, which, index, None, 0, ctypes.byref(length)))
        out = ctypes.create_string_buffer(max(1, length.value))
        check(library().gq8_gemma_file(self.handle, which, index, out, length.value,
                                       ctypes.byref(length)))
        return os.fsdecode(out.raw[:length.value])

    def shards(self) -> list[str]:
        count = check(library().gq8_gemma_shard_count(self.handle))
        return [self.file(FILE_SHARD, i) for i in range(count)]

    def config(self):
        """(DecoderShape, (bos, eos, pad)) of the loaded config.json with
        generation_config.json applied."""
        c = _Shape()
        ids = _TokenIds()
        check(library().gq8_gemma_config(self.handle, ctypes.byref(c), ctypes.byref(ids)))
        shape = DecoderShape(c.width, c.heads, c.kv_heads, c.head_dim, c.layers, c.intermediate,
                             c.vocab, c.max_positions, c.max_step_rows, c.rms_epsilon,
                             c.rope_theta, c.embedding_scale)
        return shape, (ids.bos, ids.eos, ids.pad)

    @property
    def maximum_tokens(self) -> int:
        return check(library().gq8_gemma_maximum_tokens(self.handle))

    @maximum_tokens.setter
    def maximum_tokens(self, count: int) -> None:
        check(library().gq8_gemma_set_maximum_tokens(self.handle, int(count)))

    @property
    def prompt_capacity(self) -> int:
        return check(library().gq8_gemma_prompt_capacity(self.handle))

    @prompt_capacity.setter
    def prompt_capacity(self, rows: int) -> None:
        check(library().gq8_gemma_set_prompt_capacity(self.handle, int(rows)))

    def set_sampling(self, options: SamplingOptions) -> None:
        c = options.as_c()
        check(library().gq8_gemma_set_sampling(self.handle, ctypes.byref(c)))

    @property
    def on_token(self):
        return self._on_token

    @on_token.setter
    def on_token(self, fn) -> None:
        self._on_token = fn
        self._callback = TOKEN_CALLBACK(lambda token, user: fn(int(token))) if fn else None
        check(library().gq8_gemma_set_on_token(self.handle, self._callback or TOKEN_CALLBACK(),
                                               None))

    def prepare(self) -> None:
        check(library().gq8_gemma_prepare(self.handle))

    def _window_cap(self, prompt_length: int) -> int:
        shape, _ = self.config()
        window = shape.max_positions - prompt_length
        limit = self.maximum_tokens
        return max(1, min(limit, window) if limit > 0 else window)

    def generate(self, prompt) -> list[int]:
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        cap = self._window_cap(prompt.size)
        out = np.zeros(cap, dtype=np.int32)
        count = check(library().gq8_gemma_generate(self.handle, _host(prompt), prompt.size,
                                                   _host(out), cap))
        return [int(t) for t in out[:count]]

    def generate_from_text(self, text) -> list[int]:
        raw = text.encode() if isinstance(text, str) else bytes(text)
        cap = self._window_cap(1)
        out = np.zeros(cap, dtype=np.int32)
        count = check(library().gq8_gemma_generate_from_text(self.handle, raw, len(raw),
                                                             _host(out), cap))
        return [int(t) for t in out[:min(count, cap)]]

    def generate_text(self, text) -> str:
        raw = text.encode() if isinstance(text, str) else bytes(text)
        capacity = 1 << 16
        out = ctypes.create_string_buffer(capacity)
        length = ctypes.c_size_t()
        check(library().gq8_gemma_generate_text(self.handle, raw, len(raw), out, capacity,
                                                ctypes.byref(length)))
        if length.value > capacity:
            raise Gq8Error(ERR_ARGUMENT, "generate_text: text longer than the buffer")
        return out.raw[:length.value].decode("utf-8")

    def text_for_tokens(self, tokens) -> str:
        ids = (ctypes.c_int32 * max(1, len(tokens)))(*[int(t) for t in tokens])
        length = ctypes.c_size_t()
        check(library().gq8_gemma_text_for_tokens(self.handle, ids, len(tokens), None, 0,
                                                  ctypes.byref(length)))
        out = ctypes.create_string_buffer(max(1, length.value))
        check(library().gq8_gemma_text_for_tokens(self.handle, ids, len(tokens), out,
                                                  length.value, ctypes.byref(length)))
        return out.raw[:length.value].decode("utf-8")

    def last_stats(self) -> RunStats:
        st = _RunStats()
        check(library().gq8_gemma_last_stats(self.handle, ctypes.byref(st)))
        return RunStats(st.prefill_seconds, st.decode_seconds, st.step_count, st.generated)
