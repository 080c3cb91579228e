"""MI355X-native Gemma-2B Int8Blocks token loop.

The compute path is libgemma_q8.so (gfx950 HIP kernels plus a C++ decoder
runtime behind the C ABI in include/gemma_q8.h); ``gemma_q8`` binds it.
"""
from .gemma_q8 import (  # noqa: F401
    Decoder, DecoderShape, Gq8Error, RunStats, algorithmic_decode_bytes, check,
    exported_symbols, library, version,
)
