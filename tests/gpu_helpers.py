"""Shared helpers for the GPU parity tests: device buffers come from torch
(plumbing only); every computation under test goes through libgemma_q8."""
from __future__ import annotations

import numpy as np

import oracle as O


def to_device(torch, array: np.ndarray):
    array = np.ascontiguousarray(array)
    return torch.from_numpy(array.copy()).to("cuda")


def empty(torch, n: int, dtype):
    return torch.empty(n, dtype=dtype, device="cuda")


def q8_bytes(rows: int, inner: int) -> int:
    return rows * inner + rows * inner // 16


def split_q8(buffer: np.ndarray, rows: int, inner: int):
    """(q int8 [rows, inner], scale bits uint16 [rows, inner // 32])."""
    e = rows * inner
    q = buffer[:e].view(np.int8).reshape(rows, inner)
    s = buffer[e:e + e // 16].view(np.uint16).reshape(rows, inner // 32)
    return q, s


def f16_bits(values: np.ndarray) -> np.ndarray:
    return np.array([O.half_from_float(float(v)) for v in values.ravel()], dtype=np.uint16)


def spread(count: int, seed: int, scale: float) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal(count) * scale).astype(np.float32)


def exact_fraction(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a).ravel()
    b = np.asarray(b).ravel()
    return float(np.mean(a.view(np.uint32) == b.view(np.uint32))) if a.dtype == np.float32 \
        else float(np.mean(a == b))


def worst_error(actual: np.ndarray, expected: np.ndarray) -> float:
    """max |a - e| / (1 + |e|) (Tests/Decoder/Common.h:391-406)."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    return float(np.max(np.abs(actual - expected) / (1.0 + np.abs(expected))))
