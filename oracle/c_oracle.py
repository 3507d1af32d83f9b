"""ctypes loader for the C restatement (test infrastructure only)."""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from oracle import build_oracle
from oracle.ffn_oracle import bf16_bits, bf16_from_bits

_LIBRARY: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    global _LIBRARY
    if _LIBRARY is None:
        if not build_oracle.LIBRARY.exists():
            build_oracle.build()
        lib = ctypes.CDLL(str(build_oracle.LIBRARY))
        p, i64, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        lib.xpo_bf16_from_float.argtypes = [f32]
        lib.xpo_bf16_from_float.restype = ctypes.c_uint16
        lib.xpo_copy_bytes.argtypes = [p, ctypes.c_size_t, p, ctypes.c_size_t]
        lib.xpo_copy_bytes.restype = ctypes.c_int
        lib.xpo_gather.argtypes = [p, i64, i64, p, i64, p]
        lib.xpo_gather.restype = ctypes.c_int
        lib.xpo_scatter.argtypes = [p, i64, i64, p, i64, p]
        lib.xpo_scatter.restype = ctypes.c_int
        lib.xpo_rmsnorm.argtypes = [p, i64, i64, p, f32, p]
        lib.xpo_rmsnorm.restype = None
        lib.xpo_gated_silu.argtypes = [ctypes.c_uint16, ctypes.c_uint16, f32, f32, f32]
        lib.xpo_gated_silu.restype = ctypes.c_uint16
        lib.xpo_dense_partial.argtypes = [p, i64, i64, p, p, i64, p, p]
        lib.xpo_dense_partial.restype = None
        _LIBRARY = lib
    return _LIBRARY


def _ptr(array: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(array.ctypes.data)


def bf16_from_float(values: np.ndarray) -> np.ndarray:
    lib = library()
    flat = np.asarray(values, dtype=np.float32).ravel()
    return np.array([lib.xpo_bf16_from_float(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(values))


def gather(pool: torch.Tensor, slots: np.ndarray) -> torch.Tensor:
    bits = np.ascontiguousarray(bf16_bits(pool))
    slots = np.ascontiguousarray(slots, dtype=np.int32)
    out = np.zeros((slots.size, bits.shape[1]), dtype=np.uint16)
    if library().xpo_gather(_ptr(bits), bits.shape[0], bits.shape[1], _ptr(slots), slots.size, _ptr(out)) != 0:
        raise IndexError("slot id outside the mailbox pool")
    return bf16_from_bits(out)


def scatter(pool: torch.Tensor, slots: np.ndarray, rows: torch.Tensor) -> torch.Tensor:
    bits = np.ascontiguousarray(bf16_bits(pool)).copy()
    slots = np.ascontiguousarray(slots, dtype=np.int32)
    values = np.ascontiguousarray(bf16_bits(rows))
    if library().xpo_scatter(_ptr(bits), bits.shape[0], bits.shape[1], _ptr(slots), slots.size, _ptr(values)) != 0:
        raise IndexError("slot id outside the mailbox pool")
    return bf16_from_bits(bits)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    bits = np.ascontiguousarray(bf16_bits(x))
    w = np.ascontiguousarray(bf16_bits(weight))
    out = np.zeros_like(bits)
    library().xpo_rmsnorm(_ptr(bits), bits.shape[0], bits.shape[1], _ptr(w), eps, _ptr(out))
    return bf16_from_bits(out)


def dense_partial(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    xb = np.ascontiguousarray(bf16_bits(x))
    gu = np.ascontiguousarray(bf16_bits(w_gate_up))
    dn = np.ascontiguousarray(bf16_bits(w_down))
    rows, hidden = xb.shape
    intermediate = dn.shape[1]
    activated = np.zeros((rows, intermediate), dtype=np.uint16)
    out = np.zeros((rows, hidden), dtype=np.uint16)
    library().xpo_dense_partial(_ptr(xb), rows, hidden, _ptr(gu), _ptr(dn), intermediate, _ptr(activated), _ptr(out))
    return bf16_from_bits(out), bf16_from_bits(activated)
