"""ctypes binding of the C ABI in ``include/xpool_amd.h``.

Replaces the pybind11 module ``xpool.native`` (src/cext-bindings/module.cpp:16)
for the FfnAgent execution path.  The library is loaded lazily from
``crosspool_amd/_lib/libxpool_amd.so``; when it is missing every entry point
raises :class:`NativeUnavailableError` -- there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "_lib" / "libxpool_amd.so"
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "xpool_amd.h"

XP_OK = 0
XP_ERROR_INVALID_ARGUMENT = 1
XP_ERROR_HIP = 2
XP_ERROR_STATE = 3
XP_ERROR_NOT_FOUND = 4
XP_ERROR_CAPACITY = 5
XP_ERROR_UNSUPPORTED = 6
XP_FAULT_SLOT_OUT_OF_RANGE = 1

class ActivationDesc(ctypes.Structure):
    """``xp_activation_desc`` of the header."""

    _fields_ = [
        ("function", ctypes.c_int),
        ("approximate_tanh", ctypes.c_int),
        ("gated", ctypes.c_int),
        ("has_limit", ctypes.c_int),
        ("alpha", ctypes.c_float),
        ("limit", ctypes.c_float),
        ("up_offset", ctypes.c_float),
    ]


class MoeLayerDesc(ctypes.Structure):
    """``xp_moe_layer_desc`` of the header."""

    _fields_ = [
        ("hidden", ctypes.c_int64),
        ("intermediate", ctypes.c_int64),
        ("experts", ctypes.c_int64),
        ("routed_experts", ctypes.c_int64),
        ("routed_topk", ctypes.c_int64),
        ("algorithm", ctypes.c_int),
        ("precision", ctypes.c_int),
        ("renormalize", ctypes.c_int),
        ("weight_rounding", ctypes.c_int),
        ("routed_scaling_factor", ctypes.c_float),
        ("alpha", ctypes.c_float),
        ("limit", ctypes.c_float),
        ("up_offset", ctypes.c_float),
        ("payload", ctypes.c_int),
        ("activation", ctypes.c_int),
        ("approximate_tanh", ctypes.c_int),
        ("biases", ctypes.c_int),
    ]


XP_DTYPE_BF16 = 1
XP_DTYPE_F16 = 2
XP_DTYPE_F32 = 3
XP_GATE_UP_CONCATENATED = 1
XP_GATE_UP_INTERLEAVED = 2
XP_ACTIVATION_NONE = 0
XP_ACTIVATION_SILU = 1
XP_ACTIVATION_RELU = 2
XP_ACTIVATION_GELU = 3

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_F32 = ctypes.c_float
_SIZE = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "xp_abi_version": (_INT, []),
    "xp_last_error": (_SIZE, [ctypes.c_char_p, _SIZE]),
    "xp_copy_bytes": (_INT, [_P, _P, _SIZE, _P]),
    "xp_reduce_partials": (_INT, [ctypes.POINTER(_P), _INT, _P, _I64, _P]),
    "xp_gather_rmsnorm": (_INT, [_P, _I64, _I64, _P, _I64, _P, _F32, _P, _P, _P]),
    "xp_scatter": (_INT, [_P, _I64, _I64, _P, _P, _I64, _P, _P]),
    "xp_gemm_gate_up_silu": (_INT, [_P, _I64, _I64, _P, _I64, _P, _F32, _F32, _F32, _P, _SIZE, _P]),
    "xp_gemm_down": (_INT, [_P, _I64, _I64, _P, _I64, _P, _P, _I64, _P, _SIZE, _P]),
    "xp_gemm_workspace_bytes": (_SIZE, [_I64, _I64, _I64, _INT]),
    "xp_projection": (_INT, [_P, _I64, _I64, _P, _I64, _P, _P, _INT, ctypes.POINTER(ActivationDesc), _P]),
    "xp_activation": (_INT, [_P, _P, _I64, _I64, _INT, _INT, ctypes.POINTER(ActivationDesc), _P]),
    "xp_dense_workspace_bytes": (_SIZE, [_I64, _I64, _I64]),
    "xp_dense_workspace_layout": (_INT, [_I64, _I64, _I64, ctypes.POINTER(_SIZE)]),
    "xp_dense_step": (_INT, [_P, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _F32, _P, _SIZE, _P, _P]),
    "xp_dense_step_static": (_INT, [_P, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _F32, _P, _P]),
    "xp_gemm_variant": (_SIZE, [_I64, _I64, _I64, _INT, ctypes.c_char_p, _SIZE]),
    "xp_dense_gate_up_variant": (_SIZE, [_I64, _I64, _I64, ctypes.c_char_p, _SIZE]),
    "xp_agent_create": (_INT, [_INT, ctypes.POINTER(_P)]),
    "xp_agent_destroy": (_INT, [_P]),
    "xp_layer_register": (_INT, [_P, _INT, _INT, _I64, _I64, _INT, _P, _P, _P, _F32]),
    "xp_lane_create": (_INT, [_P, _P, _SIZE, ctypes.POINTER(_P)]),
    "xp_lane_destroy": (_INT, [_P]),
    "xp_lane_stream": (_INT, [_P, ctypes.POINTER(_P)]),
    "xp_lane_check_health": (_INT, [_P, ctypes.POINTER(ctypes.c_uint32)]),
    "xp_lane_clear_fault": (_INT, [_P]),
    "xp_lane_synchronize": (_INT, [_P]),
    "xp_lane_set_graph_dispatch": (_INT, [_P, _INT]),
    "xp_template_capture": (_INT, [_P, _I64, _I64, _INT, _I64]),
    "xp_template_capacities": (_INT, [_P, _I64, _I64, _INT, ctypes.POINTER(_I64), _INT, ctypes.POINTER(_INT)]),
    "xp_replay": (_INT, [_P, _INT, _INT, _I64, _P, _P, _I64, _P, _P]),
    "xp_lane_fault_word": (_INT, [_P, ctypes.POINTER(_P)]),
    "xp_transport_create": (_INT, [_INT, _INT, ctypes.POINTER(_I64), ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(_P)]),
    "xp_transport_destroy": (_INT, [_P]),
    "xp_transport_open": (_INT, [_P, _P]),
    "xp_transport_submit": (_INT, [_P, _INT, _I64, _I64, _INT, _INT, _INT, _P, _I64, _INT, _P]),
    "xp_transport_evaluate": (_INT, [_P, _INT, _P, _P]),
    "xp_transport_complete": (_INT, [_P, _INT, _P, _I64, _INT, _I64, _P]),
    "xp_transport_settle": (_INT, [_P, _INT, _P, _P, _I64, _INT, _P]),
    "xp_transport_drain": (_INT, [_P, _P]),
    "xp_transport_publish_failure": (_INT, [_P, _INT, _INT, _P]),
    "xp_transport_snapshot": (_INT, [_P, _INT, _P]),
    "xp_transport_probe": (_INT, [_P, _INT, _INT, ctypes.POINTER(ctypes.c_uint32), _INT]),
    "xp_moe_router_topk": (_INT, [_P, _INT, _I64, _I64, _I64, _INT, _P, _INT, _INT, _P, _P, _P]),
    "xp_moe_router_workspace_bytes": (_SIZE, [_I64, _I64, _I64, _INT]),
    "xp_moe_router": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _INT, _INT, _INT, _P, _INT, _INT, _P, _P, _P, _SIZE, _P]),
    "xp_moe_finalize_routing": (_INT, [_P, _P, _I64, _I64, _P, _P, _I64, _P, _I64, _F32, _P]),
    "xp_moe_workspace_bytes": (_SIZE, [_I64, _I64, _I64, _I64, _I64]),
    "xp_moe_workspace_layout": (_INT, [_I64, _I64, _I64, _I64, _I64, ctypes.POINTER(_SIZE)]),
    "xp_moe_experts": (
        _INT,
        [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _F32, _INT, _INT, _F32, _F32, _F32, _INT, _P, _P,
         _SIZE, _P],
    ),
    "xp_moe_layer_register": (_INT, [_P, _INT, _INT, ctypes.POINTER(MoeLayerDesc), _P, _P, _P, _P, _P, _P, _P, _F32]),
    "xp_moe_step_workspace_bytes": (_SIZE, [ctypes.POINTER(MoeLayerDesc), _I64]),
    "xp_moe_step_workspace_layout": (_INT, [ctypes.POINTER(MoeLayerDesc), _I64, ctypes.POINTER(_SIZE)]),
    "xp_moe_template_capture": (_INT, [_P, ctypes.POINTER(MoeLayerDesc), _I64]),
}


class NativeUnavailableError(RuntimeError):
    """The HIP library has not been built (run ``__graft_entry__.build()``)."""


class NativeError(RuntimeError):
    """A C-ABI call returned a non-zero status; ``status`` holds it."""

    def __init__(self, status: int, message: str) -> None:
        super().__init__(message)
        self.status = status


_lock = threading.Lock()
_library: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """Load (once) and return the native library, raising if it is absent."""

    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is None:
            if not LIBRARY_PATH.exists():
                raise NativeUnavailableError(
                    f"{LIBRARY_PATH} is missing; build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                )
            lib = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                function = getattr(lib, name)
                function.restype = restype
                function.argtypes = argtypes
            _library = lib
    return _library


def last_error() -> str:
    lib = library()
    size = lib.xp_last_error(None, 0)
    buffer = ctypes.create_string_buffer(size + 1)
    lib.xp_last_error(buffer, size + 1)
    return buffer.value.decode(errors="replace")


def check(status: int, what: str) -> None:
    """Raise :class:`NativeError` (a RuntimeError) for a failed C-ABI call."""

    if status != XP_OK:
        raise NativeError(status, f"{what}: {last_error()}")


def call(name: str, *args: object) -> int:
    """Call ``name`` and raise on a non-zero status."""

    status = getattr(library(), name)(*args)
    check(status, name)
    return status


def payload_dtype_code(dtype: object) -> int:
    """XP_DTYPE_BF16 / XP_DTYPE_F16 of a payload dtype (torch.bfloat16 / torch.float16)."""

    import torch

    if dtype is torch.bfloat16:
        return XP_DTYPE_BF16
    if dtype is torch.float16:
        return XP_DTYPE_F16
    raise ValueError(f"payloads are bf16 or fp16, not {dtype}")


def gemm_variant(capacity: int, n: int, k: int, gated: bool) -> str:
    lib = library()
    buffer = ctypes.create_string_buffer(64)
    lib.xp_gemm_variant(capacity, n, k, int(gated), buffer, 64)
    return buffer.value.decode()


def dense_gate_up_variant(capacity: int, hidden: int, intermediate: int) -> str:
    """The Dense step's gate_up variant at ``capacity`` rows ("+gather" when the gather is fused)."""

    lib = library()
    buffer = ctypes.create_string_buffer(64)
    lib.xp_dense_gate_up_variant(capacity, hidden, intermediate, buffer, 64)
    return buffer.value.decode()


def gemm_workspace_bytes(rows: int, n: int, k: int, gated: bool) -> int:
    return int(library().xp_gemm_workspace_bytes(rows, n, k, int(gated)))


def gemm_workspace_bytes_upto(capacity: int, n: int, k: int, gated: bool) -> int:
    """Scratch that serves a kernel-level projection at every live row count up to ``capacity``.

    ``xp_gemm_gate_up_silu`` / ``xp_gemm_down`` choose their kernel at the live row count, and a
    smaller count can take a K split with more ranges than the capacity's choice (down 1024 x
    3072: 3833856 bytes at 117 rows, 3866624 at 59), so a plan prepared at the capacity sizes
    its scratch as the largest need over 1..capacity.
    """

    query = library().xp_gemm_workspace_bytes
    return max((int(query(rows, n, k, int(gated))) for rows in range(1, capacity + 1)), default=0)


def dense_workspace_bytes(capacity: int, hidden: int, intermediate: int) -> int:
    return int(library().xp_dense_workspace_bytes(capacity, hidden, intermediate))


def dense_workspace_layout(capacity: int, hidden: int, intermediate: int) -> tuple[int, ...]:
    """(batch, activated, gate_up partials, down partials, total) byte offsets of a Lane workspace."""

    offsets = (_SIZE * 5)()
    call("xp_dense_workspace_layout", capacity, hidden, intermediate, offsets)
    return tuple(int(value) for value in offsets)


def moe_step_workspace_bytes(desc: MoeLayerDesc, capacity: int) -> int:
    """Lane workspace bytes of one MoE template (0 for an invalid descriptor)."""

    return int(library().xp_moe_step_workspace_bytes(ctypes.byref(desc), capacity))


def moe_step_workspace_layout(desc: MoeLayerDesc, capacity: int) -> tuple[int, ...]:
    """(batch, logits, routed ids, routed weights, final ids, final weights, experts, total) offsets."""

    offsets = (_SIZE * 8)()
    call("xp_moe_step_workspace_layout", ctypes.byref(desc), capacity, offsets)
    return tuple(int(value) for value in offsets)
