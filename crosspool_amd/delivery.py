"""Fixed-order reduction of tensor-parallel FFN partials on one device.

In true TP every FfnAgent of a layer computes an unreduced ``[T, H]`` partial from its
intermediate slice; delivery folds the partials in fixed PE order in fp32 and casts once
(src/cext/ffnagent/delivery.cu:74-127, ``ordered_sum`` / ``reduce_tp_partials``), so the
result does not depend on arrival order.  This module is that fold for partials already
in one device's memory (``xp_reduce_partials``); bringing peer partials there (NVSHMEM in
the reference, xGMI peer copies or RCCL on MI355X) is not part of this single-GPU build.
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from crosspool_amd import _native

MAX_PARTIALS = 16


def reduce_tp_partials(
    partials: Sequence[torch.Tensor], *, out: torch.Tensor | None = None, stream: torch.cuda.Stream | None = None
) -> torch.Tensor:
    """``bf16(((0 + p0) + p1) + ... )`` elementwise in fp32, partials in the given (rank) order.

    All partials are bf16 tensors of one shape on one device, contiguous and 16-byte
    aligned with a multiple of 8 elements; ``out`` (allocated when omitted) may be one of
    them.  Runs on ``stream`` (default: the current stream).
    """

    if not 1 <= len(partials) <= MAX_PARTIALS:
        raise ValueError(f"between 1 and {MAX_PARTIALS} partials are supported")
    first = partials[0]
    for partial in partials:
        if partial.device.type != "cuda" or partial.device != first.device:
            raise ValueError("partials must share one GPU")
        if partial.dtype is not torch.bfloat16 or partial.shape != first.shape or not partial.is_contiguous():
            raise ValueError("partials must be contiguous bf16 tensors of one shape")
    if out is None:
        out = torch.empty_like(first)
    elif out.dtype is not torch.bfloat16 or out.shape != first.shape or not out.is_contiguous() or out.device != first.device:
        raise ValueError("out must be a contiguous bf16 tensor of the partials' shape on their device")
    pointers = (ctypes.c_void_p * len(partials))(*(partial.data_ptr() for partial in partials))
    stream = stream if stream is not None else torch.cuda.current_stream(first.device)
    _native.call(
        "xp_reduce_partials", pointers, len(partials), ctypes.c_void_p(out.data_ptr()), first.numel(),
        ctypes.c_void_p(stream.cuda_stream),
    )
    return out
