"""MI355X-native FfnAgent Dense-FFN execution path (gfx950 HIP kernels behind a C ABI).

Public surface, mirroring the reference's FfnAgent API:

* :mod:`crosspool_amd.agent`     -- ``FfnAgent``, ``ExecutorLane``, ``GraphTemplate``
* :mod:`crosspool_amd.ops`       -- ``ffn_shim`` (SGLang drop-in Tensor op), ``attach``
* :mod:`crosspool_amd.dense`     -- ``DenseExecutionPlan``, ``Dense`` and kernel-level ops
* :mod:`crosspool_amd.execution` -- Execution Signatures, capacity buckets, workspaces
* :mod:`crosspool_amd.weights`   -- Dense weight containers (interleaved Gate/Up)
* :mod:`crosspool_amd.ffn`       -- closed FFN enums and activation semantics

All compute runs in ``crosspool_amd/_lib/libxpool_amd.so``; importing the
package does not load it, calling any operator without it raises
``NativeUnavailableError``.
"""

from crosspool_amd._native import LIBRARY_PATH, NativeError, NativeUnavailableError

__all__ = ["LIBRARY_PATH", "NativeError", "NativeUnavailableError"]
