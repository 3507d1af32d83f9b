"""FfnAgent, Executor Lanes and GraphTemplates on one MI355X.

Mirrors the FfnAgent execution API of the reference:
``FfnExecutionRegistry`` (src/xpool/runtime/ffnagent/registry.py:348-584),
``LaneCaptureResources`` (registry.py:25-137) and ``capture_dense_signature``
(registry.py:189-239), with the native install / replay of
src/cext/ffnagent/runtime.cu.  A layer signature maps to one GraphTemplate;
each Lane instantiates one hipGraph per template and replays it with the
layer's weights bound.  Python retains every tensor the native side borrows
(weights, workspaces, slot buffers) until the Lane is destroyed.
"""

from __future__ import annotations

import ctypes
import logging
from collections import deque
from dataclasses import dataclass
from time import monotonic

import torch

from crosspool_amd import _native
from crosspool_amd.execution import (
    DenseFfnExecutionSignature,
    MoeFfnExecutionSignature,
    derive_payload_row_capacities,
)
from crosspool_amd.ffn import LayerKind, ResultCode
from crosspool_amd.moe import MoeFfnWeights, MoeLayerSpec
from crosspool_amd.weights import DenseFfnWeights, validate_weight_tensor

logger = logging.getLogger(__name__)


def _moe_biases(weights) -> int:
    """The projection-bias bits of MoE weights (bit 0 i_proj, bit 1 o_proj)."""

    return int(weights.i_proj_bias is not None) | 2 * int(weights.o_proj_bias is not None)


@dataclass(frozen=True, slots=True)
class GraphTemplate:
    """One captured graph identity: the Execution Signature (execution.py:73-149).

    Dense templates are keyed by (payload dtype, hidden, intermediate, capacity); MoE
    templates by their whole signature.
    """

    signature: DenseFfnExecutionSignature | MoeFfnExecutionSignature

    @property
    def kind(self) -> LayerKind:
        return LayerKind.MOE if isinstance(self.signature, MoeFfnExecutionSignature) else LayerKind.DENSE

    @property
    def key(self) -> tuple[torch.dtype, int, int, int] | MoeFfnExecutionSignature:
        s = self.signature
        if isinstance(s, MoeFfnExecutionSignature):
            return s
        return s.payload_dtype, s.hidden_size, s.local_intermediate_size, s.payload_row_capacity

    @property
    def workspace_bytes(self) -> int:
        """Lane workspace bytes of this template, K-slice partial sums included (native query)."""

        s = self.signature
        if isinstance(s, MoeFfnExecutionSignature):
            nbytes = _native.moe_step_workspace_bytes(s.native_descriptor(), s.payload_row_capacity)
            if nbytes == 0:
                raise ValueError(f"MoE signature is outside the native limits: {s}")
            return nbytes
        return _native.dense_workspace_bytes(s.payload_row_capacity, s.hidden_size, s.local_intermediate_size)


@dataclass(frozen=True, slots=True)
class LayerBinding:
    instance_index: int
    layer_ordinal: int
    weights: DenseFfnWeights | MoeFfnWeights
    norm_weight: torch.Tensor | None
    eps: float
    moe: MoeLayerSpec | None = None

    @property
    def kind(self) -> LayerKind:
        return LayerKind.DENSE if self.moe is None else LayerKind.MOE

    @property
    def payload_dtype(self) -> torch.dtype:
        """The dtype of the layer's mailboxes: its weights' (bf16 or fp16)."""

        return self.weights.payload_dtype


class FfnHealthError(RuntimeError):
    """A Lane's sticky device fault word is set (canonical asynchronous failure)."""

    def __init__(self, fault_bits: int) -> None:
        super().__init__(f"FfnAgent Lane reported fault bits {fault_bits:#x} (slot id outside the mailbox)")
        self.fault_bits = fault_bits
        self.result = ResultCode.PROTOCOL_MISMATCH


class ExecutorLane:
    """One concurrent execution context: stream, workspace and instantiated templates."""

    def __init__(self, agent: FfnAgent, workspace_bytes: int, *, graph_dispatch: bool = False) -> None:
        self.agent = agent
        self.workspace = torch.empty(max(workspace_bytes, 16), dtype=torch.uint8, device=agent.device)
        handle = ctypes.c_void_p()
        _native.call(
            "xp_lane_create", agent.handle, ctypes.c_void_p(self.workspace.data_ptr()), self.workspace.numel(),
            ctypes.byref(handle),
        )
        self.handle = handle
        # Replays launch the template's kernels directly unless graph dispatch is asked for
        # (each hipGraphLaunch adds GPU time per replay on ROCm, measured by bench.py; same kernels).
        self.graph_dispatch = bool(graph_dispatch)
        _native.call("xp_lane_set_graph_dispatch", self.handle, int(self.graph_dispatch))
        stream = ctypes.c_void_p()
        _native.call("xp_lane_stream", self.handle, ctypes.byref(stream))
        self.stream = torch.cuda.ExternalStream(stream.value or 0, device=agent.device)
        fault = ctypes.c_void_p()
        _native.call("xp_lane_fault_word", self.handle, ctypes.byref(fault))
        # Device address of the Lane's sticky fault word (read by the Transport's evaluate).
        self.fault_word = int(fault.value or 0)
        self.templates: dict[object, GraphTemplate] = {}
        self._in_flight: deque[tuple[torch.cuda.Event | None, tuple[torch.Tensor, ...], torch.cuda.Stream]] = deque()

    def set_graph_dispatch(self, enabled: bool) -> None:
        """Launch later replays as the template's instantiated hipGraph (True) or as its
        kernels directly (False); both run the same kernels with the same arguments."""

        self._require_open()
        _native.call("xp_lane_set_graph_dispatch", self.handle, int(bool(enabled)))
        self.graph_dispatch = bool(enabled)

    def capture(self, template: GraphTemplate) -> None:
        """Instantiate the template's hipGraph on this Lane (idempotent)."""

        self._require_open()
        s = template.signature
        if isinstance(s, MoeFfnExecutionSignature):
            _native.call("xp_moe_template_capture", self.handle, ctypes.byref(s.native_descriptor()),
                         s.payload_row_capacity)
        else:
            _native.call("xp_template_capture", self.handle, s.hidden_size, s.local_intermediate_size,
                         _native.payload_dtype_code(s.payload_dtype), s.payload_row_capacity)
        self.templates[template.key] = template

    def capacities(self, hidden: int, intermediate: int, payload_dtype: torch.dtype = torch.bfloat16) -> tuple[int, ...]:
        self._require_open()
        count = ctypes.c_int()
        buffer = (ctypes.c_int64 * 64)()
        _native.call("xp_template_capacities", self.handle, hidden, intermediate,
                     _native.payload_dtype_code(payload_dtype), buffer, 64, ctypes.byref(count))
        return tuple(buffer[index] for index in range(min(count.value, 64)))

    def replay(
        self,
        *,
        instance_index: int,
        layer_ordinal: int,
        pool: torch.Tensor,
        slots: torch.Tensor,
        rows: int | None = None,
        out_pool: torch.Tensor | None = None,
        stream: torch.cuda.Stream | None = None,
    ) -> None:
        """Run one mailbox step of a registered layer (stream-ordered, no host sync).

        ``rows`` live slot ids of ``slots`` are gathered from ``pool`` (with the
        layer's RMSNorm when it has one), run through the layer's FFN (Dense, or MoE:
        Router, routing finalisation, Experts) and written back to the same slots of
        ``out_pool`` (default: ``pool``).

        With ``stream=None`` the replay runs on the Lane's stream after the
        current torch stream's pending work; results are visible to other
        streams after :meth:`synchronize` or ``wait_stream(lane.stream)``.  The
        tensors must stay alive until then.  With an explicit ``stream`` the
        replay is ordered on that stream only; replays of one Lane must not
        overlap (they share its workspace).
        """

        self._require_open()
        out_pool = pool if out_pool is None else out_pool
        binding = self.agent.layers.get((instance_index, layer_ordinal))
        payload = binding.payload_dtype if binding is not None else torch.bfloat16
        for name, tensor in (("pool", pool), ("out_pool", out_pool)):
            if tensor.device != self.agent.device or tensor.dtype is not payload or tensor.ndim != 2:
                raise ValueError(f"{name} must be a {payload} matrix on the agent's device (the layer's payload dtype)")
            if not tensor.is_contiguous():
                raise ValueError(f"{name} must be contiguous")
        if out_pool.shape != pool.shape:
            raise ValueError("input and output mailboxes must have one shape")
        if binding is not None and pool.shape[1] != binding.weights.hidden_size:
            # The kernels index mailbox rows by the layer's hidden size.
            raise ValueError(f"mailbox rows must hold the layer's hidden size {binding.weights.hidden_size}")
        if slots.device != self.agent.device or slots.dtype is not torch.int32 or slots.ndim != 1:
            raise ValueError("slots must be a device int32 vector")
        rows = slots.numel() if rows is None else rows
        if not 0 < rows <= slots.numel():
            raise ValueError("row count must be positive and covered by the slot ids")
        current = torch.cuda.current_stream(self.agent.device)
        run_on = self.stream if stream is None else stream
        if stream is None:
            # Lane stream: order after the caller's pending work on the current stream.
            self.stream.wait_stream(current)
        # A handle of 0 is the legacy default stream (torch's default stream).
        stream_handle = ctypes.c_void_p(run_on.cuda_stream)
        _native.call(
            "xp_replay", self.handle, instance_index, layer_ordinal, rows, ctypes.c_void_p(pool.data_ptr()),
            ctypes.c_void_p(out_pool.data_ptr()), pool.shape[0], ctypes.c_void_p(slots.data_ptr()), stream_handle,
        )
        if run_on.cuda_stream != current.cuda_stream and not torch.cuda.is_current_stream_capturing():
            # (Under an outer stream capture the kernels become graph nodes and the tensors
            # belong to the capturing caller; no event may be recorded or queried for them.)
            self._retain(run_on, (pool, out_pool, slots))

    def _retain(self, stream: torch.cuda.Stream, tensors: tuple[torch.Tensor, ...]) -> None:
        """Keep borrowed tensors alive until the replay that reads them has run.

        The caching allocator only tracks the stream a tensor was allocated on;
        without this a tensor freed by the caller could be handed out again
        while this Lane's stream still reads it.
        """

        while self._in_flight and self._in_flight[0][0] is not None and self._in_flight[0][0].query():
            self._in_flight.popleft()
        if self._in_flight:
            _, last_tensors, last_stream = self._in_flight[-1]
            if last_stream == stream and all(a is b for a, b in zip(last_tensors, tensors)):
                # Same tensors on the same stream as the previous replay (the common
                # layer-after-layer case): hold them until that stream is drained instead of
                # recording an event per replay, a marker packet that delays the next kernels.
                self._in_flight[-1] = (None, tensors, stream)
                return
        event = torch.cuda.Event()
        event.record(stream)
        self._in_flight.append((event, tensors, stream))

    def _release_retained(self) -> None:
        """Drop retained tensors once the work that reads them has run."""

        for event, _, stream in self._in_flight:
            if event is None:
                stream.synchronize()
            else:
                event.synchronize()
        self._in_flight.clear()

    def check_health(self) -> int:
        """Synchronise the Lane and return its sticky fault bits (0 = healthy)."""

        self._require_open()
        bits = ctypes.c_uint32()
        _native.call("xp_lane_check_health", self.handle, ctypes.byref(bits))
        self._release_retained()
        return int(bits.value)

    def clear_fault(self) -> None:
        self._require_open()
        _native.call("xp_lane_clear_fault", self.handle)

    def synchronize(self) -> None:
        self._require_open()
        _native.call("xp_lane_synchronize", self.handle)
        self._release_retained()

    def close(self) -> None:
        """Drain the Lane (its stream is destroyed), then drop retained tensors."""

        if self.handle is not None:
            self._release_retained()
            _native.call("xp_lane_destroy", self.handle)
            self.handle = None
            self.templates.clear()

    def _require_open(self) -> None:
        if self.handle is None:
            raise RuntimeError("Executor Lane is closed")


class FfnAgent:
    """FFN execution owner on one device: layer weights, GraphTemplates and Lanes.

    ``executor_lane_count`` plays the role of ``scheduler.ffn_concurrency``
    (src/xpool/config.py:457): independent Lanes may replay concurrently on
    their own streams.
    """

    def __init__(
        self, device: int | torch.device | None = None, *, executor_lane_count: int = 1, graph_dispatch: bool = False
    ) -> None:
        if executor_lane_count <= 0:
            raise ValueError("an FfnAgent needs at least one Executor Lane")
        if device is None:
            device = torch.cuda.current_device()
        self.device = torch.device("cuda", device if isinstance(device, int) else device.index)
        handle = ctypes.c_void_p()
        _native.call("xp_agent_create", self.device.index, ctypes.byref(handle))
        self.handle = handle
        self.executor_lane_count = executor_lane_count
        self.graph_dispatch = graph_dispatch
        self.layers: dict[tuple[int, int], LayerBinding] = {}
        self.templates: dict[object, GraphTemplate] = {}
        self.lanes: list[ExecutorLane] = []
        self.materialized = False

    # -------------------------------------------------------------- layers
    def register_layer(
        self,
        *,
        instance_index: int,
        layer_ordinal: int,
        weights: DenseFfnWeights,
        norm_weight: torch.Tensor | None = None,
        eps: float = 1e-6,
    ) -> None:
        """Bind one Dense layer's weights (and optional fused RMSNorm weight)."""

        if weights.device != self.device:
            raise ValueError("local FFN resources must reside on the agent's device")
        if not weights.template_ready:
            raise ValueError(
                "captured Dense templates take gated bf16 or fp16 INTERLEAVED weights without biases and 16-byte "
                "rows; run other layers through crosspool_amd.operators"
            )
        payload = weights.payload_dtype
        if norm_weight is not None:
            validate_weight_tensor(norm_weight, name="RMSNorm weight")
            if norm_weight.dtype is not payload or tuple(norm_weight.shape) != (weights.hidden_size,):
                raise ValueError(f"RMSNorm weight must be a {payload} [H] vector (the layer's payload dtype)")
            if norm_weight.device != self.device:
                raise ValueError("RMSNorm weight must reside on the agent's device")
        _native.call(
            "xp_layer_register", self.handle, instance_index, layer_ordinal, weights.hidden_size,
            weights.local_intermediate_size, _native.payload_dtype_code(payload),
            ctypes.c_void_p(weights.i_proj.values.data_ptr()),
            ctypes.c_void_p(weights.o_proj.values.data_ptr()),
            None if norm_weight is None else ctypes.c_void_p(norm_weight.data_ptr()), float(eps),
        )
        self.layers[(instance_index, layer_ordinal)] = LayerBinding(
            instance_index, layer_ordinal, weights, norm_weight, float(eps)
        )

    def register_moe_layer(
        self,
        *,
        instance_index: int,
        layer_ordinal: int,
        weights: MoeFfnWeights,
        spec: MoeLayerSpec,
        norm_weight: torch.Tensor | None = None,
        eps: float = 1e-6,
    ) -> None:
        """Bind one MoE layer: expert projections, Router (+ correction bias), optional fused RMSNorm.

        On one device the Lane owns the Router: each replay projects and routes the gathered
        rows itself (the reference's TP rank 0 role, src/cext/ffnagent/runtime.cu:649).
        """

        if weights.i_proj.device != self.device:
            raise ValueError("local FFN resources must reside on the agent's device")
        spec.validate_weights(weights)
        if norm_weight is not None:
            validate_weight_tensor(norm_weight, name="RMSNorm weight")
            if norm_weight.dtype is not weights.payload_dtype or tuple(norm_weight.shape) != (weights.hidden_size,):
                raise ValueError(f"RMSNorm weight must be a {weights.payload_dtype} [H] vector")
            if norm_weight.device != self.device:
                raise ValueError("RMSNorm weight must reside on the agent's device")
        signature = spec.signature(
            hidden_size=weights.hidden_size, local_intermediate_size=weights.local_intermediate_size,
            payload_row_capacity=1, payload_dtype=weights.payload_dtype, biases=_moe_biases(weights),
        )
        router = weights.router
        _native.call(
            "xp_moe_layer_register", self.handle, instance_index, layer_ordinal,
            ctypes.byref(signature.native_descriptor()), ctypes.c_void_p(weights.i_proj.data_ptr()),
            ctypes.c_void_p(weights.o_proj.data_ptr()),
            None if weights.i_proj_bias is None else ctypes.c_void_p(weights.i_proj_bias.data_ptr()),
            None if weights.o_proj_bias is None else ctypes.c_void_p(weights.o_proj_bias.data_ptr()),
            ctypes.c_void_p(router.projection.data_ptr()),
            None if router.correction_bias is None else ctypes.c_void_p(router.correction_bias.data_ptr()),
            None if norm_weight is None else ctypes.c_void_p(norm_weight.data_ptr()), float(eps),
        )
        self.layers[(instance_index, layer_ordinal)] = LayerBinding(
            instance_index, layer_ordinal, weights, norm_weight, float(eps), spec
        )

    def register_checkpoint(
        self,
        model_path,
        *,
        instance_index: int,
        tp_size: int = 1,
        tp_rank: int = 0,
        layers=None,
        fuse_norm: bool = True,
        parallelism: int = 4,
    ):
        """Load a local checkpoint's Dense layers and bind each at ``layer_ordinal`` = its layer id.

        The loading follows the reference's Plan materialisation for one FfnAgent
        (loader.py:148-284) through ``crosspool_amd.checkpoint.load_dense_layers``.  With
        ``fuse_norm`` the post-attention RMSNorm weight and ``rms_norm_eps`` of the
        checkpoint are bound for the fused gather; without it the caller applies the
        norm, as SGLang does for the reference.  Returns the loaded layers.
        """

        from crosspool_amd.checkpoint import load_dense_layers

        loaded = load_dense_layers(
            model_path, device=self.device, tp_size=tp_size, tp_rank=tp_rank, layers=layers, norm=fuse_norm,
            parallelism=parallelism,
        )
        for layer in loaded:
            self.register_layer(
                instance_index=instance_index,
                layer_ordinal=layer.layer_id,
                weights=DenseFfnWeights.from_tensors(layer.i_proj, layer.o_proj),
                norm_weight=layer.norm_weight,
                eps=layer.eps,
            )
        return tuple(loaded)

    # -------------------------------------------------------------- bring-up
    def materialize(self, *, maximum_row_capacity: int) -> tuple[GraphTemplate, ...]:
        """Create the Lanes and capture every signature of every registered layer.

        Signatures are deduplicated across layers (registry.py:466-474): layers of
        one shape share templates.  One attempt only (registry.py:400-402).
        """

        if self.materialized:
            raise RuntimeError("FFN execution materialization cannot be retried")
        if not self.layers:
            raise RuntimeError("register at least one layer before materializing")
        self.materialized = True
        started = monotonic()
        capacities = derive_payload_row_capacities(maximum_row_capacity)
        dense = self._dense_layers()
        shapes = sorted({(str(b.payload_dtype), b.payload_dtype, b.weights.hidden_size,
                          b.weights.local_intermediate_size) for b in dense})
        for _, payload, hidden, intermediate in shapes:
            for capacity in capacities:
                signature = DenseFfnExecutionSignature(
                    payload_dtype=payload,
                    payload_row_capacity=capacity,
                    hidden_size=hidden,
                    local_intermediate_size=intermediate,
                )
                template = GraphTemplate(signature)
                self.templates[template.key] = template
        for binding in self.layers.values():
            if binding.moe is None:
                continue
            for capacity in capacities:
                template = GraphTemplate(binding.moe.signature(
                    hidden_size=binding.weights.hidden_size,
                    local_intermediate_size=binding.weights.local_intermediate_size,
                    payload_row_capacity=capacity,
                    payload_dtype=binding.payload_dtype,
                    biases=_moe_biases(binding.weights),
                ))
                self.templates.setdefault(template.key, template)
        workspace_bytes = max(t.workspace_bytes for t in self.templates.values())
        for _ in range(self.executor_lane_count):
            lane = ExecutorLane(self, workspace_bytes, graph_dispatch=self.graph_dispatch)
            self.lanes.append(lane)
            for template in self.templates.values():
                lane.capture(template)
        logger.info(
            "graph templates captured device=%s signature_count=%s dense_count=%s moe_count=%s lane_count=%s "
            "row_capacities=%s elapsed=%.3fs",
            self.device, len(self.templates),
            sum(t.kind is LayerKind.DENSE for t in self.templates.values()),
            sum(t.kind is LayerKind.MOE for t in self.templates.values()),
            len(self.lanes), list(capacities), monotonic() - started,
        )
        return tuple(self.templates.values())

    def _dense_layers(self) -> list[LayerBinding]:
        return [binding for binding in self.layers.values() if binding.moe is None]

    # -------------------------------------------------------------- execution
    def execute(
        self,
        *,
        instance_index: int,
        layer_ordinal: int,
        pool: torch.Tensor,
        slots: torch.Tensor,
        rows: int | None = None,
        out_pool: torch.Tensor | None = None,
        lane: int = 0,
        stream: torch.cuda.Stream | None = None,
    ) -> None:
        """Replay one layer on ``lane`` (see :meth:`ExecutorLane.replay`)."""

        if not self.materialized:
            raise RuntimeError("FfnAgent has not been materialized")
        if (instance_index, layer_ordinal) not in self.layers:
            raise KeyError(f"no layer registered for instance {instance_index} ordinal {layer_ordinal}")
        self.lanes[lane].replay(
            instance_index=instance_index, layer_ordinal=layer_ordinal, pool=pool, slots=slots, rows=rows,
            out_pool=out_pool, stream=stream,
        )

    def check_health(self) -> None:
        """Raise :class:`FfnHealthError` if any Lane raised a fault (reference ``check_health``)."""

        for lane in self.lanes:
            bits = lane.check_health()
            if bits:
                raise FfnHealthError(bits)

    def close(self) -> None:
        """Destroy Lanes (after their streams drain), then the agent; weights are released last."""

        while self.lanes:
            self.lanes[-1].close()
            self.lanes.pop()
        if self.handle is not None:
            _native.call("xp_agent_destroy", self.handle)
            self.handle = None
        self.layers.clear()
        self.templates.clear()

    def __enter__(self) -> FfnAgent:
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()
