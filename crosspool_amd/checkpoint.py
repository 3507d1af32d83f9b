"""Local checkpoint loading for the Dense FFN path.

Reads a local Hugging Face checkpoint directory (``config.json`` plus safetensors
shards) of a gated Dense family and places each layer's tensor-parallel shard on
the GPU in the layout the kernels take: INTERLEAVED ``i_proj [2 L, H]`` (row 2j =
gate_j, row 2j+1 = up_j), ``o_proj [H, L]`` and, for the fused RMSNorm, the
post-attention norm weight ``[H]``.  L = I / tp_size, and rank r owns intermediate
rows ``[r L, (r + 1) L)``.

Reference behaviour followed (file:line in the CrossPool checkout):

- family compilers: ``runtime/ffnagent/models/qwen3.py:13-45`` (Qwen2 and Llama are
  the same gated Dense profile), ``architecture.py:22-137`` (strict ``config.json``
  fields, ``architecture.py:177-215`` load);
- key view: ``checkpoint.py:18-76`` (index or one canonical file, duplicate JSON members
  and unsafe shard names rejected);
- FFN key coverage: ``checkpoint.py:79-93``;
- TP geometry: ``preparation.py:160-241``; Gate/Up row order ``ffn.py:57-68``;
- reading: ``loader.py:451-519`` (slices, dtype and shape checks), ``loader.py:593-720``
  (bounded pinned slots, reader threads that never touch the GPU, the owner thread
  installs each value before its slot is reused).

The post-attention norm weight (``model.layers.{i}.post_attention_layernorm.weight``)
is read in addition, because this build fuses the norm into the gather; the reference
leaves the norm to SGLang.  Payloads are bf16: bf16 sources are copied bit for bit,
fp16 / fp32 sources are rounded to nearest even.
"""

from __future__ import annotations

import concurrent.futures
import json
import math
import queue
import threading
from dataclasses import dataclass
from pathlib import Path
from typing import Callable, Iterable

import torch

INDEX_FILENAME = "model.safetensors.index.json"
SINGLE_FILE_NAME = "model.safetensors"

# Gated Dense families: architecture name -> model_type (all use ``model.layers.{i}.mlp``).
DENSE_FAMILIES = {
    "Qwen3ForCausalLM": "qwen3",
    "Qwen2ForCausalLM": "qwen2",
    "LlamaForCausalLM": "llama",
}
ADMITTED_SOURCE_DTYPES = ("bfloat16", "float16")


# ---------------------------------------------------------------- config and key view
def parse_json_object(payload: bytes, *, source: Path) -> dict:
    """One JSON object; a duplicated member at any level is an error (checkpoint.py:18-34)."""

    def unique(pairs: list[tuple[str, object]]) -> dict:
        result: dict = {}
        for key, value in pairs:
            if key in result:
                raise ValueError(f"duplicate JSON member {key!r} in {source}")
            result[key] = value
        return result

    value = json.loads(payload, object_pairs_hook=unique)
    if not isinstance(value, dict):
        raise ValueError(f"{source} must contain one JSON object")
    return value


def read_checkpoint_key_view(model_path: Path) -> dict[str, Path]:
    """Tensor key -> shard file, from the index or the one canonical file (checkpoint.py:37-76)."""

    model_path = Path(model_path)
    index_path = model_path / INDEX_FILENAME
    if index_path.exists():
        index = parse_json_object(index_path.read_bytes(), source=index_path)
        weight_map = index.get("weight_map")
        if not isinstance(weight_map, dict) or not weight_map:
            raise ValueError(f"{index_path} must contain one nonempty object-valued weight_map")
        view: dict[str, Path] = {}
        for key, shard in weight_map.items():
            if not key:
                raise ValueError(f"{index_path} contains an invalid weight key")
            if not isinstance(shard, str) or not shard:
                raise ValueError(f"{index_path} contains an invalid shard name for {key!r}")
            if "/" in shard or "\\" in shard or not shard.endswith(".safetensors"):
                raise ValueError(f"{index_path} contains unsafe shard name {shard!r}")
            path = model_path / shard
            if path.is_symlink() or not path.is_file():
                raise ValueError(f"checkpoint shard {path} is not an existing regular file")
            view[key] = path
        return view

    canonical = model_path / SINGLE_FILE_NAME
    files = [entry for entry in model_path.iterdir() if entry.suffix == ".safetensors"]
    if len(files) != 1 or files[0] != canonical:
        raise ValueError(f"{model_path} must contain exactly one unindexed canonical {SINGLE_FILE_NAME} checkpoint")
    if canonical.is_symlink() or not canonical.is_file():
        raise ValueError(f"checkpoint {canonical} is not an existing regular file")
    from safetensors import safe_open

    with safe_open(str(canonical), framework="pt", device="cpu") as handle:
        keys = tuple(handle.keys())
    if not keys or any(not isinstance(key, str) or not key for key in keys):
        raise ValueError(f"checkpoint {canonical} must contain only nonempty tensor keys")
    return dict.fromkeys(keys, canonical)


def _config_int(config: dict, name: str) -> int:
    value = config.get(name)
    if not isinstance(value, int) or isinstance(value, bool):
        raise ValueError(f"{name} must be a JSON integer")
    if value < 1:
        raise ValueError(f"{name} must be greater than or equal to 1")
    return value


def mlp_keys(layer_id: int) -> tuple[str, str, str]:
    """Gate, up and down weight keys of one layer (architecture.py:120-137)."""

    prefix = f"model.layers.{layer_id}.mlp"
    return (f"{prefix}.gate_proj.weight", f"{prefix}.up_proj.weight", f"{prefix}.down_proj.weight")


def norm_key(layer_id: int) -> str:
    return f"model.layers.{layer_id}.post_attention_layernorm.weight"


@dataclass(frozen=True, slots=True)
class DenseModelSpec:
    """FFN semantics of a gated Dense checkpoint (the FfnModelSpec of qwen3.py:24-45)."""

    architecture: str
    hidden_size: int
    intermediate_size: int
    layer_count: int
    rms_norm_eps: float
    key_view: dict[str, Path]


def load_model_spec(model_path: Path) -> DenseModelSpec:
    """Compile ``config.json`` and check the FFN key coverage (architecture.py:177-215).

    Raises RuntimeError naming the checkpoint, as the reference does.
    """

    model_path = Path(model_path)
    try:
        config_path = model_path / "config.json"
        config = parse_json_object(config_path.read_bytes(), source=config_path)
        architectures = config.get("architectures")
        if (
            not isinstance(architectures, list)
            or len(architectures) != 1
            or not isinstance(architectures[0], str)
            or not architectures[0]
        ):
            raise ValueError("architectures must be a one-element array containing a nonempty string")
        architecture = architectures[0]
        model_type = DENSE_FAMILIES.get(architecture)
        if model_type is None:
            raise ValueError(f"unsupported FFN architecture {architecture!r}")
        if config.get("model_type") != model_type:
            raise ValueError(f"model_type must equal {model_type!r}")
        if config.get("hidden_act") != "silu":
            raise ValueError("hidden_act must equal 'silu'")
        if config.get("torch_dtype") not in ADMITTED_SOURCE_DTYPES:
            raise ValueError("torch_dtype must be 'bfloat16' or 'float16'")
        hidden = _config_int(config, "hidden_size")
        layers = _config_int(config, "num_hidden_layers")
        intermediate = _config_int(config, "intermediate_size")
        eps = config.get("rms_norm_eps", 1e-6)
        if isinstance(eps, bool) or not isinstance(eps, (int, float)) or not math.isfinite(eps) or eps <= 0:
            raise ValueError("rms_norm_eps must be a finite positive JSON number")
        key_view = read_checkpoint_key_view(model_path)
        validate_ffn_coverage(key_view, layers)
        return DenseModelSpec(architecture, hidden, intermediate, layers, float(eps), key_view)
    except Exception as error:
        raise RuntimeError(f"failed to compile FFN model at {model_path}: {error}") from error


def validate_ffn_coverage(key_view: dict[str, Path], layer_count: int) -> None:
    """Each layer's ``mlp.`` namespace holds exactly its three weights (checkpoint.py:79-93)."""

    keys = set(key_view)
    for layer_id in range(layer_count):
        prefix = f"model.layers.{layer_id}.mlp."
        actual = {key for key in keys if key.startswith(prefix)}
        expected = set(mlp_keys(layer_id))
        if actual != expected:
            missing = sorted(expected - actual)
            extra = sorted(actual - expected)
            raise ValueError(f"FFN checkpoint namespace for layer {layer_id} differs: missing={missing}, extra={extra}")


# ---------------------------------------------------------------- TP geometry and reads
@dataclass(frozen=True, slots=True)
class ShardGeometry:
    """One rank's slice of the intermediate dimension (preparation.py:160-241)."""

    hidden_size: int
    intermediate_size: int
    tp_size: int
    tp_rank: int

    def __post_init__(self) -> None:
        for value in (self.tp_size, self.tp_rank):
            if isinstance(value, bool) or not isinstance(value, int):
                raise ValueError("FFN preparation coordinates must be integers")
        if self.tp_size <= 0 or not 0 <= self.tp_rank < self.tp_size:
            raise ValueError("FFN preparation coordinate is outside the TP domain")
        if self.intermediate_size % self.tp_size:
            raise ValueError("FFN intermediate size is not divisible by FFN TP")

    @property
    def local_width(self) -> int:
        return self.intermediate_size // self.tp_size

    @property
    def source_start(self) -> int:
        return self.tp_rank * self.local_width


@dataclass(frozen=True, slots=True)
class _Read:
    """One staged value: the keys it reads, its host shape and how the slices combine."""

    layer_id: int
    kind: str  # "i_proj", "o_proj" or "norm"
    keys: tuple[str, ...]
    shape: tuple[int, ...]

    @property
    def staged_bytes(self) -> int:
        return math.prod(self.shape) * 2


def _to_payload(source: torch.Tensor, *, key: str) -> torch.Tensor:
    if not source.is_floating_point():
        raise ValueError(f"checkpoint tensor {key!r} has incompatible dtype {source.dtype}")
    return source.to(torch.bfloat16)  # bf16 is a copy; wider floats round to nearest even


def _read_slice(handle, key: str, expected: tuple[int, ...], select: Callable) -> torch.Tensor:
    piece = handle.get_slice(key)
    shape = tuple(piece.get_shape())
    if shape != expected:
        raise ValueError(f"checkpoint tensor {key!r} has incompatible shape: expected {expected}, found {shape}")
    return _to_payload(select(piece), key=key)


def stage_read(read: _Read, geometry: ShardGeometry, key_view: dict[str, Path], out: torch.Tensor) -> None:
    """Fill ``out`` (host, bf16, ``read.shape``) from the checkpoint; no GPU work.

    ``i_proj``: rows 2j and 2j+1 of ``out`` are gate and up row ``start + j``.
    ``o_proj``: columns ``[start, start + L)`` of ``down``.  ``norm``: the vector.
    """

    from safetensors import safe_open

    hidden, intermediate = geometry.hidden_size, geometry.intermediate_size
    start, width = geometry.source_start, geometry.local_width
    handles: dict[Path, object] = {}
    try:
        def handle_of(key: str):
            path = key_view.get(key)
            if path is None:
                raise ValueError(f"checkpoint key {key!r} is absent from its authoritative key view")
            if path not in handles:
                handles[path] = safe_open(str(path), framework="pt", device="cpu").__enter__()
            return handles[path]

        if read.kind == "i_proj":
            pairs = out.view(width, 2, hidden)
            for column, key in enumerate(read.keys):  # gate -> rows 2j, up -> rows 2j + 1
                rows = _read_slice(handle_of(key), key, (intermediate, hidden), lambda p: p[start : start + width])
                pairs[:, column, :].copy_(rows)
        elif read.kind == "o_proj":
            (key,) = read.keys
            out.copy_(_read_slice(handle_of(key), key, (hidden, intermediate), lambda p: p[:, start : start + width]))
        else:
            (key,) = read.keys
            out.copy_(_read_slice(handle_of(key), key, (hidden,), lambda p: p[:]))
    finally:
        for handle in handles.values():
            handle.__exit__(None, None, None)


def layer_reads(spec: DenseModelSpec, geometry: ShardGeometry, layer_ids: Iterable[int], *, norm: bool) -> list[_Read]:
    hidden, width = geometry.hidden_size, geometry.local_width
    reads = []
    for layer_id in layer_ids:
        gate, up, down = mlp_keys(layer_id)
        reads.append(_Read(layer_id, "i_proj", (gate, up), (2 * width, hidden)))
        reads.append(_Read(layer_id, "o_proj", (down,), (hidden, width)))
        if norm:
            reads.append(_Read(layer_id, "norm", (norm_key(layer_id),), (hidden,)))
    return reads


# ---------------------------------------------------------------- materialisation
@dataclass(frozen=True, slots=True)
class LoadedDenseLayer:
    """One layer's local shard on the device, ready for ``FfnAgent.register_layer``."""

    layer_id: int
    i_proj: torch.Tensor
    o_proj: torch.Tensor
    norm_weight: torch.Tensor | None
    eps: float


def load_dense_layers(
    model_path: Path,
    *,
    device: torch.device | int | None = None,
    tp_size: int = 1,
    tp_rank: int = 0,
    layers: Iterable[int] | None = None,
    norm: bool = True,
    parallelism: int = 4,
) -> list[LoadedDenseLayer]:
    """Materialise the selected layers' local shards on ``device`` (default: current GPU).

    Reader threads fill at most ``parallelism`` pinned host slots (each sized for the
    largest value); this thread copies every staged value to its device tensor and
    returns the slot once the copy has completed (loader.py:228-284, 593-720).  The
    device tensors are allocated up front; a failure anywhere stops the readers and
    raises RuntimeError.
    """

    if parallelism <= 0:
        raise ValueError("loader parallelism must be positive")
    spec = load_model_spec(Path(model_path))
    geometry = ShardGeometry(spec.hidden_size, spec.intermediate_size, tp_size, tp_rank)
    if spec.hidden_size % 8 or geometry.local_width % 8:
        raise ValueError("hidden size and local intermediate size must be multiples of 8 on this path")
    layer_ids = list(range(spec.layer_count)) if layers is None else list(layers)
    for layer_id in layer_ids:
        if not 0 <= layer_id < spec.layer_count:
            raise ValueError(f"layer {layer_id} is outside the model")
    if device is None:
        device = torch.cuda.current_device()
    device = torch.device("cuda", device if isinstance(device, int) else device.index)

    reads = layer_reads(spec, geometry, layer_ids, norm=norm)
    try:
        destinations = {(read.layer_id, read.kind): torch.empty(read.shape, dtype=torch.bfloat16, device=device)
                        for read in reads}
        _copy_staged(reads, geometry, spec.key_view, destinations, parallelism)
    except Exception as error:
        raise RuntimeError(f"failed to materialize local FFN weights: {error}") from error
    return [
        LoadedDenseLayer(
            layer_id=layer_id,
            i_proj=destinations[(layer_id, "i_proj")],
            o_proj=destinations[(layer_id, "o_proj")],
            norm_weight=destinations.get((layer_id, "norm")),
            eps=spec.rms_norm_eps,
        )
        for layer_id in layer_ids
    ]


def _copy_staged(
    reads: list[_Read],
    geometry: ShardGeometry,
    key_view: dict[str, Path],
    destinations: dict[tuple[int, str], torch.Tensor],
    parallelism: int,
) -> None:
    slot_bytes = max(read.staged_bytes for read in reads)
    slots: queue.Queue[torch.Tensor] = queue.Queue()
    for _ in range(min(parallelism, len(reads))):
        slots.put(torch.empty(slot_bytes, dtype=torch.uint8, pin_memory=True))
    staged: queue.Queue = queue.Queue()
    cancelled = threading.Event()

    def acquire() -> torch.Tensor | None:
        while not cancelled.is_set():
            try:
                return slots.get(timeout=0.1)
            except queue.Empty:
                continue
        return None

    def reader(read: _Read) -> None:
        slot = acquire()
        if slot is None:
            staged.put(("done", read, None))
            return
        try:
            view = slot[: read.staged_bytes].view(torch.bfloat16).view(read.shape)
            stage_read(read, geometry, key_view, view)
        except Exception as error:
            slots.put(slot)
            cancelled.set()
            staged.put(("failed", read, error))
            return
        staged.put(("staged", read, slot))

    first_error: Exception | None = None
    with concurrent.futures.ThreadPoolExecutor(max_workers=parallelism) as pool:
        futures = [pool.submit(reader, read) for read in reads]
        for _ in reads:
            state, read, payload = staged.get()
            if state == "failed":
                first_error = first_error or payload
                continue
            if state == "done":
                continue
            try:
                if first_error is None:
                    view = payload[: read.staged_bytes].view(torch.bfloat16).view(read.shape)
                    destinations[(read.layer_id, read.kind)].copy_(view, non_blocking=False)
            except Exception as error:  # a failed copy stops the readers too
                first_error = first_error or error
                cancelled.set()
            finally:
                slots.put(payload)
        for future in futures:
            future.result()
    if first_error is not None:
        raise first_error
