"""Local checkpoint loading for the Dense FFN path.

Reads a local Hugging Face checkpoint directory (``config.json`` plus safetensors
shards) of a gated Dense family and places each layer's tensor-parallel shard on
the GPU in the layout the kernels take: INTERLEAVED ``i_proj [2 L, H]`` (row 2j =
gate_j, row 2j+1 = up_j), ``o_proj [H, L]`` and, for the fused RMSNorm, the
post-attention norm weight ``[H]``.  L = I / tp_size, and rank r owns intermediate
rows ``[r L, (r + 1) L)``.

Contract kept from the reference (file:line in the CrossPool checkout); the code is
this module's own:

- accepted families and ``config.json`` fields: ``runtime/ffnagent/models/qwen3.py:13-45``
  and ``architecture.py:22-137,177-215`` (Qwen3, Qwen2 and Llama share the gated
  Dense profile; integer fields are strict JSON integers; the source dtype is bf16 or
  fp16, named ``torch_dtype`` or ``dtype``);
- which file holds each tensor: ``checkpoint.py:18-76`` (the index's weight map, or a
  lone canonical ``model.safetensors``; duplicate JSON members, path-like or
  non-safetensors shard names and missing shard files are refused);
- each layer's ``mlp.`` keys are exactly gate, up and down: ``checkpoint.py:79-93``;
- TP slice and Gate/Up row order: ``preparation.py:160-241``, ``ffn.py:57-68``;
- payload conversion and shape checks: ``loader.py:451-519``.

Error messages the reference's tests match are kept word for word (``exactly one
unindexed canonical``, ``duplicate JSON member``, ``missing=`` / ``extra=``, ``must be a
JSON integer``, ``must be greater than or equal to``, the offending field's name).

The post-attention norm weight (``model.layers.{i}.post_attention_layernorm.weight``)
is read as well, because this build fuses the norm into the gather; the reference
leaves the norm to SGLang.  The payload dtype is the checkpoint's source dtype, bf16 or
fp16, as the reference's loader keeps it (``loader.py:485-508``): tensors of that dtype
are copied bit for bit, wider floats are rounded to it (nearest even).
"""

from __future__ import annotations

import json
import math
import re
from collections import Counter, defaultdict
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path, PurePosixPath
from typing import Iterable

import torch

INDEX_FILENAME = "model.safetensors.index.json"
SINGLE_FILE_NAME = "model.safetensors"

# Gated Dense families (architecture name -> required model_type); all keep their FFN under
# ``model.layers.{i}.mlp``.
DENSE_FAMILIES = {
    "Qwen3ForCausalLM": "qwen3",
    "Qwen2ForCausalLM": "qwen2",
    "LlamaForCausalLM": "llama",
}
SOURCE_DTYPES = frozenset({"bfloat16", "float16"})
MLP_PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
_MLP_KEY = re.compile(r"model\.layers\.(\d+)\.mlp\.(.+)")


# ---------------------------------------------------------------- JSON and config fields
def _json_object(path: Path) -> dict:
    """The JSON object stored at ``path``; a member name repeated in any object is refused."""

    def build(pairs: list[tuple[str, object]]) -> dict:
        built = dict(pairs)
        if len(built) != len(pairs):
            repeated = next(name for name, count in Counter(name for name, _ in pairs).items() if count > 1)
            raise ValueError(f"duplicate JSON member {repeated!r} in {path}")
        return built

    document = json.loads(path.read_bytes(), object_pairs_hook=build)
    if not isinstance(document, dict):
        raise ValueError(f"{path} does not hold a JSON object")
    return document


class _Fields:
    """Typed reads of ``config.json`` members (strict JSON types, bounds in the message)."""

    def __init__(self, document: dict) -> None:
        self.document = document

    def integer(self, name: str, minimum: int = 1) -> int:
        value = self.document.get(name)
        if type(value) is not int:  # bool and float are not JSON integers here
            raise ValueError(f"{name} must be a JSON integer")
        if value < minimum:
            raise ValueError(f"{name} must be greater than or equal to {minimum}")
        return value

    def positive_number(self, name: str, default: float) -> float:
        value = self.document.get(name, default)
        if type(value) not in (int, float) or not math.isfinite(value) or value <= 0:
            raise ValueError(f"{name} must be a finite positive JSON number")
        return float(value)

    def text(self, name: str, required: str) -> None:
        if self.document.get(name) != required:
            raise ValueError(f"{name} is {self.document.get(name)!r}; this family requires {required!r}")

    def architecture(self) -> str:
        names = self.document.get("architectures")
        if type(names) is not list or len(names) != 1 or type(names[0]) is not str or not names[0]:
            raise ValueError("architectures must name exactly one architecture (a one-element array)")
        return names[0]

    def source_dtype(self) -> str:
        field = "dtype" if "dtype" in self.document and "torch_dtype" not in self.document else "torch_dtype"
        value = self.document.get(field)
        if value not in SOURCE_DTYPES:
            raise ValueError(f"{field} is {value!r}; the Dense FFN path reads 'bfloat16' or 'float16' checkpoints")
        return value


# ---------------------------------------------------------------- tensor key -> shard file
def _shard_file(model_path: Path, name: object, *, index_path: Path) -> Path:
    """The shard file an index entry names: a plain ``*.safetensors`` file name in the model
    directory that exists as a regular file (no directories, no symlinks)."""

    if type(name) is not str or not name:
        raise ValueError(f"{index_path} names an empty or non-string shard")
    if PurePosixPath(name).name != name or "\\" in name or not name.endswith(".safetensors"):
        raise ValueError(f"{index_path} names unsafe shard name {name!r} (a plain *.safetensors file name is required)")
    path = model_path / name
    if path.is_symlink() or not path.is_file():
        raise ValueError(f"shard file {path} is missing, a symlink or not a regular file")
    return path


def read_checkpoint_key_view(model_path: Path) -> dict[str, Path]:
    """Map every tensor key of the checkpoint to the file holding it, reading no tensor data.

    An index (``model.safetensors.index.json``) is authoritative when present; otherwise the
    directory must hold one safetensors file, ``model.safetensors``, whose header lists the keys.
    """

    model_path = Path(model_path)
    index_path = model_path / INDEX_FILENAME
    if index_path.exists():
        weight_map = _json_object(index_path).get("weight_map")
        if type(weight_map) is not dict or not weight_map:
            raise ValueError(f"{index_path} has no weight_map object with at least one entry")
        resolved: dict[str, Path] = {}
        files: dict[str, Path] = {}  # each distinct shard name is checked once
        for key, name in weight_map.items():
            if not key:
                raise ValueError(f"{index_path} maps an empty tensor key")
            if type(name) is not str or name not in files:
                files[name] = _shard_file(model_path, name, index_path=index_path)
            resolved[key] = files[name]
        return resolved

    candidates = sorted(entry for entry in model_path.iterdir() if entry.suffix == ".safetensors")
    canonical = model_path / SINGLE_FILE_NAME
    if candidates != [canonical]:
        raise ValueError(f"{model_path} must contain exactly one unindexed canonical {SINGLE_FILE_NAME} checkpoint")
    if canonical.is_symlink() or not canonical.is_file():
        raise ValueError(f"{canonical} is a symlink or not a regular file")
    from safetensors import safe_open

    with safe_open(str(canonical), framework="pt", device="cpu") as handle:
        keys = list(handle.keys())
    if not keys or not all(type(key) is str and key for key in keys):
        raise ValueError(f"checkpoint {canonical} lists an empty tensor key (or none)")
    return {key: canonical for key in keys}


def mlp_keys(layer_id: int) -> tuple[str, str, str]:
    """Gate, up and down weight keys of one layer (architecture.py:120-137)."""

    return tuple(f"model.layers.{layer_id}.mlp.{projection}.weight" for projection in MLP_PROJECTIONS)


def norm_key(layer_id: int) -> str:
    return f"model.layers.{layer_id}.post_attention_layernorm.weight"


def validate_ffn_coverage(key_view: dict[str, Path], layer_count: int) -> None:
    """Each layer below ``layer_count`` holds exactly its gate, up and down weights under ``mlp.``.

    Keys are grouped by the layer their ``model.layers.{i}.mlp.`` name gives; keys of other
    modules and of layers past the count do not take part.
    """

    by_layer: dict[int, set[str]] = defaultdict(set)
    for key in key_view:
        match = _MLP_KEY.fullmatch(key)
        if match is not None:
            by_layer[int(match.group(1))].add(key)
    for layer_id in range(layer_count):
        wanted = set(mlp_keys(layer_id))
        found = by_layer.get(layer_id, set())
        if found != wanted:
            raise ValueError(
                f"FFN checkpoint namespace for layer {layer_id} differs: missing={sorted(wanted - found)}, "
                f"extra={sorted(found - wanted)}"
            )


@dataclass(frozen=True, slots=True)
class DenseModelSpec:
    """FFN facts of a gated Dense checkpoint (the reference's FfnModelSpec, qwen3.py:24-45)."""

    architecture: str
    hidden_size: int
    intermediate_size: int
    layer_count: int
    rms_norm_eps: float
    key_view: dict[str, Path]
    payload_dtype: torch.dtype = torch.bfloat16  # the source dtype (bf16 or fp16)


def load_model_spec(model_path: Path) -> DenseModelSpec:
    """Read ``config.json`` and the key view, and check the FFN keys of every layer.

    Any failure is re-raised as RuntimeError naming the checkpoint (architecture.py:177-215).
    """

    model_path = Path(model_path)
    try:
        fields = _Fields(_json_object(model_path / "config.json"))
        architecture = fields.architecture()
        if architecture not in DENSE_FAMILIES:
            raise ValueError(f"unsupported FFN architecture {architecture!r} (gated Dense families: "
                             f"{', '.join(sorted(DENSE_FAMILIES))})")
        fields.text("model_type", DENSE_FAMILIES[architecture])
        fields.text("hidden_act", "silu")
        source_dtype = fields.source_dtype()
        spec = DenseModelSpec(
            architecture=architecture,
            hidden_size=fields.integer("hidden_size"),
            intermediate_size=fields.integer("intermediate_size"),
            layer_count=fields.integer("num_hidden_layers"),
            rms_norm_eps=fields.positive_number("rms_norm_eps", 1e-6),
            key_view=read_checkpoint_key_view(model_path),
            payload_dtype=torch.float16 if source_dtype == "float16" else torch.bfloat16,
        )
        validate_ffn_coverage(spec.key_view, spec.layer_count)
        return spec
    except Exception as error:
        raise RuntimeError(f"checkpoint at {model_path} is not a loadable gated Dense FFN model: {error}") from error


# ---------------------------------------------------------------- TP geometry and reads
@dataclass(frozen=True, slots=True)
class ShardGeometry:
    """One rank's slice of the intermediate dimension (preparation.py:160-241)."""

    hidden_size: int
    intermediate_size: int
    tp_size: int
    tp_rank: int

    def __post_init__(self) -> None:
        if type(self.tp_size) is not int or type(self.tp_rank) is not int:
            raise ValueError("TP size and rank must be integers")
        if not 0 <= self.tp_rank < self.tp_size:
            raise ValueError(f"TP rank {self.tp_rank} is outside the TP domain of size {self.tp_size}")
        if self.intermediate_size % self.tp_size:
            raise ValueError(f"intermediate size {self.intermediate_size} is not divisible by TP size {self.tp_size}")

    @property
    def local_width(self) -> int:
        return self.intermediate_size // self.tp_size

    @property
    def source_start(self) -> int:
        return self.tp_rank * self.local_width


@dataclass(frozen=True, slots=True)
class StagedValue:
    """One device value of one layer and the checkpoint keys it is assembled from."""

    layer_id: int
    kind: str  # "i_proj", "o_proj" or "norm"
    keys: tuple[str, ...]
    shape: tuple[int, ...]

    @property
    def nbytes(self) -> int:
        return math.prod(self.shape) * 2


def layer_reads(spec: DenseModelSpec, geometry: ShardGeometry, layer_ids: Iterable[int], *,
                norm: bool) -> list[StagedValue]:
    hidden, width = geometry.hidden_size, geometry.local_width
    values = []
    for layer_id in layer_ids:
        gate, up, down = mlp_keys(layer_id)
        values.append(StagedValue(layer_id, "i_proj", (gate, up), (2 * width, hidden)))
        values.append(StagedValue(layer_id, "o_proj", (down,), (hidden, width)))
        if norm:
            values.append(StagedValue(layer_id, "norm", (norm_key(layer_id),), (hidden,)))
    return values


def _checked_slice(handle, key: str, full_shape: tuple[int, ...], region: tuple[slice, ...],
                   dtype: torch.dtype) -> torch.Tensor:
    """``region`` of tensor ``key`` in the payload ``dtype``, after checking the tensor's full
    shape and type."""

    lazy = handle.get_slice(key)
    found = tuple(lazy.get_shape())
    if found != full_shape:
        raise ValueError(f"tensor {key!r} is {found}, the model config implies {full_shape}")
    data = lazy[region]
    if not data.is_floating_point():
        raise ValueError(f"tensor {key!r} holds {data.dtype}, not a floating-point type")
    return data.to(dtype)  # a copy in the payload dtype, nearest-even rounding for wider floats


def stage_read(value: StagedValue, geometry: ShardGeometry, key_view: dict[str, Path], out: torch.Tensor) -> None:
    """Fill the host tensor ``out`` (payload dtype, ``value.shape``) from the checkpoint; no GPU work.

    ``i_proj``: rows 2j and 2j+1 are gate and up row ``start + j``; ``o_proj``: columns
    ``[start, start + L)`` of down; ``norm``: the whole vector.
    """

    from safetensors import safe_open

    hidden, intermediate = geometry.hidden_size, geometry.intermediate_size
    rows = slice(geometry.source_start, geometry.source_start + geometry.local_width)
    files = []
    for key in value.keys:
        if key not in key_view:
            raise ValueError(f"no shard file holds tensor {key!r}")
        files.append(key_view[key])
    handles = {path: safe_open(str(path), framework="pt", device="cpu") for path in set(files)}
    if value.kind == "i_proj":
        # out viewed as [L, 2, H]: plane 0 takes the gate rows, plane 1 the up rows.
        pairs = out.view(geometry.local_width, 2, hidden)
        for plane, (key, path) in enumerate(zip(value.keys, files)):
            pairs[:, plane].copy_(_checked_slice(handles[path], key, (intermediate, hidden), (rows,), out.dtype))
    elif value.kind == "o_proj":
        out.copy_(_checked_slice(handles[files[0]], value.keys[0], (hidden, intermediate), (slice(None), rows),
                                 out.dtype))
    else:
        out.copy_(_checked_slice(handles[files[0]], value.keys[0], (hidden,), (slice(None),), out.dtype))


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

    The device tensors are allocated first; host reads then run ``parallelism`` at a time
    into a ring of pinned buffers, and each staged value goes to its device tensor by an
    asynchronous copy on a side stream.  Any failure raises RuntimeError after the reads in
    flight have ended.
    """

    if parallelism <= 0:
        raise ValueError("loader parallelism must be positive")
    spec = load_model_spec(Path(model_path))
    geometry = ShardGeometry(spec.hidden_size, spec.intermediate_size, tp_size, tp_rank)
    if spec.hidden_size % 8 or geometry.local_width % 8:
        raise ValueError("hidden size and local intermediate size must be multiples of 8 on this path")
    layer_ids = list(range(spec.layer_count)) if layers is None else list(layers)
    outside = [layer_id for layer_id in layer_ids if not 0 <= layer_id < spec.layer_count]
    if outside:
        raise ValueError(f"layers {outside} are outside the model's {spec.layer_count} layers")
    if device is None:
        device = torch.cuda.current_device()
    device = torch.device("cuda", device if isinstance(device, int) else device.index)

    values = layer_reads(spec, geometry, layer_ids, norm=norm)
    try:
        targets = [torch.empty(value.shape, dtype=spec.payload_dtype, device=device) for value in values]
        _PinnedRing(min(parallelism, len(values)), max(value.nbytes for value in values), device,
                    spec.payload_dtype).run(
            values, targets, geometry, spec.key_view
        )
    except Exception as error:
        raise RuntimeError(f"loading the FFN shards of {model_path} onto {device} failed: {error}") from error
    placed = {(value.layer_id, value.kind): target for value, target in zip(values, targets)}
    return [
        LoadedDenseLayer(layer_id, placed[(layer_id, "i_proj")], placed[(layer_id, "o_proj")],
                         placed.get((layer_id, "norm")), spec.rms_norm_eps)
        for layer_id in layer_ids
    ]


class _PinnedRing:
    """A ring of pinned host buffers between host reads and device copies.

    Value i is read into buffer i mod N by a worker thread; the calling thread then copies
    it to the device on a side stream and records an event.  Buffer b is handed to its next
    read only after that event has completed, so at most N host reads and the copies behind
    them overlap.  Worker threads never touch the GPU.
    """

    def __init__(self, count: int, nbytes: int, device: torch.device, dtype: torch.dtype = torch.bfloat16) -> None:
        self.buffers = [torch.empty(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(count)]
        self.copied: list[torch.cuda.Event | None] = [None] * count
        self.device = device
        self.dtype = dtype

    def _view(self, index: int, value: StagedValue) -> torch.Tensor:
        buffer = self.buffers[index % len(self.buffers)]
        return buffer[: value.nbytes].view(self.dtype).view(value.shape)

    def run(self, values: list[StagedValue], targets: list[torch.Tensor], geometry: ShardGeometry,
            key_view: dict[str, Path]) -> None:
        count = len(self.buffers)
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))  # the targets' allocation
        reads: dict[int, Future] = {}
        with ThreadPoolExecutor(max_workers=count) as workers:

            def start(index: int) -> None:
                ring_slot = index % count
                if self.copied[ring_slot] is not None:
                    self.copied[ring_slot].synchronize()
                reads[index] = workers.submit(stage_read, values[index], geometry, key_view,
                                              self._view(index, values[index]))

            try:
                for index in range(min(count, len(values))):
                    start(index)
                for index, (value, target) in enumerate(zip(values, targets)):
                    reads.pop(index).result()
                    with torch.cuda.stream(stream):
                        target.copy_(self._view(index, value), non_blocking=True)
                        event = torch.cuda.Event()
                        event.record(stream)
                    self.copied[index % count] = event
                    if index + count < len(values):
                        start(index + count)
            finally:
                for pending in reads.values():
                    pending.cancel()
                # Copies already issued write into the targets: they must land before a
                # failure lets the targets go back to the allocator.
                stream.synchronize()
