"""CPU tests of the local checkpoint loader (crosspool_amd.checkpoint).

Cases follow the reference's own loader tests: single-file and indexed key views
(test_checkpoint.py:12-28), exact FFN key coverage and strict configs
(test_architecture.py:60-110, 186-230), and the true-TP packing known answer
(integration test_loader.py:153-240: I = 6, TP 2, rank 1 takes rows 3..5 of gate and
up interleaved and columns 3..5 of down).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from crosspool_amd import checkpoint as ck


def dense_keys(layer_id: int) -> tuple[str, ...]:
    return ck.mlp_keys(layer_id)


def qwen3_config(hidden: int, intermediate: int, layers: int, **overrides) -> dict:
    config = {
        "architectures": ["Qwen3ForCausalLM"],
        "model_type": "qwen3",
        "hidden_act": "silu",
        "torch_dtype": "bfloat16",
        "hidden_size": hidden,
        "intermediate_size": intermediate,
        "num_hidden_layers": layers,
        "rms_norm_eps": 1e-6,
    }
    config.update(overrides)
    return config


def write_checkpoint(path: Path, config: dict, shards: list[dict[str, torch.Tensor]]) -> None:
    path.mkdir()
    (path / "config.json").write_text(json.dumps(config), encoding="utf-8")
    weight_map = {}
    for index, tensors in enumerate(shards, start=1):
        name = f"model-{index:05d}-of-{len(shards):05d}.safetensors"
        save_file(tensors, path / name)
        weight_map.update(dict.fromkeys(tensors, name))
    (path / ck.INDEX_FILENAME).write_text(json.dumps({"weight_map": weight_map}), encoding="utf-8")


def tensor_values(shape: tuple[int, ...], start: int) -> torch.Tensor:
    """Recognisable bf16 values (exact integers)."""

    return torch.arange(start, start + int(np.prod(shape)), dtype=torch.float32).reshape(shape).to(torch.bfloat16)


# ---------------------------------------------------------------- key view
def test_single_file_checkpoint_uses_safetensors_header(tmp_path: Path) -> None:
    path = tmp_path / "model.safetensors"
    save_file({"model.layers.0.mlp.gate_proj.weight": torch.zeros(1)}, path)
    assert ck.read_checkpoint_key_view(tmp_path) == {"model.layers.0.mlp.gate_proj.weight": path}


def test_unindexed_checkpoint_rejects_ambiguous_files(tmp_path: Path) -> None:
    for name in ("model.safetensors", "other.safetensors"):
        save_file({name: torch.zeros(1)}, tmp_path / name)
    with pytest.raises(ValueError, match="exactly one unindexed canonical"):
        ck.read_checkpoint_key_view(tmp_path)


@pytest.mark.parametrize(
    ("shard_name", "message"),
    [("../escape.safetensors", "unsafe shard name"), ("model.bin", "unsafe shard name"), ("absent.safetensors", "missing, a symlink")],
)
def test_index_rejects_unsafe_or_missing_shards(tmp_path: Path, shard_name: str, message: str) -> None:
    (tmp_path / ck.INDEX_FILENAME).write_text(json.dumps({"weight_map": {"a": shard_name}}), encoding="utf-8")
    with pytest.raises(ValueError, match=message):
        ck.read_checkpoint_key_view(tmp_path)


def test_duplicate_json_members_are_rejected(tmp_path: Path) -> None:
    model = tmp_path / "model"
    model.mkdir()
    (model / "config.json").write_bytes(b'{"architectures":[],"architectures":[]}')
    with pytest.raises(RuntimeError, match="duplicate JSON member 'architectures'"):
        ck.load_model_spec(model)


# ---------------------------------------------------------------- config and coverage
def _indexed_model(path: Path, config: dict, keys: tuple[str, ...]) -> None:
    path.mkdir()
    (path / "config.json").write_text(json.dumps(config), encoding="utf-8")
    (path / "model-00001-of-00001.safetensors").write_bytes(b"")
    (path / ck.INDEX_FILENAME).write_text(
        json.dumps({"weight_map": dict.fromkeys(keys, "model-00001-of-00001.safetensors")}), encoding="utf-8"
    )


@pytest.mark.parametrize(
    ("layer_keys", "message"),
    [
        ((*dense_keys(0), "model.layers.0.mlp.unowned.weight"), r"extra=.*unowned"),
        (dense_keys(0)[1:], r"missing=.*gate_proj"),
    ],
)
def test_load_requires_exact_declared_ffn_keys(tmp_path: Path, layer_keys, message: str) -> None:
    keys = (*layer_keys, *(key for layer in range(1, 3) for key in dense_keys(layer)))
    _indexed_model(tmp_path / "model", qwen3_config(16, 32, 3), keys)
    with pytest.raises(RuntimeError, match=message):
        ck.load_model_spec(tmp_path / "model")


@pytest.mark.parametrize(
    ("architecture", "model_type"),
    [("Qwen3ForCausalLM", "qwen3"), ("Qwen2ForCausalLM", "qwen2"), ("LlamaForCausalLM", "llama")],
)
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_load_compiles_gated_dense_families(tmp_path: Path, architecture: str, model_type: str, dtype: str) -> None:
    config = qwen3_config(16, 32, 3, architectures=[architecture], model_type=model_type, torch_dtype=dtype)
    keys = tuple(key for layer in range(3) for key in dense_keys(layer))
    # Keys of other modules (attention, norms, a layer past the count) are outside the FFN namespaces.
    _indexed_model(tmp_path / "model", config, (*keys, *dense_keys(3), "model.layers.0.self_attn.q_proj.weight"))
    spec = ck.load_model_spec(tmp_path / "model")
    assert (spec.architecture, spec.hidden_size, spec.intermediate_size, spec.layer_count) == (architecture, 16, 32, 3)
    assert spec.rms_norm_eps == 1e-6


@pytest.mark.parametrize(
    ("override", "message"),
    [
        ({"torch_dtype": "float32"}, "torch_dtype"),
        ({"torch_dtype": None}, "torch_dtype"),
        ({"model_type": "llama"}, "model_type"),
        ({"hidden_act": "relu"}, "hidden_act"),
        ({"architectures": ["OPTForCausalLM"]}, "unsupported FFN architecture"),
        ({"architectures": ["Qwen3ForCausalLM", "Qwen3ForCausalLM"]}, "one-element array"),
        ({"hidden_size": 0}, "hidden_size must be greater than or equal to 1"),
        ({"intermediate_size": 32.0}, "intermediate_size must be a JSON integer"),
        ({"num_hidden_layers": True}, "num_hidden_layers must be a JSON integer"),
        ({"rms_norm_eps": -1.0}, "rms_norm_eps"),
    ],
)
def test_load_rejects_inadmissible_configs(tmp_path: Path, override: dict, message: str) -> None:
    keys = tuple(key for layer in range(3) for key in dense_keys(layer))
    _indexed_model(tmp_path / "model", qwen3_config(16, 32, 3, **override), keys)
    with pytest.raises(RuntimeError, match=message):
        ck.load_model_spec(tmp_path / "model")


# ---------------------------------------------------------------- TP packing
def _layer_tensors(layer_id: int, hidden: int, intermediate: int, base: int) -> dict[str, torch.Tensor]:
    gate, up, down = dense_keys(layer_id)
    return {
        gate: tensor_values((intermediate, hidden), base),
        up: tensor_values((intermediate, hidden), base + 100),
        down: tensor_values((hidden, intermediate), base + 200),
        ck.norm_key(layer_id): tensor_values((hidden,), base + 60),
    }


def _stage(spec: ck.DenseModelSpec, geometry: ck.ShardGeometry, layer_id: int) -> dict[str, torch.Tensor]:
    out = {}
    for read in ck.layer_reads(spec, geometry, [layer_id], norm=True):
        out[read.kind] = torch.empty(read.shape, dtype=torch.bfloat16)
        ck.stage_read(read, geometry, spec.key_view, out[read.kind])
    return out


def test_true_tp_packing_known_answer(tmp_path: Path) -> None:
    # The reference's packing case: H = 4, I = 6, TP 2, rank 1.  Layer 0's gate and up sit
    # in different shards from its down and norm, so one value reads two files.
    hidden, intermediate = 4, 6
    tensors = _layer_tensors(0, hidden, intermediate, 0)
    gate, up, down = dense_keys(0)
    write_checkpoint(
        tmp_path / "model",
        qwen3_config(hidden, intermediate, 1),
        [{gate: tensors[gate]}, {up: tensors[up], down: tensors[down], ck.norm_key(0): tensors[ck.norm_key(0)]}],
    )
    spec = ck.load_model_spec(tmp_path / "model")
    geometry = ck.ShardGeometry(hidden, intermediate, tp_size=2, tp_rank=1)
    assert (geometry.source_start, geometry.local_width) == (3, 3)
    staged = _stage(spec, geometry, 0)
    # Row 2j = gate row 3 + j, row 2j + 1 = up row 3 + j: gate rows start at 12 (3 x 4),
    # up rows at 100 + 12.
    expected_i = torch.tensor(
        [[12 + 4 * j + h if parity == 0 else 112 + 4 * j + h for h in range(4)] for j in range(3) for parity in (0, 1)],
        dtype=torch.float32,
    )
    assert torch.equal(staged["i_proj"].float(), expected_i)
    # down [4, 6] starts at 200; columns 3..5 of row h are 200 + 6 h + 3 ..
    expected_o = torch.tensor([[200 + 6 * h + 3 + c for c in range(3)] for h in range(4)], dtype=torch.float32)
    assert torch.equal(staged["o_proj"].float(), expected_o)
    assert torch.equal(staged["norm"].float(), torch.arange(60, 64, dtype=torch.float32))


def test_wider_sources_round_to_nearest_even(tmp_path: Path) -> None:
    hidden, intermediate = 8, 8
    generator = torch.Generator().manual_seed(5)
    tensors = {key: torch.randn(value.shape, generator=generator) for key, value in
               _layer_tensors(0, hidden, intermediate, 0).items()}
    tensors[dense_keys(0)[1]] = tensors[dense_keys(0)[1]].to(torch.float16)  # up in fp16
    write_checkpoint(tmp_path / "model", qwen3_config(hidden, intermediate, 1), [tensors])
    spec = ck.load_model_spec(tmp_path / "model")
    staged = _stage(spec, ck.ShardGeometry(hidden, intermediate, 1, 0), 0)

    def rne(values: torch.Tensor) -> np.ndarray:
        # bf16 bits of float32 values by the round-to-nearest-even bit formula.
        bits = values.float().numpy().view(np.uint32).astype(np.uint64)
        return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)

    gate, up, _ = dense_keys(0)
    got = staged["i_proj"].view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[0::2], rne(tensors[gate]))
    assert np.array_equal(got[1::2], rne(tensors[up].float()))


def test_reads_reject_wrong_shapes_and_integer_tensors(tmp_path: Path) -> None:
    hidden, intermediate = 4, 6
    tensors = _layer_tensors(0, hidden, intermediate, 0)
    gate, up, down = dense_keys(0)
    tensors[down] = tensor_values((hidden, intermediate + 2), 0)
    tensors[up] = torch.zeros((intermediate, hidden), dtype=torch.int32)
    write_checkpoint(tmp_path / "model", qwen3_config(hidden, intermediate, 1), [tensors])
    spec = ck.load_model_spec(tmp_path / "model")
    geometry = ck.ShardGeometry(hidden, intermediate, 1, 0)
    reads = {read.kind: read for read in ck.layer_reads(spec, geometry, [0], norm=True)}
    with pytest.raises(ValueError, match=r"is \(4, 8\), the model config implies \(4, 6\)"):
        ck.stage_read(reads["o_proj"], geometry, spec.key_view, torch.empty(reads["o_proj"].shape, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="not a floating-point type"):
        ck.stage_read(reads["i_proj"], geometry, spec.key_view, torch.empty(reads["i_proj"].shape, dtype=torch.bfloat16))


@pytest.mark.parametrize(
    ("tp_size", "tp_rank", "message"),
    [(4, 0, "not divisible"), (2, 2, "outside the TP domain"), (0, 0, "outside the TP domain"), (2, True, "integers")],
)
def test_shard_geometry_rejects_bad_coordinates(tp_size, tp_rank, message: str) -> None:
    with pytest.raises(ValueError, match=message):
        ck.ShardGeometry(16, 6, tp_size=tp_size, tp_rank=tp_rank)
