"""GPU tests of checkpoint loading into the FfnAgent (crosspool_amd.checkpoint).

A synthetic two-layer Qwen3-style checkpoint (bf16 or fp16 shards plus one fp32 tensor,
gate and up of a layer in different files) is loaded as TP rank 1 of 2.  The device
shards must be the checkpoint's dtype (the payload dtype the reference's loader keeps,
loader.py:485-508) and equal the closed-form TP slice of the source tensors bit for bit,
and a mailbox step through the loaded layers must meet the FFN parity gates against the
oracle run on those same slices.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from crosspool_amd import checkpoint as ck
from crosspool_amd.agent import FfnAgent
from oracle import ffn_oracle as o
from parity import assert_bitwise_equal, assert_ffn_parity, slots_tensor, to_device

pytestmark = pytest.mark.gpu

HIDDEN, INTERMEDIATE, LAYERS, TP_SIZE, TP_RANK = 256, 1024, 2, 2, 1


def _write_model(path: Path, dtype: torch.dtype = torch.bfloat16) -> dict[str, torch.Tensor]:
    generator = torch.Generator().manual_seed(18)
    tensors: dict[str, torch.Tensor] = {}
    for layer in range(LAYERS):
        gate, up, down = ck.mlp_keys(layer)
        tensors[gate] = (torch.randn(INTERMEDIATE, HIDDEN, generator=generator) * 0.05).to(dtype)
        tensors[up] = (torch.randn(INTERMEDIATE, HIDDEN, generator=generator) * 0.05).to(dtype)
        tensors[down] = (torch.randn(HIDDEN, INTERMEDIATE, generator=generator) * 0.05).to(dtype)
        tensors[ck.norm_key(layer)] = (1.0 + 0.1 * torch.randn(HIDDEN, generator=generator)).to(dtype)
    tensors[ck.mlp_keys(1)[2]] = tensors[ck.mlp_keys(1)[2]].float()  # one fp32 source (exact in the dtype)
    path.mkdir()
    config = {
        "architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3", "hidden_act": "silu",
        "torch_dtype": "float16" if dtype is torch.float16 else "bfloat16", "hidden_size": HIDDEN,
        "intermediate_size": INTERMEDIATE,
        "num_hidden_layers": LAYERS, "rms_norm_eps": 1e-6,
    }
    (path / "config.json").write_text(json.dumps(config), encoding="utf-8")
    first = {key: value for key, value in tensors.items() if not key.endswith("up_proj.weight")}
    second = {key: value for key, value in tensors.items() if key.endswith("up_proj.weight")}
    weight_map = {}
    for index, shard in enumerate((first, second), start=1):
        name = f"model-{index:05d}-of-00002.safetensors"
        save_file(shard, path / name)
        weight_map.update(dict.fromkeys(shard, name))
    (path / ck.INDEX_FILENAME).write_text(json.dumps({"weight_map": weight_map}), encoding="utf-8")
    return tensors


def _expected_shard(tensors: dict[str, torch.Tensor], layer: int,
                    dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    width = INTERMEDIATE // TP_SIZE
    start = TP_RANK * width
    gate, up, down = (tensors[key].to(dtype) for key in ck.mlp_keys(layer))
    i_proj = torch.empty(2 * width, HIDDEN, dtype=dtype)
    for j in range(width):
        i_proj[2 * j] = gate[start + j]
        i_proj[2 * j + 1] = up[start + j]
    return i_proj, down[:, start : start + width].contiguous(), tensors[ck.norm_key(layer)]


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16), ids=("bf16", "fp16"))
def test_checkpoint_layers_load_and_run(device, tmp_path: Path, dtype: torch.dtype) -> None:
    tensors = _write_model(tmp_path / "model", dtype)
    pool = o.generate_hidden_states(128, HIDDEN, 17).to(dtype)
    slots = o.generate_slots(128, 24, 19)
    with FfnAgent(device) as agent:
        loaded = agent.register_checkpoint(
            tmp_path / "model", instance_index=0, tp_size=TP_SIZE, tp_rank=TP_RANK, parallelism=2
        )
        assert [layer.layer_id for layer in loaded] == [0, 1]
        for layer in loaded:
            assert layer.i_proj.dtype is dtype and layer.o_proj.dtype is dtype and layer.norm_weight.dtype is dtype
            i_proj, o_proj, norm = _expected_shard(tensors, layer.layer_id, dtype)
            assert_bitwise_equal(layer.i_proj.cpu(), i_proj)
            assert_bitwise_equal(layer.o_proj.cpu(), o_proj)
            assert_bitwise_equal(layer.norm_weight.cpu(), norm)
            assert layer.eps == 1e-6
        agent.materialize(maximum_row_capacity=32)
        pool_gpu = to_device(pool, device)
        current = pool
        for layer in (0, 1):
            agent.execute(instance_index=0, layer_ordinal=layer, pool=pool_gpu, slots=slots_tensor(slots, device))
            agent.check_health()
            new_pool = pool_gpu.cpu()
            # The oracle step of this layer on the closed-form shard, from the pool as it was.
            i_proj, o_proj, norm = _expected_shard(tensors, layer, dtype)
            _, normalized, stage_rows = o.mailbox_step(current, slots, i_proj, o_proj, norm_weight=norm, eps=1e-6)
            untouched = np.setdiff1d(np.arange(pool.shape[0]), slots)
            assert_bitwise_equal(new_pool[untouched], pool[untouched])
            assert_ffn_parity(o.gather(new_pool, slots), stage_rows, o.dense_fp32(normalized, i_proj, o_proj))
            current = new_pool


def test_checkpoint_loading_reports_missing_layers(device, tmp_path: Path) -> None:
    _write_model(tmp_path / "model")
    with FfnAgent(device) as agent:
        with pytest.raises(ValueError, match="outside the model"):
            agent.register_checkpoint(tmp_path / "model", instance_index=0, layers=[2])
        with pytest.raises(ValueError, match="not divisible"):
            agent.register_checkpoint(tmp_path / "model", instance_index=0, tp_size=3)
