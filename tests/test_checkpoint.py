"""Packed-expert storage and its safetensors loader / saver (CPU only)."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from oxidizr_amd.checkpoint import (CheckpointError, PackedExperts, from_checkpoint_name,
                                    load_packed, moe_layer_names, save_packed,
                                    to_checkpoint_name)


def test_checkpoint_names_follow_the_reference():
    # the cases of src/checkpoint_names.rs's own tests
    n = "layers.0.self_attn.q_proj.weight"
    assert to_checkpoint_name(n) == "model.layers.0.self_attn.q_proj.weight"
    assert from_checkpoint_name(to_checkpoint_name(n)) == n
    assert to_checkpoint_name("lm_head.weight") == "lm_head.weight"
    assert from_checkpoint_name("lm_head.weight") == "lm_head.weight"
    lora = "layers.3.self_attn.q_proj.lora_a"
    assert from_checkpoint_name(to_checkpoint_name(lora)) == lora
    assert from_checkpoint_name("layers.1.mlp.up_proj.weight") == "layers.1.mlp.up_proj.weight"


def test_moe_layer_names_order():
    names = moe_layer_names(2, 2, shared=True)
    assert names == [
        "layers.2.moe.router.gate.weight",
        "layers.2.moe.experts.0.gate_proj.weight", "layers.2.moe.experts.0.up_proj.weight",
        "layers.2.moe.experts.0.down_proj.weight",
        "layers.2.moe.experts.1.gate_proj.weight", "layers.2.moe.experts.1.up_proj.weight",
        "layers.2.moe.experts.1.down_proj.weight",
        "layers.2.moe.shared_expert.gate_proj.weight", "layers.2.moe.shared_expert.up_proj.weight",
        "layers.2.moe.shared_expert.down_proj.weight"]


def _random_packed(H=16, E=3, I=8, S=8, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    pk = PackedExperts.empty(H, E, I, S, dtype=dtype, device="cpu")
    for t in [pk.router, pk.gate, pk.up, pk.down, *(pk.shared or ())]:
        t.copy_(torch.randn(t.shape, generator=g).to(dtype))
    return pk


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_save_then_load_round_trips_bitwise(tmp_path, dtype):
    pk = _random_packed(dtype=dtype)
    path = str(tmp_path / "layer.safetensors")
    save_packed(path, 5, pk)
    back = load_packed(path, 5, 16, 3, 8, 8, device="cpu")
    for a, b in [(pk.router, back.router), (pk.gate, back.gate), (pk.up, back.up),
                 (pk.down, back.down)] + list(zip(pk.shared, back.shared)):
        assert a.dtype == b.dtype and torch.equal(a, b)


def test_load_from_per_expert_tensors_in_any_order_and_files(tmp_path):
    # a checkpoint written tensor by tensor (as the reference stores experts),
    # split over two files in shuffled order
    H, E, I = 16, 4, 8
    rng = np.random.default_rng(1)
    tensors = {}
    for n in moe_layer_names(0, E, shared=False):
        if n.endswith("router.gate.weight"):
            shape = (E, H)
        elif n.endswith("down_proj.weight"):
            shape = (H, I)
        else:
            shape = (I, H)
        tensors[to_checkpoint_name(n)] = torch.tensor(rng.standard_normal(shape), dtype=torch.float32)
    keys = list(tensors)
    rng.shuffle(keys)
    save_file({k: tensors[k] for k in keys[:7]}, str(tmp_path / "a.safetensors"))
    save_file({k: tensors[k] for k in keys[7:]}, str(tmp_path / "b.safetensors"))
    pk = load_packed([str(tmp_path / "a.safetensors"), str(tmp_path / "b.safetensors")], 0, H, E, I,
                     device="cpu")
    assert pk.shared is None
    for e in range(E):
        p = f"model.layers.0.moe.experts.{e}"
        assert torch.equal(pk.gate[e], tensors[f"{p}.gate_proj.weight"])
        assert torch.equal(pk.up[e], tensors[f"{p}.up_proj.weight"])
        assert torch.equal(pk.down[e], tensors[f"{p}.down_proj.weight"])
    assert torch.equal(pk.router, tensors["model.layers.0.moe.router.gate.weight"])
    # expert e is a view at a fixed stride of one allocation: the pointer table
    # of a plan takes these addresses as they are
    g, u, d = pk.experts()
    esz = pk.gate.element_size()
    for e in range(E):
        assert g[e].data_ptr() == pk.gate.data_ptr() + e * I * H * esz
        assert d[e].data_ptr() == pk.down.data_ptr() + e * H * I * esz


def test_missing_and_misshaped_tensors_are_errors(tmp_path):
    pk = _random_packed(S=0)
    path = str(tmp_path / "l.safetensors")
    save_packed(path, 0, pk)
    with pytest.raises(CheckpointError, match="model.layers.0.moe.shared_expert.gate_proj.weight"):
        load_packed(path, 0, 16, 3, 8, 8, device="cpu")
    with pytest.raises(CheckpointError, match=r"shape mismatch for 'model.layers.0.moe.router"
                                              r".gate.weight': expected \[3, 32\], got \[3, 16\]"):
        load_packed(path, 0, 32, 3, 8, 0, device="cpu")
