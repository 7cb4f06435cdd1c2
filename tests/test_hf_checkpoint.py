"""Routed-expert banks from a Hugging Face block-FP8 safetensors checkpoint
(freetoken_amd/checkpoint/hf.py; reference models/qwen3_5_moe/weight.py:834-1055,
checkpoint/convert.py:163-330), on small synthetic checkpoints in the HF layout
written with safetensors: both name prefixes, a dense prefix layer, shards
split mid-layer, non-expert tensors that must be ignored.  CPU only."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import experts as X
from oracle import synth
from oracle.numerics import bf16_round
from freetoken_amd.checkpoint import load_ftw_banks
from freetoken_amd.checkpoint.hf import convert_hf_experts_to_ftw, load_hf_expert_banks, scan_experts


def write_hf_checkpoint(path, prefix: str, dense: int, L: int, E: int, H: int, I: int, seed: int = 0,
                        scale_dtype=torch.bfloat16, shards: int = 2, mtp: bool = True):
    """A block-FP8 checkpoint: ``dense`` dense layers, then ``L`` MoE layers of
    ``E`` experts; returns the oracle banks per MoE layer (scales as stored).

    With ``mtp`` the checkpoint also holds a multi-token-prediction head's
    experts where the two model families store them: ``mtp.layers.0`` (Qwen3.5,
    ``model.language_model`` stem) or ``model.layers.<num_hidden_layers>``
    (DeepSeek-V3, ``model.layers`` stem), which the loader must drop."""
    import safetensors.torch as st

    rng = np.random.default_rng(seed)
    tensors, banks = {}, []
    if mtp:
        mtp_prefix = "mtp.layers.0" if prefix.startswith("model.language_model") else f"{prefix}.{dense + L}"
        junk = synth.make_bank("fp8", E, H, I, np.random.default_rng(seed + 99))
        for e in range(E):
            p = f"{mtp_prefix}.mlp.experts.{e}"
            gu = torch.from_numpy(junk.gate_up[e]).view(torch.float8_e4m3fn)
            tensors[f"{p}.gate_proj.weight"] = gu[:I].contiguous()
            tensors[f"{p}.up_proj.weight"] = gu[I:].contiguous()
            tensors[f"{p}.down_proj.weight"] = torch.from_numpy(junk.down[e]).view(torch.float8_e4m3fn).contiguous()
            s_gu = torch.from_numpy(junk.gate_up_scale[e]).to(scale_dtype)
            tensors[f"{p}.gate_proj.weight_scale_inv"] = s_gu[: I // 128].contiguous()
            tensors[f"{p}.up_proj.weight_scale_inv"] = s_gu[I // 128:].contiguous()
            tensors[f"{p}.down_proj.weight_scale_inv"] = torch.from_numpy(junk.down_scale[e]).to(scale_dtype)
    for li in range(L):
        bank = synth.make_bank("fp8", E, H, I, rng)
        sc = torch.from_numpy(bank.gate_up_scale).to(scale_dtype)
        sd = torch.from_numpy(bank.down_scale).to(scale_dtype)
        bank.gate_up_scale = sc.float().numpy()
        bank.down_scale = sd.float().numpy()
        banks.append(bank)
        layer = dense + li
        for e in range(E):
            p = f"{prefix}.{layer}.mlp.experts.{e}"
            gu = torch.from_numpy(bank.gate_up[e]).view(torch.float8_e4m3fn)
            tensors[f"{p}.gate_proj.weight"] = gu[:I].contiguous()
            tensors[f"{p}.up_proj.weight"] = gu[I:].contiguous()
            tensors[f"{p}.down_proj.weight"] = torch.from_numpy(bank.down[e]).view(torch.float8_e4m3fn).contiguous()
            tensors[f"{p}.gate_proj.weight_scale_inv"] = sc[e, : I // 128].contiguous()
            tensors[f"{p}.up_proj.weight_scale_inv"] = sc[e, I // 128:].contiguous()
            tensors[f"{p}.down_proj.weight_scale_inv"] = sd[e].contiguous()
        tensors[f"{prefix}.{layer}.mlp.gate.weight"] = torch.randn(E, H).to(torch.bfloat16)
        tensors[f"{prefix}.{layer}.mlp.shared_experts.down_proj.weight"] = torch.zeros(H, I, dtype=torch.float8_e4m3fn)
    for d in range(dense):
        tensors[f"{prefix}.{d}.mlp.down_proj.weight"] = torch.randn(H, I).to(torch.bfloat16)
    tensors["lm_head.weight"] = torch.randn(8, H).to(torch.bfloat16)
    names = list(tensors)
    np.random.default_rng(seed + 1).shuffle(names)  # experts of one layer spread over the shards
    wmap = {}
    os.makedirs(path, exist_ok=True)
    for s in range(shards):
        file = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        part = {n: tensors[n] for n in names[s::shards]}
        st.save_file(part, os.path.join(path, file))
        wmap.update({n: file for n in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)
    with open(os.path.join(path, "config.json"), "w") as f:
        cfg = {"hidden_size": H, "moe_intermediate_size": I, "n_routed_experts": E, "num_hidden_layers": dense + L,
               "num_nextn_predict_layers": int(mtp)}
        if prefix.startswith("model.language_model"):
            cfg = {"text_config": cfg}
        json.dump(cfg, f)
    os.makedirs(os.path.join(path, "tok"), exist_ok=True)
    with open(os.path.join(path, "tok", "tokenizer.json"), "w") as f:
        f.write("{}")
    return banks


@pytest.mark.parametrize("prefix,dense", [("model.layers", 3), ("model.language_model.layers", 1)])
def test_fp8_banks_hold_the_checkpoint_bytes(tmp_path, prefix, dense):
    L, E, H, I = 2, 4, 256, 128
    banks = write_hf_checkpoint(tmp_path, prefix, dense, L, E, H, I)
    lay, _ = scan_experts(str(tmp_path))
    assert (lay.num_layers, lay.num_experts, lay.hidden, lay.inter, lay.first_moe_layer) == (L, E, H, I, dense)
    assert lay.scale_dtype == torch.bfloat16
    fmt, src, _ = load_hf_expert_banks(str(tmp_path), pinned=False, workers=3)
    assert fmt == "fp8_block" and list(src) == ["gate_up", "gate_up_scale", "down", "down_scale"]
    for li, b in enumerate(banks):
        np.testing.assert_array_equal(src["gate_up"][li].view(torch.uint8).numpy(), b.gate_up)
        np.testing.assert_array_equal(src["down"][li].view(torch.uint8).numpy(), b.down)
        assert src["gate_up_scale"][li].dtype == torch.float32  # widened for the kernels
        np.testing.assert_array_equal(src["gate_up_scale"][li].numpy(), b.gate_up_scale)
        np.testing.assert_array_equal(src["down_scale"][li].numpy(), b.down_scale)
    _, src16, _ = load_hf_expert_banks(str(tmp_path), pinned=False, scales_to_float32=False)
    assert src16["down_scale"][0].dtype == torch.bfloat16


def test_bf16_mode_dequantises_every_expert(tmp_path):
    """The FREETOKEN_FP8_EXPERTS=bf16 route: bf16(fp8 * block scale), the oracle's dequant rounded to bf16."""
    L, E, H, I = 2, 3, 256, 256
    banks = write_hf_checkpoint(tmp_path, "model.layers", 1, L, E, H, I, seed=4, scale_dtype=torch.float32)
    fmt, src, lay = load_hf_expert_banks(str(tmp_path), mode="bf16", pinned=False)
    assert fmt == "bf16" and list(src) == ["gate_up", "down"] and lay.scale_dtype == torch.float32
    for li, b in enumerate(banks):
        np.testing.assert_array_equal(src["gate_up"][li].float().numpy(),
                                      bf16_round(X.dequant_fp8_block(b.gate_up, b.gate_up_scale)))
        np.testing.assert_array_equal(src["down"][li].float().numpy(),
                                      bf16_round(X.dequant_fp8_block(b.down, b.down_scale)))


@pytest.mark.parametrize("per_layer", [True, False])
def test_convert_to_ftw_round_trip(tmp_path, per_layer):
    """HF -> FTW (the reference's converter for the expert banks): bf16 scales kept
    as stored, metadata files copied, and loading the FTW gives the same banks as
    loading the HF checkpoint."""
    src_dir, out_dir = tmp_path / "hf", tmp_path / "ftw"
    L, E, H, I = 3, 4, 256, 128
    write_hf_checkpoint(src_dir, "model.layers", 2, L, E, H, I, seed=7, shards=3)
    index = convert_hf_experts_to_ftw(str(src_dir), str(out_dir), per_layer=per_layer, shard_limit=1 << 18)
    assert index["quant_format"] == "fp8_block" and index["expert_bank_num_layers"] == L
    assert index["first_moe_layer"] == 2 and len(index["shards"]) > 1
    dtypes = {t["name"].split("#")[0]: t["dtype"] for t in index["tensors"]}
    assert dtypes["gate_up_scale"] == "bfloat16" and dtypes["gate_up"] == "float8_e4m3fn"
    assert os.path.isfile(out_dir / "config.json") and os.path.isfile(out_dir / "tok" / "tokenizer.json")
    assert not os.path.exists(out_dir / "model.safetensors.index.json")
    fmt, ftw, _ = load_ftw_banks(str(out_dir), L, pinned=False)
    _, hf, _ = load_hf_expert_banks(str(src_dir), pinned=False)
    assert fmt == "fp8_block" and list(ftw) == list(hf)
    for name in hf:
        for li in range(L):
            assert ftw[name][li].dtype == hf[name][li].dtype
            assert torch.equal(ftw[name][li].view(torch.uint8), hf[name][li].view(torch.uint8)), (name, li)


def test_scan_rejects_incomplete_checkpoints(tmp_path):
    write_hf_checkpoint(tmp_path, "model.layers", 0, 1, 2, 128, 128)
    with open(tmp_path / "model.safetensors.index.json") as f:
        idx = json.load(f)
    del idx["weight_map"]["model.layers.0.mlp.experts.1.up_proj.weight_scale_inv"]
    with open(tmp_path / "model.safetensors.index.json", "w") as f:
        json.dump(idx, f)
    with pytest.raises(ValueError, match="expert tensors"):
        scan_experts(str(tmp_path))
    with pytest.raises(ValueError, match="mode"):
        load_hf_expert_banks(str(tmp_path), mode="int4")


@pytest.mark.parametrize("prefix", ["model.layers", "model.language_model.layers"])
def test_mtp_experts_are_dropped(tmp_path, prefix):
    """The MTP head's experts (``mtp.layers.0`` for Qwen3.5, ``model.layers.<num_hidden_layers>``
    for DeepSeek-V3) are not decoder layers: the layer count stays L and the banks hold
    only the decoder layers' experts."""
    L, E, H, I = 2, 3, 256, 128
    banks = write_hf_checkpoint(tmp_path, prefix, 1, L, E, H, I, seed=11, mtp=True)
    lay, per_file = scan_experts(str(tmp_path))
    assert (lay.num_layers, lay.first_moe_layer) == (L, 1)
    assert all(not n.startswith("mtp.") and int(n.split(".layers.")[1].split(".")[0]) < 1 + L
               for items in per_file.values() for n, _ in items)
    _, src, _ = load_hf_expert_banks(str(tmp_path), pinned=False)
    assert len(src["gate_up"]) == L
    for li, b in enumerate(banks):
        np.testing.assert_array_equal(src["gate_up"][li].view(torch.uint8).numpy(), b.gate_up)


def test_expert_names_outside_the_decoder_stems_are_ignored(tmp_path):
    """Without a layer count in config.json the anchored stems alone decide: a
    vision tower's or an MTP head's experts never join the banks."""
    L, E, H, I = 1, 2, 128, 128
    write_hf_checkpoint(tmp_path, "model.language_model.layers", 0, L, E, H, I, seed=3, mtp=True)
    os.remove(tmp_path / "config.json")
    lay, _ = scan_experts(str(tmp_path))
    assert lay.num_layers == L
