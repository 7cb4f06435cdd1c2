"""FTW expert-bank checkpoints (reference checkpoint/ftw.py): the on-disk
contract (4096-aligned tensors, shards cut at aligned points, a tensor that
fits one shard never straddles two, the index fields) and byte-exact round
trips of per-layer and flat bank layouts through the loader, with shards
small enough that large tensors span several of them."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from freetoken_amd.checkpoint import ftw

L, E, H, I = 3, 4, 256, 128


def _banks(seed=0):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, shape in (("gate_up", (E, 2 * I, H)), ("gate_up_scale", (E, 2 * I // 128, H // 128)),
                        ("down", (E, H, I)), ("down_scale", (E, H // 128, I // 128))):
        if name.endswith("scale"):
            out[name] = [torch.rand(shape, generator=g).to(torch.bfloat16) for _ in range(L)]
        else:
            out[name] = [torch.randint(0, 256, shape, generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn)
                         for _ in range(L)]
    return out


def _bytes(t):
    return t.contiguous().view(-1).view(torch.uint8).numpy()


@pytest.mark.parametrize("per_layer", [True, False])
@pytest.mark.parametrize("shard_limit", [3 * 4096, 1 << 20])
def test_round_trip(tmp_path, per_layer, shard_limit):
    src = _banks()
    index = ftw.save_ftw_banks(str(tmp_path), "fp8_block", src, per_layer=per_layer, shard_limit=shard_limit)
    assert ftw.is_ftw_checkpoint(str(tmp_path))
    for widen in (False, True):
        fmt, got, alphas = ftw.load_ftw_banks(str(tmp_path), L, pinned=False, scales_to_float32=widen, workers=4)
        assert fmt == "fp8_block" and not alphas
        assert list(got) == list(src)
        for name in src:
            for l in range(L):
                a, b = got[name][l], src[name][l]
                assert tuple(a.shape) == tuple(b.shape)
                if widen and name.endswith("_scale"):
                    assert a.dtype == torch.float32 and torch.equal(a, b.float())
                else:
                    assert a.dtype == b.dtype and np.array_equal(_bytes(a), _bytes(b))
    # the on-disk contract
    assert index["format"] == "freetoken_weight" and index["version"] == 1 and index["align"] == 4096
    total = 0
    for sh in index["shards"]:
        assert sh["global_off"] == total and sh["global_off"] % 4096 == 0 and sh["nbytes"] <= shard_limit
        assert os.path.getsize(tmp_path / sh["file"]) == sh["nbytes"]
        total += sh["nbytes"]
    assert total == index["total_bytes"]
    for t in index["tensors"]:
        assert t["global_off"] % 4096 == 0 and t["kind"] == "experts_bank"
        if t["nbytes"] <= shard_limit:  # fits a shard: lies in one
            assert any(s["global_off"] <= t["global_off"] and t["global_off"] + t["nbytes"] <= s["global_off"] + s["nbytes"]
                       for s in index["shards"])
    names = [t["name"] for t in index["tensors"]]
    assert ("gate_up#L00002" in names) == per_layer
    with open(tmp_path / "freetoken_weight.json") as f:
        assert json.load(f)["expert_bank_num_layers"] == L


def test_errors(tmp_path):
    src = _banks(1)
    ftw.save_ftw_banks(str(tmp_path), "fp8_block", src, shard_limit=1 << 20)
    with pytest.raises(ValueError):
        ftw.load_ftw_banks(str(tmp_path), L + 1, pinned=False)  # written for 3 layers
    shard = tmp_path / "freetoken-00000.ftw"
    with open(shard, "r+b") as f:
        f.truncate(os.path.getsize(shard) // 2)
    with pytest.raises((OSError, ValueError)):
        ftw.load_ftw_banks(str(tmp_path), L, pinned=False)
    with pytest.raises(ValueError):
        ftw.FTWWriter(str(tmp_path / "x"), shard_limit=1000)


def test_reader_pieces_split_at_shards(tmp_path):
    w = ftw.FTWWriter(str(tmp_path), shard_limit=2 * 4096)
    big = torch.arange(5000, dtype=torch.int32)  # 20000 bytes: spans three shards
    w.add_tensor("a", torch.ones(10, dtype=torch.float32))
    w.add_tensor("big", big)
    w.finalize()
    r = ftw.FTWReader(str(tmp_path))
    e = {t["name"]: t for t in r.entries()}["big"]
    ps = r.pieces(e["global_off"], e["nbytes"])
    assert len(ps) >= 3 and sum(p[3] for p in ps) == e["nbytes"]
    buf = torch.empty(ftw._align_up(e["nbytes"]), dtype=torch.uint8)
    r.read_into(buf, e["global_off"], e["nbytes"])
    assert torch.equal(buf[:e["nbytes"]].view(torch.int32), big)
    r.close()
