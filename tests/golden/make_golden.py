"""Writes the golden fixtures of the MoE-layer hot path (tests/golden/*.npz).

The reference keeps no golden files and its CUDA-RNG seeds are not
reproducible on a CPU, so the vectors here come from the CPU restatement
(oracle/) on seeded numpy inputs shaped like BASELINE.json's configurations:

  c1_decode          C1 in full: hidden 1024, 16 experts, top-2 softmax
                     renormalised, intermediate 512, bf16, 4 tokens, seed 0
  c2r_decode         C2 reduced: FP8 128x128 block scales, top-8 softmax
  c3r_decode         C3 reduced: MXFP4 routed experts, grouped sigmoid with one
                     group, bf16 shared expert
  c4r_decode         C4 reduced: FP8, 8 groups / top-4 groups / top-8 sigmoid
                     with bias and scale 2.5, 16 of 32 experts resident behind a
                     slot table (misses excluded), FP8 shared expert
  c5r_prefill_fp8    C5 reduced: the grouped GEMM regime (W8A8) with shared
  c5r_prefill_mxfp4  C5 reduced: the grouped GEMM regime (MXFP4 x e4m3)
  kat_routing        tie known-answer cases of both routers
  kat_align          the align docstring example and a ragged random case

Each fixture holds the inputs, the routing results and the expected outputs.
Weight banks are not stored (C1's alone is 50 MB): the file records the seed
and the SHA-256 of every bank, and `build(name)` regenerates them with the
same calls, so a fixture also detects a change of the generator.

usage: python tests/golden/make_golden.py        (rewrites every fixture)
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from oracle import synth  # noqa: E402
from oracle.numerics import bf16_bits  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def bank_digest(bank) -> str:
    h = hashlib.sha256()
    for a in (bank.gate_up, bank.down, bank.gate_up_scale, bank.down_scale):
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# ---------------------------------------------------------------- case recipes
# Every recipe returns (inputs: dict of arrays, banks: dict name -> Bank,
# meta: dict) from its seed alone; run(name, ...) produces the expected outputs.


def _c1():
    rng = np.random.default_rng(0)
    bank = synth.make_bank("bf16", 16, 1024, 512, rng)
    x = synth.activations(rng, 4, 1024)
    router = synth.normal(rng, (16, 1024), 0.02)
    logits = (x @ router.T).astype(np.float32)
    return dict(x=x, logits=logits), dict(bank=bank), dict(regime="decode", router="softmax", k=2, renorm=1)


def _c2r():
    rng = np.random.default_rng(2)
    bank = synth.make_bank("fp8", 16, 256, 128, rng)
    x = synth.activations(rng, 8, 256)
    logits = synth.normal(rng, (8, 16))
    return dict(x=x, logits=logits), dict(bank=bank), dict(regime="decode", router="softmax", k=8, renorm=1)


def _c3r():
    rng = np.random.default_rng(3)
    bank = synth.make_bank("mxfp4", 20, 256, 128, rng)
    shared = synth.make_bank("bf16", 1, 256, 128, rng)
    x = synth.activations(rng, 8, 256)
    logits = synth.normal(rng, (8, 20))
    bias = synth.normal(rng, (20,), 0.1)
    meta = dict(regime="decode", router="sigmoid", k=8, renorm=1, n_group=1, topk_group=1, scale=2.5)
    return dict(x=x, logits=logits, bias=bias), dict(bank=bank, shared=shared), meta


def _c4r():
    rng = np.random.default_rng(4)
    e_all, slots = 32, 16
    bank = synth.make_bank("fp8", slots, 256, 128, rng)
    shared = synth.make_bank("fp8", 1, 256, 128, rng)
    x = synth.activations(rng, 8, 256)
    logits = synth.normal(rng, (8, e_all))
    bias = synth.normal(rng, (e_all,), 0.1)
    resident = np.sort(rng.choice(e_all, slots, replace=False))
    table = np.full(e_all, -1, dtype=np.int32)
    table[resident] = np.arange(slots, dtype=np.int32)
    meta = dict(regime="decode", router="sigmoid", k=8, renorm=1, n_group=8, topk_group=4, scale=2.5)
    return dict(x=x, logits=logits, bias=bias, slot_for_id=table), dict(bank=bank, shared=shared), meta


def _c5r(fmt: str, seed: int):
    rng = np.random.default_rng(seed)
    e = 16
    bank = synth.make_bank(fmt, e, 256, 128, rng)
    shared = synth.make_bank(fmt, 1, 256, 128, rng)
    x = synth.activations(rng, 96, 256)
    logits = synth.normal(rng, (96, e)) + synth.zipf_bias(rng, e)[None, :]
    bias = synth.normal(rng, (e,), 0.1)
    meta = dict(regime="prefill", router="sigmoid", k=8, renorm=1, n_group=4, topk_group=2, scale=2.5)
    return dict(x=x, logits=logits.astype(np.float32), bias=bias), dict(bank=bank, shared=shared), meta


RECIPES = {
    "c1_decode": _c1,
    "c2r_decode": _c2r,
    "c3r_decode": _c3r,
    "c4r_decode": _c4r,
    "c5r_prefill_fp8": lambda: _c5r("fp8", 5),
    "c5r_prefill_mxfp4": lambda: _c5r("mxfp4", 6),
}


def route(inputs: dict, meta: dict):
    if meta["router"] == "softmax":
        return oracle.routing.softmax_topk(inputs["logits"], meta["k"], bool(meta["renorm"]))
    return oracle.routing.grouped_sigmoid_topk(inputs["logits"], inputs["bias"], meta["n_group"],
                                               meta["topk_group"], meta["k"], bool(meta["renorm"]), meta["scale"])


def run(name: str, inputs: dict, banks: dict, meta: dict) -> dict:
    """Expected outputs of a layer case from the oracle."""
    w, ids = route(inputs, meta)
    out = dict(topk_w=w, topk_ids=ids)
    if "slot_for_id" in inputs:
        slots, miss, stats = oracle.slots.slot_map(ids, inputs["slot_for_id"])
        out.update(slot_ids=slots, miss_mask=miss, slot_stats=stats)
        ids = slots
    y = oracle.experts.moe_layer(meta["regime"], inputs["x"], w, ids, banks["bank"], banks.get("shared"))
    out["y_bits"] = bf16_bits(y)
    return out


def build(name: str):
    """(inputs, banks, meta) of a layer case, regenerated from its seed."""
    return RECIPES[name]()


# ---------------------------------------------------------------- KATs


def kat_routing() -> dict:
    """Tie cases.  Softmax: bf16-quantised logits with many exact ties, all
    equal rows; grouped sigmoid: equal groups and a bias that flips the pick."""
    rng = np.random.default_rng(11)
    tied = synth.tied_logits(rng, 64, 64)
    tied[0] = 0.5
    tied[1, :] = np.float32(-1.0)
    tied[1, 17] = 2.0
    w_s, ids_s = oracle.routing.softmax_topk(tied, 8, True)
    w_n, ids_n = oracle.routing.softmax_topk(tied, 8, False)
    g = np.zeros((4, 32), dtype=np.float32)          # every group and expert equal
    g[1, :] = np.tile(np.array([0.0, 1.0, 1.0, 0.0], np.float32), 8)
    g[2, :] = rng.standard_normal(32).astype(np.float32)
    g[3, :] = g[2, :]
    bias = np.zeros(32, dtype=np.float32)
    bias[5] = 1.5                                     # lifts expert 5 (group 1) into the pick
    w_g, ids_g = oracle.routing.grouped_sigmoid_topk(g, bias, 8, 4, 8, True, 2.5)
    w_g0, ids_g0 = oracle.routing.grouped_sigmoid_topk(g, np.zeros(32, np.float32), 8, 4, 8, True, 2.5)
    return dict(softmax_logits=tied, softmax_renorm_w=w_s, softmax_renorm_ids=ids_s, softmax_w=w_n,
                softmax_ids=ids_n, sigmoid_logits=g, sigmoid_bias=bias, sigmoid_w=w_g, sigmoid_ids=ids_g,
                sigmoid_nobias_w=w_g0, sigmoid_nobias_ids=ids_g0)


def kat_align() -> dict:
    doc_ids = np.array([[2, 3, 4], [1, 2, 4], [1, 3, 4], [1, 2, 3]], dtype=np.int32)
    s, e, n = oracle.align.moe_align_block_size(doc_ids, 4, 4)
    rng = np.random.default_rng(12)
    ids = rng.integers(-1, 17, size=(37, 6)).astype(np.int32)   # ragged, with skips and the sentinel id 16
    s2, e2, n2 = oracle.align.moe_align_block_size(ids, 8, 16)
    return dict(doc_ids=doc_ids, doc_sorted=s, doc_expert_ids=e, doc_ntpp=n, rand_ids=ids, rand_sorted=s2,
                rand_expert_ids=e2, rand_ntpp=n2)


def _meta_array(meta: dict) -> np.ndarray:
    return np.array(repr(sorted(meta.items())))


def main() -> None:
    for name in RECIPES:
        inputs, banks, meta = build(name)
        out = run(name, inputs, banks, meta)
        arrays = {f"in_{k}": v for k, v in inputs.items()}
        arrays.update({f"out_{k}": v for k, v in out.items()})
        arrays["meta"] = _meta_array(meta)
        for bname, b in banks.items():
            arrays[f"sha256_{bname}"] = np.array(bank_digest(b))
        arrays["x_bits"] = bf16_bits(inputs["x"])
        del arrays["in_x"]
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        print(f"wrote {name}.npz")
    np.savez_compressed(os.path.join(HERE, "kat_routing.npz"), **kat_routing())
    np.savez_compressed(os.path.join(HERE, "kat_align.npz"), **kat_align())
    print("wrote kat_routing.npz kat_align.npz")


if __name__ == "__main__":
    main()
