#!/usr/bin/env python3
"""Benchmark of the MI355X fused MoE-layer hot path.

Headline workload (one JSON line on stdout): the DeepSeek-V3-shaped FP8 MoE
layer in decode -- hidden 7168, 256 routed experts with grouped sigmoid routing
(8 groups, top-4 groups, top-8, bias, scale 2.5), intermediate 2048, one FP8
shared expert, 64 experts resident in cache slots behind the slot table -- at
batch 64.  One step = one layer call: router -> slot lookup -> experts ->
combine, captured in a HIP graph and replayed; successive steps rotate through
different synthetic routings so the touched experts change.  ``value`` is the
algorithmic HBM traffic of the step (distinct resident experts x expert bytes
+ shared expert + activations + logits) divided by the measured time.

Also reported in the same line: the roofline of the dominant kernel (the
gate_up GEMV stage, timed with HIP events on the library's stream), a bounded
sweep over the other configurations (decode batches 1..64 of the Qwen3-30B
FP8, GLM MXFP4 and DeepSeek-V3 layers; 8K-token ragged prefill in FP8 and
MXFP4 against the dense FP8 MFMA peak), and the CPU baseline: the C++
restatement of the reference's CPU MoE executor on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
import zlib

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from freetoken_amd import _lib, ops  # noqa: E402

METRIC = "MoE layer tok/s + HBM GB/s (decode b=1..64) and MFMA TFLOPS (8K prefill)"
HBM_PEAK_GBS = 8000.0
PEAK_TFLOPS = {"fp8": 5000.0, "mxfp4": 10100.0, "bf16": 2500.0}

C2 = dict(name="c2_qwen3_30b_a3b_fp8", H=2048, I=768, E=128, k=8, router="softmax", fmt="fp8_block",
          shared=None, Is=0, slots=128)
C3 = dict(name="c3_glm_mxfp4", H=5120, I=1536, E=160, k=8, router="sigmoid", n_group=1, topk_group=1,
          scale=2.5, fmt="mxfp4", shared="bf16", Is=1536, slots=160)
C4 = dict(name="c4_deepseek_v3_fp8", H=7168, I=2048, E=256, k=8, router="sigmoid", n_group=8, topk_group=4,
          scale=2.5, fmt="fp8_block", shared="fp8_block", Is=2048, slots=64)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ----------------------------------------------------------------------------- synthetic weights


def _e2m1_codes(v: torch.Tensor) -> torch.Tensor:
    """Round |v| <= 6 to e2m1 codes, ties to even (same rule as the oracle)."""
    m = v.abs()
    code = torch.full_like(m, 7, dtype=torch.uint8)
    for thr, c, le in ((5.0, 6, True), (3.5, 5, False), (2.5, 4, True), (1.75, 3, False), (1.25, 2, True),
                       (0.75, 1, False), (0.25, 0, True)):
        hit = (m <= thr) if le else (m < thr)
        code = torch.where(hit, torch.full_like(code, c), code)
    return code | (torch.signbit(v).to(torch.uint8) << 3)


def make_bank(fmt: str, rows: int, H: int, I: int, gen: torch.Generator, dev, std: float = 0.02) -> ops.ExpertBank:
    """Bank of ``rows`` SwiGLU experts drawn from N(0, std) and quantised on the GPU."""

    def one(n, k):
        outs = []
        for e0 in range(0, rows, 4):
            e1 = min(rows, e0 + 4)
            w = torch.randn((e1 - e0, n, k), generator=gen, device=dev, dtype=torch.float32) * std
            if fmt == "bf16":
                outs.append((w.to(torch.bfloat16), None))
            elif fmt == "fp8_block":
                b = w.view(e1 - e0, n // 128, 128, k // 128, 128)
                s = b.abs().amax(dim=(2, 4)).clamp_min(1e-12) / 448.0
                q = (b / s[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(e1 - e0, n, k)
                outs.append((q, s))
            else:
                b = w.view(e1 - e0, n, k // 32, 32)
                amax = b.abs().amax(-1).clamp_min(1e-30)
                e = torch.ceil(torch.log2(amax / 6.0)).clamp(-127, 127)
                codes = _e2m1_codes(b / torch.exp2(e)[..., None]).view(e1 - e0, n, k)
                packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).contiguous()
                outs.append((packed, (e + 127).to(torch.uint8)))
            del w
        q = torch.cat([o[0] for o in outs])
        s = torch.cat([o[1] for o in outs]) if outs[0][1] is not None else None
        return q, s

    gu, gus = one(2 * I, H)
    dn, dns = one(H, I)
    return ops.ExpertBank(fmt, gu, dn, gus, dns)


def expert_bytes(fmt: str, H: int, I: int) -> int:
    if fmt == "bf16":
        return 3 * H * I * 2
    if fmt == "fp8_block":
        return 3 * H * I + 4 * ((2 * I // 128) * (H // 128) + (H // 128) * (I // 128))
    return 3 * H * I // 2 + 3 * H * I // 32


def gate_up_bytes(fmt: str, H: int, I: int) -> int:
    if fmt == "bf16":
        return 2 * H * I * 2
    if fmt == "fp8_block":
        return 2 * H * I + 4 * (2 * I // 128) * (H // 128)
    return H * I + 2 * H * I // 32


# ----------------------------------------------------------------------------- decode layer


class DecodeLayer:
    """One decode configuration on the GPU: router inputs, slot table, banks."""

    def __init__(self, cfg: dict, dev, gen: torch.Generator):
        self.cfg = cfg
        self.dev = dev
        H, I, E = cfg["H"], cfg["I"], cfg["E"]
        self.bank = make_bank(cfg["fmt"], cfg["slots"], H, I, gen, dev)
        self.shared = make_bank(cfg["shared"], 1, H, cfg["Is"], gen, dev) if cfg["shared"] else None
        self.bias = (torch.randn((E,), generator=gen, device=dev) * 0.1) if cfg["router"] == "sigmoid" else None
        # resident set: the `slots` most popular experts under the seeded router
        # (popularity estimated on 4096 calibration tokens); all experts when slots == E
        self.table = torch.full((E,), -1, dtype=torch.int32, device=dev)
        if cfg["slots"] >= E:
            self.table = torch.arange(E, dtype=torch.int32, device=dev)
        else:
            lg = torch.randn((4096, E), generator=gen, device=dev)
            _, ids = self.route(lg)
            freq = torch.bincount(ids.view(-1).long(), minlength=E)
            top = torch.sort(torch.argsort(freq, descending=True, stable=True)[: cfg["slots"]]).values
            self.table[top] = torch.arange(cfg["slots"], dtype=torch.int32, device=dev)
        self.stats = torch.zeros(4, dtype=torch.int64, device=dev)
        if cfg["router"] == "softmax":
            self.router = ops.Router("softmax", cfg["k"], True)
        else:
            self.router = ops.Router("grouped_sigmoid", cfg["k"], True, self.bias, cfg["n_group"], cfg["topk_group"],
                                     cfg["scale"])

    def route(self, logits):
        c = self.cfg
        if c["router"] == "softmax":
            return ops.route_softmax_topk(logits, c["k"], True)
        return ops.route_grouped_sigmoid(logits, self.bias, c["n_group"], c["topk_group"], c["k"], True, c["scale"])

    def step(self, logits, x, out):
        """Router, expert ids -> slot ids (ensure_experts) and the experts of the
        offload layer's decode in one call (the router and the permutation
        share a launch for up to 16 tokens and 64 routes)."""
        _, _, ids = ops.experts_decode_routed(x, logits, self.router, self.bank, shared=self.shared, out=out,
                                              slot_for_id=self.table, stats=self.stats)
        return ids

    def shared_in_router(self, M: int) -> bool:
        """Whether the shared expert's gate_up runs in the router's launch (the
        library's route_shared_fits: grouped router, shared expert, at most four
        tokens and 64 routes, at most 256 experts); its bytes then belong to
        that launch, not to the gate_up stage."""
        c = self.cfg
        return (c["router"] == "sigmoid" and bool(c["shared"]) and M <= 4 and M * c["k"] <= 64
                and c["E"] <= 256)

    def step_bytes(self, ids: torch.Tensor, M: int) -> tuple[int, int, int]:
        """(algorithmic bytes of the step, gate_up-stage bytes, distinct resident experts)."""
        c = self.cfg
        valid = ids[ids >= 0]
        u = int(torch.unique(valid).numel())
        eb = expert_bytes(c["fmt"], c["H"], c["I"])
        sh = expert_bytes(c["shared"], c["H"], c["Is"]) if c["shared"] else 0
        io = M * c["H"] * 2 * 2 + M * c["E"] * 4
        gu = u * gate_up_bytes(c["fmt"], c["H"], c["I"])
        gu += M * c["H"] * 2 + int(valid.numel()) * c["I"] * 2
        if c["shared"] and not self.shared_in_router(M):
            gu += gate_up_bytes(c["shared"], c["H"], c["Is"]) + M * c["Is"] * 2
        return u * eb + sh + io, gu, u


def run_decode(layer: DecodeLayer, M: int, steps: int, warmup: int, gen, graphs: int = 8, stage_timing=False,
               min_ms: float = 0.0):
    """Times `steps` graph replays (rotating over `graphs` routings); returns a dict.  With
    `min_ms` > 0 the warm-up and the timed region each last at least that long (more replays
    than `warmup` / `steps` for short steps, whose first replays after an idle stretch run at
    lower clocks and whose timed region would otherwise be a millisecond or two)."""
    c, dev = layer.cfg, layer.dev
    G = max(1, min(graphs, steps))
    logits = [torch.randn((M, c["E"]), generator=gen, device=dev) for _ in range(G)]
    xs = [torch.randn((M, c["H"]), generator=gen, device=dev).to(torch.bfloat16) for _ in range(G)]
    outs = [torch.empty((M, c["H"]), dtype=torch.bfloat16, device=dev) for _ in range(G)]
    ids_eager = [layer.step(logits[g], xs[g], outs[g]) for g in range(G)]  # sizes the workspace
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)
    graphs_ = []
    ids_graph = []
    with torch.cuda.stream(stream):
        for g in range(G):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                ids_graph.append(layer.step(logits[g], xs[g], outs[g]))
            graphs_.append(gr)
    torch.cuda.synchronize()
    for i in range(warmup):
        graphs_[i % G].replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if min_ms > 0:
        t0.record()
        for i in range(G):
            graphs_[i % G].replay()
        t1.record()
        torch.cuda.synchronize()
        est = max(t0.elapsed_time(t1) / G, 1e-3)
        n = min(4000, math.ceil(min_ms / est))
        for i in range(n):
            graphs_[i % G].replay()
        torch.cuda.synchronize()
        steps = max(steps, n)
    t0.record()
    for i in range(steps):
        graphs_[i % G].replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1)
    total_bytes = 0
    gu_bytes = 0
    us = []
    for i in range(steps):
        b, gb, u = layer.step_bytes(ids_eager[i % G], M)
        total_bytes += b
        gu_bytes += gb
        us.append(u)
    res = dict(batch=M, steps=steps, ms_per_step=ms / steps, tok_s=M * steps / (ms / 1e3),
               gbs=total_bytes / (ms / 1e3) / 1e9, bytes_per_step=total_bytes / steps,
               resident_experts_per_step=statistics.mean(us))
    res["hbm_frac"] = res["gbs"] / HBM_PEAK_GBS
    if stage_timing:
        # instrumented eager pass over the same inputs: per-kernel durations
        L = _lib.lib()
        L.ftmoe_stage_timing_begin()
        for i in range(min(steps, 64)):
            layer.step(logits[i % G], xs[i % G], outs[i % G])
        torch.cuda.synchronize()
        import ctypes

        arr = (ctypes.c_double * 8)()
        ns, nc = ctypes.c_int(), ctypes.c_int()
        _lib.check(L.ftmoe_stage_timing_end(arr, 8, ctypes.byref(ns), ctypes.byref(nc)), "stage timing")
        if nc.value == 0 or ns.value < 4:
            raise RuntimeError(f"stage timing recorded {nc.value} calls / {ns.value} stages")
        names = ["align", "gate_up", "down", "combine"]
        res["stage_us"] = {names[j]: arr[j] / max(1, nc.value) * 1e3 for j in range(min(ns.value, 4))}
        res["gate_up_bytes_per_launch"] = gu_bytes / steps
    del graphs_
    return res


# ----------------------------------------------------------------------------- prefill


def prefill_workload(fmt: str, gen, dev, M: int = 8192) -> dict:
    """The C5 workload: the C4 layer (256 experts + shared, in ``fmt``) and an
    M-token ragged batch of 16 sequences whose router logits carry a Zipf(1.1)
    expert-popularity bias, routed by the grouped sigmoid router."""
    c = C4
    H, I, E, k = c["H"], c["I"], c["E"], c["k"]
    bank = make_bank(fmt, E, H, I, gen, dev)
    shared = make_bank(fmt, 1, H, I, gen, dev)
    # 16 ragged sequences, lengths U[64, 1024] normalised to M (largest remainder);
    # the MoE layer sees the packed [M, H] rows, so lengths only document the batch
    g = torch.Generator().manual_seed(5)
    raw = torch.randint(64, 1025, (16,), generator=g).double()
    exact = raw / raw.sum() * M
    lens = exact.floor().long()
    rem = M - int(lens.sum())
    lens[torch.argsort(exact - lens, descending=True)[:rem]] += 1
    ranks = torch.randperm(E, generator=gen, device=dev).double() + 1
    p = ranks ** -1.1
    zipf = torch.log(p / p.sum()).float()
    bias = torch.randn((E,), generator=gen, device=dev) * 0.1
    logits = torch.randn((M, E), generator=gen, device=dev) + zipf[None, :]
    x = torch.randn((M, H), generator=gen, device=dev).to(torch.bfloat16)
    w, ids = ops.route_grouped_sigmoid(logits, bias, 8, 4, k, True, 2.5)
    return dict(bank=bank, shared=shared, lens=lens, bias=bias, logits=logits, x=x, w=w, ids=ids)


def run_prefill(fmt: str, steps: int, warmup: int, gen, dev, M: int = 8192):
    c = C4
    H, I, E = c["H"], c["I"], c["E"]
    wl = prefill_workload(fmt, gen, dev, M)
    bank, shared, lens, x, w, ids = wl["bank"], wl["shared"], wl["lens"], wl["x"], wl["w"], wl["ids"]
    del wl
    out = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    for _ in range(max(1, warmup)):
        ops.experts_prefill(x, w, ids, bank, shared=shared, out=out)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        ops.experts_prefill(x, w, ids, bank, shared=shared, out=out)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    # instrumented eager pass: per-kernel durations of one call
    import ctypes

    L = _lib.lib()
    L.ftmoe_stage_timing_begin()
    for _ in range(steps):
        ops.experts_prefill(x, w, ids, bank, shared=shared, out=out)
    torch.cuda.synchronize()
    arr = (ctypes.c_double * 8)()
    ns, nc = ctypes.c_int(), ctypes.c_int()
    _lib.check(L.ftmoe_stage_timing_end(arr, 8, ctypes.byref(ns), ctypes.byref(nc)), "stage timing")
    names = ["align", "x_quant", "gate_up", "act_quant", "down", "combine"]
    stage_us = {names[j]: arr[j] / max(1, nc.value) * 1e3 for j in range(min(ns.value, len(names)))}
    routes = int((ids >= 0).sum())
    flops = (routes + M) * 6 * H * I
    counts = torch.bincount(ids.view(-1).long(), minlength=E)
    peak = PEAK_TFLOPS["fp8"]
    bm = 128 if fmt == "bf16" else 256  # routes per M block of the prefill GEMMs
    padded = int(((counts + bm - 1) // bm * bm).sum()) + (M + bm - 1) // bm * bm
    res = dict(tokens=M, sequences=lens.tolist(), ms=ms, tflops=flops / (ms / 1e3) / 1e12, flops=flops,
               max_expert_tokens=int(counts.max()), min_expert_tokens=int(counts.min()),
               padded_rows_per_real_row=round(padded / (routes + M), 4), stage_us=stage_us)
    res["frac_of_fp8_peak"] = res["tflops"] / peak
    if fmt == "mxfp4":
        # the reference's MXFP4 prefill FP8-round-trips its activations, so the
        # GEMMs are FP8 x FP4 scaled MFMAs, which issue at the FP8 rate (32 busy
        # cycles per 16x16x128, as FP8 x FP8): frac_of_fp8_peak is this path's
        # roofline, the FP4 figure only a reference point
        res["frac_of_fp4_peak"] = res["tflops"] / PEAK_TFLOPS["mxfp4"]
        res["roofline_peak"] = "fp8 (FP8 x FP4 scaled MFMAs issue at the FP8 rate)"
    del bank, shared
    torch.cuda.empty_cache()
    return res


def run_dense_fp8_library(dev, steps: int = 10, warmup: int = 3) -> list[dict]:
    """A library reference point for the prefill GEMMs, not part of the path:
    ``torch._scaled_mm`` (hipBLASLt) on dense FP8 GEMMs of C5's shapes.  The
    C5 gate_up and down GEMMs as single dense problems (all routes + shared
    rows in one M), and one expert's gate_up at C5's mean routes per expert
    (256), with per-tensor and per-row/column float scales.  Block scales of
    128 x 128 (the path's format) are tried as well and reported unsupported
    if the library refuses them."""
    c = C4
    H, I = c["H"], c["I"]
    Mall = 8192 * c["k"] + 8192  # C5: routes + shared-expert rows
    shapes = [("gate_up_dense", Mall, H, 2 * I), ("down_dense", Mall, I, H), ("gate_up_one_expert", 256, H, 2 * I)]
    f8 = torch.float8_e4m3fn
    g = torch.Generator(device=dev).manual_seed(77)
    out = []
    for name, M, K, N in shapes:
        a = (torch.randn((M, K), generator=g, device=dev) * 0.5).to(f8)
        w = (torch.randn((N, K), generator=g, device=dev) * 0.5).to(f8)
        b = w.t()  # column-major [K, N], as the library wants its second operand
        scales = {
            "tensorwise": (torch.tensor(0.01, device=dev), torch.tensor(0.02, device=dev)),
            "rowwise": (torch.full((M, 1), 0.01, device=dev), torch.full((1, N), 0.02, device=dev)),
            "blockwise_1x128_128x128": (torch.full((M, K // 128), 0.01, device=dev),
                                        torch.full((K // 128, N // 128), 0.02, device=dev)),
        }
        for kind, (sa, sb) in scales.items():
            rec = dict(gemm=name, M=M, K=K, N=N, scales=kind)
            try:
                for _ in range(warmup):
                    y = torch._scaled_mm(a, b, scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
                torch.cuda.synchronize()
                reps = steps if M > 1024 else 50 * steps
                t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                t0.record()
                for _ in range(reps):
                    y = torch._scaled_mm(a, b, scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
                t1.record()
                torch.cuda.synchronize()
                us = t0.elapsed_time(t1) / reps * 1e3
                tf = 2.0 * M * K * N / (us * 1e-6) / 1e12
                rec.update(us=round(us, 2), tflops=round(tf, 1), frac_of_fp8_peak=round(tf / PEAK_TFLOPS["fp8"], 4))
                del y
            except Exception as e:  # the library refuses this scale layout
                rec["unsupported"] = f"{type(e).__name__}: {str(e).splitlines()[0][:160]}"
            out.append(rec)
        del a, w, b, scales
        torch.cuda.empty_cache()
    return out


# ----------------------------------------------------------------------------- CPU baseline


PCIE_PEAK_GBS = 64.0  # PCIe Gen5 x16, one direction


def run_miss_fetch(gen, dev, n_fetch: int = 8, steps: int = 10):
    """Miss path at C4 shape: each step routes n_fetch experts none of which is
    resident (two disjoint expert sets alternate over n_fetch slots), so the
    admission evicts and the gather moves n_fetch whole experts from pinned host
    banks over PCIe.  Reports the gather's GB/s against the link and the
    admission kernel's time."""
    c = C4
    H, I = c["H"], c["I"]
    E, S = 2 * n_fetch, n_fetch
    rows = {"gate_up": (2 * I, H), "gate_up_scale": (2 * I // 128 * (H // 128) * 4,), "down": (H, I),
            "down_scale": (H // 128 * (I // 128) * 4,)}
    host, slots = [], []
    for shape in rows.values():
        h = ops.alloc_pinned_tensor(E, *shape, dtype=torch.uint8)
        h.view(-1)[:: 4097] = 1
        host.append(h)
        slots.append(torch.empty((S,) + shape, dtype=torch.uint8, device=dev))
    expert_bytes = sum(int(h[0].numel()) for h in host)
    slot_for_id = torch.full((1, E), -1, dtype=torch.int32, device=dev)
    id_of_slot = torch.full((S,), -1, dtype=torch.int32, device=dev)
    usage = torch.zeros((S,), dtype=torch.int64, device=dev)
    step = torch.zeros((1,), dtype=torch.int64, device=dev)
    evict = torch.zeros((E,), dtype=torch.int32, device=dev)
    src = torch.zeros((E,), dtype=torch.int32, device=dev)
    num = torch.zeros((1,), dtype=torch.int32, device=dev)
    nmiss = torch.zeros((1,), dtype=torch.int32, device=dev)
    sets = [torch.arange(g * n_fetch, (g + 1) * n_fetch, dtype=torch.int32, device=dev) for g in range(2)]
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps + 1)]
    for i in range(steps + 1):  # call 0 warms up
        ids = sets[i % 2].clone()
        ev[i][0].record()
        ops.lru_ensure(ids, 0, slot_for_id, id_of_slot, usage, step, evict, src, num, nmiss)
        ev[i][1].record()
        ops.fetch_experts(host, slots, evict, src, num, max_entries=n_fetch)
        ev[i][2].record()
    torch.cuda.synchronize()
    adm = statistics.median(ev[i][0].elapsed_time(ev[i][1]) for i in range(1, steps + 1))
    fet = statistics.median(ev[i][1].elapsed_time(ev[i][2]) for i in range(1, steps + 1))
    assert int(num.item()) == n_fetch and int(nmiss.item()) == n_fetch
    gbs = n_fetch * expert_bytes / (fet * 1e-3) / 1e9
    return dict(experts_per_step=n_fetch, expert_bytes=expert_bytes, admission_us=adm * 1e3, fetch_ms=fet,
                fetch_gbs=gbs, pcie_frac=gbs / PCIE_PEAK_GBS)


def run_ep_share(gen, dev, ep: int = 8, per_gpu_batch: int = 64, steps: int = 20, warmup: int = 3, graphs: int = 4):
    """One GPU's share of an expert-parallel C4 layer, the per-GPU kernel work
    at its real shape: `ep` GPUs hold 256/ep experts each; every GPU routes its
    own `per_gpu_batch` tokens and sends each route to the owner of its expert,
    so GPU 0's experts see the routes of the whole global batch
    (ep * per_gpu_batch tokens) that fall on experts [0, 256/ep).  The dispatch
    sends each token with at least one route here once (its activations, its
    k expert ids with -1 for the other GPUs' experts, its weights), and the
    same decode entry point runs the received tokens over the local bank; the
    return all-to-all and the home GPU's sum of the GPUs' partial outputs are
    the combine.  Timed: the share's routed-expert call, replayed
    from graphs (routing precomputed; the all-to-alls and the shared expert,
    which runs on each token's home GPU, are not part of it)."""
    c = C4
    H, I, E, k = c["H"], c["I"], c["E"], c["k"]
    e_loc = E // ep
    B = ep * per_gpu_batch
    bank = make_bank("fp8_block", e_loc, H, I, gen, dev)
    bias = torch.randn((E,), generator=gen, device=dev) * 0.1
    G = max(1, min(graphs, steps))
    ws, ids_loc, xs, outs = [], [], [], []
    for _ in range(G):
        w, ids = ops.route_grouped_sigmoid(torch.randn((B, E), generator=gen, device=dev), bias, c["n_group"],
                                           c["topk_group"], k, True, c["scale"])
        x = torch.randn((B, H), generator=gen, device=dev).to(torch.bfloat16)
        local = ids < e_loc  # this GPU's routes
        tok = torch.nonzero(local.any(1))[:, 0]  # received tokens, in token order
        ws.append(w[tok].contiguous())
        ids_loc.append(torch.where(local[tok], ids[tok], torch.full_like(ids[tok], -1)).contiguous())
        xs.append(x[tok].contiguous())
        outs.append(torch.empty((int(tok.numel()), H), dtype=torch.bfloat16, device=dev))
    for g in range(G):  # eager calls size the workspace
        ops.experts_decode(xs[g], ws[g], ids_loc[g], bank, out=outs[g])
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)
    grs = []
    with torch.cuda.stream(stream):
        for g in range(G):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                ops.experts_decode(xs[g], ws[g], ids_loc[g], bank, out=outs[g])
            grs.append(gr)
    torch.cuda.synchronize()
    for i in range(warmup):
        grs[i % G].replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        grs[i % G].replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    # instrumented eager pass over the same inputs: per-kernel durations
    import ctypes

    L = _lib.lib()
    L.ftmoe_stage_timing_begin()
    for i in range(min(steps, 64)):
        ops.experts_decode(xs[i % G], ws[i % G], ids_loc[i % G], bank, out=outs[i % G])
    torch.cuda.synchronize()
    arr = (ctypes.c_double * 8)()
    ns, nc = ctypes.c_int(), ctypes.c_int()
    _lib.check(L.ftmoe_stage_timing_end(arr, 8, ctypes.byref(ns), ctypes.byref(nc)), "stage timing")
    names = ["align", "gate_up", "down", "combine"]
    stage_us = {names[j]: arr[j] / max(1, nc.value) * 1e3 for j in range(min(ns.value, 4))}
    eb = expert_bytes("fp8_block", H, I)
    us = [int(torch.unique(t[t >= 0]).numel()) for t in ids_loc]
    routes = [int((t >= 0).sum()) for t in ids_loc]
    tokens = [int(t.shape[0]) for t in ids_loc]
    step_bytes = statistics.mean(us) * eb + 2 * statistics.mean(tokens) * H * 2
    return dict(ep=ep, experts_per_gpu=e_loc, global_batch=B, per_gpu_batch=per_gpu_batch,
                received_tokens_per_step=statistics.mean(tokens),
                local_routes_per_step=statistics.mean(routes), local_experts_per_step=statistics.mean(us),
                ms_per_step=ms, gbs=step_bytes / (ms * 1e-3) / 1e9, hbm_frac=step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                global_tok_s_bound=B / (ms * 1e-3), stage_us=stage_us)


def run_hybrid(gen, dev, M: int = 1, n_sets: int = 4, slots: int = 8, max_fetch: int = 1, steps: int = 8,
               warmup: int = 8, fetch_fraction: float | None = None):
    """Hybrid decode at C4 shape (FP8 experts, one layer): each step routes the
    M tokens to one of n_sets disjoint sets of k experts in turn, over a slot
    cache of ``slots`` experts, so every step has misses; the admission fetches
    at most max_fetch of them over PCIe and the CPU executor computes the rest
    while the GPU runs its share.  Besides the step time it times the two
    shares alone on the same routing (the CPU job; the gather plus the GPU
    experts), so the overlap is (cpu + gpu) / step.  ``fetch_fraction`` (the
    bandwidth-matched share of the misses, from measured rates) replaces the
    fixed ``max_fetch`` cap when given."""
    from freetoken_amd.core import moe_phase
    from freetoken_amd.layers.moe import OffloadMoELayer
    from freetoken_amd.moe.cpu_decode import CpuMoeDecoder
    from freetoken_amd.moe.offload_cache import ExpertSlotCache

    c = C4
    H, I, k = c["H"], c["I"], c["k"]
    E = n_sets * k
    shapes = {"gate_up": (2 * I, H), "gate_up_scale": (2 * I // 128, H // 128), "down": (H, I),
              "down_scale": (H // 128, I // 128)}
    host = {}
    for name, shape in shapes.items():
        if name.endswith("scale"):
            d = torch.rand((E,) + shape, generator=gen, device=dev) * 1e-3 + 1e-4
        else:
            d = torch.randint(0, 256, (E,) + shape, generator=gen, device=dev, dtype=torch.uint8)
            d[(d & 0x7F) == 0x7F] = 0  # no NaN codes
        h = ops.alloc_pinned_tensor(*d.shape, dtype=d.dtype)
        h.copy_(d)
        host[name] = h
        del d
    cache = ExpertSlotCache(1, E, slots, "fp8_block", device=dev, decode_target="hybrid", hybrid_max_fetch=max_fetch,
                            hybrid_fetch_fraction=fetch_fraction or 0.0)
    cache.set_bank_caches(**{n: torch.zeros((slots,) + h.shape[1:], dtype=h.dtype, device=dev)
                             for n, h in host.items()})
    cache.set_bank_sources({n: [h] for n, h in host.items()})
    cache.reset()
    dec = CpuMoeDecoder(cache, k)
    cache.set_cpu_executor(dec)
    layer = OffloadMoELayer(0, E, k, H, I, device=dev)
    layer.offload_cache = cache
    x = torch.randn((M, H), generator=gen, device=dev).to(torch.bfloat16)
    w = torch.full((M, k), 1.0 / k, device=dev)
    sets = [torch.arange(s * k, (s + 1) * k, dtype=torch.int32, device=dev).repeat(M, 1) for s in range(n_sets)]
    eb = expert_bytes("fp8_block", H, I)
    rec = []
    with moe_phase("decode", backend="hybrid"):
        for i in range(warmup + steps):
            raw = sets[i % n_sets]
            ids = raw.clone()
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
            torch.cuda.synchronize()
            ev[0].record()
            layer.routed_forward(x, w, ids)
            ev[1].record()
            torch.cuda.synchronize()
            cpu_ids = torch.where(ids < 0, raw, torch.full_like(raw, -1))
            ev[2].record()
            dec.decode(0, x, w, cpu_ids)
            ev[3].record()
            cache.copy_missing()
            ops.experts_decode(x, w, ids, layer._views_bank(cache.bank_views()))
            ev[4].record()
            torch.cuda.synchronize()
            if i >= warmup:
                n_cpu = int(torch.unique(cpu_ids[cpu_ids >= 0]).numel())
                n_fetch = int(cache.num_indices.item())
                n_gpu = int(torch.unique(ids[ids >= 0]).numel())
                rec.append((ev[0].elapsed_time(ev[1]), ev[2].elapsed_time(ev[3]), ev[3].elapsed_time(ev[4]),
                            n_cpu, n_fetch, n_gpu))
    threads, isa = dec.executor.threads, dec.executor.isa
    dec.close()
    med = lambda j: statistics.median(r[j] for r in rec)  # noqa: E731
    step, cpu_ms, gpu_ms = med(0), med(1), med(2)
    n_cpu, n_fetch, n_gpu = med(3), med(4), med(5)
    return dict(batch=M, experts_per_step=k, slots=slots, max_fetch=max_fetch, fetch_fraction=fetch_fraction, step_ms=step,
                cpu_experts=n_cpu, fetched_experts=n_fetch, gpu_experts=n_gpu, cpu_ms=cpu_ms, gpu_ms=gpu_ms,
                overlap=(cpu_ms + gpu_ms) / step, cpu_gbs=n_cpu * eb / (cpu_ms * 1e-3) / 1e9,
                cpu_threads=threads, cpu_isa=isa)


def run_prefill_offload(gen, dev, L: int = 3, E: int = 32, M: int = 8192, reps: int = 2):
    """Prefill movement of the expert cache at C4 expert shape (FP8), L layers
    of E experts each held only in pinned host memory, M tokens routed top-8
    uniformly: per-layer time of (a) materialize + PCIe gather + experts, one
    after the other, (b) the double buffer, layer l+1's host copy on a copy
    stream behind layer l's experts, and (c) the double buffer with half of
    every layer's experts already resident, with and without the hit/miss
    split.  E is reduced from 256 so that L layers
    of host banks stay a few GB."""
    from freetoken_amd.core import moe_phase
    from freetoken_amd.layers.moe import OffloadMoELayer
    from freetoken_amd.moe.offload_cache import ExpertSlotCache

    c = C4
    H, I, k = c["H"], c["I"], c["k"]
    shapes = {"gate_up": (2 * I, H), "gate_up_scale": (2 * I // 128, H // 128), "down": (H, I),
              "down_scale": (H // 128, I // 128)}
    host = {n: [] for n in shapes}
    for _ in range(L):
        for name, shape in shapes.items():
            if name.endswith("scale"):
                d = torch.rand((E,) + shape, generator=gen, device=dev) * 1e-3 + 1e-4
            else:
                d = torch.randint(0, 256, (E,) + shape, generator=gen, device=dev, dtype=torch.uint8)
                d[(d & 0x7F) == 0x7F] = 0
            h = ops.alloc_pinned_tensor(*d.shape, dtype=d.dtype)
            h.copy_(d)
            host[name].append(h)
            del d
    layer_bytes = sum(int(h[0].numel()) * h[0].element_size() for h in host.values())
    x = torch.randn((M, H), generator=gen, device=dev).to(torch.bfloat16)
    w, ids = ops.route_softmax_topk(torch.randn((M, E), generator=gen, device=dev), k, True)
    res = {"layers": L, "experts_per_layer": E, "tokens": M, "layer_bytes": layer_bytes}
    for overlap in (False, True):
        S = 2 * E if overlap else E
        cache = ExpertSlotCache(L, E, S, "fp8_block", device=dev, prefill_overlap=overlap)
        cache.set_bank_caches(**{n: torch.zeros((S,) + h[0].shape[1:], dtype=h[0].dtype, device=dev)
                                 for n, h in host.items()})
        cache.set_bank_sources(host)
        cache.reset()
        layers = [OffloadMoELayer(l, E, k, H, I, device=dev) for l in range(L)]
        for lay in layers:
            lay.offload_cache = cache
        times = []
        with moe_phase("prefill", backend="offload"):
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                e0.record()
                for lay in layers:
                    lay.routed_forward(x, w, ids.clone())
                e1.record()
                torch.cuda.synchronize()
                times.append(e0.elapsed_time(e1))
        t = min(times) / L
        key = "double_buffer" if overlap else "materialize"
        res[f"{key}_ms_per_layer"] = t
        res[f"{key}_gbs"] = layer_bytes / (t * 1e-3) / 1e9
        del cache, layers
        torch.cuda.empty_cache()
    # half of every layer's experts already resident outside the two buffers (slots >= 2E, as a
    # decode leaves them): the double buffer with and without the hit/miss split
    # (moe/offload_cache.py:703-773), hits gathered device to device, only misses over PCIe
    half = E // 2
    for split in (False, True):
        S = 2 * E + L * half
        cache = ExpertSlotCache(L, E, S, "fp8_block", device=dev, prefill_overlap=True, prefill_hit_d2d=split)
        cache.set_bank_caches(**{n: torch.zeros((S,) + h[0].shape[1:], dtype=h[0].dtype, device=dev)
                                 for n, h in host.items()})
        cache.set_bank_sources(host)
        cache.reset()
        for l in range(L):
            experts = list(range(0, E, 2))
            slots = [2 * E + l * half + j for j in range(half)]
            for e, sl in zip(experts, slots):
                for n, h in host.items():
                    cache.banks[n][sl].copy_(h[l][e], non_blocking=True)
            cache.assign(l, experts, slots)
        torch.cuda.synchronize()
        layers = [OffloadMoELayer(l, E, k, H, I, device=dev) for l in range(L)]
        for lay in layers:
            lay.offload_cache = cache
        times = []
        with moe_phase("prefill", backend="offload"):
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                e0.record()
                for lay in layers:
                    lay.routed_forward(x, w, ids.clone())
                e1.record()
                torch.cuda.synchronize()
                times.append(e0.elapsed_time(e1))
        key = "half_resident_split" if split else "half_resident_no_split"
        res[f"{key}_ms_per_layer"] = min(times) / L
        if split:
            res["half_resident_hit_rate"] = cache.prefill_hit_rate()
        del cache, layers
        torch.cuda.empty_cache()
    # the experts alone on resident banks, for the overlap bound
    bank = ops.ExpertBank("fp8_block", *(h[0].to(dev) for h in (host["gate_up"], host["down"])),
                          host["gate_up_scale"][0].to(dev), host["down_scale"][0].to(dev))
    ops.experts_prefill(x, w, ids, bank)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    ops.experts_prefill(x, w, ids, bank)
    e1.record()
    torch.cuda.synchronize()
    res["experts_ms"] = e0.elapsed_time(e1)
    return res


def _host_cpu_info() -> dict:
    """CPU model, physical cores of the machine, SMT state and NUMA nodes with
    the CPUs of this process's share on each."""
    from pathlib import Path

    from oracle.cpu_moe import physical_cores

    info = {"model": "unknown", "smt_active": None, "physical_cores_total": None, "numa_nodes": {}}
    try:
        info["model"] = [ln.split(":", 1)[1].strip() for ln in open("/proc/cpuinfo") if ln.startswith("model name")][0]
    except (OSError, IndexError):
        pass
    try:
        info["smt_active"] = Path("/sys/devices/system/cpu/smt/active").read_text().strip() == "1"
    except OSError:
        pass
    keys = set()
    for d in Path("/sys/devices/system/cpu").glob("cpu[0-9]*"):
        try:
            keys.add((d.joinpath("topology/physical_package_id").read_text().strip(),
                      d.joinpath("topology/core_id").read_text().strip()))
        except OSError:
            pass
    info["physical_cores_total"] = len(keys) or None
    allowed = set(os.sched_getaffinity(0))

    def parse(text):
        out = set()
        for part in text.strip().split(","):
            if part:
                a, _, b = part.partition("-")
                out.update(range(int(a), int(b or a) + 1))
        return out

    for node in sorted(Path("/sys/devices/system/node").glob("node[0-9]*")):
        try:
            cpus = parse(node.joinpath("cpulist").read_text())
        except OSError:
            continue
        mine = sorted(cpus & allowed)
        if mine:
            info["numa_nodes"][node.name] = mine
    phys = physical_cores()
    info["share_physical_cores"] = phys
    return info


# (name, CPU format, H, I, host experts, top_k, batches, bf16 shared expert I or 0).  C2 and C4 run
# bf16-dequantised banks (the reference's CPU route for block-FP8 checkpoints); C4 holds the 64
# experts of the GPU's resident set on the host, the others every expert of the config.
CPU_CONFIGS = [
    ("c1_tiny_bf16", "bf16", 1024, 512, 16, 2, (4,), 0),
    ("c2_qwen3_30b_a3b_bf16_dequant", "bf16", 2048, 768, 128, 8, (1, 8, 32, 64), 0),
    ("c3_glm_mxfp4_bf16_shared", "mxfp4", 5120, 1536, 160, 8, (1, 8, 32, 64), 1536),
    ("c4_deepseek_v3_bf16_dequant_64_experts", "bf16", 7168, 2048, 64, 8, (1, 8, 32, 64), 0),
]


def _cpu_config_runs(cfg, cores, step_budget_s: float, seed: int) -> list[dict]:
    """One CPU configuration at its batch sizes on ``cores``: the reference's
    bs=1 method (``moe/benchbw.py:463-499``: 8 warm-up steps, then the median
    of up to 64 timed steps, each routed to the next window of k experts so
    consecutive steps touch disjoint experts and read DRAM); at batch > 1
    (2 warm-up steps, at least 3 timed) each token takes k distinct experts
    drawn from all host experts."""
    import numpy as np

    from oracle.cpu_moe import CpuMoe, lib as cpulib

    name, fmt, H, I, E, k, batches, Is = cfg
    nth = len(cores)
    if fmt == "bf16":
        gu = np.empty((E, 2 * I, H), dtype=np.uint16)
        dn = np.empty((E, H, I), dtype=np.uint16)
        cpulib().cpumoe_fill_bf16(gu.ctypes.data, gu.size, 0.02 * math.sqrt(3), seed, nth)
        cpulib().cpumoe_fill_bf16(dn.ctypes.data, dn.size, 0.02 * math.sqrt(3), seed + 1, nth)
        banks = (gu, dn)
    else:  # any byte is a valid pair of e2m1 codes; scales 2^-7..2^-5
        gu = np.empty((E, 2 * I, H // 2), dtype=np.uint8)
        dn = np.empty((E, H, I // 2), dtype=np.uint8)
        cpulib().cpumoe_fill_bf16(gu.ctypes.data, gu.size // 2, 1.0, seed, nth)
        cpulib().cpumoe_fill_bf16(dn.ctypes.data, dn.size // 2, 1.0, seed + 1, nth)
        rng = np.random.default_rng(seed)
        banks = (gu, dn, rng.integers(120, 123, (E, 2 * I, H // 32), dtype=np.uint8),
                 rng.integers(120, 123, (E, H, I // 32), dtype=np.uint8))
    cpu = CpuMoe(H, I, k, E, fmt, cpus=cores)
    cpu.set_bank(*banks)
    sh = None
    if Is:
        sgu = np.empty((1, 2 * Is, H), dtype=np.uint16)
        sdn = np.empty((1, H, Is), dtype=np.uint16)
        cpulib().cpumoe_fill_bf16(sgu.ctypes.data, sgu.size, 0.02 * math.sqrt(3), seed + 2, nth)
        cpulib().cpumoe_fill_bf16(sdn.ctypes.data, sdn.size, 0.02 * math.sqrt(3), seed + 3, nth)
        sh = CpuMoe(H, Is, 1, 1, "bf16", cpus=cores)
        sh.set_bank(sgu, sdn)
    eb = expert_bytes("bf16" if fmt == "bf16" else "mxfp4", H, I)
    sh_bytes = expert_bytes("bf16", H, Is) if Is else 0
    rng = np.random.default_rng(seed + 7)
    out = []
    for M in batches:
        x = (rng.standard_normal((M, H)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        w = np.full((M, k), 1.0 / k, dtype=np.float32)
        base = np.arange(k, dtype=np.int32)

        def ids_for(i):
            if M == 1:
                return ((i * k + base) % E).reshape(1, k).astype(np.int32)
            return np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)

        def step(ids):
            t0 = time.perf_counter()
            cpu.run(x, w, ids)
            if sh is not None:
                sh.run(x, np.ones((M, 1), np.float32), np.zeros((M, 1), np.int32))
            return time.perf_counter() - t0

        warm = 8 if M == 1 else 2  # the reference's method is for bs=1; larger batches warm up briefly
        for i in range(warm):
            step(ids_for(i))
        times, us = [], []
        t_end = time.perf_counter() + step_budget_s
        i = warm
        while len(times) < 64 and (len(times) < 3 or time.perf_counter() < t_end):
            ids = ids_for(i)
            times.append(step(ids))
            us.append(len(np.unique(ids)))
            i += 1
        t = statistics.median(times)
        nbytes = statistics.mean(us) * eb + sh_bytes
        out.append({"config": name, "batch": M, "ms": round(t * 1e3, 3), "tok_s": round(M / t, 1),
                    "gbs": round(nbytes / t / 1e9, 2), "experts_per_step": round(statistics.mean(us), 2),
                    "timed_steps": len(times)})
    isa = cpu.isa
    cpu.close()
    if sh is not None:
        sh.close()
    for r in out:
        r["isa"] = isa
    return out


def cpu_baseline(step_budget_s: float = 0.6) -> dict:
    """The C++ restatement of the reference's CPU MoE executor on this host:
    every CPU configuration at its batch sizes, on all physical cores of this
    process's CPU share and on the physical cores of one NUMA node (the
    reference assumes a single node, ``cpu_moe_ext.cpp:1094-1095``).  ``value``
    is C4 at batch 64 on all cores (the headline workload); the rest is in
    ``sweep``."""
    host = _host_cpu_info()
    all_cores = host["share_physical_cores"]
    node, node_cpus = max(host["numa_nodes"].items(), key=lambda kv: len(kv[1])) if host["numa_nodes"] else (None, [])
    node_cores = [c for c in all_cores if c in set(node_cpus)] or all_cores
    variants = {"all_physical_cores": all_cores}
    if node_cores != all_cores:
        variants[f"numa_{node}"] = node_cores
    sweep = []
    for vname, cores in variants.items():
        for i, cfg in enumerate(CPU_CONFIGS):
            log(f"[bench] CPU baseline {cfg[0]} on {vname} ({len(cores)} threads)")
            for r in _cpu_config_runs(cfg, cores, step_budget_s, seed=11 + i):
                r["variant"] = vname
                r["threads"] = len(cores)
                sweep.append(r)
    head = next(r for r in sweep if r["variant"] == "all_physical_cores" and r["config"].startswith("c4")
                and r["batch"] == 64)
    same = "" if len(variants) > 1 else (f"; the process's CPU share lies on one NUMA node ({node}), so the "
                                         f"single-node variant is the all-cores run")
    return {
        "value": head["gbs"],
        "unit": "GB/s",
        "cores": len(all_cores),
        "kind": "port",
        "sample": (f"C4 decode batch 64: {head['timed_steps']} timed steps after 2 warm-up (median "
                   f"{head['ms']} ms/step, {head['tok_s']} tok/s), routed experts only over 64 host experts as "
                   f"bf16 banks (the reference's CPU route for FP8 checkpoints), two-pass GEMV restatement of "
                   f"cpu_moe_ext.cpp, ISA {head['isa']}, {len(all_cores)} pinned threads on physical cores{same}"),
        "host": {"cpu_model": host["model"], "isa": head["isa"], "smt_active": host["smt_active"],
                 "physical_cores_total": host["physical_cores_total"], "threads_all_cores": len(all_cores),
                 "numa_node": node, "threads_numa_node": len(node_cores),
                 "numa_nodes_of_share": {k: len(v) for k, v in host["numa_nodes"].items()}},
        "sweep": sweep,
    }


# ----------------------------------------------------------------------------- main

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_c4_b64_gate_up_traffic.json")


def measured_traffic(batch: int):
    """HBM bytes per launch of the gate_up kernel, from the two rocprofv3 counter
    runs (FETCH_SIZE, WRITE_SIZE, each scaled by a 1 GiB copy) summarised in
    profiles/; only for the workload they were measured on, else None."""
    if batch != 64 or not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        return int(json.load(f)["traffic_bytes_per_launch"])



def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--config", choices=("c2", "c3", "c4"), default="c4",
                    help="decode configuration of the timed layer (c4: the headline line; c2/c3: that layer "
                         "alone at --batch, printed as its own line -- a profiling aid)")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-step-seconds", type=float, default=0.6,
                    help="time budget of each CPU baseline point (at least 3 timed steps, at most 64)")
    ap.add_argument("--cpu-only", action="store_true", help="run only the CPU baseline and print it")
    ap.add_argument("--miss-only", action="store_true", help="time the miss path (admission + PCIe gather) alone")
    ap.add_argument("--hybrid-only", action="store_true", help="time the hybrid CPU/GPU decode alone")
    ap.add_argument("--prefill-offload-only", action="store_true",
                    help="time the expert cache's prefill movement (materialize vs double buffer) alone")
    ap.add_argument("--prefill-only", choices=("fp8_block", "mxfp4"), default=None,
                    help="profiling aid: run only the C5 prefill of this format and print its result")
    ap.add_argument("--dense-fp8-library", action="store_true",
                    help="reference point only: time hipBLASLt (torch._scaled_mm) on dense FP8 GEMMs of C5's shapes")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="run one device copy of this many MiB first (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (the MoE-layer hot path is measured on one MI355X); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    if args.cpu_only:  # host cores only
        print(json.dumps(cpu_baseline(args.cpu_step_seconds)), flush=True)
        return 0
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(1234)

    if args.calib_copy_mib:
        a = torch.empty((args.calib_copy_mib << 20,), dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    if args.miss_only:
        res = run_miss_fetch(gen, dev)
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in res.items()}), flush=True)
        return 0

    if args.prefill_offload_only:
        res = run_prefill_offload(gen, dev)
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in res.items()}), flush=True)
        return 0

    if args.hybrid_only:
        for M in (1, 4):
            res = run_hybrid(gen, dev, M=M)
            print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in res.items()}), flush=True)
        return 0

    if args.dense_fp8_library:
        for rec in run_dense_fp8_library(dev):
            print(json.dumps(rec), flush=True)
        return 0

    if args.prefill_only:
        res = run_prefill(args.prefill_only, args.steps, args.warmup, gen, dev)
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in res.items()}), flush=True)
        return 0

    hcfg = {"c2": C2, "c3": C3, "c4": C4}[args.config]
    if hcfg is not C4:  # one decode configuration alone (profiling aid)
        log(f"[bench] building {hcfg['name']}")
        layer = DecodeLayer(hcfg, dev, gen)
        res = run_decode(layer, args.batch, args.steps, args.warmup, gen, stage_timing=True)
        print(json.dumps({"config": hcfg["name"], **{k: (round(v, 4) if isinstance(v, float) else v)
                                                    for k, v in res.items()}}), flush=True)
        return 0
    log("[bench] building C4 layer (64 resident FP8 experts + shared)")
    c4 = DecodeLayer(C4, dev, gen)
    log(f"[bench] C4 decode batch {args.batch}: {args.steps} steps")
    head = run_decode(c4, args.batch, args.steps, args.warmup, gen, stage_timing=True)
    gu_us = head["stage_us"]["gate_up"]
    gu_gbs = head["gate_up_bytes_per_launch"] / (gu_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(args.batch),
                "kernel": "decode_stage_kernel<FP8,FP8,0> (gate_up + SwiGLU)",
                "avg_launch_us": round(gu_us, 2),
                "algorithmic_bytes_per_launch": int(head["gate_up_bytes_per_launch"])}

    def seeded(tag: str) -> torch.Generator:
        # each sweep line draws from its own seed, so that adding or removing a
        # line leaves the others' inputs (routings, weights) unchanged
        return torch.Generator(device=dev).manual_seed(zlib.crc32(tag.encode()) & 0x7FFFFFFF)

    sweep = {}
    if not args.no_sweep:
        for M in (1, 2, 4, 8, 16, 32, 128, 192, 256):
            log(f"[bench] sweep C4 decode batch {M}")
            sweep[f"{C4['name']}_b{M}"] = run_decode(c4, M, 20, 3, seeded(f"{C4['name']}_b{M}"), stage_timing=True,
                                                     min_ms=20.0)
    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline")
        cpu = cpu_baseline(args.cpu_step_seconds)
    del c4
    torch.cuda.empty_cache()
    if not args.no_sweep:
        for cfg in (C2, C3):
            log(f"[bench] sweep {cfg['name']}")
            layer = DecodeLayer(cfg, dev, seeded(cfg["name"]))
            for M in (1, 8, 32, 64):
                sweep[f"{cfg['name']}_b{M}"] = run_decode(layer, M, 20, 3, seeded(f"{cfg['name']}_b{M}"),
                                                          stage_timing=True, min_ms=20.0)
            del layer
            torch.cuda.empty_cache()
        for fmt in ("fp8_block", "mxfp4"):
            log(f"[bench] sweep C5 prefill {fmt}")
            sweep[f"c5_prefill_8192_{fmt}"] = run_prefill(fmt, 10, 3, seeded(f"c5_prefill_8192_{fmt}"), dev)
        log("[bench] sweep C4 miss path (admission + PCIe gather of 8 experts per step)")
        sweep["c4_miss_fetch_8_experts"] = run_miss_fetch(seeded("c4_miss_fetch_8_experts"), dev)
        log("[bench] sweep C4 prefill movement (3 layers x 32 host-resident experts, 8192 tokens)")
        sweep["c4_prefill_offload_3x32_experts"] = run_prefill_offload(seeded("c4_prefill_offload_3x32_experts"), dev)
        log("[bench] sweep C4 hybrid decode (1 expert fetched per step, the other misses on the CPU)")
        sweep["c4_hybrid_b1"] = run_hybrid(seeded("c4_hybrid_b1"), dev, M=1)
        log("[bench] sweep C4 expert-parallel share (EP-8: 32 experts on this GPU, 64 tokens per GPU)")
        sweep["c4_ep8_share_b64_per_gpu"] = run_ep_share(seeded("c4_ep8_share_b64_per_gpu"), dev)
        # the reference's benched rules (moe/bench_profile.py:156-191): the fetch share from the measured
        # PCIe and CPU rates, pcie / cpu for rates taken under DRAM contention, pcie / (pcie + cpu) for
        # rates of transfers that overlap without contending; both from this run's standalone rates
        from freetoken_amd.moe.cpu_decode import hybrid_fetch_fraction

        pcie, cpu_rate = sweep["c4_miss_fetch_8_experts"]["fetch_gbs"], sweep["c4_hybrid_b1"]["cpu_gbs"]
        for rule, overlapped in (("contention", False), ("overlap", True)):
            frac = hybrid_fetch_fraction(pcie, cpu_rate, overlapped=overlapped)
            log(f"[bench] sweep C4 hybrid decode, measured fetch fraction {frac} ({rule} rule)")
            sweep[f"c4_hybrid_b1_fraction_{rule}_rule"] = run_hybrid(seeded(f"c4_hybrid_b1_fraction_{rule}_rule"), dev, M=1,
                                                                     fetch_fraction=frac)

    def rnd(d):
        return {k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}

    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 weights x bf16 activations (W8A16, bf16 MFMA, fp32 accumulate)",
        "data": "synthetic (seeded N(0,0.02) weights quantised to 128x128-block FP8, N(0,1) activations/logits)",
        "config": {"workload": f"C4 DeepSeek-V3-shaped FP8 MoE layer decode, batch {args.batch}",
                   "hidden": 7168, "experts": 256, "resident_slots": 64, "top_k": 8,
                   "router": "grouped sigmoid 8 groups / top-4 groups, bias, scale 2.5",
                   "intermediate": 2048, "shared_expert": "1 x FP8 (I=2048)",
                   "tok_s": round(head["tok_s"], 1), "hbm_frac": round(head["hbm_frac"], 4),
                   "resident_experts_per_step": round(head["resident_experts_per_step"], 2),
                   "stage_us": {k: round(v, 2) for k, v in head["stage_us"].items()},
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "sweep": {k: rnd(v) for k, v in sweep.items()},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
