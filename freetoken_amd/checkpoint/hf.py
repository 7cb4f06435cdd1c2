"""Routed-expert banks from a Hugging Face block-FP8 safetensors checkpoint
(Qwen3-30B-A3B / DeepSeek-V3-class models), and their FTW conversion.

Reference: ``setup_offload_expert_banks`` / ``_build_fp8_expert_banks`` /
``_setup_bf16_dequant_banks`` (``models/qwen3_5_moe/weight.py:834-1055``) and
``convert_checkpoint`` (``checkpoint/convert.py:163-330``).

Tensor names follow the HF layout the reference matches
(``models/qwen3_5_moe/weight.py:720-723``), under one of the two decoder
stems, ``model.language_model.layers`` (Qwen3.5) or ``model.layers``
(DeepSeek-V3)::

    <stem>.<L>.mlp.experts.<e>.{gate,up,down}_proj.{weight,weight_scale_inv}

Multi-token-prediction heads are not decoder layers and are dropped, as the
reference drops them: Qwen3.5's ``mtp.layers.N.mlp.experts.*`` do not match the
anchored stems (``weight.py:36-38,718-723``), and DeepSeek-V3's MTP layer,
stored as ``model.layers.<num_hidden_layers>`` after the decoder layers, is
cut by the ``num_hidden_layers`` of ``config.json`` (or of its
``text_config``), as the reference's model config counts only those
(``models/glm4_moe/config.py:28-30``).

``weight`` is e4m3 ``[N, K]``; ``weight_scale_inv`` the 128x128 block scale
``[N/128, K/128]`` (bf16 in the reference's checkpoints, float32 in some).
MoE layer ``li`` is checkpoint layer ``first_moe_layer + li`` (the dense
prefix, e.g. DeepSeek-V3's ``first_k_dense_replace`` = 3, comes first).

Banks, per MoE layer, ``[E, ...]`` host tensors (pinned for the slot cache's
PCIe gather, ``ExpertSlotCache.set_bank_sources``):

* ``mode="fp8"`` (the reference default): ``gate_up`` e4m3 ``[E, 2I, H]``
  (gate rows ``[0, I)``, up rows ``[I, 2I)``), ``gate_up_scale``
  ``[E, 2I/128, H/128]``, ``down`` ``[E, H, I]``, ``down_scale``
  ``[E, H/128, I/128]``; scales widened to float32 for this build's kernels
  unless ``scales_to_float32=False`` (the FTW converter keeps the
  checkpoint's dtype, as the reference's FTW files do);
* ``mode="bf16"`` (the reference's ``FREETOKEN_FP8_EXPERTS=bf16``): every
  expert dequantised at load, ``W[n, k] = fp8(W[n, k]) * s[n/128, k/128]``
  rounded to bf16 (``dequant_block_fp8``, ``kernel/triton/fp8_block_linear.py:262-271``):
  ``gate_up`` ``[E, 2I, H]`` and ``down`` ``[E, H, I]`` bf16 (twice the bytes).

Reading: each safetensors shard is opened (memory-mapped) by one worker of a
thread pool and its expert tensors are copied straight into their bank rows,
so no layer is materialised twice.
"""

from __future__ import annotations

import hashlib
import json
import os
import re
import shutil
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass

import torch

from .ftw import DEFAULT_SHARD_LIMIT, _host_buffer, save_ftw_banks

BLOCK = 128
INDEX_FILE = "model.safetensors.index.json"
_EXPERT_RE = re.compile(
    r"^(?P<stem>model\.(?:language_model\.)?)layers\.(?P<layer>\d+)\.mlp\.experts\.(?P<expert>\d+)\."
    r"(?P<proj>gate|up|down)_proj\.(?P<kind>weight|weight_scale_inv)$"
)
_WEIGHT_SUFFIXES = (".safetensors", ".gguf", ".ftw")
_SKIP_NAMES = (INDEX_FILE,)
_SKIP_DIRS = (".git", ".cache", ".freetoken_expert_cache")


@dataclass(frozen=True)
class ExpertLayout:
    """Shape of the routed experts found in a checkpoint."""

    num_layers: int        # MoE layers
    num_experts: int
    hidden: int
    inter: int
    first_moe_layer: int   # checkpoint index of MoE layer 0
    scale_dtype: torch.dtype


def _weight_map(model_path: str) -> dict[str, str]:
    """tensor name -> shard file, from the index (or the one shard without one)."""
    idx = os.path.join(model_path, INDEX_FILE)
    if os.path.isfile(idx):
        with open(idx) as f:
            return json.load(f)["weight_map"]
    single = os.path.join(model_path, "model.safetensors")
    if not os.path.isfile(single):
        raise FileNotFoundError(f"{model_path}: neither {INDEX_FILE} nor model.safetensors")
    from safetensors import safe_open

    with safe_open(single, "pt") as f:
        return {k: "model.safetensors" for k in f.keys()}


def _num_hidden_layers(model_path: str) -> int | None:
    """Decoder layers of the checkpoint's ``config.json`` (``num_hidden_layers``,
    or that of ``text_config`` for multimodal configs); None when not stated."""
    path = os.path.join(model_path, "config.json")
    if not os.path.isfile(path):
        return None
    with open(path) as f:
        cfg = json.load(f)
    n = cfg.get("num_hidden_layers")
    if n is None and isinstance(cfg.get("text_config"), dict):
        n = cfg["text_config"].get("num_hidden_layers")
    return int(n) if n is not None else None


def scan_experts(model_path: str) -> tuple[ExpertLayout, dict[str, list[tuple[str, tuple]]]]:
    """The checkpoint's expert layout and, per shard file, its expert tensors as
    (name, (layer, expert, proj, kind)); raises on a missing or misshapen tensor."""
    from safetensors import safe_open

    wmap = _weight_map(model_path)
    n_layers = _num_hidden_layers(model_path)
    per_file: dict[str, list[tuple[str, tuple]]] = {}
    layers, experts, stems = set(), set(), set()
    for name, file in wmap.items():
        m = _EXPERT_RE.match(name)
        if m is None:
            continue
        if n_layers is not None and int(m["layer"]) >= n_layers:
            continue  # an MTP layer stored after the decoder layers
        stems.add(m["stem"])
        key = (int(m["layer"]), int(m["expert"]), m["proj"], m["kind"])
        per_file.setdefault(file, []).append((name, key))
        layers.add(key[0])
        experts.add(key[1])
    if not per_file:
        raise ValueError(f"{model_path}: no routed-expert tensors (model[.language_model].layers.L.mlp.experts.e.*_proj.*)")
    if len(stems) > 1:
        raise ValueError(f"{model_path}: routed experts under two decoder stems {sorted(stems)}")
    first, L, E = min(layers), len(layers), len(experts)
    if sorted(layers) != list(range(first, first + L)) or sorted(experts) != list(range(E)):
        raise ValueError(f"{model_path}: expert layers {sorted(layers)} / experts 0..{E - 1} not contiguous")
    n_expected = L * E * 6
    n_found = sum(len(v) for v in per_file.values())
    if n_found != n_expected:
        raise ValueError(f"{model_path}: {n_found} expert tensors, expected {n_expected} (gate/up/down x weight/scale)")
    # shapes from one expert's headers
    file0, (name0, _) = next((f, v[0]) for f, v in per_file.items())
    stem = _EXPERT_RE.match(name0)["stem"] or ""
    shapes, sdt = {}, None
    probe = f"{stem}layers.{first}.mlp.experts.0."
    for proj in ("gate", "up", "down"):
        for kind in ("weight", "weight_scale_inv"):
            n = f"{probe}{proj}_proj.{kind}"
            with safe_open(os.path.join(model_path, wmap[n]), "pt") as f:
                sl = f.get_slice(n)
                shapes[(proj, kind)] = tuple(sl.get_shape())
                if kind == "weight" and sl.get_dtype() != "F8_E4M3":
                    raise ValueError(f"{n}: dtype {sl.get_dtype()}, the block-FP8 banks need F8_E4M3")
                if kind == "weight_scale_inv":
                    sdt = {"BF16": torch.bfloat16, "F32": torch.float32}.get(sl.get_dtype())
                    if sdt is None:
                        raise ValueError(f"{n}: scale dtype {sl.get_dtype()}")
    I, H = shapes[("gate", "weight")]
    if (shapes[("up", "weight")] != (I, H) or shapes[("down", "weight")] != (H, I) or H % BLOCK or I % BLOCK
            or shapes[("gate", "weight_scale_inv")] != (I // BLOCK, H // BLOCK)
            or shapes[("down", "weight_scale_inv")] != (H // BLOCK, I // BLOCK)):
        raise ValueError(f"{model_path}: inconsistent expert shapes {shapes}")
    return ExpertLayout(L, E, H, I, first, sdt), per_file


def _alloc(shape, dtype, pinned: bool) -> torch.Tensor:
    n = 1
    for s in shape:
        n *= s
    nbytes = n * torch.empty((), dtype=dtype).element_size()
    return _host_buffer(nbytes, pinned)[:nbytes].view(dtype).view(shape)


def load_hf_expert_banks(model_path: str, *, mode: str = "fp8", pinned: bool = True,
                         scales_to_float32: bool = True, workers: int = 8):
    """Per-layer routed-expert banks of a block-FP8 HF checkpoint.

    Returns (quant_format, sources, layout): quant_format "fp8_block" (mode
    "fp8") or "bf16" (mode "bf16"); ``sources[bank][layer]`` the ``[E, ...]``
    host tensors in the slot cache's bank order."""
    mode = mode.strip().lower()
    if mode not in ("fp8", "bf16"):
        raise ValueError(f"mode must be 'fp8' or 'bf16', got {mode!r}")
    from safetensors import safe_open

    lay, per_file = scan_experts(model_path)
    L, E, H, I = lay.num_layers, lay.num_experts, lay.hidden, lay.inter
    sdt = torch.float32 if (scales_to_float32 or mode == "bf16") else lay.scale_dtype
    if mode == "fp8":
        specs = {"gate_up": ((E, 2 * I, H), torch.float8_e4m3fn),
                 "gate_up_scale": ((E, 2 * I // BLOCK, H // BLOCK), sdt),
                 "down": ((E, H, I), torch.float8_e4m3fn),
                 "down_scale": ((E, H // BLOCK, I // BLOCK), sdt)}
    else:
        specs = {"gate_up": ((E, 2 * I, H), torch.bfloat16), "down": ((E, H, I), torch.bfloat16)}
    sources = {name: [_alloc(shape, dt, pinned) for _ in range(L)] for name, (shape, dt) in specs.items()}

    def dest(li, e, proj, kind):
        if mode == "fp8":
            if kind == "weight":
                return (sources["gate_up"][li][e, :I] if proj == "gate" else
                        sources["gate_up"][li][e, I:] if proj == "up" else sources["down"][li][e])
            return (sources["gate_up_scale"][li][e, : I // BLOCK] if proj == "gate" else
                    sources["gate_up_scale"][li][e, I // BLOCK:] if proj == "up" else sources["down_scale"][li][e])
        return (sources["gate_up"][li][e, :I] if proj == "gate" else
                sources["gate_up"][li][e, I:] if proj == "up" else sources["down"][li][e])

    def read_file(file: str, items: list) -> None:
        with safe_open(os.path.join(model_path, file), "pt") as f:
            if mode == "fp8":
                for name, (layer, e, proj, kind) in items:
                    dest(layer - lay.first_moe_layer, e, proj, kind).copy_(f.get_tensor(name))
                return
            # bf16: dequantise each projection from its weight and scale (both in this
            # shard in practice; a scale elsewhere is fetched from its own shard)
            weights = [(n, key) for n, key in items if key[3] == "weight"]
            names = {key: n for n, key in items}
            for name, (layer, e, proj, _) in weights:
                sname = names.get((layer, e, proj, "weight_scale_inv"))
                scale = f.get_tensor(sname) if sname else _tensor(model_path, name.replace(".weight", ".weight_scale_inv"))
                dest(layer - lay.first_moe_layer, e, proj, "weight").copy_(dequant_block_fp8(f.get_tensor(name), scale))

    with ThreadPoolExecutor(max(1, min(workers, len(per_file)))) as pool:
        for fut in [pool.submit(read_file, file, items) for file, items in per_file.items()]:
            fut.result()
    return ("fp8_block" if mode == "fp8" else "bf16"), sources, lay


def _tensor(model_path: str, name: str) -> torch.Tensor:
    from safetensors import safe_open

    with safe_open(os.path.join(model_path, _weight_map(model_path)[name]), "pt") as f:
        return f.get_tensor(name)


def dequant_block_fp8(weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16(fp8(W[n, k]) * s[n/128, k/128]) in float32 (``dequant_block_fp8``,
    ``kernel/triton/fp8_block_linear.py:262-271``)."""
    n, k = weight.shape
    s = scale.to(torch.float32).repeat_interleave(BLOCK, 0)[:n].repeat_interleave(BLOCK, 1)[:, :k]
    return (weight.to(torch.float32) * s).to(torch.bfloat16)


def _fingerprint(model_path: str, mode: str) -> str:
    """Identity of the source (file names, sizes, times) and the bank mode."""
    h = hashlib.sha256(f"mode={mode}|".encode())
    for name in sorted(os.listdir(model_path)):
        if name.endswith(".safetensors"):
            st = os.stat(os.path.join(model_path, name))
            h.update(f"{name}:{st.st_size}:{int(st.st_mtime)}|".encode())
    return h.hexdigest()[:16]


def _copy_metadata(model_path: str, out_dir: str) -> list[str]:
    """Every non-weight file (config, tokenizer, remote code) with its relative
    path, so the FTW directory is a checkpoint of its own (``checkpoint/convert.py:60-107``)."""
    out_abs = os.path.abspath(out_dir)
    copied = []
    for root, dirs, files in os.walk(model_path):
        dirs[:] = [d for d in dirs if d not in _SKIP_DIRS and os.path.abspath(os.path.join(root, d)) != out_abs]
        for name in files:
            if name.endswith(_WEIGHT_SUFFIXES) or name in _SKIP_NAMES:
                continue
            src = os.path.join(root, name)
            rel = os.path.relpath(src, model_path)
            dst = os.path.join(out_dir, rel)
            os.makedirs(os.path.dirname(dst), exist_ok=True)
            shutil.copy2(src, dst)
            copied.append(rel)
    return copied


def convert_hf_experts_to_ftw(model_path: str, out_dir: str, *, mode: str = "fp8", per_layer: bool = True,
                              shard_limit: int = DEFAULT_SHARD_LIMIT, workers: int = 8) -> dict:
    """Writes the checkpoint's routed-expert banks as an FTW checkpoint
    (``experts_bank`` entries, one per (bank, layer) or one flat region per
    bank) with the source's metadata files; scales keep the checkpoint's dtype.
    The dense weights are outside the MoE-layer path and are not converted.
    Returns the index."""
    if os.path.abspath(model_path) == os.path.abspath(out_dir):
        raise ValueError("out_dir must differ from the source checkpoint")
    fmt, sources, lay = load_hf_expert_banks(model_path, mode=mode, pinned=False, scales_to_float32=False,
                                             workers=workers)
    copied = _copy_metadata(model_path, out_dir)
    meta = {"source_fingerprint": _fingerprint(model_path, mode), "first_moe_layer": lay.first_moe_layer,
            "copied_files": copied}
    return save_ftw_banks(out_dir, fmt, sources, per_layer=per_layer, shard_limit=shard_limit, meta=meta)


__all__ = ["ExpertLayout", "scan_experts", "load_hf_expert_banks", "dequant_block_fp8", "convert_hf_experts_to_ftw"]
