"""FreeToken Weight (FTW) checkpoints: the on-disk expert banks of the offload
cache (reference ``checkpoint/ftw.py``).

On-disk contract kept from the reference (``checkpoint/ftw.py:1-61,110-190``)
so that its checkpoints load here and these files load there:

* ``<dir>/freetoken_weight.json`` -- index: ``format`` "freetoken_weight",
  ``version`` 1, ``align`` 4096, ``shard_limit``, ``total_bytes``,
  ``tensors[]`` (``name``, ``kind``, ``dtype`` as torch's name without
  ``torch.``, ``shape``, ``global_off``, ``nbytes``), ``shards[]`` (``file``,
  ``global_off``, ``nbytes``) and free metadata (``quant_format``,
  ``expert_bank_num_layers``);
* ``<dir>/freetoken-NNNNN.ftw`` -- one logical byte region cut into shards of
  at most ``shard_limit`` bytes at 4096-aligned points; every tensor starts
  4096-aligned and is padded to 4096; a tensor no larger than a shard never
  straddles two;
* expert banks are ``kind="experts_bank"`` entries, either one flat
  ``[num_layers * E, ...]`` region per bank or one entry per (bank, layer)
  named ``f"{bank}#L{layer:05d}"``.

Loading (``load_ftw_banks``) reads every (bank, layer) straight into pinned
host memory from a thread pool -- with O_DIRECT where the filesystem and the
destination mapping allow it (HIP's pinned allocations do not: direct I/O
into them fails with EFAULT, and those reads go through the page cache) --
and returns the per-layer ``[E, ...]`` tensors that
``ExpertSlotCache.set_bank_sources`` takes.  A flat region's layer is read
through its enclosing aligned window and viewed at its offset.  bf16 block
scales (the reference's FP8 banks) can be widened to float32 on load, the
scale type of this build's kernels.
"""

from __future__ import annotations

import errno
import json
import math
import os
import re
import threading
from concurrent.futures import ThreadPoolExecutor

import torch

INDEX_NAME = "freetoken_weight.json"
FORMAT_TAG = "freetoken_weight"
FORMAT_VERSION = 1
ALIGN = 4096
DEFAULT_SHARD_LIMIT = 8 << 30
SHARD_NAME = "freetoken-{:05d}.ftw"
CHUNK = 8 << 20
ALPHA_NAMES = ("gate_up_alpha", "down_alpha")
_LAYER_RE = re.compile(r"^(?P<base>.+)#L(?P<layer>\d{5})$")


def layer_bank_entry_name(bank_name: str, layer_id: int) -> str:
    return f"{bank_name}#L{layer_id:05d}"


def is_ftw_checkpoint(path: str) -> bool:
    return os.path.isfile(os.path.join(path, INDEX_NAME))


def _align_up(n: int) -> int:
    return -(-n // ALIGN) * ALIGN


def _dtype_name(dt: torch.dtype) -> str:
    return str(dt).split(".", 1)[1]


def _dtype(name: str) -> torch.dtype:
    dt = getattr(torch, name, None)
    if not isinstance(dt, torch.dtype):
        raise ValueError(f"unknown FTW dtype {name!r}")
    return dt


class FTWWriter:
    """Appends tensors to the logical region in call order; ``finalize``
    writes the index."""

    def __init__(self, out_dir: str, shard_limit: int = DEFAULT_SHARD_LIMIT):
        if shard_limit <= 0 or shard_limit % ALIGN:
            raise ValueError("shard_limit must be a positive multiple of 4096")
        os.makedirs(out_dir, exist_ok=True)
        self.out_dir = out_dir
        self.shard_limit = shard_limit
        self.tensors: list[dict] = []
        self.shards: list[dict] = []
        self._pos = 0          # logical offset of the next byte
        self._file = None
        self._used = 0         # bytes in the open shard

    def _next_shard(self) -> None:
        self._close_shard()
        self.shards.append({"file": SHARD_NAME.format(len(self.shards)), "global_off": self._pos, "nbytes": 0})
        self._file = open(os.path.join(self.out_dir, self.shards[-1]["file"]), "wb")
        self._used = 0

    def _close_shard(self) -> None:
        if self._file is not None:
            self.shards[-1]["nbytes"] = self._used
            self._file.close()
            self._file = None

    def _write(self, data) -> None:
        mv = memoryview(data).cast("B")
        while len(mv):
            if self._file is None or self._used == self.shard_limit:
                self._next_shard()
            n = min(len(mv), self.shard_limit - self._used)
            self._file.write(mv[:n])
            mv = mv[n:]
            self._used += n
            self._pos += n

    def add_tensor(self, name: str, tensor: torch.Tensor, kind: str = "weight") -> None:
        t = tensor.detach().to("cpu").contiguous()
        raw = t.reshape(-1).view(torch.uint8).numpy()
        nbytes = raw.size
        if self._file is None or (nbytes <= self.shard_limit and self._used + nbytes > self.shard_limit):
            self._next_shard()  # a tensor that fits one shard starts a fresh one rather than straddle
        start = self._pos
        self._write(raw)
        pad = _align_up(self._pos) - self._pos
        if pad:
            self._write(bytes(pad))
        self.tensors.append({"name": name, "kind": kind, "dtype": _dtype_name(t.dtype), "shape": list(t.shape),
                             "global_off": start, "nbytes": int(nbytes)})

    def finalize(self, meta: dict | None = None) -> dict:
        self._close_shard()
        index = {"format": FORMAT_TAG, "version": FORMAT_VERSION, "align": ALIGN, "shard_limit": self.shard_limit,
                 "total_bytes": self._pos, "tensors": self.tensors, "shards": self.shards, **(meta or {})}
        tmp = os.path.join(self.out_dir, INDEX_NAME + ".tmp")
        with open(tmp, "w") as f:
            json.dump(index, f)
        os.replace(tmp, os.path.join(self.out_dir, INDEX_NAME))
        return index


class FTWReader:
    """Positional reads of FTW byte ranges into caller memory."""

    def __init__(self, path: str):
        with open(os.path.join(path, INDEX_NAME)) as f:
            self.index = json.load(f)
        if self.index.get("format") != FORMAT_TAG or self.index.get("version") != FORMAT_VERSION:
            raise ValueError(f"{path}: not a {FORMAT_TAG} v{FORMAT_VERSION} index")
        if self.index.get("align", ALIGN) != ALIGN:
            raise ValueError(f"{path}: alignment {self.index.get('align')} != {ALIGN}")
        self.dir = path
        self.shards = sorted(self.index["shards"], key=lambda s: s["global_off"])
        self._fds: dict[tuple[str, bool], int] = {}
        self._lock = threading.Lock()
        self._direct: bool | None = None

    def meta(self, key: str, default=None):
        return self.index.get(key, default)

    def entries(self, *kinds: str) -> list[dict]:
        return [t for t in self.index["tensors"] if not kinds or t["kind"] in kinds]

    def _fd(self, file: str, direct: bool) -> int:
        key = (file, direct)
        with self._lock:
            fd = self._fds.get(key)
            if fd is None:
                flags = os.O_RDONLY | (getattr(os, "O_DIRECT", 0) if direct else 0)
                fd = os.open(os.path.join(self.dir, file), flags)
                self._fds[key] = fd
            return fd

    def _use_direct(self) -> bool:
        with self._lock:
            if self._direct is None:
                self._direct = False
                if hasattr(os, "O_DIRECT") and self.shards:
                    try:  # tmpfs and several overlay filesystems refuse O_DIRECT at open
                        os.close(os.open(os.path.join(self.dir, self.shards[0]["file"]),
                                         os.O_RDONLY | os.O_DIRECT))
                        self._direct = True
                    except OSError:
                        pass
            return self._direct

    def pieces(self, global_off: int, nbytes: int):
        """(file, file offset, destination offset, length) covering the range,
        cut at shard boundaries."""
        out, pos, end = [], global_off, global_off + nbytes
        for sh in self.shards:
            s0, s1 = sh["global_off"], sh["global_off"] + sh["nbytes"]
            if pos >= end:
                break
            if pos >= s1:
                continue
            if pos < s0:
                raise ValueError("FTW index has a gap between shards")
            take = min(end, s1) - pos
            out.append((sh["file"], pos - s0, pos - global_off, take))
            pos += take
        if pos < end:
            raise ValueError("byte range runs past the last FTW shard")
        return out

    def read_into(self, dest: torch.Tensor, global_off: int, nbytes: int, pool: ThreadPoolExecutor | None = None):
        """Reads [global_off, +nbytes) into the uint8 CPU tensor ``dest``
        (at least ``nbytes`` long).  O_DIRECT is used for the 4096-aligned
        body of each piece when ``dest`` is page-aligned; the rest is read
        buffered.  Raises on a short file."""
        if dest.dtype != torch.uint8 or dest.device.type != "cpu" or not dest.is_contiguous() or dest.numel() < nbytes:
            raise ValueError("dest must be a contiguous uint8 CPU tensor of at least nbytes")
        mv = memoryview(dest.numpy()).cast("B")
        aligned_dest = dest.data_ptr() % ALIGN == 0
        jobs = []
        for file, foff, doff, length in self.pieces(global_off, nbytes):
            for c in range(0, length, CHUNK):
                jobs.append((file, foff + c, doff + c, min(CHUNK, length - c)))
        direct = self._use_direct() and aligned_dest

        def run(job):
            file, foff, doff, length = job
            body = length // ALIGN * ALIGN if direct and foff % ALIGN == 0 and doff % ALIGN == 0 else 0
            if body:
                try:
                    _pread_all(self._fd(file, True), mv[doff:doff + body], foff)
                except OSError as err:
                    # direct I/O cannot target every mapping: HIP's pinned host
                    # allocations refuse it (EFAULT); read those buffered
                    if err.errno not in (errno.EFAULT, errno.EINVAL):
                        raise
                    body = 0
            if length > body:
                _pread_all(self._fd(file, False), mv[doff + body:doff + length], foff + body)

        if pool is None or len(jobs) == 1:
            for j in jobs:
                run(j)
        else:
            for f in [pool.submit(run, j) for j in jobs]:
                f.result()

    def close(self) -> None:
        with self._lock:
            for fd in self._fds.values():
                os.close(fd)
            self._fds.clear()


def _pread_all(fd: int, mv: memoryview, off: int) -> None:
    done = 0
    while done < len(mv):
        n = os.preadv(fd, [mv[done:]], off + done)
        if n <= 0:
            raise OSError(f"FTW shard ends early: {done}/{len(mv)} bytes at offset {off}")
        done += n


def _host_buffer(nbytes: int, pinned: bool) -> torch.Tensor:
    n = _align_up(max(nbytes, 1))
    if pinned:  # exact size: torch's pinned allocator would round each layer up to a power of two
        from ..ops import alloc_pinned_tensor

        return alloc_pinned_tensor(n, dtype=torch.uint8)
    return torch.empty((n,), dtype=torch.uint8)


def load_ftw_banks(path: str, num_layers: int, *, pinned: bool = True, scales_to_float32: bool = True,
                   workers: int = 8) -> tuple[str | None, dict[str, list[torch.Tensor]], dict[str, torch.Tensor]]:
    """The FTW's ``experts_bank`` entries as per-layer host banks (reference
    ``load_ftw_banks``, ``checkpoint/ftw.py:415-630``).

    Returns (quant_format, sources, alphas): ``sources[name][layer]`` is an
    ``[E, ...]`` tensor (pinned when ``pinned``), in the index's bank order;
    ``alphas`` holds the flat ``gate_up_alpha`` / ``down_alpha`` vectors when
    present.  With ``scales_to_float32`` bf16 ``*_scale`` banks are widened."""
    reader = FTWReader(path)
    try:
        entries = reader.entries("experts_bank")
        meta_layers = reader.meta("expert_bank_num_layers")
        if meta_layers is not None and meta_layers != num_layers:
            raise ValueError(f"{path}: banks written for {meta_layers} layers, {num_layers} asked")
        flat, per_layer, alpha = {}, {}, {}
        for e in entries:
            if e["name"] in ALPHA_NAMES:
                alpha[e["name"]] = e
                continue
            m = _LAYER_RE.match(e["name"])
            if m is None:
                flat[e["name"]] = e
            else:
                per_layer.setdefault(m.group("base"), {})[int(m.group("layer"))] = e
        if set(flat) & set(per_layer):
            raise ValueError(f"banks in both layouts: {sorted(set(flat) & set(per_layer))}")
        plan = []  # (name, layer, global_off, nbytes, head, shape, dtype)
        order = []
        for e in entries:
            m = _LAYER_RE.match(e["name"])
            base = m.group("base") if m else e["name"]
            if base not in order and base not in ALPHA_NAMES:
                order.append(base)
        for name, e in flat.items():
            total, *row = e["shape"]
            if total % num_layers:
                raise ValueError(f"bank {name}: {total} rows do not split into {num_layers} layers")
            E = total // num_layers
            dt = _dtype(e["dtype"])
            layer_bytes = E * math.prod(row) * dt.itemsize
            if layer_bytes * num_layers != e["nbytes"]:
                raise ValueError(f"bank {name}: size does not match its shape")
            for l in range(num_layers):
                off = e["global_off"] + l * layer_bytes
                win = off // ALIGN * ALIGN
                plan.append((name, l, win, off + layer_bytes - win, off - win, [E] + row, dt))
        for name, by_layer in per_layer.items():
            if sorted(by_layer) != list(range(num_layers)):
                raise ValueError(f"bank {name}: per-layer entries {sorted(by_layer)} != range({num_layers})")
            for l, e in by_layer.items():
                plan.append((name, l, e["global_off"], e["nbytes"], 0, e["shape"], _dtype(e["dtype"])))
        bufs = {}
        with ThreadPoolExecutor(max(1, workers)) as pool:
            for name, l, off, nbytes, head, shape, dt in plan:
                buf = _host_buffer(nbytes, pinned)
                reader.read_into(buf, off, nbytes, pool)
                bufs[(name, l)] = buf[head:head + math.prod(shape) * dt.itemsize].view(dt).view(shape)
            alphas = {}
            for name, e in alpha.items():
                buf = _host_buffer(e["nbytes"], False)
                reader.read_into(buf, e["global_off"], e["nbytes"], pool)
                alphas[name] = buf[:e["nbytes"]].view(_dtype(e["dtype"])).view(e["shape"])
        sources = {}
        for name in order:
            layers = [bufs[(name, l)] for l in range(num_layers)]
            if scales_to_float32 and name.endswith("_scale") and layers[0].dtype == torch.bfloat16:
                widened = []
                for t in layers:
                    f = _host_buffer(t.numel() * 4, pinned)[: t.numel() * 4].view(torch.float32).view(t.shape)
                    f.copy_(t)
                    widened.append(f)
                layers = widened
            sources[name] = layers
        return reader.meta("quant_format"), sources, alphas
    finally:
        reader.close()


def save_ftw_banks(path: str, quant_format: str, sources: dict[str, list[torch.Tensor]], *, per_layer: bool = True,
                   shard_limit: int = DEFAULT_SHARD_LIMIT, meta: dict | None = None) -> dict:
    """Writes per-layer banks as ``experts_bank`` entries: one per (bank,
    layer) (``per_layer``) or one flat ``[L * E, ...]`` region per bank."""
    w = FTWWriter(path, shard_limit)
    num_layers = len(next(iter(sources.values())))
    for name, layers in sources.items():
        if per_layer:
            for l, t in enumerate(layers):
                w.add_tensor(layer_bank_entry_name(name, l), t, kind="experts_bank")
        else:
            w.add_tensor(name, torch.cat([t.to("cpu") for t in layers]), kind="experts_bank")
    return w.finalize({"quant_format": quant_format, "expert_bank_num_layers": num_layers, **(meta or {})})


__all__ = ["INDEX_NAME", "FORMAT_TAG", "FORMAT_VERSION", "ALIGN", "DEFAULT_SHARD_LIMIT", "FTWWriter", "FTWReader",
           "is_ftw_checkpoint", "layer_bank_entry_name", "load_ftw_banks", "save_ftw_banks"]
