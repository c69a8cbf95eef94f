"""Expert host-store builder: checkpoint rows -> pinned [E, ...] host stores.

The reference never reads a checkpoint itself: it moves each MoE layer's
per-expert params to host memory before vLLM's loader runs
(src/sluice/offloader.py:509-571), lets the loader fill them, and pins them
at install (965-967).  ``ExpertStreamOffloader._prepare_layer`` does the same
with the params already viewing pinned stores, so nothing is copied twice.

This module is the same step for engines without vLLM's loader (the
synthetic decoders, tools): it reads Hugging Face safetensors checkpoints
and writes each expert's rows straight into the fused layout the slot
buffers use --

    w13_weight [E, 2I, H]   rows 0..I-1 = experts.{e}.gate_proj, I..2I-1 = up_proj
    w2_weight  [E, H, I]    experts.{e}.down_proj
    (fp8 block-quantised checkpoints, e4m3 weights + fp32 weight_scale_inv
     [ceil(rows/128), ceil(cols/128)])
    w13_weight_scale [E, 2*ceil(I/128), ceil(H/128)], w2_weight_scale [E, ceil(H/128), ceil(I/128)]

-- from a read-only memory map of each file (the safetensors layout: a
little-endian u64 header length, a JSON header of name -> dtype / shape /
data_offsets, then the data), one copy per row from the page cache into the
pinned store, spread over threads.
"""

from __future__ import annotations

import json
import mmap
import os
import struct
import threading
from concurrent.futures import ThreadPoolExecutor
from typing import Optional

import numpy as np
import torch

_DTYPES = {
    "BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32,
    "F8_E4M3": torch.float8_e4m3fn, "U8": torch.uint8, "I8": torch.int8, "I32": torch.int32,
    "I64": torch.int64,
}

EXPERT_KEY = "model.layers.{layer}.mlp.experts.{e}.{proj}.{kind}"


class Checkpoint:
    """Tensors of one safetensors file, a list of files, or a directory of
    them, by name, as zero-copy CPU views of read-only memory maps."""

    def __init__(self, path):
        paths = path if isinstance(path, (list, tuple)) else [path]
        files = []
        for p in paths:
            if os.path.isdir(p):
                files += sorted(os.path.join(p, f) for f in os.listdir(p)
                                if f.endswith(".safetensors"))
            else:
                files.append(p)
        if not files:
            raise FileNotFoundError(f"no .safetensors files under {path!r}")
        self._maps = []
        self._where: dict[str, tuple] = {}
        for fn in files:
            with open(fn, "rb") as f:
                mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
            (n,) = struct.unpack("<Q", mm[:8])
            if n <= 0 or 8 + n > len(mm):
                raise ValueError(f"{fn}: bad safetensors header length {n}")
            header = json.loads(bytes(mm[8:8 + n]))
            base = 8 + n
            arr = np.frombuffer(mm, dtype=np.uint8)
            self._maps.append((mm, arr))
            for name, info in header.items():
                if name == "__metadata__":
                    continue
                dt = _DTYPES.get(info["dtype"])
                if dt is None:
                    raise ValueError(f"{fn}: tensor {name} has unsupported dtype {info['dtype']}")
                b0, b1 = info["data_offsets"]
                shape = tuple(int(v) for v in info["shape"])
                esz = torch.empty((), dtype=dt).element_size()
                nbytes = int(np.prod(shape, dtype=np.int64)) * esz
                if b1 - b0 != nbytes or base + b1 > len(mm):
                    raise ValueError(f"{fn}: tensor {name} offsets do not match its shape")
                self._where[name] = (len(self._maps) - 1, base + b0, base + b1, dt, shape)

    def __contains__(self, name: str) -> bool:
        return name in self._where

    def names(self):
        return list(self._where)

    def info(self, name: str):
        _, _, _, dt, shape = self._where[name]
        return dt, shape

    def tensor(self, name: str) -> torch.Tensor:
        """Read-only view (do not write to it)."""
        i, b0, b1, dt, shape = self._where[name]
        raw = self._maps[i][1][b0:b1]
        import warnings

        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)  # non-writable buffer
            t = torch.from_numpy(raw)
        return t.view(dt).view(shape)

    def close(self):
        maps, self._maps = self._maps, []
        for i in range(len(maps)):
            mm = maps[i][0]
            maps[i] = None  # drop the array over the map first
            try:
                mm.close()
            except BufferError:
                pass  # a tensor view is still alive; the map closes with it


def expert_layout(ck: Checkpoint, layer: int, key: str = EXPERT_KEY):
    """(E, I, H, fp8) of a layer's routed experts in the checkpoint."""
    E = 0
    while key.format(layer=layer, e=E, proj="gate_proj", kind="weight") in ck:
        E += 1
    if E == 0:
        raise KeyError(f"layer {layer}: no experts under {key!r}")
    dt, (I, H) = ck.info(key.format(layer=layer, e=0, proj="gate_proj", kind="weight"))
    return E, I, H, dt == torch.float8_e4m3fn


def store_shapes(E: int, I: int, H: int, fp8: bool, block: int = 128) -> dict:
    """Name -> (shape, dtype) of a layer's host stores in the slot layout.
    fp8 needs I % block == 0: the fused w13 rows are scaled in blocks of
    `block` rows, so a block must not straddle the gate / up boundary."""
    if fp8 and I % block:
        raise ValueError(f"fp8 experts need the intermediate size ({I}) to be a multiple of the "
                         f"scale block ({block})")
    cd = lambda a: (a + block - 1) // block  # noqa: E731
    wdt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    out = {"w13_weight": ((E, 2 * I, H), wdt), "w2_weight": ((E, H, I), wdt)}
    if fp8:
        out["w13_weight_scale"] = ((E, 2 * cd(I), cd(H)), torch.float32)
        out["w2_weight_scale"] = ((E, cd(H), cd(I)), torch.float32)
    return out


def load_experts(ck: Checkpoint, layer: int, stores: dict, experts: Optional[list] = None,
                 key: str = EXPERT_KEY, threads: int = 8) -> int:
    """Copy layer ``layer``'s experts into ``stores`` (name -> CPU tensor in
    the slot layout, usually pinned): store row j <- checkpoint expert
    experts[j] (default: all, in order; an EP rank passes its owned global
    ids).  Returns the bytes copied."""
    w13, w2 = stores["w13_weight"], stores["w2_weight"]
    n, two_i, H = w13.shape
    I = two_i // 2
    ids = list(range(n)) if experts is None else [int(g) for g in experts]
    if len(ids) != n:
        raise ValueError(f"{len(ids)} experts for a store of {n} rows")
    fp8 = w13.dtype == torch.float8_e4m3fn
    jobs = []
    for j, g in enumerate(ids):
        k = lambda proj, kind="weight": key.format(layer=layer, e=g, proj=proj, kind=kind)  # noqa
        jobs.append((w13[j, :I], k("gate_proj")))
        jobs.append((w13[j, I:], k("up_proj")))
        jobs.append((w2[j], k("down_proj")))
        if fp8:
            s13, s2 = stores["w13_weight_scale"], stores["w2_weight_scale"]
            nI = s13.shape[1] // 2
            jobs.append((s13[j, :nI], k("gate_proj", "weight_scale_inv")))
            jobs.append((s13[j, nI:], k("up_proj", "weight_scale_inv")))
            jobs.append((s2[j], k("down_proj", "weight_scale_inv")))
    total = [0]
    lock = threading.Lock()

    def run(job):
        dst, name = job
        if name not in ck:
            raise KeyError(f"checkpoint has no tensor {name}")
        src = ck.tensor(name)
        if tuple(src.shape) != tuple(dst.shape) or src.dtype != dst.dtype:
            raise ValueError(f"{name}: checkpoint {tuple(src.shape)} {src.dtype} does not fit "
                             f"the store row {tuple(dst.shape)} {dst.dtype}")
        dst.copy_(src)
        with lock:
            total[0] += dst.numel() * dst.element_size()

    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        for _ in ex.map(run, jobs):
            pass
    return total[0]


def expert_stores_from_checkpoint(path, layer: int, pinned: bool = True, threads: int = 8,
                                  key: str = EXPERT_KEY) -> dict:
    """Build a layer's host stores (pinned ``ops.HostStore`` objects when
    ``pinned``, else plain CPU tensors wrapped alike) from a checkpoint.
    Returns name -> object with ``.tensor``."""
    ck = Checkpoint(path)
    try:
        E, I, H, fp8 = expert_layout(ck, layer, key)
        stores = {}
        for name, (shape, dt) in store_shapes(E, I, H, fp8).items():
            if pinned:
                from sluice_amd import ops

                stores[name] = ops.HostStore(shape, dt)
            else:
                stores[name] = _PlainStore(torch.empty(shape, dtype=dt))
        load_experts(ck, layer, {n: s.tensor for n, s in stores.items()}, key=key,
                     threads=threads)
        return stores
    finally:
        ck.close()


class _PlainStore:
    def __init__(self, t: torch.Tensor):
        self.tensor = t


def _bench(argv=None) -> dict:
    """Loader throughput on a synthetic checkpoint of a model's expert shape:
    one safetensors file per MoE layer (every expert's gate/up/down rows, and
    fp8 block scales for an fp8 shape; each expert's rows hold a distinct
    byte value) written to --dir (default: a fresh directory in /dev/shm, so
    the files are in memory as a warm page cache would be), then each layer
    loaded into pinned host stores: the stores' allocation timed apart from
    the copies, every expert's placement spot-checked."""
    import argparse
    import shutil
    import tempfile
    import time

    from safetensors.torch import save_file

    from sluice_amd import ops
    from sluice_amd.decoder import SPECS

    ap = argparse.ArgumentParser(description=_bench.__doc__)
    ap.add_argument("--bench", action="store_true")
    ap.add_argument("--shape", choices=sorted(SPECS), default="qwen3")
    ap.add_argument("--layers", type=int, default=2)
    ap.add_argument("--threads", type=int, default=8)
    ap.add_argument("--dir", default=None)
    a = ap.parse_args(argv)
    sp = SPECS[a.shape]
    E, I, H, fp8 = sp["E"], sp["I"], sp["H"], sp["fp8"]
    cd = lambda n: (n + 127) // 128  # noqa: E731
    own = a.dir is None
    d = a.dir or tempfile.mkdtemp(prefix="sluice_ckpt_",
                                  dir="/dev/shm" if os.path.isdir("/dev/shm") else None)
    try:
        t0 = time.perf_counter()
        for L in range(a.layers):
            tensors = {}
            for e in range(E):
                v = (L * 37 + e) % 120 + 1
                for proj, (r, c) in (("gate_proj", (I, H)), ("up_proj", (I, H)),
                                     ("down_proj", (H, I))):
                    name = EXPERT_KEY.format(layer=L, e=e, proj=proj, kind="weight")
                    raw = torch.full((r, c * (1 if fp8 else 2)), v, dtype=torch.uint8)
                    tensors[name] = raw.view(torch.float8_e4m3fn) if fp8 else \
                        raw.view(torch.bfloat16)
                    if fp8:
                        tensors[EXPERT_KEY.format(layer=L, e=e, proj=proj,
                                                  kind="weight_scale_inv")] = torch.full(
                            (cd(r), cd(c)), float(v), dtype=torch.float32)
            save_file(tensors, os.path.join(d, f"layer-{L:03d}.safetensors"))
            del tensors
        write_s = time.perf_counter() - t0
        ck = Checkpoint(d)
        try:
            t0 = time.perf_counter()
            stores = {n: ops.HostStore(shape, dt)
                      for n, (shape, dt) in store_shapes(E, I, H, fp8).items()}
            alloc_s = time.perf_counter() - t0
            views = {n: s.tensor for n, s in stores.items()}
            per_layer = []
            for L in range(a.layers):
                t0 = time.perf_counter()
                nbytes = load_experts(ck, L, views, threads=a.threads)
                dt = time.perf_counter() - t0
                w13 = views["w13_weight"].view(torch.uint8)
                w2 = views["w2_weight"].view(torch.uint8)
                for e in (0, E // 2, E - 1):
                    v = (L * 37 + e) % 120 + 1
                    if int(w13[e, 0, 0]) != v or int(w13[e, -1, -1]) != v or \
                            int(w2[e, -1, -1]) != v:
                        raise RuntimeError(f"layer {L} expert {e}: rows misplaced")
                per_layer.append({"bytes": nbytes, "s": dt, "GBs": nbytes / dt / 1e9})
            store_bytes = sum(t.numel() * t.element_size() for t in views.values())
        finally:
            ck.close()
        out = {"shape": a.shape, "experts": E, "layers": a.layers, "threads": a.threads,
               "fp8": fp8, "store_GB": store_bytes / 1e9, "write_s": write_s,
               "pinned_alloc_s": alloc_s, "pinned_alloc_GBs": store_bytes / alloc_s / 1e9,
               "per_layer": per_layer,
               "load_GBs": sum(x["bytes"] for x in per_layer) / sum(x["s"] for x in per_layer)
               / 1e9,
               "source": "/dev/shm" if d.startswith("/dev/shm") else d}
        del stores, views
        return out
    finally:
        if own:
            shutil.rmtree(d, ignore_errors=True)


if __name__ == "__main__":
    print(json.dumps(_bench()), flush=True)
