"""On-disk packed int4 weights: save a quantized model once, load it without quantizing again.

The reference quantizes every projection from the fp16 checkpoint on each run (lowbit/model.py:30-40, about a minute
per 3B model on its CPU path). This module stores what quantization produced, in the interchange format of
lowbit.quant: for each projection, the canonical packed bytes (uint8 [N, K/2], two nibbles per byte, low nibble
first) and the fp16 group scales ([N, K/G]). The file is a safetensors file:

    "<name>.packed"  uint8   [N, K/2]
    "<name>.scales"  float16 [N, K/G]
    metadata: format = "lowbit-w4", version = "1", group = G, layout = "canonical", and an optional clip_grid
    (JSON list) recording how the scales were chosen

Device layouts are not stored: the GPU builds them from the canonical bytes with its relayout kernel when a W4Weight
is made, which is cheaper than reading a second copy from disk.
"""
import json

import numpy as np
import torch

FORMAT = "lowbit-w4"
VERSION = "1"


def _as_tensor(a, dtype):
    t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))
    if t.dtype != dtype:
        raise ValueError(f"expected {dtype}, got {t.dtype}")
    return t.detach().to("cpu").contiguous()


def save_w4(path, entries, group, clip_grid=None):
    """Write {name: (packed, scales)} (numpy arrays or tensors, canonical layout) to `path`.
    Checks every entry against the format before writing anything."""
    if group % 32:
        raise ValueError(f"group size {group} must be a multiple of 32")
    tensors = {}
    for name, (packed, scales) in entries.items():
        if name.endswith((".packed", ".scales")):
            raise ValueError(f"entry name {name!r} ends in a reserved suffix")
        p, s = _as_tensor(packed, torch.uint8), _as_tensor(scales, torch.float16)
        if p.dim() != 2 or s.dim() != 2:
            raise ValueError(f"{name}: packed and scales must be 2-D")
        n, k = p.shape[0], p.shape[1] * 2
        if k % group:
            raise ValueError(f"{name}: K={k} must be a multiple of the group size {group}")
        if tuple(s.shape) != (n, k // group):
            raise ValueError(f"{name}: scales are {tuple(s.shape)}, expected {(n, k // group)}")
        tensors[f"{name}.packed"], tensors[f"{name}.scales"] = p, s
    meta = {"format": FORMAT, "version": VERSION, "group": str(group), "layout": "canonical"}
    if clip_grid is not None:
        meta["clip_grid"] = json.dumps([float(a) for a in clip_grid])
    from safetensors.torch import save_file
    save_file(tensors, str(path), metadata=meta)


def read_meta(path):
    """The file's metadata, checked: {"group": int, "clip_grid": tuple or None, "names": [entry names]}."""
    from safetensors import safe_open
    with safe_open(str(path), framework="pt") as f:
        meta = f.metadata() or {}
        keys = list(f.keys())
    if meta.get("format") != FORMAT:
        raise ValueError(f"{path} is not a lowbit int4 file (format {meta.get('format')!r})")
    if meta.get("version") != VERSION:
        raise ValueError(f"{path}: unsupported format version {meta.get('version')!r}")
    if meta.get("layout") != "canonical":
        raise ValueError(f"{path}: unsupported layout {meta.get('layout')!r}")
    stray = [k for k in keys if not k.endswith((".packed", ".scales"))]
    if stray:
        raise ValueError(f"{path}: unexpected tensor {stray[0]!r}")
    names = sorted({k.rsplit(".", 1)[0] for k in keys})
    for name in names:
        if f"{name}.packed" not in keys or f"{name}.scales" not in keys:
            raise ValueError(f"{path}: entry {name!r} lacks its packed bytes or its scales")
    grid = meta.get("clip_grid")
    return {"group": int(meta["group"]), "clip_grid": tuple(json.loads(grid)) if grid else None, "names": names}


def load_w4(path, device="cpu", names=None):
    """({name: (packed uint8 [N, K/2], scales fp16 [N, K/G])} as tensors on `device`, group). `names` limits which
    entries are read; asking for one the file lacks raises."""
    meta = read_meta(path)
    group = meta["group"]
    want = meta["names"] if names is None else list(names)
    missing = [n for n in want if n not in meta["names"]]
    if missing:
        raise KeyError(f"{path} has no entry {missing[0]!r}")
    from safetensors import safe_open
    out = {}
    with safe_open(str(path), framework="pt", device=str(device)) as f:
        for name in want:
            p, s = f.get_tensor(f"{name}.packed"), f.get_tensor(f"{name}.scales")
            if p.dtype != torch.uint8 or s.dtype != torch.float16 or p.dim() != 2:
                raise ValueError(f"{path}: entry {name!r} has the wrong dtype or rank")
            if tuple(s.shape) != (p.shape[0], p.shape[1] * 2 // group) or (p.shape[1] * 2) % group:
                raise ValueError(f"{path}: entry {name!r} has scales {tuple(s.shape)} for packed {tuple(p.shape)}")
            out[name] = (p, s)
    return out, group
