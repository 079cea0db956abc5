"""Binding packed expert shards to a model — the expert part of
load_w4 in kernels/load_w4_checkpoint.py:56-83.

The encoder and decoder layer N of DiffusionGemma hold the same expert
weights, so a checkpoint ships one shard per layer (experts_*.safetensors,
keys "<prefix>.<buffer>" for the six EXPERT_BUFS). bind_expert_shards loads
each layer's shard once and registers the same six tensors on every experts
module of that layer (modules named "...layers.<N>.experts"), binds the
fused forward, then runs the load-time repack once per shared tensor (the
tiled down layout, optionally the one-launch FFN pack) so the modules keep
sharing. Shards are read with safetensors only (no pickle). As the
reference's load_w4 does (kernels/load_w4_checkpoint.py:38-41, :100), a
directory without w4_meta.json is refused: it is not a dg-w4a16 checkpoint.
"""
from __future__ import annotations

import json
import pathlib
import re

import torch

from .fused_moe_w4_v2 import enable_pack, enable_tiled_down
from .pack_experts import EXPERT_BUFS, fused_experts_forward

_LAYER_RE = re.compile(r"\.layers\.(\d+)\.experts$")


def experts_by_layer(model) -> dict:
    """{layer index: [(name, module), ...]} of the experts modules of model."""
    out: dict = {}
    for name, mod in model.named_modules():
        m = _LAYER_RE.search(name)
        if m:
            out.setdefault(int(m.group(1)), []).append((name, mod))
    return out


def expert_shards(ckpt) -> dict:
    """{layer index: (shard path, key prefix)} of the experts_*.safetensors
    files in ckpt; the first file naming a layer wins."""
    from safetensors import safe_open
    found: dict = {}
    for f in sorted(pathlib.Path(ckpt).glob("experts_*.safetensors")):
        with safe_open(str(f), framework="pt") as h:
            key = next(iter(h.keys()))
        m = re.search(r"\.layers\.(\d+)\.experts\.", key)
        if not m:
            raise ValueError(f"{f.name}: key {key!r} names no experts layer")
        found.setdefault(int(m.group(1)), (f, key.rsplit(".", 1)[0]))
    return found


def checkpoint_meta(ckpt) -> dict:
    """w4_meta.json of a dg-w4a16 checkpoint directory (its "format" names the
    pack format); AssertionError with the reference's message if absent."""
    ckpt = pathlib.Path(ckpt).resolve()
    assert (ckpt / "w4_meta.json").exists(), (
        f"{ckpt} is not a dg-w4a16 checkpoint (no w4_meta.json). Point this at the directory "
        f"holding model.safetensors + experts_*.safetensors, not at the bf16 base model."
    )
    meta = json.loads((ckpt / "w4_meta.json").read_text())
    if not isinstance(meta, dict):
        raise ValueError(f"{ckpt / 'w4_meta.json'}: expected a JSON object")
    return meta


@torch.no_grad()
def bind_expert_shards(model, ckpt, device="cuda", tile_down: bool = True, pack: bool = False) -> int:
    """Register each layer's six packed buffers on all of its experts modules
    (one tensor per buffer per layer), bind the fused forward, and repack at
    load time (tile_down: the tiled down layout; pack: also the one-launch
    expert FFN pack). Returns the number of modules bound."""
    from safetensors.torch import load_file
    checkpoint_meta(ckpt)  # a dg-w4a16 checkpoint, else AssertionError
    by_layer = experts_by_layer(model)
    shards = expert_shards(ckpt)
    missing = sorted(set(by_layer) - set(shards))
    if missing:
        raise ValueError(f"no expert shard for layer(s) {missing}")
    tiled: dict = {}
    packs: dict = {}
    n = 0
    for i, (path, prefix) in sorted(shards.items()):
        if i not in by_layer:
            continue
        d = load_file(str(path), device=str(device))  # once per layer
        for _, mod in by_layer[i]:
            for attr in ("gate_up_proj", "down_proj"):
                if hasattr(mod, attr):
                    setattr(mod, attr, None)
            for b in EXPERT_BUFS:
                mod.register_buffer(b, d[f"{prefix}.{b}"], persistent=False)
            mod.forward = fused_experts_forward.__get__(mod, mod.__class__)
            if tile_down:
                enable_tiled_down(mod, tiled)
            if pack:
                enable_pack(mod, packs)
            n += 1
    return n
