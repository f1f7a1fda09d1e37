"""Block-FP8 expert weights straight from DeepSeek-style safetensors.

The fp8 branch of the reference's checkpoint importer
(``src/mlops/sequential_moe/precision/checkpoint.py:18-267``,
``safetensors.py:1-209``), reading into this package's `BlockFP8Weight`.
A checkpoint directory holds ``config.json`` and either ``model.safetensors``
or shards named by ``model.safetensors.index.json``. The encoding is checked
before any tensor is read. ``quantization_config`` must say ``quant_method:
"fp8"``, ``fmt: "e4m3"`` and ``weight_block_size: [128, 128]``; anything else
is refused with the reason, since bytes are never interpreted from a dtype
name alone.

Each projection ``<prefix>.weight`` is e4m3 ``[out, in]``, with
``<prefix>.weight_scale_inv`` fp32 ``[ceil(out/128), ceil(in/128)]``. That is
the descale, ``value ~ weight * scale_inv`` per block, which is
`BlockFP8Weight`'s own layout. Gate and up projections join row-wise (gate
rows, then up rows: ``w13``'s order), which needs the boundary on a block
edge. Experts stack along a new leading dimension. Tensors are read one
projection at a time from memory-mapped shards; no whole-model state dict is
built.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

from .block_fp8 import BLOCK, BlockFP8Weight

FP8 = torch.float8_e4m3fn


class BlockFP8Checkpoint:
    """Read access to the block-FP8 projections of one checkpoint directory."""

    def __init__(self, directory):
        self.directory = Path(directory)
        config_path = self.directory / "config.json"
        config = json.loads(config_path.read_text()) if config_path.exists() else {}
        quant = (config.get("quantization_config")
                 or config.get("text_config", {}).get("quantization_config") or {})
        method = quant.get("quant_method")
        if method is None:
            raise ValueError(f"{self.directory}: no quantization_config; this importer reads "
                             "block-FP8 checkpoints (load dense weights as plain tensors)")
        if method != "fp8":
            raise ValueError(f"Unsupported checkpoint quant_method={method!r}; only block FP8 "
                             "is imported into BlockFP8Weight")
        if quant.get("fmt", "e4m3") != "e4m3" or quant.get("weight_block_size") != [BLOCK, BLOCK]:
            raise ValueError("FP8 checkpoint importer requires E4M3 weight_block_size=[128,128]")
        index = self.directory / "model.safetensors.index.json"
        if index.exists():
            self.files = dict(json.loads(index.read_text())["weight_map"])
        else:
            from safetensors import safe_open

            single = self.directory / "model.safetensors"
            with safe_open(str(single), framework="pt") as handle:
                self.files = {name: single.name for name in handle.keys()}
        self._handles = {}

    def close(self):
        self._handles.clear()

    def __enter__(self):
        return self

    def __exit__(self, *args):
        self.close()

    def _tensor(self, name: str) -> torch.Tensor:
        if name not in self.files:
            raise KeyError(f"{self.directory}: checkpoint has no tensor {name!r}")
        shard = self.files[name]
        if shard not in self._handles:
            from safetensors import safe_open

            self._handles[shard] = safe_open(str(self.directory / shard), framework="pt")
        return self._handles[shard].get_tensor(name).contiguous()

    def projection(self, prefix: str, shape) -> tuple[torch.Tensor, torch.Tensor]:
        """``(weight e4m3 [out, in], scale_inv fp32 [ceil(out/128), ceil(in/128)])``
        of one ``nn.Linear`` projection, checked against ``shape = (out, in)``."""
        rows, cols = (int(x) for x in shape)
        data = self._tensor(prefix + ".weight")
        if data.dtype != FP8 or tuple(data.shape) != (rows, cols):
            raise ValueError(f"{prefix}.weight: expected float8_e4m3fn {(rows, cols)}, got "
                             f"{data.dtype} {tuple(data.shape)}")
        scale = self._tensor(prefix + ".weight_scale_inv")
        expected = (-(-rows // BLOCK), -(-cols // BLOCK))
        if tuple(scale.shape) != expected or not scale.is_floating_point():
            raise ValueError(f"{prefix}.weight_scale_inv: expected {expected} floating scales, "
                             f"got {scale.dtype} {tuple(scale.shape)}")
        scale = scale.float()
        if not torch.isfinite(scale).all() or (scale < 0).any():
            raise ValueError("Weight scales must be finite and nonnegative")
        return data, scale


def join_gate_up(gate, up):
    """Gate rows then up rows of two projections (reference checkpoint.py:226-244)."""
    (g, gs), (u, us) = gate, up
    if g.shape != u.shape or gs.shape != us.shape:
        raise ValueError("Gate/up need matching shape and scale layout")
    if g.shape[0] % BLOCK:
        raise ValueError("Gate/up boundary must align with weight scale blocks")
    return torch.cat((g, u), 0), torch.cat((gs, us), 0)


def load_block_fp8_experts(checkpoint, *, experts, gate, up, down, hidden, inter,
                           device=None, dtype=torch.bfloat16):
    """``(w13, w2)`` as `BlockFP8Weight` containers of logical ``dtype``:
    ``w13 [E, 2*inter, hidden]`` (gate rows, then up rows) and
    ``w2 [E, hidden, inter]``. ``gate``, ``up`` and ``down`` are tensor-name
    prefixes with an ``{expert}`` field, e.g.
    ``"model.layers.3.mlp.experts.{expert}.gate_proj"``; ``experts`` is the
    count or the list of expert indices to read (reference
    ``load_hf_expert``, checkpoint.py:247-267, over a layer's experts)."""
    indices = list(range(experts)) if isinstance(experts, int) else [int(e) for e in experts]
    if not indices:
        raise ValueError("no experts to load")
    source = checkpoint if isinstance(checkpoint, BlockFP8Checkpoint) else BlockFP8Checkpoint(checkpoint)
    w13_data, w13_scale, w2_data, w2_scale = [], [], [], []
    try:
        for e in indices:
            g = source.projection(gate.format(expert=e), (inter, hidden))
            u = source.projection(up.format(expert=e), (inter, hidden))
            data, scale = join_gate_up(g, u)
            w13_data.append(data)
            w13_scale.append(scale)
            data, scale = source.projection(down.format(expert=e), (hidden, inter))
            w2_data.append(data)
            w2_scale.append(scale)
    finally:
        if source is not checkpoint:
            source.close()
    to = (lambda t: t.to(device)) if device is not None else (lambda t: t)
    w13 = BlockFP8Weight(to(torch.stack(w13_data)), to(torch.stack(w13_scale)), dtype=dtype)
    w2 = BlockFP8Weight(to(torch.stack(w2_data)), to(torch.stack(w2_scale)), dtype=dtype)
    return w13, w2


__all__ = ["BlockFP8Checkpoint", "join_gate_up", "load_block_fp8_experts"]
