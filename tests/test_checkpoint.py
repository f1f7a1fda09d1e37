"""Block-FP8 safetensors checkpoints into `BlockFP8Weight` (CPU, plus one GPU
layer run). The checkpoints are written here with ``safetensors`` in the
DeepSeek layout: e4m3 ``weight`` with fp32 ``weight_scale_inv`` per 128x128
block, ``config.json`` with the fp8 ``quantization_config``, and sharded with
an index. The encoding refusals follow the reference importer
(sequential_moe/precision/checkpoint.py:42-64, :151-223)."""

import json
import math

import pytest
import torch
from safetensors.torch import save_file

from mlops_amd import BlockFP8Weight
from mlops_amd.checkpoint import BlockFP8Checkpoint, load_block_fp8_experts
from oracle import moe_oracle as O

E, H, I = 3, 256, 128
PREFIX = "model.layers.1.mlp.experts.{expert}.{proj}"
FP8_CONFIG = {"quant_method": "fp8", "fmt": "e4m3", "weight_block_size": [128, 128],
              "activation_scheme": "dynamic"}


def _projections(seed=0):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for e in range(E):
        for proj, shape in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            w = (torch.randn(1, *shape, generator=g) * 0.02).to(torch.bfloat16)
            q, s = O.quantize_blocks(w)
            out[PREFIX.format(expert=e, proj=proj)] = (q[0], s[0])
    return out


def _write(directory, projections, *, config=FP8_CONFIG, shards=2):
    (directory / "config.json").write_text(json.dumps({"quantization_config": config}))
    tensors = {}
    for prefix, (q, s) in projections.items():
        tensors[prefix + ".weight"] = q
        tensors[prefix + ".weight_scale_inv"] = s
    names = sorted(tensors)
    if shards == 1:
        (directory / "model.safetensors.index.json").unlink(missing_ok=True)
        save_file(tensors, str(directory / "model.safetensors"))
        return
    weight_map = {}
    per = math.ceil(len(names) / shards)
    for k in range(shards):
        part = names[k * per:(k + 1) * per]
        file = f"model-{k + 1:05d}-of-{shards:05d}.safetensors"
        save_file({n: tensors[n] for n in part}, str(directory / file))
        weight_map.update({n: file for n in part})
    (directory / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))


def _load(directory, **kw):
    return load_block_fp8_experts(
        directory, experts=E, gate=PREFIX.replace("{proj}", "gate_proj"),
        up=PREFIX.replace("{proj}", "up_proj"), down=PREFIX.replace("{proj}", "down_proj"),
        hidden=H, inter=I, **kw)


@pytest.mark.parametrize("shards", [1, 2])
def test_loads_components_bit_for_bit(tmp_path, shards):
    projections = _projections()
    _write(tmp_path, projections, shards=shards)
    w13, w2 = _load(tmp_path)
    assert isinstance(w13, BlockFP8Weight) and w13.shape == (E, 2 * I, H)
    assert w2.shape == (E, H, I) and w13.dtype == torch.bfloat16
    data, scale = w13.components()
    assert scale.shape == (E, 2 * I // 128, H // 128)
    for e in range(E):
        g, gs = projections[PREFIX.format(expert=e, proj="gate_proj")]
        u, us = projections[PREFIX.format(expert=e, proj="up_proj")]
        d, ds = projections[PREFIX.format(expert=e, proj="down_proj")]
        # gate rows, then up rows (w13's order)
        assert torch.equal(data[e, :I].view(torch.uint8), g.view(torch.uint8))
        assert torch.equal(data[e, I:].view(torch.uint8), u.view(torch.uint8))
        assert torch.equal(scale[e], torch.cat((gs, us)))
        assert torch.equal(w2.components()[0][e].view(torch.uint8), d.view(torch.uint8))
        assert torch.equal(w2.components()[1][e], ds)
    # The containers represent the checkpoint's values.
    logical = w13.dequantize(dtype=torch.float32)
    g, gs = projections[PREFIX.format(expert=1, proj="gate_proj")]
    assert torch.equal(logical[1, :I], O.dequantize_blocks(g[None], gs[None])[0])


def test_a_subset_of_experts(tmp_path):
    projections = _projections(seed=1)
    _write(tmp_path, projections)
    w13, w2 = load_block_fp8_experts(
        tmp_path, experts=[2, 0], gate=PREFIX.replace("{proj}", "gate_proj"),
        up=PREFIX.replace("{proj}", "up_proj"), down=PREFIX.replace("{proj}", "down_proj"),
        hidden=H, inter=I)
    g, _ = projections[PREFIX.format(expert=2, proj="gate_proj")]
    assert w13.shape[0] == 2
    assert torch.equal(w13.components()[0][0, :I].view(torch.uint8), g.view(torch.uint8))


@pytest.mark.parametrize("config,reason", [
    ({**FP8_CONFIG, "weight_block_size": [1, 128]}, "weight_block_size"),
    ({**FP8_CONFIG, "fmt": "e5m2"}, "E4M3"),
    ({"quant_method": "awq"}, "quant_method"),
    (None, "quantization_config"),
])
def test_refuses_other_encodings(tmp_path, config, reason):
    _write(tmp_path, _projections(), config=config if config is not None else {})
    if config is None:
        (tmp_path / "config.json").write_text(json.dumps({}))
    with pytest.raises(ValueError, match=reason):
        BlockFP8Checkpoint(tmp_path)


def test_refuses_bad_tensors(tmp_path):
    projections = _projections()
    prefix = PREFIX.format(expert=1, proj="down_proj")
    q, s = projections[prefix]
    projections[prefix] = (q, -s)
    _write(tmp_path, projections)
    with pytest.raises(ValueError, match="nonnegative"):
        _load(tmp_path)
    projections[prefix] = (q[:, :64].contiguous(), s)
    _write(tmp_path, projections, shards=1)
    with pytest.raises(ValueError, match="down_proj.weight"):
        _load(tmp_path)
    projections[prefix] = (q, s)
    _write(tmp_path, projections, shards=1)
    with pytest.raises(KeyError, match="no tensor"):
        load_block_fp8_experts(tmp_path, experts=E + 1, gate=PREFIX.replace("{proj}", "gate_proj"),
                               up=PREFIX.replace("{proj}", "up_proj"),
                               down=PREFIX.replace("{proj}", "down_proj"), hidden=H, inter=I)


@pytest.mark.gpu
def test_loaded_experts_run_the_layer(tmp_path, device):
    """The loaded containers, moved to the GPU, drive mlops_amd.moe; the
    output matches the fp8 oracle on the same components."""
    import mlops_amd
    from mlops_amd import router
    from tests.conftest import frob_rel

    _write(tmp_path, _projections(seed=2))
    w13, w2 = _load(tmp_path, device=device)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, H, generator=g).to(torch.bfloat16).to(device)
    res = torch.zeros_like(x)
    wr = (torch.randn(E, H, generator=g) / math.sqrt(H)).to(device)
    out, _, counts, _ = mlops_amd.moe(x, res, wr, w13, w2, top_k=2, routing_mode="softmax_then_topk")
    (q13, s13), (q2, s2) = w13.components(), w2.components()
    fwd = O.fp8_moe_forward(x.cpu(), res.cpu(), wr.cpu(), q13.cpu(), s13.cpu(), q2.cpu(), s2.cpu(),
                            top_k=2, routing_mode="softmax_then_topk",
                            logits=router.router_logits(x, wr).cpu())
    assert torch.equal(counts.cpu(), fwd["counts"])
    assert frob_rel(out.cpu().float(), fwd["out"].float()) < 1e-2


@pytest.mark.gpu
def test_copy_publication_from_masters(device):
    """``container.copy_(master)`` re-quantizes the master into the container's
    storage, exactly as ``quantize`` does; a container source copies its
    components (reference block_fp8.py:117-129)."""
    g = torch.Generator().manual_seed(5)
    master = (torch.randn(2, 256, 384, generator=g) * 0.02).to(device)
    target = BlockFP8Weight.quantize(torch.zeros_like(master)).detach()
    storage = [t.data_ptr() for t in target.components()]
    target.copy_(master)
    fresh = BlockFP8Weight.quantize(master)
    for a, b in zip(target.components(), fresh.components()):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    assert [t.data_ptr() for t in target.components()] == storage
    other = BlockFP8Weight.quantize(master * 3)
    target.copy_(other)
    for a, b in zip(target.components(), other.components()):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
