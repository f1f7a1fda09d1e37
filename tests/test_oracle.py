"""Pins the CPU oracle (``oracle/moe_oracle.py``) with checks independent of
its own formulas: a bit-level e4m3 encoder written from the format
definition, brute-force selection and sorting in plain Python, closed forms,
torch autograd of the closed-form losses, and a dense-vs-sparse evaluation of
the layer. The reference ships no golden vectors (its tests recompute every
reference from seeded inputs); the hand-made cases under ``tests/golden``
follow the reference tests' edge cases."""

import json
import math
import os
import struct

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests.conftest import frob_rel

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------- e4m3 rounding
def e4m3_encode(x: float) -> int:
    """OCP e4m3fn encode with round-to-nearest-even, from the format definition
    (bias 7, 3 mantissa bits, subnormals below 2^-6, max 448, no inf)."""
    if x != x:
        return 0x7F
    sign = 0x80 if (x < 0 or (x == 0 and math.copysign(1.0, x) < 0)) else 0
    a = abs(x)
    best, best_err, best_code = None, None, 0
    # enumerate all finite magnitudes (exact, small table)
    for code in range(0x7F):  # 0x7F is NaN
        e, m = code >> 3, code & 7
        v = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        err = abs(v - a)
        if best is None or err < best_err or (err == best_err and (code & 1) == 0 and (best_code & 1)):
            best, best_err, best_code = v, err, code
    return sign | best_code


def test_torch_e4m3_cast_matches_format_definition():
    rng = np.random.default_rng(0)
    values = list(rng.uniform(-448, 448, 2000)) + list(rng.uniform(-1, 1, 2000) * 2.0 ** -5)
    # exact ties between neighbouring codes
    for code in range(0x7E):
        e, m = code >> 3, code & 7
        v = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        e2, m2 = (code + 1) >> 3, (code + 1) & 7
        v2 = (m2 / 8.0) * 2.0 ** -6 if e2 == 0 else (1 + m2 / 8.0) * 2.0 ** (e2 - 7)
        values.append((v + v2) / 2)
    values = [float(np.float32(v)) for v in values]
    got = torch.tensor(values, dtype=torch.float32).to(O.FP8).view(torch.uint8).tolist()
    want = [e4m3_encode(v) for v in values]
    assert got == want


# ------------------------------------------------------------- quantizers
def _step(value_abs):
    """Spacing of e4m3 values around |value| (in the quantized domain)."""
    e = max(math.floor(math.log2(max(value_abs, 2.0 ** -9))), -6)
    return 2.0 ** (e - 3)


def test_quantize_blocks_closed_form():
    torch.manual_seed(0)
    w = torch.randn(2, 200, 300) * 0.02
    w[1, :128, :128] = 0.0  # a zero block (test_sonicmoe_block_fp8.py:67-75)
    data, scale = O.quantize_blocks(w)
    assert scale.shape == (2, 2, 3) and data.shape == w.shape
    assert torch.all(data[1, :128, :128].float() == 0)
    assert scale[1, 0, 0] == np.float32(1e-12)
    # scale = amax / 448 with an IEEE fp32 division
    blk = w[0, :128, 128:256].abs().max().numpy().astype(np.float32)
    assert scale[0, 0, 1].item() == float(np.float32(blk) / np.float32(448.0))
    # the amax element maps to +-448 exactly; every element within half a step
    q = data.float()
    for e in range(2):
        for bo in range(2):
            for bi in range(3):
                blockw = w[e, bo * 128:(bo + 1) * 128, bi * 128:(bi + 1) * 128]
                blockq = q[e, bo * 128:(bo + 1) * 128, bi * 128:(bi + 1) * 128]
                s = scale[e, bo, bi].item()
                if blockw.abs().max() == 0:
                    continue
                assert blockq.abs().max().item() == 448.0
                ratio = (blockw / s).double()
                for val, got in zip(ratio.flatten()[:500].tolist(), blockq.flatten()[:500].tolist()):
                    assert abs(val - got) <= _step(abs(val)) / 2 + 1e-9
    # round trip relative error (test_sonicmoe_block_fp8.py:31-55)
    rt = O.dequantize_blocks(data, scale)
    assert frob_rel(rt, w) < 4e-2


def test_quantize_rows_1x128_closed_form():
    torch.manual_seed(1)
    x = (torch.randn(7, 384) * 3).to(torch.bfloat16)
    x[3] = 0
    q, s = O.quantize_rows_1x128(x)
    assert q.shape == (7, 384) and s.shape == (3, 7)
    xf = x.float().numpy()
    for r in range(7):
        for g in range(3):
            amax = np.float32(np.abs(xf[r, g * 128:(g + 1) * 128]).max())
            want = max(np.float32(amax * (np.float32(1.0) / np.float32(448.0))), np.float32(1e-12))
            assert s[g, r].item() == float(want)
    assert torch.all(q[3].float() == 0)
    deq = O.dequantize_rows(q, s)
    assert frob_rel(deq, x.float()) < 4e-2


def test_gate_up_columns_and_transpose_layout():
    cols = O.gate_up_columns(8).tolist()
    assert cols == [0, 2, 4, 6, 1, 3, 5, 7]
    torch.manual_seed(2)
    rows = torch.randn(300, 128).to(torch.bfloat16)
    offsets = torch.tensor([0, 100, 100, 300], dtype=torch.int32)  # an empty expert
    starts, total = O.padded_layout(offsets)
    assert starts == [0, 128, 128] and total == 128 + 256
    qt, st, _ = O.quantize_transpose_padded(rows, offsets, 512)
    assert qt.shape == (128, 512) and st.shape == (4, 128)
    # expert 2's rows start at padded column 128; padding is zero
    assert torch.all(qt[:, 100:128].float() == 0)
    # Scales by frexp on Python floats (independent of the oracle's exponent
    # bit arithmetic): the smallest power of two >= fp32(amax * fp32(1/448)).
    x = rows.float()
    block_rows = {0: x[0:100], 1: x[100:228], 2: x[228:300]}
    for b, src in block_rows.items():
        amax = src.abs().amax(0)
        for f in range(0, 128, 7):
            prod = float(np.float32(np.float32(amax[f].item()) * np.float32(1.0 / 448.0)))
            prod = max(prod, float(np.float32(1e-12)))
            m, e = math.frexp(prod)
            want = prod if m == 0.5 else math.ldexp(1.0, e)
            assert st[b, f].item() == want
            # amax lands in (224, 448] (saturating at 448)
            assert 224.0 < amax[f].item() / want <= 448.0 * (1 + 2 ** -20)
            got = qt[f, 128 * b:128 * b + src.shape[0]].float() * want
            step = (src[:, f].abs() * 2 ** -3).clamp_min(want * 2 ** -9)
            assert torch.all((got - src[:, f]).abs() <= step / 2 * (1 + 1e-6))
    assert torch.all(st[3] == 2.0 ** -39)  # all-zero block: pow2 ceiling of 1e-12


# ---------------------------------------------------------------- routing
def _brute_topk(values, k):
    order = sorted(range(len(values)), key=lambda e: (-values[e], e))
    return order[:k]


@pytest.mark.parametrize("mode", ["topk_then_softmax", "softmax_then_topk", "sigmoid_noaux_tc"])
def test_route_matches_brute_force(mode):
    torch.manual_seed(3)
    logits = torch.randn(40, 12)
    logits[5] = 0.0  # all ties: lowest ids win
    logits[6, 3] = logits[6, 7] = 5.0  # tie at the top
    w, ids = O.route(logits, 3, mode)
    for t in range(40):
        lv = logits[t].tolist()
        if mode == "sigmoid_noaux_tc":
            sel = [1 / (1 + math.exp(-v)) for v in lv]
        else:
            sel = lv  # softmax is monotonic; ties stay ties
        want = _brute_topk(sel, 3)
        assert ids[t].tolist() == want, (t, ids[t].tolist(), want)
    assert ids[5].tolist() == [0, 1, 2]
    assert ids[6].tolist()[:2] == [3, 7]
    if mode == "sigmoid_noaux_tc":
        assert torch.allclose(w.sum(-1), torch.ones(40))
    elif mode == "topk_then_softmax":
        assert torch.allclose(w.sum(-1), torch.ones(40))
    else:
        p = torch.softmax(logits, -1)
        assert torch.allclose(w, p.gather(1, ids.long()))


def test_route_group_limited_brute_force():
    torch.manual_seed(4)
    logits = torch.randn(25, 16)
    bias = torch.randn(16) * 0.1
    w, ids = O.route(logits, 4, "sigmoid_noaux_tc", bias=bias, n_group=4, topk_group=2,
                     routed_scaling=2.5)
    for t in range(25):
        s = [1 / (1 + math.exp(-v)) for v in logits[t].tolist()]
        sel = [a + b for a, b in zip(s, bias.tolist())]
        groups = []
        for g in range(4):
            top2 = sorted(sel[g * 4:(g + 1) * 4], reverse=True)[:2]
            groups.append(top2[0] + top2[1])
        keep = _brute_topk(groups, 2)
        masked = [sel[e] if e // 4 in keep else -math.inf for e in range(16)]
        assert ids[t].tolist() == _brute_topk(masked, 4)
        picked = [s[e] for e in ids[t].tolist()]
        want = [p / sum(picked) * 2.5 for p in picked]
        assert np.allclose(w[t].tolist(), want, rtol=1e-6)


def test_sort_assignments_brute_force():
    rng = np.random.default_rng(5)
    ids = torch.from_numpy(rng.integers(0, 6, size=(50, 3)).astype(np.int32))
    ids[:, 0] = 2  # heavy expert; expert 5 may be empty
    order, offsets, slots = O.sort_assignments(ids, 7)
    flat = ids.reshape(-1).tolist()
    want = sorted(range(len(flat)), key=lambda i: (flat[i], i))
    assert order.tolist() == want
    counts = [flat.count(e) for e in range(7)]
    assert offsets.tolist() == [0] + list(np.cumsum(counts))
    assert offsets[-1] == len(flat) and offsets[7] == offsets[6]  # expert 6 empty
    for i, o in enumerate(order.tolist()):
        assert slots.reshape(-1)[o] == i


def test_routing_statistics_closed_forms():
    tokens, experts, k = 32, 8, 2
    logits = torch.zeros(tokens, experts)  # uniform probabilities
    ids = torch.tensor([[e % experts, (e + 1) % experts] for e in range(tokens)], dtype=torch.int32)
    aux, counts, psum = O.routing_statistics(logits, ids, "topk_then_softmax", (tokens,), experts)
    assert torch.allclose(psum, torch.full((experts,), tokens / experts))
    assert counts.tolist() == [8] * 8
    assert abs(aux.item() - 1.0) < 1e-6  # E * sum_e f_e / E = 1
    # one-hot probabilities concentrate on expert 0
    logits = torch.full((tokens, experts), -1e4)
    logits[:, 0] = 0
    ids = torch.zeros(tokens, 1, dtype=torch.int32)
    aux, _, psum = O.routing_statistics(logits, ids, "softmax_then_topk", (tokens,), experts)
    assert abs(aux.item() - experts) < 1e-4 and abs(psum[0].item() - tokens) < 1e-3


@pytest.mark.parametrize("mode", ["topk_then_softmax", "softmax_then_topk", "sigmoid_noaux_tc"])
def test_routing_gradient_matches_autograd(mode):
    torch.manual_seed(6)
    tokens, experts, k = 24, 10, 3
    lengths = (10, 14)
    logits = torch.randn(tokens, experts, dtype=torch.float64)
    w, ids = O.route(logits.float(), k, mode, routed_scaling=1.7 if mode == "sigmoid_noaux_tc" else 1.0)
    gw = torch.randn(tokens, k, dtype=torch.float64)
    ga = torch.tensor(0.37, dtype=torch.float64)
    gps = torch.randn(experts, dtype=torch.float64)
    lv = logits.clone().requires_grad_(True)
    live = O._live_weights(lv, ids, mode, 1.7 if mode == "sigmoid_noaux_tc" else 1.0)
    p = O.probabilities(lv, mode) if mode != "sigmoid_noaux_tc" else (
        torch.sigmoid(lv) / torch.sigmoid(lv).sum(-1, keepdim=True))
    counts_all = torch.bincount(ids.reshape(-1).long(), minlength=experts).double()
    if mode == "sigmoid_noaux_tc":
        aux = 0
        start = 0
        for length in lengths:
            seg = torch.bincount(ids[start:start + length].reshape(-1).long(), minlength=experts).double()
            f = seg * experts / (k * length)
            aux = aux + (f * p[start:start + length].mean(0)).sum()
            start += length
    else:
        f = counts_all / ids.numel()
        aux = experts * (f * p.mean(0)).sum()
    loss = (live * gw).sum() + ga * aux + (p.sum(0) * gps).sum()
    (expected,) = torch.autograd.grad(loss, lv)
    got = O.routing_gradient(ga.float(), gps.float(), gw.float(), live.detach().float(), ids,
                             logits.float(), mode, lengths)
    assert torch.allclose(got.double(), expected, atol=2e-6, rtol=1e-4)


# ---------------------------------------------------------------- SwiGLU
@pytest.mark.parametrize("limit", [None, 0.8])
def test_routed_swiglu_backward_matches_autograd(limit):
    torch.manual_seed(7)
    rows, width = 9, 16
    h = (torch.randn(rows, 2 * width, dtype=torch.float64) * 1.5).requires_grad_(True)
    score = torch.rand(rows, dtype=torch.float64).requires_grad_(True)
    r = torch.randn(rows, width, dtype=torch.float64)
    g, u = h[:, 0::2], h[:, 1::2]
    if limit is not None:
        g, u = g.clamp(max=limit), u.clamp(-limit, limit)
    act = torch.nn.functional.silu(g) * u
    loss = (r * act * score[:, None]).sum()
    dh_ref, ds_ref = torch.autograd.grad(loss, (h, score))
    ds, dh, ap = O.routed_swiglu_backward(r, h.detach(), score.detach(), limit)
    assert torch.allclose(ds.double(), ds_ref, atol=1e-5)
    assert torch.allclose(dh.double(), dh_ref, atol=1e-5)
    assert torch.allclose(ap.double(), (act * score[:, None]).detach(), atol=1e-5)
    assert torch.allclose(O.swiglu(h.detach(), limit).double(), act.detach(), atol=1e-5)


# ----------------------------------------------------------------- GEMMs
def test_grouped_gemm_matches_loop():
    torch.manual_seed(8)
    w = torch.randn(3, 256, 128) * 0.02
    wq, ws = O.quantize_blocks(w)
    offsets = torch.tensor([0, 5, 5, 12], dtype=torch.int32)
    x = torch.randn(12, 128).to(torch.bfloat16)
    xq, xs = O.quantize_rows_1x128(x)
    out = O.grouped_gemm(xq, xs, wq, ws, offsets)
    a = O.dequantize_rows(xq, xs).double()
    wd = O.dequantize_blocks(wq, ws).double()
    for row in range(12):
        e = 0 if row < 5 else 2
        for n in (0, 77, 255):
            want = sum(a[row, kk].item() * wd[e, n, kk].item() for kk in range(128))
            assert abs(out[row, n].item() - want) < 1e-9
    inter = O.grouped_gemm(xq, xs, wq, ws, offsets, interleave=True)
    assert torch.equal(inter[:, 0::2], out[:, :128]) and torch.equal(inter[:, 1::2], out[:, 128:])
    y = torch.randn(12, 256).to(torch.bfloat16)
    yq, ys = O.quantize_rows_1x128(y)
    dg = O.grouped_gemm(yq, ys, wq, ws, offsets, transposed=True)
    yd = O.dequantize_rows(yq, ys).double()
    assert torch.allclose(dg[5:], yd[5:] @ wd[2], atol=1e-9)


# ------------------------------------------------------------- full layer
def _layer_inputs(tokens=64, hidden=256, experts=4, inter=128, seed=9):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    res = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    wr = torch.randn(experts, hidden, generator=g) / math.sqrt(hidden)
    w13 = (torch.randn(experts, 2 * inter, hidden, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(experts, hidden, inter, generator=g) * 0.02).to(torch.bfloat16)
    return x, res, wr, w13, w2


def test_native_moe_dense_equals_sparse():
    x, res, wr, w13, w2 = _layer_inputs()
    out, aux, counts, psum = O.native_moe(x, res, wr, w13, w2, top_k=2,
                                          routing_mode="topk_then_softmax",
                                          compute_dtype=torch.float64)
    logits = O.router_logits(x, wr)
    w, ids = O.route(logits, 2, "topk_then_softmax")
    want = res.double().clone()
    for t in range(x.shape[0]):
        for j in range(2):
            e = int(ids[t, j])
            h = x[t].double() @ w13[e].double().t()
            a = torch.nn.functional.silu(h[:128]) * h[128:]
            want[t] += w[t, j].double() * (a @ w2[e].double().t())
    assert frob_rel(out.float(), want.to(torch.bfloat16).float()) < 1e-2
    assert counts.sum().item() == 128


def test_fp8_layer_close_to_native_on_dequantized_weights():
    x, res, wr, w13, w2 = _layer_inputs(seed=10)
    res = torch.zeros_like(res)  # compare the routed part without bf16 residual rounding
    w13q, w13s = O.quantize_blocks(w13)
    w2q, w2s = O.quantize_blocks(w2)
    w13d, w2d = O.dequantize_blocks(w13q, w13s), O.dequantize_blocks(w2q, w2s)
    fwd = O.fp8_moe_forward(x, res, wr, w13q, w13s, w2q, w2s, top_k=2,
                            routing_mode="topk_then_softmax")
    xr = x.clone().float().requires_grad_(True)
    w13r = w13d.clone().requires_grad_(True)
    w2r = w2d.clone().requires_grad_(True)
    wrr = wr.clone().requires_grad_(True)
    out, aux, counts, psum = O.native_moe(xr, res.float(), wrr, w13r, w2r, top_k=2,
                                          routing_mode="topk_then_softmax")
    # Forward: activation quantization error only (reference BOUNDS, test_sonicmoe_block_fp8.py:350)
    routed_fp8 = fwd["out"].float() - res.float()
    routed_ref = out.float() - res.float()
    # two e4m3 activation quantizations (x, act) at ~3% RMS each
    assert frob_rel(routed_fp8, routed_ref.detach()) < 6e-2
    x2, res2, *_ = _layer_inputs(seed=10)
    full = O.fp8_moe_forward(x2, res2, wr, w13q, w13s, w2q, w2s, top_k=2,
                             routing_mode="topk_then_softmax")["out"]
    full_ref = O.native_moe(x2.float(), res2.float(), wr, w13d, w2d, top_k=2,
                            routing_mode="topk_then_softmax")[0]
    assert frob_rel(full.float(), full_ref.detach().float()) < 4e-2
    assert torch.equal(fwd["counts"], counts)
    gy = torch.randn_like(out)
    out.backward(gy)
    bwd = O.fp8_moe_backward(fwd, x, gy.to(torch.bfloat16), wr, w13q, w13s, w2q, w2s, top_k=2,
                             routing_mode="topk_then_softmax")
    assert frob_rel(bwd["dw2"], w2r.grad) < 8e-2
    assert frob_rel(bwd["dw13"], w13r.grad) < 8e-2
    assert frob_rel(bwd["grad_x"].float(), xr.grad) < 6e-2
    assert frob_rel(bwd["grad_router"], wrr.grad) < 8e-2


def test_golden_cases():
    """Hand-made edge cases (ties, empty experts, zero blocks), independent of
    the oracle: expected values were written by hand / brute force."""
    with open(os.path.join(GOLDEN, "routing_cases.json")) as f:
        cases = json.load(f)
    for case in cases["route"]:
        logits = torch.tensor(case["logits"], dtype=torch.float32)
        w, ids = O.route(logits, case["top_k"], case["mode"])
        assert ids.tolist() == case["ids"], case["name"]
    for case in cases["sort"]:
        ids = torch.tensor(case["ids"], dtype=torch.int32)
        order, offsets, slots = O.sort_assignments(ids, case["experts"])
        assert order.tolist() == case["order"], case["name"]
        assert offsets.tolist() == case["offsets"], case["name"]
        assert slots.reshape(-1).tolist() == case["slots"], case["name"]


# --------------------------------------------------------------------------
# Expert LoRA terms of the oracle (lora/experts.py:46-50, :160-163), pinned by
# the LoRA identity W -> W + scale * B @ A, not by restating the formula.
def _lora_case(seed=3, experts=4, width=24, inter=16, rank=5, tokens=20, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape, s=1.0):
        return (torch.randn(*shape, generator=g, dtype=torch.float64) * s).to(dtype)

    x, res = rnd(tokens, width), rnd(tokens, width)
    wr = rnd(experts, width, s=width ** -0.5)
    w13, w2 = rnd(experts, 2 * inter, width, s=width ** -0.5), rnd(experts, width, inter, s=inter ** -0.5)
    a13, b13 = rnd(experts, rank, width, s=width ** -0.5), rnd(experts, 2 * inter, rank, s=rank ** -0.5)
    a2, b2 = rnd(experts, rank, inter, s=inter ** -0.5), rnd(experts, width, rank, s=rank ** -0.5)
    return x, res, wr, w13, w2, a13, b13, a2, b2


def test_oracle_lora_equals_the_merged_weights_forward_and_gradients():
    """Expert LoRA is the layer with W' = W + s B@A: equal outputs, and the
    factor gradients follow from the merged weight's by the chain rule
    (dB = s dW' A^T, dA = s B^T dW'). A dropped scale, a transposed factor or
    a gate/up mix-up in the LoRA terms fails this."""
    x, res, wr, w13, w2, a13, b13, a2, b2 = _lora_case()
    s = 0.7
    opts = dict(top_k=2, routing_mode="softmax_then_topk", compute_dtype=torch.float64,
                swiglu_limit=1.5)
    leaves = [t.clone().requires_grad_(True) for t in (a13, b13, a2, b2)]
    out, aux, _, _ = O.native_moe(x, res, wr, w13, w2, lora=(*leaves, s), **opts)
    m13 = (w13 + s * b13 @ a13).requires_grad_(True)
    m2 = (w2 + s * b2 @ a2).requires_grad_(True)
    ref, ref_aux, _, _ = O.native_moe(x, res, wr, m13, m2, **opts)
    assert torch.allclose(out, ref, rtol=1e-12, atol=1e-12)
    upstream = torch.randn(out.shape, generator=torch.Generator().manual_seed(9), dtype=out.dtype)
    ga13, gb13, ga2, gb2 = torch.autograd.grad((out * upstream).sum() + 0.3 * aux, leaves)
    gm13, gm2 = torch.autograd.grad((ref * upstream).sum() + 0.3 * ref_aux, (m13, m2))
    assert torch.allclose(gb13, s * gm13 @ a13.transpose(1, 2), rtol=1e-10, atol=1e-12)
    assert torch.allclose(ga13, s * b13.transpose(1, 2) @ gm13, rtol=1e-10, atol=1e-12)
    assert torch.allclose(gb2, s * gm2 @ a2.transpose(1, 2), rtol=1e-10, atol=1e-12)
    assert torch.allclose(ga2, s * b2.transpose(1, 2) @ gm2, rtol=1e-10, atol=1e-12)


def test_oracle_lora_with_zero_b_factors_is_the_plain_layer():
    """lora/experts.py resets B to zero (:39-43): the layer is then mlops.moe's
    (the reference's test_zero_factors_are_mlops_moe)."""
    x, res, wr, w13, w2, a13, b13, a2, b2 = _lora_case(dtype=torch.float32)
    opts = dict(top_k=2, routing_mode="sigmoid_noaux_tc", n_group=2, topk_group=1,
                routed_scaling=1.5)
    zero = (a13, torch.zeros_like(b13), a2, torch.zeros_like(b2), 0.5)
    got = O.native_moe(x, res, wr, w13, w2, lora=zero, **opts)
    ref = O.native_moe(x, res, wr, w13, w2, **opts)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


# --------------------------------------------------------------------------
# fp8_current (per-row scaling) functions of the oracle.
def test_quantize_rows_current_closed_form():
    """128-wide rows are the pinned 1x128 quantizer's single group; wider rows
    follow the per-row closed form (numpy fp32); zero rows stay zero; the
    amax element maps to +-448."""
    torch.manual_seed(21)
    x = (torch.randn(9, 128) * 5).to(torch.bfloat16)
    q, s = O.quantize_rows_current(x)
    q1, s1 = O.quantize_rows_1x128(x)
    assert torch.equal(q.view(torch.uint8), q1.view(torch.uint8))
    assert torch.equal(s, s1[0])
    x = (torch.randn(7, 384) * 3).to(torch.bfloat16)
    x[2] = 0
    q, s = O.quantize_rows_current(x)
    assert q.shape == (7, 384) and s.shape == (7,)
    xf = x.float().numpy()
    for r in range(7):
        amax = np.float32(np.abs(xf[r]).max())
        want = max(np.float32(amax * (np.float32(1.0) / np.float32(448.0))), np.float32(1e-12))
        assert s[r].item() == float(want)
        if amax > 0:
            assert q[r].float().abs().max().item() == 448.0
    assert torch.all(q[2].float() == 0)
    assert frob_rel(q.float() * s[:, None], x.float()) < 4e-2


def test_quantize_weights_current_container_bounds():
    """The reference's container checks (tests/test_sonicmoe_fp8.py:261-291):
    per-row relative error < 0.07 of the row maximum in both orientations; the
    interleaved container stores row 2j = gate j, 2j + 1 = up j in both, and
    dequantizes to the same logical weight."""
    torch.manual_seed(22)
    w = torch.randn(3, 8, 32).to(torch.bfloat16)
    data, transposed, scale, tscale = O.quantize_weights_current(w)
    assert data.shape == (3, 8, 32) and transposed.shape == (3, 32, 8)
    assert scale.shape == (3, 8) and tscale.shape == (3, 32)
    row_max = w.float().abs().amax(-1, keepdim=True)
    restored = data.float() * scale[..., None]
    assert float(((restored - w.float()).abs() / row_max).max()) < 0.07
    restored_t = (transposed.float() * tscale[..., None]).transpose(1, 2)
    assert float(((restored_t - w.float()).abs() / row_max).max()) < 0.07
    i_data, i_transposed, i_scale, _ = O.quantize_weights_current(w, interleaved=True)
    expected = torch.stack(data.chunk(2, dim=1), dim=2).reshape(data.shape)
    assert torch.equal(i_data.view(torch.uint8), expected.view(torch.uint8))
    expected_t = torch.stack(transposed.chunk(2, dim=2), dim=3).reshape(transposed.shape)
    assert torch.equal(i_transposed.view(torch.uint8), expected_t.view(torch.uint8))
    logical = (i_data.float() * i_scale[..., None]).view(3, 4, 2, 32).transpose(1, 2)
    assert torch.equal(logical.reshape(3, 8, 32), restored)


def test_rowwise_gemm_matches_loop():
    torch.manual_seed(23)
    w = torch.randn(3, 64, 128) * 0.02
    wq, _, ws, _ = O.quantize_weights_current(w)
    offsets = torch.tensor([0, 5, 5, 12], dtype=torch.int32)
    xq, xs = O.quantize_rows_current(torch.randn(12, 128).to(torch.bfloat16))
    out = O.rowwise_gemm(xq, xs, wq, ws, offsets)
    for row in range(12):
        e = 0 if row < 5 else 2
        for n in (0, 33, 63):
            want = sum(xq[row, kk].double().item() * wq[e, n, kk].double().item()
                       for kk in range(128)) * xs[row].item() * ws[e, n].item()
            assert abs(out[row, n].item() - want) < 1e-9 * max(1.0, abs(want))


def test_current_forward_is_the_layer_when_quantizers_are_identities(monkeypatch):
    """With the e4m3 rounding replaced by the identity, the fp8_current
    forward is the native layer up to its bf16 roundings: a wrong gather,
    gate/up order, scale or orientation fails this."""
    monkeypatch.setattr(O, "_e4m3", lambda values: values)
    x, res, wr, w13, w2 = _layer_inputs(seed=24)
    res = torch.zeros_like(res)  # the routed part alone, without bf16 residual rounding
    w13c = O.quantize_weights_current(w13, interleaved=True)
    w2c = O.quantize_weights_current(w2)
    fwd = O.current_moe_forward(x, res, wr, w13c, w2c, top_k=2, routing_mode="softmax_then_topk",
                                swiglu_limit=0.05)
    out, _, counts, _ = O.native_moe(x.float(), res.float(), wr, w13.float(), w2.float(), top_k=2,
                                     routing_mode="softmax_then_topk", swiglu_limit=0.05)
    assert torch.equal(fwd["counts"], counts)
    assert frob_rel(fwd["out"].float(), out.detach().float()) < 1e-2


def test_fp8_layer_is_the_native_layer_when_quantizers_are_identities(monkeypatch):
    """With the e4m3 rounding replaced by the identity, the block-FP8 forward
    and backward are the native layer up to their bf16 roundings: a wrong
    gather, slot, gate/up order, scale layout, padding or orientation in any
    of the layer's products (forward, both input gradients, both weight
    gradients, router) fails this."""
    monkeypatch.setattr(O, "_e4m3", lambda values: values)
    x, res, wr, w13, w2 = _layer_inputs(tokens=96, seed=31)
    res = torch.zeros_like(res)  # the routed part alone, without bf16 residual rounding
    w13q, w13s = O.quantize_blocks(w13)
    w2q, w2s = O.quantize_blocks(w2)
    for mode, limit in (("topk_then_softmax", None), ("softmax_then_topk", 0.3)):
        fwd = O.fp8_moe_forward(x, res, wr, w13q, w13s, w2q, w2s, top_k=2, routing_mode=mode,
                                swiglu_limit=limit)
        xr = x.float().requires_grad_(True)
        w13r = w13.float().requires_grad_(True)
        w2r = w2.float().requires_grad_(True)
        wrr = wr.clone().requires_grad_(True)
        out, aux, counts, _ = O.native_moe(xr, res.float(), wrr, w13r, w2r, top_k=2,
                                           routing_mode=mode, swiglu_limit=limit)
        assert torch.equal(fwd["counts"], counts)
        assert frob_rel(fwd["out"].float(), out.detach().float()) < 1e-2
        g = torch.Generator().manual_seed(32)
        gy = torch.randn(out.shape, generator=g).to(torch.bfloat16)
        out.backward(gy.float())
        bwd = O.fp8_moe_backward(fwd, x, gy, wr, w13q, w13s, w2q, w2s, top_k=2,
                                 routing_mode=mode, swiglu_limit=limit)
        assert frob_rel(bwd["dw2"], w2r.grad) < 1e-2, mode
        assert frob_rel(bwd["dw13"], w13r.grad) < 1e-2, mode
        assert frob_rel(bwd["grad_x"].float(), xr.grad) < 1e-2, mode
        assert frob_rel(bwd["grad_router"], wrr.grad) < 1e-2, mode


def test_wgrad_is_a_sum_of_row_outer_products(monkeypatch):
    """``O.wgrad`` against a row-by-row outer-product accumulation over each
    expert's own (unpadded) rows. With identity e4m3 rounding the power-of-two
    descales make the dequantized operands equal the inputs exactly, so the
    padded layout, the per-expert starts and the transposition are what is
    checked; the real rounding is then held within one e4m3 step."""
    g = torch.Generator().manual_seed(33)
    counts = [3, 0, 130, 1]
    offsets = torch.tensor([0, *np.cumsum(counts)], dtype=torch.int32)
    rows = int(offsets[-1])
    p = torch.randn(rows, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(rows, 256, generator=g).to(torch.bfloat16)
    _, padded = O.padded_layout(offsets)
    want = np.zeros((len(counts), 128, 256))
    pn, qn = p.double().numpy(), q.double().numpy()
    for e in range(len(counts)):
        for r in range(int(offsets[e]), int(offsets[e + 1])):
            want[e] += np.outer(pn[r], qn[r])
    with monkeypatch.context() as m:
        m.setattr(O, "_e4m3", lambda values: values)
        pt, pts, _ = O.quantize_transpose_padded(p, offsets, padded)
        qt, qts, _ = O.quantize_transpose_padded(q, offsets, padded)
        exact = O.wgrad(pt, pts, qt, qts, offsets).numpy()
    assert np.abs(exact - want).max() < 1e-9 * np.abs(want).max()
    assert np.all(exact[1] == 0)
    pt, pts, _ = O.quantize_transpose_padded(p, offsets, padded)
    qt, qts, _ = O.quantize_transpose_padded(q, offsets, padded)
    rounded = O.wgrad(pt, pts, qt, qts, offsets).numpy()
    assert np.linalg.norm(rounded - want) / np.linalg.norm(want) < 6e-2


def test_combine_and_token_sum_by_loops():
    """``O.combine`` / ``O.unpermute_sum`` against per-token loops in fp64,
    rounded to bf16 once: every output within one bf16 step."""
    g = torch.Generator().manual_seed(34)
    tokens, top_k, width, experts = 40, 3, 256, 5
    ids = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(tokens)]).int()
    _, _, slots = O.sort_assignments(ids, experts)
    y = torch.randn(tokens * top_k, width, generator=g).to(torch.bfloat16)
    w = torch.rand(tokens, top_k, generator=g)
    res = torch.randn(tokens, width, generator=g).to(torch.bfloat16)
    want = torch.zeros(tokens, width, dtype=torch.float64)
    want_sum = torch.zeros(tokens, width, dtype=torch.float64)
    for t in range(tokens):
        acc = res[t].double().clone()
        s = torch.zeros(width, dtype=torch.float64)
        for j in range(top_k):
            row = y[int(slots[t, j])].double()
            acc += float(w[t, j]) * row
            s += row
        want[t], want_sum[t] = acc, s
    for got, exp in ((O.combine(y, slots, w, res), want), (O.unpermute_sum(y, slots), want_sum)):
        step = exp.abs().clamp_min(1e-3) * 2.0 ** -7
        assert torch.all((got.double() - exp).abs() <= step)
