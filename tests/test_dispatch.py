"""Registry, resolution and context contracts (CPU).

Mirrors the reference's registry tests (tests/test_implementation_registry.py)
and support-refusal tests (tests/test_sonicmoe_moe.py:226-259): duplicate IDs
raise, the highest priority wins with ties by ID, forced choices must be
supported, the explicit surface needs forward/backward, and the MI355X
provider refuses anything it cannot serve -- with the reason."""

import pytest
import torch
from torch.utils.flop_counter import FlopCounterMode

import mlops_amd
from mlops_amd.dispatch import (
    Implementation,
    SupportResult,
    capture_dispatch,
    dispatch_manifest,
    explain_implementation,
    implementation_registry,
    resolve_implementation,
    use_implementation,
    weight_gradient_dtype,
    weight_gradients_at,
)
from mlops_amd.dispatch import context, registry
from mlops_amd.dispatch.logical_costs import moe_flops
from mlops_amd.providers.mi355x import moe as provider


def _args(tokens=4, hidden=256, experts=8, inter=128, device="cpu", dtype=torch.bfloat16):
    x = torch.zeros(tokens, hidden, dtype=dtype, device=device)
    return (x, x.clone(), torch.zeros(experts, hidden), torch.zeros(experts, 2 * inter, hidden),
            torch.zeros(experts, hidden, inter))


def test_catalog_contains_the_provider():
    table = implementation_registry()["moe"]
    assert sorted(table) == ["mi355x.moe.block_fp8", "mi355x.moe.composed",
                             "mi355x.moe.fp8_current"]
    current = table["mi355x.moe.fp8_current"]
    assert current.deterministic and current.forward and current.backward
    impl = table["mi355x.moe.block_fp8"]
    assert impl.priority > 110 and impl.deterministic and impl.forward and impl.backward
    # The two-region form is semantic-only (no explicit forward/backward, as
    # the reference's composed implementations) and ranks below the fused op.
    composed = table["mi355x.moe.composed"]
    assert composed.deterministic and composed.forward is None and composed.backward is None
    assert 110 < composed.priority < impl.priority


def test_composed_refuses_the_explicit_surface():
    from mlops_amd.providers.mi355x import moe_composed

    result = moe_composed._supports(*_args(), surface="explicit", top_k=2,
                                    routing_mode="topk_then_softmax",
                                    compute_precision="fp8_block")
    assert not result and "semantic-only" in result.reason


def test_duplicate_id_and_pairing_rules():
    with pytest.raises(ValueError, match="duplicate"):
        registry.register_implementation(provider.IMPLEMENTATION)
    with pytest.raises(ValueError, match="together"):
        Implementation("moe", "x", "p", 0, True, lambda *a, **k: True, lambda: None,
                       forward=lambda: None)


def test_priority_selection_and_forcing():
    calls = []

    def yes(*a, **k):
        return SupportResult.yes()

    registry._catalog.tables["toy"] = {}
    try:
        for name, prio in (("b.low", 1), ("a.high", 5), ("c.high", 5)):
            registry.register_implementation(
                Implementation("toy", name, "t", prio, True, yes, lambda *a, **k: calls.append(name)))
        assert resolve_implementation("toy").implementation_id == "a.high"
        with use_implementation("toy", "b.low"):
            assert resolve_implementation("toy").implementation_id == "b.low"
        with pytest.raises(ValueError, match="unknown implementation"):
            with use_implementation("toy", "missing"):
                pass
        explanation = explain_implementation("toy", surface="explicit")
        assert explanation.selected is None
        assert "explicit" in explanation.candidates["a.high"].reason
    finally:
        del registry._catalog.tables["toy"]


def test_resolution_error_lists_reasons():
    with pytest.raises(RuntimeError, match="mi355x.moe.block_fp8: .*GPU"):
        mlops_amd.moe(*_args(), top_k=2, routing_mode="topk_then_softmax",
                      compute_precision="fp8_block")


@pytest.mark.parametrize("kwargs,reason", [
    (dict(compute_precision="bf16"), "not served"),
    (dict(compute_precision="fp8_current"), "not served"),
    (dict(compute_precision=None), "compute in bf16"),
])
def test_support_refusals_precision(kwargs, reason):
    result = provider.supports(*_args(), surface="semantic", top_k=2,
                               routing_mode="topk_then_softmax", **kwargs)
    assert not result and reason in result.reason


def test_support_refusals_with_a_gfx950_device(monkeypatch):
    """Shape rules, checked past the device gate (monkeypatched, as the
    reference's support tests monkeypatch capability)."""
    monkeypatch.setattr(torch.version, "hip", "7.0", raising=False)
    monkeypatch.setattr(provider, "_arch", lambda device: "gfx950:sramecc+:xnack-")

    class FakeCuda(torch.Tensor):
        pass

    def gpu(t):
        t = t.as_subclass(FakeCuda)
        return t

    monkeypatch.setattr(FakeCuda, "is_cuda", property(lambda self: True))
    base = dict(surface="semantic", top_k=2, routing_mode="topk_then_softmax",
                compute_precision="fp8_block")
    ok = provider.supports(*map(gpu, _args()), **base)
    assert ok, ok.reason
    cases = [
        (_args(hidden=200), {}, "multiples of 128"),
        (_args(inter=96), {}, "multiples of 128"),
        (_args(dtype=torch.float32), {}, "bf16"),
        (_args(), dict(top_k=9), "top_k"),
        (_args(), dict(routing_mode="nope"), "routing mode"),
        (_args(), dict(routing_mode="sigmoid_noaux_tc", n_group=3), "n_group"),
        (_args(), dict(lengths=(1, 2)), "lengths"),
    ]
    for args, extra, reason in cases:
        result = provider.supports(*map(gpu, args), **{**base, **extra})
        assert not result and reason in result.reason, (extra, result.reason)


def test_fp8_current_support_rules(monkeypatch):
    """Which operator serves which precision and container (reference
    tests/test_sonicmoe_fp8.py:314-341, 386-423), past the device gate."""
    from mlops_amd import RowFP8Weight
    from mlops_amd.providers.mi355x import moe_current

    monkeypatch.setattr(torch.version, "hip", "7.0", raising=False)
    monkeypatch.setattr(provider, "_arch", lambda device: "gfx950:sramecc+:xnack-")

    class FakeCuda(torch.Tensor):
        pass

    monkeypatch.setattr(FakeCuda, "is_cuda", property(lambda self: True))
    gpu = lambda t: t.as_subclass(FakeCuda)
    base = dict(surface="semantic", top_k=2, routing_mode="topk_then_softmax")

    def container(w, interleaved=False):
        e, out, inner = w.shape
        fp8 = torch.float8_e4m3fn
        return RowFP8Weight(torch.zeros(e, out, inner, dtype=fp8), torch.zeros(e, inner, out, dtype=fp8),
                            torch.ones(e, out), torch.ones(e, inner), dtype=torch.bfloat16,
                            interleaved=interleaved)

    x, res, wr, w13, w2 = map(gpu, _args(hidden=256, inter=256))
    ok = moe_current.supports(x, res, wr, w13, w2, compute_precision="fp8_current", **base)
    assert ok, ok.reason
    # The block operator refuses fp8_current; the current one refuses block weights.
    refused = provider.supports(x, res, wr, w13, w2, compute_precision="fp8_current", **base)
    assert not refused and "block-FP8 only" in refused.reason
    c13, c2 = container(w13, interleaved=True), container(w2)
    assert moe_current.supports(x, res, wr, c13, c2, **base)
    refused = provider.supports(x, res, wr, c13, c2, compute_precision="fp8_block", **base)
    assert not refused and "fp8_current" in refused.reason
    refused = moe_current.supports(x, res, wr, container(w13), c2, **base)
    assert not refused and "interleaved=True" in refused.reason
    narrow = map(gpu, _args(hidden=256, inter=128))
    refused = moe_current.supports(*narrow, compute_precision="fp8_current", **base)
    assert not refused and "multiples of 256" in refused.reason
    refused = moe_current.supports(x, res, wr, w13, w2, compute_precision="fp8_block", **base)
    assert not refused


def test_row_fp8_container_on_cpu():
    """Components, shapes and the interleaved row order in both orientations
    (reference tests/test_sonicmoe_fp8.py:261-303), built from components."""
    from mlops_amd import QuackFP8Weight, RowFP8Weight

    assert QuackFP8Weight is RowFP8Weight
    g = torch.Generator().manual_seed(0)
    e, out, inner = 2, 8, 16
    data = (torch.randn(e, out, inner, generator=g) * 50).to(torch.float8_e4m3fn)
    scale = torch.rand(e, out, generator=g) + 0.5
    logical = data.float() * scale[..., None]
    # The interleaved container of the same rows: stored 2j = gate j, 2j+1 = up j.
    stored = torch.stack(data.chunk(2, dim=1), dim=2).reshape(data.shape)
    stored_scale = torch.stack(scale.chunk(2, dim=1), dim=2).reshape(scale.shape)
    fp8 = torch.float8_e4m3fn
    weight = RowFP8Weight(stored, torch.zeros(e, inner, out, dtype=fp8), stored_scale,
                          torch.ones(e, inner), dtype=torch.bfloat16, interleaved=True)
    assert weight.shape == (e, out, inner) and weight.dtype == torch.bfloat16
    assert weight.interleaved and len(weight.components()) == 4
    assert torch.equal(weight.dequantize(dtype=torch.float32), logical)
    clone = weight.clone()
    assert torch.equal(clone._data.view(torch.uint8), stored.view(torch.uint8))
    with pytest.raises(ValueError, match="row orders"):
        clone.copy_(RowFP8Weight(*weight.components(), interleaved=False))
    with pytest.raises(ValueError, match="MI355X"):
        RowFP8Weight.quantize(torch.randn(e, out, inner))
    with pytest.raises(ValueError, match="transpose"):
        RowFP8Weight(data, torch.zeros(e, out, inner, dtype=fp8), scale, torch.ones(e, inner))


def test_facade_validation():
    args = _args()
    with pytest.raises(ValueError, match="compute precision"):
        mlops_amd.moe(*args, top_k=2, routing_mode="topk_then_softmax", compute_precision="fp4")
    with pytest.raises(ValueError, match="positive"):
        mlops_amd.moe(*args, top_k=2, routing_mode="topk_then_softmax", swiglu_limit=0)
    with pytest.raises(ValueError, match="together"):
        mlops_amd.moe(*args, top_k=2, routing_mode="topk_then_softmax", shared_w13=args[2])
    with pytest.raises(ValueError, match="shared_gate_weight"):
        mlops_amd.moe(*args, top_k=2, routing_mode="topk_then_softmax", shared_mode="sigmoid")


def test_environment_override(monkeypatch):
    monkeypatch.setenv("MLOPS_IMPLEMENTATIONS", "moe=mi355x.moe.block_fp8")
    token = context._SETTINGS.set(context._SETTINGS.get())
    try:
        applied = context.apply_environment_overrides()
        assert dict(applied) == {"moe": "mi355x.moe.block_fp8"}
        assert context.implementation_override("moe") == "mi355x.moe.block_fp8"
    finally:
        context._SETTINGS.reset(token)
    monkeypatch.setenv("MLOPS_IMPLEMENTATIONS", "garbage")
    with pytest.raises(ValueError):
        context.apply_environment_overrides()


def test_weight_gradient_dtype_context():
    assert weight_gradient_dtype() is None
    with weight_gradients_at(torch.float32):
        assert weight_gradient_dtype() is torch.float32
    with pytest.raises(ValueError):
        with weight_gradients_at(torch.int32):
            pass


def test_dispatch_manifest():
    assert dict(dispatch_manifest({"moe": {"a": 2}})) == {"moe": "a"}
    with pytest.raises(ValueError):
        dispatch_manifest({"moe": {"a": 1, "b": 1}})
    with capture_dispatch() as trace:
        context.record_dispatch("moe", "x")
    assert trace == {"moe": {"x": 1}}


def test_flop_formulas_on_fake_tensors():
    """The op pair is priced by FlopCounterMode under fake tensors
    (reference tests/test_flop_formulas.py:288,403)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    tokens, hidden, inter, experts, k = 64, 256, 128, 4, 2
    with FakeTensorMode():
        x = torch.empty(tokens, hidden, dtype=torch.bfloat16)
        wr = torch.empty(experts, hidden)
        w13 = torch.empty(experts, 2 * inter, hidden, dtype=torch.float8_e4m3fn)
        w2 = torch.empty(experts, hidden, inter, dtype=torch.float8_e4m3fn)
        s13 = torch.empty(experts, 2, 2)
        s2 = torch.empty(experts, 2, 1)
        with FlopCounterMode(display=False) as counter:
            torch.ops.mlops_mi355x.moe_mi355x_block_fp8_fwd(
                x, x, wr, w13, w2, torch.empty(0), k, "topk_then_softmax", 1, 1, 1.0, [tokens],
                "float32", None, None, [s13, s2])
    expected = moe_flops(x, wr, w13, w2, k, forward=True)
    assert counter.get_total_flops() == expected
    a = tokens * k
    assert expected == (2 * tokens * hidden * experts + 3 * tokens * experts
                        + 2 * a * hidden * 2 * inter + 5 * a * inter + 2 * a * inter * hidden
                        + 2 * a * hidden)


def test_composed_flop_formulas_sum_to_the_layer():
    """prepare + finish price the same logical FLOPs as the fused operator
    (reference logical_costs.py:418-494), forward and backward."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    import mlops_amd.providers.mi355x.moe_composed  # noqa: F401  (registers the ops)

    tokens, hidden, inter, experts, k = 64, 256, 128, 4, 2
    a = tokens * k
    ops = torch.ops.mlops_mi355x
    with FakeTensorMode():
        x = torch.empty(tokens, hidden, dtype=torch.bfloat16)
        wr = torch.empty(experts, hidden)
        w13 = torch.empty(experts, 2 * inter, hidden, dtype=torch.float8_e4m3fn)
        w2 = torch.empty(experts, hidden, inter, dtype=torch.float8_e4m3fn)
        s13, s2 = torch.empty(experts, 2, 2), torch.empty(experts, 2, 1)
        with FlopCounterMode(display=False) as forward:
            outs = ops.moe_mi355x_prepare_fwd(x, wr, w13, torch.empty(0), k,
                                              "topk_then_softmax", 1, 1, 1.0, [tokens],
                                              "float32", None, [s13])
            (aux, counts, psum, logits, weights, ids, order, offsets, slots, h13) = outs
            out = ops.moe_mi355x_finish_fwd(h13, w2, weights, order, offsets, slots, x, k, None,
                                            None, [s2])
        with FlopCounterMode(display=False) as backward:
            ops.moe_mi355x_finish_bwd(out, h13, w2, weights, order, offsets, slots, k, None,
                                      None, [s2], True)
            ops.moe_mi355x_prepare_bwd(aux, psum, weights, h13, x, wr, w13, logits, weights, ids,
                                       order, offsets, slots, k, "topk_then_softmax", [tokens],
                                       None, [s13], True, True)
    assert tuple(h13.shape) == (a, 2 * inter) and tuple(out.shape) == (tokens, hidden)
    assert forward.get_total_flops() == moe_flops(x, wr, w13, w2, k, forward=True)
    assert backward.get_total_flops() == moe_flops(x, wr, w13, w2, k, forward=False)


def test_op_namespace_is_separate():
    """New ops live in mlops_mi355x:: so the reference's exact torch.ops.mlops
    manifest test (tests/test_custom_op_contracts.py:787) is unaffected."""
    assert hasattr(torch.ops.mlops_mi355x, "moe_mi355x_block_fp8_fwd")
    assert hasattr(torch.ops.mlops_mi355x, "moe_mi355x_block_fp8_bwd")


def test_block_fp8_container_on_cpu():
    from oracle import moe_oracle as O

    w = torch.randn(2, 256, 128) * 0.02
    data, scale = O.quantize_blocks(w)
    c = mlops_amd.BlockFP8Weight(data, scale)
    assert c.shape == (2, 256, 128) and c.dtype == torch.bfloat16
    assert torch.equal(c.detach()._data.view(torch.uint8), data.view(torch.uint8))
    d = c.dequantize(dtype=torch.float32)
    assert torch.allclose(d, O.dequantize_blocks(data, scale))
    cl = c.clone()
    assert isinstance(cl, mlops_amd.BlockFP8Weight)
    flat, meta = c.__tensor_flatten__()
    assert flat == ["_data", "_scale"]
    with pytest.raises(ValueError, match="MI355X"):
        mlops_amd.BlockFP8Weight.quantize(w)
    with pytest.raises(ValueError, match="E4M3"):
        mlops_amd.BlockFP8Weight(w, scale)
    with pytest.raises(NotImplementedError):
        c + 1
    assert c.to(torch.float32).dtype == torch.float32  # dequantizing copy


def test_routing_override_validation():
    from mlops_amd.routing import next_override, routing_override

    ids = torch.tensor([[0, 1], [2, 3]])
    with pytest.raises(RuntimeError, match="consumed 0"):
        with routing_override([ids]):
            pass
    with routing_override([torch.tensor([[0, 0], [1, 2]])]):
        with pytest.raises(ValueError, match="duplicate"):
            next_override(2, 4, 2, "cpu")
    with routing_override([ids]):
        with pytest.raises(ValueError, match="shape"):
            next_override(3, 4, 2, "cpu")


def test_protocol_containers_are_recognised(monkeypatch):
    """A container class that only carries the reference's block-FP8
    component protocol is served by the block-FP8 operator (and refused by
    the fp8_current one), as the reference's own BlockFP8Weight would be."""
    from mlops_amd.providers.mi355x import moe_current
    from mlops_amd.weight_formats import block_parts, is_row_fp8
    from tests.foreign_container import ProtocolBlockWeight

    monkeypatch.setattr(torch.version, "hip", "7.0", raising=False)
    monkeypatch.setattr(provider, "_arch", lambda device: "gfx950:sramecc+:xnack-")

    class FakeCuda(torch.Tensor):
        pass

    monkeypatch.setattr(FakeCuda, "is_cuda", property(lambda self: True))
    gpu = lambda t: t.as_subclass(FakeCuda)
    x, res, wr, w13, w2 = _args()
    fp8 = torch.float8_e4m3fn

    def foreign(w):
        e, out, inner = w.shape
        return ProtocolBlockWeight(torch.zeros(e, out, inner, dtype=fp8),
                                   torch.ones(e, -(-out // 128), -(-inner // 128)))

    c13, c2 = foreign(w13), foreign(w2)
    assert block_parts(c13) is not None and not is_row_fp8(c13)
    base = dict(surface="semantic", top_k=2, routing_mode="topk_then_softmax")
    ok = provider.supports(gpu(x), gpu(res), gpu(wr), c13, c2, **base)
    assert ok, ok.reason
    refused = moe_current.supports(gpu(x), gpu(res), gpu(wr), c13, c2, **base)
    assert not refused and "fp8_block" in refused.reason
    # A wrong scale shape is not the protocol: treated as a plain weight.
    bad = ProtocolBlockWeight(torch.zeros(8, 256, 256, dtype=fp8), torch.ones(8, 1, 1))
    assert block_parts(bad) is None


class _WrongCube(torch.autograd.Function):
    """x**3 with a backward that misses the factor 3."""

    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return x ** 3

    @staticmethod
    def backward(ctx, grad):
        (x,) = ctx.saved_tensors
        return grad * x * x


def _toy_catalog():
    def yes(*a, **k):
        return SupportResult.yes()

    def float32_only(x, **k):
        return SupportResult.yes() if x.dtype == torch.float32 else SupportResult.no("float32 only")

    registry._catalog.tables["toy.cube"] = {}
    for name, provider_name, prio, supports, apply in (
            ("toy.native", "native_torch", 0, yes, lambda x: x ** 3),
            ("toy.wrong", "t", 7, yes, _WrongCube.apply),
            ("toy.narrow", "t", 9, float32_only, lambda x: x ** 3)):
        registry.register_implementation(
            Implementation("toy.cube", name, provider_name, prio, True, supports, apply))


def test_gradcheck_reports_each_implementation_exactly():
    from mlops_amd.dispatch import GradcheckCase, gradcheck_implementation, gradcheck_implementations

    _toy_catalog()
    try:
        x = torch.randn(5, dtype=torch.float64, requires_grad=True)
        results = {r.implementation_id: r for r in gradcheck_implementations(
            [GradcheckCase("toy.cube", (x,))])}
        assert list(results) == ["toy.narrow", "toy.native", "toy.wrong"]  # sorted IDs
        assert results["toy.native"].status == "passed"
        assert results["toy.wrong"].status == "failed"
        # the float32-only record declines float64 and is skipped, not replaced
        assert results["toy.narrow"].status == "skipped"
        assert "float32 only" in results["toy.narrow"].reason
        with pytest.raises(Exception):
            gradcheck_implementation("toy.cube", "toy.wrong", (x,), raise_exception=True)
        with pytest.raises(ValueError, match="no implementation 'toy.none'"):
            gradcheck_implementation("toy.cube", "toy.none", (x,))
    finally:
        del registry._catalog.tables["toy.cube"]


def test_gradcheck_of_the_mi355x_moe_is_skipped_off_gpu():
    from mlops_amd.dispatch import gradcheck_implementation

    args = [a.double().requires_grad_() if a.is_floating_point() else a for a in _args()]
    result = gradcheck_implementation(
        "moe", provider.IMPLEMENTATION_ID, args,
        kwargs=dict(top_k=2, routing_mode="topk_then_softmax", compute_precision="fp8_block"))
    assert result.status == "skipped" and result.reason


def test_implementation_pairs():
    from mlops_amd.dispatch import implementation_pairs

    _toy_catalog()
    try:
        pairs = implementation_pairs(["toy.cube"])
        assert dict(pairs["toy.cube"]["default"]) == {"toy.cube": "toy.narrow"}
        assert dict(pairs["toy.cube"]["native_torch"]) == {"toy.cube": "toy.native"}
        with use_implementation("toy.cube", pairs["toy.cube"]["native_torch"]["toy.cube"]):
            x = torch.tensor([2.0])
            assert resolve_implementation("toy.cube", x).apply(x).item() == 8.0
    finally:
        del registry._catalog.tables["toy.cube"]
    # The MoE catalog has no plain-torch record: the hot path has no fallback.
    with pytest.raises(ValueError, match="no native_torch"):
        implementation_pairs(["moe"])
