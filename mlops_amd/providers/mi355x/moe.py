"""The MI355X (gfx950) block-FP8 routed-MoE implementation: ``mi355x.moe.block_fp8``.

Registered behind the same registry contract as the reference providers
(``src/mlops/providers/builtin/moe.py:21-554`` for the record, custom-op pair,
fakes, autograd and FLOP formulas; ``providers/sonicmoe/moe.py:441-620`` and
``providers/sonicmoe/block_fp8.py`` for the block-FP8 math it serves). Every
step from the fp32 router logits on is a hand-written HIP kernel of
``libmlops_mi355x.so``; the router GEMM and its two small gradient GEMMs stay on
hipBLASLt through torch, as the reference keeps them on cuBLAS.

Forward (sorted rows ``A = T * k``):
  logits = bf16 x @ bf16 Wr^T (fp32)          router GEMM
  weights, ids = router_topk(logits)          one wave per token
  counts, offsets, order, slots = plan(ids)   stable counting sort
  xq = quantize_rows(x)                       e4m3 token rows (1x128); k < 4: permuted
  h  = gemm(xq[order / k], W13) gate/up       fp8 MFMA reading each routed row's token
                                              row, bf16 out [A, 2I]
  aq = swiglu_quantize(h)                     e4m3 act (1x128)
  y  = gemm(aq, W2)                           [A, H]
  out = residual + sum_j w * y[slot]          token-parallel combine
Backward:
  r = gemm(quant(dy)[order / k], W2)         input gradient through W2 (K-major)
  dh, a', dscore = swiglu_bwd_quantize(r, h)  fused: quant(dh), dh^T, a'^T
  dW2 = wgrad(dy^T, a'^T), dW13 = wgrad(dh^T, x^T)   fp8 wgrad, 128-row blocks
  dx = gemm(quant(dh), W13^T); grad_x = sum_j dx[slot] + grad_logits @ Wr
  grad_logits = router_bwd(dscore[slots], aux / prob-sum cotangents)
"""

from __future__ import annotations

import torch

from ... import kernels, router
from ...block_fp8 import BlockFP8Weight
from ...weight_formats import (block_parts, is_block_fp8, is_row_fp8, register_container_class,
                               route_containers)
from ...dispatch import logical_costs as logical
from ...dispatch.context import weight_gradient_dtype
from ...dispatch.costs import flop_formula
from ...dispatch.registry import Implementation, SupportResult, register_implementation
from ...routing import current_route_weight_precision, next_override

IMPLEMENTATION_ID = "mi355x.moe.block_fp8"
PRIORITY = 120  # above every reference provider (sonicmoe.moe.composed is 110)
ARCH = "gfx950"
ROUTING_MODES = tuple(kernels.ROUTING_MODES)
_ARCH_CACHE: dict[int, str] = {}


def _arch(device: torch.device) -> str:
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _ARCH_CACHE:
        _ARCH_CACHE[index] = torch.cuda.get_device_properties(index).gcnArchName
    return _ARCH_CACHE[index]


def _precision(compute_precision, w13, w2):
    """``"fp8_block"`` when this implementation serves the request, else a refusal."""
    if any(is_row_fp8(w) for w in (w13, w2)):
        return None, "row-FP8 (RowFP8Weight / QuackFP8Weight) weights compute at fp8_current"
    containers = is_block_fp8(w13) or is_block_fp8(w2)
    if compute_precision == "fp8_block":
        return "fp8_block", None
    if compute_precision is None and containers:
        return "fp8_block", None
    if compute_precision is None:
        return None, "plain weights with compute_precision=None compute in bf16; ask 'fp8_block'"
    return None, f"compute_precision={compute_precision!r} is not served (block-FP8 only)"


def supports(
    h2, residual, router_weight, w13_experts, w2_experts, *, surface, top_k, routing_mode,
    router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
    compute_precision=None, shared_w13=None, shared_w2=None, shared_gate_weight=None,
    shared_mode="add", swiglu_limit=None, **_kwargs,
) -> SupportResult:
    """Metadata-only checks; never runs a kernel."""
    _, refusal = _precision(compute_precision, w13_experts, w2_experts)
    if refusal is not None:
        return SupportResult.no(refusal)
    return check_shapes(
        h2, residual, router_weight, w13_experts, w2_experts, top_k=top_k,
        routing_mode=routing_mode, router_bias=router_bias, n_group=n_group,
        topk_group=topk_group, lengths=lengths, shared_w13=shared_w13, shared_w2=shared_w2)


def check_shapes(h2, residual, router_weight, w13_experts, w2_experts, *, top_k, routing_mode,
                 router_bias=None, n_group=1, topk_group=1, lengths=None, shared_w13=None,
                 shared_w2=None) -> SupportResult:
    """The device, dtype, shape and routing rules every MI355X MoE operator shares."""
    tensors = (h2, residual, router_weight, w13_experts, w2_experts)
    if not all(isinstance(t, torch.Tensor) for t in tensors):
        return SupportResult.no("MoE core arguments must be tensors")
    if torch.version.hip is None:
        return SupportResult.no("the MI355X provider needs a ROCm build of torch")
    if not h2.is_cuda:
        return SupportResult.no("the MI355X provider runs on GPU tensors")
    if not _arch(h2.device).startswith(ARCH):
        return SupportResult.no(f"the MI355X provider needs {ARCH}, found {_arch(h2.device)}")
    if h2.dtype != torch.bfloat16 or residual.dtype != torch.bfloat16:
        return SupportResult.no("block-FP8 MoE takes bf16 activations")
    if h2.shape != residual.shape:
        return SupportResult.no("h2 and residual must have equal shape")
    width = h2.shape[-1]
    if router_weight.ndim != 2 or router_weight.shape[1] != width:
        return SupportResult.no("router_weight must have shape [experts, width]")
    experts = router_weight.shape[0]
    if w13_experts.ndim != 3 or w2_experts.ndim != 3:
        return SupportResult.no("expert weights must have shape [experts, out, in]")
    if w13_experts.shape[0] != experts or w2_experts.shape[0] != experts:
        return SupportResult.no("router and expert counts differ")
    expert_width = w2_experts.shape[2]
    if (w13_experts.shape[1] != 2 * expert_width or w13_experts.shape[2] != width
            or w2_experts.shape[1] != width):
        return SupportResult.no(
            "expert weights must be w13 [experts, 2 * expert_width, width] and "
            "w2 [experts, width, expert_width]"
        )
    if width % 128 or expert_width % 128:
        return SupportResult.no("block-FP8 MI355X GEMMs need widths that are multiples of 128")
    if experts > kernels.MAX_EXPERTS:
        return SupportResult.no(f"at most {kernels.MAX_EXPERTS} experts")
    if not 0 < int(top_k) <= min(experts, kernels.MAX_TOP_K):
        return SupportResult.no("top_k must be within the expert count (and <= 32)")
    if routing_mode not in ROUTING_MODES:
        return SupportResult.no(f"unsupported routing mode {routing_mode!r}")
    if routing_mode == "sigmoid_noaux_tc":
        if int(n_group) <= 0 or experts % int(n_group) or int(n_group) > 64:
            return SupportResult.no("n_group must divide the expert count (and be <= 64)")
    if router_bias is not None and router_bias.numel() not in (0, experts):
        return SupportResult.no("router_bias must be [experts]")
    rows = h2.numel() // width
    normalized = (rows,) if lengths is None else tuple(int(x) for x in lengths)
    if not normalized or any(x <= 0 for x in normalized) or sum(normalized) != rows:
        return SupportResult.no("lengths must be positive and cover all hidden rows")
    if (shared_w13 is None) != (shared_w2 is None):
        return SupportResult.no("shared_w13 and shared_w2 must be supplied together")
    return SupportResult.yes()


# --------------------------------------------------------------------------
# The routed math on plain tensors (weights as (data, scale) components).
def _normalized(lengths, rows):
    result = tuple(int(x) for x in lengths)
    if not result or any(x <= 0 for x in result) or sum(result) != rows:
        raise ValueError("MoE lengths must be positive and cover every hidden row")
    return result


def forward_routed(
    h2, residual, router_weight, w13, w2, *, top_k, routing_mode, router_bias=None,
    n_group=1, topk_group=1, routed_scaling=1.0, lengths=None, swiglu_limit=None,
    use_routing_override=True,
):
    """``(output, aux, counts, probability_sum, logits, route_weights, route_ids,
    order, offsets, slots, h13)``; ``w13``/``w2`` are ``(data, scale)`` pairs."""
    width = h2.shape[-1]
    rows = h2.numel() // width
    lengths = _normalized((rows,) if lengths is None else lengths, rows)
    (w13_data, w13_scale), (w2_data, w2_scale) = w13[:2], w2[:2]
    experts = router_weight.shape[0]
    with torch.no_grad():
        x = h2.reshape(rows, width).contiguous()
        base = residual.reshape(rows, width).contiguous()
        logits = router.router_logits(x, router_weight)
        forced = next_override(rows, experts, top_k, x.device) if use_routing_override else None
        bias = None if router_bias is None or router_bias.numel() == 0 else router_bias
        weights, ids = kernels.router_topk(
            logits, int(top_k), routing_mode, bias=bias, n_group=int(n_group),
            topk_group=int(topk_group), routed_scaling=float(routed_scaling), forced_ids=forced,
        )
        counts, offsets, order, slots = kernels.permute_plan(ids, experts)
        # GEMM, then the SwiGLU pass: measured faster than the fused epilogue
        # of mi355x_gemm_fp8_block_swiglu, whose activation math runs while
        # every wave of the CU is in the epilogue (no MFMA work to hide it).
        h13 = routed_rows_gemm(x, slots, order, int(top_k), (w13_data, w13_scale), offsets,
                               interleave=True)
        aq, as_ = kernels.swiglu_quantize(h13, swiglu_limit)
        y = kernels.gemm(aq, as_, w2_data, w2_scale, offsets)
        output = kernels.combine(y, slots, weights, base)
        aux, probability_sum, _, _ = kernels.router_stats(logits, ids, int(top_k), routing_mode, lengths)
    return (output.reshape(h2.shape), aux, counts, probability_sum, logits, weights, ids, order,
            offsets, slots, h13)


def _grad_at(grad: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return grad if grad.dtype == dtype else grad.to(dtype)


def skipped_gradient(like: torch.Tensor, dtype=None) -> torch.Tensor:
    """Placeholder for a gradient nobody asked for (autograd turns it into None)."""
    return torch.empty(0, dtype=like.dtype if dtype is None else dtype, device=like.device)


def backward_routed(
    grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13, w2, logits,
    route_weights, route_ids, order, offsets, slots, h13, *, top_k, routing_mode, lengths,
    weight_grad_dtype, swiglu_limit=None, need_router=True, need_w13=True, need_w2=True,
    need_residual=True,
):
    """VJPs ``(h2, residual, router_weight, w13, w2)`` with fp32 sums; the
    expert weights' gradients at ``weight_grad_dtype`` (bf16, the containers'
    logical dtype, when None), the router's at ``weight_grad_dtype`` (its own
    dtype when None); unrequested weight grads are placeholders."""
    width = h2.shape[-1]
    rows = h2.numel() // width
    lengths = _normalized(lengths, rows)
    (w13_data, w13_scale), (w2_data, w2_scale) = w13[:2], w2[:2]
    experts = router_weight.shape[0]
    assignments = order.numel()
    router_dtype = router_weight.dtype if weight_grad_dtype is None else weight_grad_dtype
    weight_grad_dtype = torch.bfloat16 if weight_grad_dtype is None else weight_grad_dtype
    direct = weight_grad_dtype if weight_grad_dtype in (torch.bfloat16, torch.float32) else torch.float32
    with torch.no_grad():
        x = h2.reshape(rows, width).contiguous()
        dy = grad_output.reshape(rows, width).contiguous()
        if dy.dtype != torch.bfloat16:
            dy = dy.to(torch.bfloat16)
        # Through the down projection: r = dy_routed @ W2, then SwiGLU backward.
        r = routed_rows_gemm(dy, slots, order, int(top_k), w2, offsets, input_gradient=True)
        # SwiGLU backward fused with the quantizers of its outputs: dh row-
        # quantized for the input gradient, dh and a' transposed for the
        # weight gradients (each only when that gradient is wanted).
        padded = kernels.wgrad_padded_rows(assignments, experts)
        blocks = kernels.padded_row_blocks(offsets, padded)
        dhq, dhs, dh_t, dh_ts, ap_t, ap_ts, dscore, _ = kernels.swiglu_bwd_quantize(
            r, h13, route_weights.reshape(-1), order, offsets, padded=padded, limit=swiglu_limit,
            transposed_dh=need_w13, transposed_ap=need_w2, row_blocks=blocks,
        )
        if need_w2:
            dy_t, dy_ts, _ = kernels.quantize_transpose(
                dy, offsets, assignments, gather=order, gather_div=int(top_k), padded=padded,
                row_blocks=blocks,
            )
            grad_w2 = _grad_at(kernels.wgrad(dy_t, dy_ts, ap_t, ap_ts, offsets, out_dtype=direct,
                                             rows=assignments),
                               weight_grad_dtype)
        else:
            grad_w2 = skipped_gradient(h2, weight_grad_dtype)
        # Through the up projection: dx = dh @ W13 (gate rows, then up rows).
        dx = input_gradient_gemm(dhq, dhs, w13, offsets)
        if need_w13:
            x_t, x_ts, _ = kernels.quantize_transpose(
                x, offsets, assignments, gather=order, gather_div=int(top_k), padded=padded,
                row_blocks=blocks,
            )
            grad_w13 = _grad_at(kernels.wgrad(dh_t, dh_ts, x_t, x_ts, offsets, out_dtype=direct,
                                              rows=assignments),
                                weight_grad_dtype)
        else:
            grad_w13 = skipped_gradient(h2, weight_grad_dtype)
        grad_h2 = kernels.unpermute_sum(dx, slots)
        grad_router = routing_backward(
            grad_h2, x, router_weight, logits, route_weights, route_ids, dscore, slots, offsets,
            grad_aux, grad_probability_sum, top_k=top_k, routing_mode=routing_mode,
            lengths=lengths, router_dtype=router_dtype, need_router=need_router,
        )
    grad_residual = grad_output.clone() if need_residual else grad_output.new_empty(0)
    return (grad_h2.reshape(h2.shape).to(h2.dtype), grad_residual, grad_router, grad_w13, grad_w2)


def routing_backward(grad_h2, x, router_weight, logits, route_weights, route_ids, dscore, slots,
                     offsets, grad_aux, grad_probability_sum, *, top_k, routing_mode, lengths,
                     router_dtype, need_router=True):
    """Score gradient ``dscore`` (per sorted row) and the aux / probability-sum
    cotangents through the router: returns the router weight's gradient (a
    placeholder when not needed) and adds the router's input gradient to
    ``grad_h2`` in place. An empty ``grad_aux`` / ``grad_probability_sum``
    stands for a zero cotangent."""
    if grad_aux is not None and grad_aux.numel() == 0:
        grad_aux = None
    if grad_probability_sum is not None and grad_probability_sum.numel() == 0:
        grad_probability_sum = None
    seg_offsets = seg_counts = None
    if routing_mode == "sigmoid_noaux_tc" and grad_aux is not None:
        _, _, seg_counts, seg_offsets = kernels.router_stats(
            logits, route_ids, int(top_k), routing_mode, lengths
        )
    # bf16 activations: the kernel writes the cotangent's bf16 pieces, the
    # operands of both router GEMMs, in place of fp32 logit gradients.
    split = (router.operand_dtype(x) == torch.bfloat16 and grad_h2.dtype == torch.bfloat16
             and x.dtype == torch.bfloat16)
    grad_logits = kernels.router_backward(
        logits, route_weights, route_ids, dscore, slots, routing_mode,
        grad_aux=grad_aux, grad_prob_sum=grad_probability_sum, offsets=offsets,
        seg_offsets=seg_offsets, seg_counts=seg_counts, pieces=split,
    )
    if split:
        if need_router:
            grad_router = router.router_weight_gradient_from_pieces(grad_logits, x, router_dtype)
            if grad_router.stride() != router_weight.stride():
                aligned = torch.empty_strided(grad_router.shape, router_weight.stride(),
                                              dtype=grad_router.dtype, device=grad_router.device)
                aligned.copy_(grad_router)
                grad_router = aligned
        else:
            grad_router = skipped_gradient(router_weight, router_dtype)
        router.add_router_input_gradient_from_pieces_(grad_h2, grad_logits, router_weight)
        return grad_router
    if need_router:
        grad_router = router.router_weight_gradient(grad_logits, x, router_dtype)
        if grad_router.stride() != router_weight.stride():
            aligned = torch.empty_strided(grad_router.shape, router_weight.stride(),
                                          dtype=grad_router.dtype, device=grad_router.device)
            aligned.copy_(grad_router)
            grad_router = aligned
    else:
        grad_router = skipped_gradient(router_weight, router_dtype)
    router.add_router_input_gradient_(grad_h2, grad_logits, router_weight)
    return grad_router


# --------------------------------------------------------------------------
# Custom operators. Weights arrive as block-FP8 containers; the dispatch
# rule below replaces each by its e4m3 data and appends its scale to
# ``weight_components`` (the reference's container protocol,
# providers/sonicmoe/fp8.py:204-236).
def _split(w13, w2, weight_components):
    """``((w13, scale[, data_t]), (w2, scale[, data_t]))``: the two scales,
    optionally followed by the two transposed e4m3 copies the per-call
    quantizer writes in the same pass (containers built elsewhere have none;
    the input-gradient GEMMs then read the data as stored or transpose on the
    fly). An empty tensor stands for the copy of a weight that has none."""
    if len(weight_components) == 2:
        return (w13, weight_components[0]), (w2, weight_components[1])
    if len(weight_components) == 4:
        parts = []
        for data, scale, data_t in ((w13, weight_components[0], weight_components[2]),
                                    (w2, weight_components[1], weight_components[3])):
            parts.append((data, scale) if data_t.numel() == 0 else (data, scale, data_t))
        return tuple(parts)
    raise ValueError("the block-FP8 operators take the two weights' scales (and optionally "
                     "their transposed data) as components")


# From this many routed rows per token, the GEMMs read token rows quantized
# once (mi355x_gemm_fp8_block_gathered) instead of a permuted copy of k rows
# per token. Measured on MI355X at C3 (k = 8): the copy's 69 us against 18 us
# for the token rows, the gathered GEMM ~3% slower on the up projection and
# ~4% faster on r = dy @ W2; at k = 2 (Mixtral) the gathered GEMMs lose more
# (4% of a 2 ms GEMM) than the copy costs.
GATHER_MIN_TOP_K = 4


def routed_rows_gemm(x, slots, order, top_k, weight, offsets, *, interleave=False,
                     input_gradient=False):
    """The GEMM on the routed rows of token rows ``x [T, K]`` (bf16): the
    projection ``rows @ W[e]^T`` (``weight = (data [E, N, K], scale)``), or
    with ``input_gradient`` the input gradient ``rows @ W[e]`` as
    :func:`input_gradient_gemm` does it. Bitwise the same whichever way the
    rows are read."""
    data, scale = weight[0], weight[1]
    n = data.shape[2] if input_gradient else data.shape[1]
    kmajor = input_gradient and len(weight) == 2
    if top_k >= GATHER_MIN_TOP_K and n % 256 == 0 and (kmajor or not input_gradient):
        tq, ts = kernels.quantize_token_rows(x)
        # Routed row r reads token order[r] // top_k, divided in the kernel.
        return kernels.gemm_gathered(tq, ts, order, data, scale, offsets, interleave=interleave,
                                     kmajor=kmajor, rows_div=top_k)
    xq, xs = kernels.permute_quantize(x, slots)
    if input_gradient:
        return input_gradient_gemm(xq, xs, weight, offsets)
    return kernels.gemm(xq, xs, data, scale, offsets, interleave=interleave)


def input_gradient_gemm(aq, a_scale, weight, offsets):
    """``rows @ W[e]`` for the input gradients (``weight = (data [E, K, N],
    scale[, data_t])``): through a transposed copy the weight carries, else
    on the data as stored (``mi355x_gemm_fp8_block_kmajor``, bitwise the
    same), else (N not a multiple of 256) through a copy transposed now."""
    data, scale = weight[0], weight[1]
    if len(weight) == 3:
        return kernels.gemm(aq, a_scale, weight[2], scale, offsets, transposed_scale=True)
    if data.shape[2] % 256 == 0:
        return kernels.gemm_kmajor(aq, a_scale, data, scale, offsets)
    return kernels.gemm(aq, a_scale, kernels.transpose_fp8(data), scale, offsets,
                        transposed_scale=True)


def available_transposed(container) -> torch.Tensor | None:
    """A transposed copy the container already has (carried from a quantizer
    or cached by :func:`transposed_data`), or None; nothing is computed."""
    carried = getattr(container, "_transposed", None)
    if carried is not None:
        return carried
    cached = getattr(container, "_transposed_cache", None)
    data = block_parts(container)[0]
    if cached is not None and cached[0] == data._version and cached[1] is data:
        return cached[2]
    return None


def transposed_data(container: BlockFP8Weight) -> torch.Tensor:
    """The container's e4m3 data transposed per expert (``[E, in, out]``), the
    operand layout of the input-gradient GEMMs. A per-call quantized weight
    carries it from the quantizer's own pass; otherwise it is made once and
    kept on the container for as long as the data's version counter (bumped
    by every in-place write through torch) is unchanged, so a frozen base is
    transposed once, not at every backward. It occupies as much memory as
    the data."""
    carried = getattr(container, "_transposed", None)
    if carried is not None:
        return carried
    data = block_parts(container)[0]
    cached = getattr(container, "_transposed_cache", None)
    if cached is not None and cached[0] == data._version and cached[1] is data:
        return cached[2]
    result = kernels.transpose_fp8(data)
    container._transposed_cache = (data._version, data, result)
    return result


@torch.library.custom_op("mlops_mi355x::moe_mi355x_block_fp8_fwd", mutates_args=())
def _forward_op(
    h2: torch.Tensor, residual: torch.Tensor, router_weight: torch.Tensor,
    w13_experts: torch.Tensor, w2_experts: torch.Tensor, router_bias: torch.Tensor,
    top_k: int, routing_mode: str, n_group: int, topk_group: int, routed_scaling: float,
    lengths: list[int], weight_precision: str, weight_grad_dtype: torch.dtype | None,
    swiglu_limit: float | None, weight_components: list[torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
           torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    del weight_precision, weight_grad_dtype
    w13, w2 = _split(w13_experts, w2_experts, weight_components)
    return forward_routed(
        h2, residual, router_weight, w13, w2, top_k=top_k, routing_mode=routing_mode,
        router_bias=router_bias, n_group=n_group, topk_group=topk_group,
        routed_scaling=routed_scaling, lengths=lengths, swiglu_limit=swiglu_limit,
    )


@_forward_op.register_fake
def _forward_fake(h2, residual, router_weight, w13_experts, w2_experts, router_bias, top_k,
                  routing_mode, n_group, topk_group, routed_scaling, lengths, weight_precision,
                  weight_grad_dtype, swiglu_limit, weight_components):
    rows = h2.numel() // h2.shape[-1]
    experts = router_weight.shape[0]
    assignments = rows * int(top_k)
    device = h2.device
    return (
        torch.empty_like(h2),
        torch.empty((), dtype=torch.float32, device=device),
        torch.empty(experts, dtype=torch.int64, device=device),
        torch.empty(experts, dtype=torch.float32, device=device),
        torch.empty((rows, experts), dtype=torch.float32, device=device),
        torch.empty((rows, int(top_k)), dtype=torch.float32, device=device),
        torch.empty((rows, int(top_k)), dtype=torch.int32, device=device),
        torch.empty(assignments, dtype=torch.int32, device=device),
        torch.empty(experts + 1, dtype=torch.int32, device=device),
        torch.empty((rows, int(top_k)), dtype=torch.int32, device=device),
        torch.empty((assignments, w13_experts.shape[1]), dtype=h2.dtype, device=device),
    )


@torch.library.custom_op("mlops_mi355x::moe_mi355x_block_fp8_bwd", mutates_args=())
def _backward_op(
    grad_output: torch.Tensor, grad_aux: torch.Tensor, grad_probability_sum: torch.Tensor,
    h2: torch.Tensor, router_weight: torch.Tensor, w13_experts: torch.Tensor,
    w2_experts: torch.Tensor, logits: torch.Tensor, route_weights: torch.Tensor,
    route_ids: torch.Tensor, order: torch.Tensor, offsets: torch.Tensor, slots: torch.Tensor,
    h13: torch.Tensor, top_k: int, routing_mode: str, lengths: list[int],
    weight_grad_dtype: torch.dtype | None, swiglu_limit: float | None, need_router: bool,
    need_w13: bool, need_w2: bool, need_residual: bool,
    weight_components: list[torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    w13, w2 = _split(w13_experts, w2_experts, weight_components)
    return backward_routed(
        grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13, w2, logits,
        route_weights, route_ids, order, offsets, slots, h13, top_k=top_k,
        routing_mode=routing_mode, lengths=lengths,
        weight_grad_dtype=weight_grad_dtype, swiglu_limit=swiglu_limit, need_router=need_router,
        need_w13=need_w13, need_w2=need_w2, need_residual=need_residual,
    )


@_backward_op.register_fake
def _backward_fake(grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13_experts,
                   w2_experts, logits, route_weights, route_ids, order, offsets, slots, h13,
                   top_k, routing_mode, lengths, weight_grad_dtype, swiglu_limit, need_router,
                   need_w13, need_w2, need_residual, weight_components):
    grad_dtype = torch.bfloat16 if weight_grad_dtype is None else weight_grad_dtype
    router_dtype = router_weight.dtype if weight_grad_dtype is None else weight_grad_dtype
    return (
        torch.empty_like(h2),
        torch.empty_like(grad_output) if need_residual else grad_output.new_empty(0),
        torch.empty(router_weight.shape, dtype=router_dtype, device=h2.device)
        if need_router else skipped_gradient(router_weight, router_dtype),
        torch.empty(w13_experts.shape, dtype=grad_dtype, device=h2.device)
        if need_w13 else skipped_gradient(h2, grad_dtype),
        torch.empty(w2_experts.shape, dtype=grad_dtype, device=h2.device)
        if need_w2 else skipped_gradient(h2, grad_dtype),
    )


@flop_formula(_forward_op)
def _forward_flops(h2, residual, router_weight, w13_experts, w2_experts, router_bias, top_k,
                   *_rest, out_val=None, **_kwargs):
    return logical.moe_flops(h2, router_weight, w13_experts, w2_experts, top_k, forward=True)


@flop_formula(_backward_op)
def _backward_flops(grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13_experts,
                    w2_experts, logits, route_weights, route_ids, order, offsets, slots, h13,
                    top_k, *_rest, out_val=None, **_kwargs):
    return logical.moe_flops(h2, router_weight, w13_experts, w2_experts, top_k, forward=False)


def _container_rule(cls, func, types, args, kwargs):
    del cls, types
    if kwargs:
        raise ValueError("use positional operator arguments")
    args = list(args)
    components = list(args[-1])
    transposed = []
    backward = func is torch.ops.mlops_mi355x.moe_mi355x_block_fp8_bwd.default
    for index, value in enumerate(args):
        parts = block_parts(value)
        if parts is not None:
            args[index] = parts[0]
            components.append(parts[1])
            # The input-gradient GEMMs read a transposed copy the container
            # already has, or the data as stored (none is made here).
            transposed.append(available_transposed(value) if backward
                              else getattr(value, "_transposed", None))
    if len(transposed) == 2 and any(t is not None for t in transposed):
        components.extend(t if t is not None else args[0].new_empty(0, dtype=torch.uint8)
                          for t in transposed)
    args[-1] = components
    return func(*args)


OPERATORS = (_forward_op, _backward_op)
register_container_class(OPERATORS, _container_rule, BlockFP8Weight)


def _setup_context(ctx, inputs, output):
    (h2, _residual, router_weight, w13, w2, _bias, top_k, routing_mode, _n_group, _topk_group,
     _scaling, lengths, _precision, weight_grad_dtype, swiglu_limit, components) = inputs
    (_out, _aux, counts, _psum, logits, route_weights, route_ids, order, offsets, slots,
     h13) = output
    ctx.save_for_backward(h2, router_weight, w13, w2, logits, route_weights, route_ids, order,
                          offsets, slots, h13, *components)
    ctx.top_k = int(top_k)
    ctx.routing_mode = routing_mode
    ctx.lengths = list(lengths)
    ctx.weight_grad_dtype = weight_grad_dtype
    ctx.swiglu_limit = swiglu_limit
    ctx.n_components = len(components)
    # Unused cotangents arrive as None (the backward builds the small ones it
    # needs) instead of autograd materializing zeros, h13's 2 bytes x A x 2I
    # among them.
    ctx.set_materialize_grads(False)
    ctx.mark_non_differentiable(counts, logits, route_weights, route_ids, order, offsets, slots,
                                h13)


def _autograd_backward(ctx, grad_output, grad_aux, _g_counts, grad_probability_sum, *_unused):
    saved = ctx.saved_tensors
    h2, router_weight = saved[:2]
    components = list(saved[11:])
    # An absent cotangent travels as an empty tensor (no fill kernel); the
    # router backward then treats it as zero.
    if grad_aux is None:
        grad_aux = torch.empty(0, dtype=torch.float32, device=h2.device)
    if grad_probability_sum is None:
        grad_probability_sum = torch.empty(0, dtype=torch.float32, device=h2.device)
    if grad_output is None:
        grad_output = torch.zeros_like(h2)
    needs = ctx.needs_input_grad
    grads = _backward_op(
        grad_output.contiguous(), grad_aux, grad_probability_sum, *saved[:11], ctx.top_k,
        ctx.routing_mode, ctx.lengths, ctx.weight_grad_dtype, ctx.swiglu_limit, bool(needs[2]),
        bool(needs[3]), bool(needs[4]), False, components,
    )
    grad_h2, _, grad_router, grad_w13, grad_w2 = grads
    # d residual is the incoming cotangent itself; the operator returns an
    # empty placeholder here rather than a copy (a custom operator's outputs
    # may not alias its inputs).
    grad_residual = grad_output if needs[1] else None
    return (grad_h2, grad_residual, grad_router if needs[2] else None,
            grad_w13 if needs[3] else None, grad_w2 if needs[4] else None, *([None] * 10),
            [None] * ctx.n_components)


_forward_op.register_autograd(_autograd_backward, setup_context=_setup_context)


# --------------------------------------------------------------------------
class _QuantizePerCall(torch.autograd.Function):
    """A plain weight quantized for one call (``BlockFP8Weight.quantize``
    semantics, straight-through gradient). The input-gradient GEMMs read the
    e4m3 data as stored (K-major), so no transposed copy is written: that
    saves a quarter of the quantizer's bytes for ~4-10% on those two GEMMs.
    A weight whose last axis (the N of that K-major GEMM) is not a multiple
    of 256 (outside the K-major kernel) still gets the copy from the same
    pass."""

    @staticmethod
    def forward(ctx, weight):
        if weight.shape[2] % 256 == 0:
            data, scale = kernels.quantize_weight_blocks(weight.detach())
            return BlockFP8Weight(data, scale, dtype=weight.dtype)
        data, scale, data_t = kernels.quantize_weight_blocks(weight.detach(), transposed=True)
        container = BlockFP8Weight(data, scale, dtype=weight.dtype)
        container._transposed = data_t
        return container

    @staticmethod
    def backward(ctx, grad):
        return grad


def _containers(w13, w2):
    """Plain weights quantized per call (straight-through); containers as they are."""
    weights = tuple(w if is_block_fp8(w) else _QuantizePerCall.apply(w) for w in (w13, w2))
    # Containers of other classes carrying the same components (the
    # reference's own BlockFP8Weight) reach the operators the same way.
    route_containers(OPERATORS, _container_rule, *weights)
    return weights


def _shared_base(h2, residual, shared_w13, shared_w2, shared_gate_weight, shared_mode, limit):
    """The optional shared expert, composed outside the routed operator as the
    reference does (``src/mlops/moe.py:12-37``): torch GEMMs on hipBLASLt."""
    if shared_w13 is None:
        return residual
    flat = h2.reshape(-1, h2.shape[-1])
    packed = torch.nn.functional.linear(flat, shared_w13)
    width = shared_w2.shape[1]
    gate, up = packed[:, :width], packed[:, width:]
    if limit is not None:
        gate, up = gate.clamp(max=limit), up.clamp(-limit, limit)
    activated = torch.nn.functional.silu(gate.float()).to(gate.dtype) * up
    shared = torch.nn.functional.linear(activated, shared_w2)
    if shared_mode == "sigmoid":
        gate_value = torch.sigmoid(torch.nn.functional.linear(flat, shared_gate_weight).float())
        shared = (gate_value * shared.float()).to(residual.dtype)
    return residual + shared.reshape_as(residual)


def apply(
    h2, residual, router_weight, w13_experts, w2_experts, *, top_k, routing_mode,
    router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
    shared_w13=None, shared_w2=None, shared_gate_weight=None, shared_mode="add",
    compute_precision=None, swiglu_limit=None,
):
    """``(out, aux, counts, probability_sum)`` with autograd through the op pair."""
    _, refusal = _precision(compute_precision, w13_experts, w2_experts)
    if refusal is not None:
        raise ValueError(refusal)
    w13, w2 = _containers(w13_experts, w2_experts)
    rows = h2.numel() // h2.shape[-1]
    normalized = (rows,) if lengths is None else tuple(int(x) for x in lengths)
    bias = torch.empty(0, dtype=torch.float32, device=h2.device) if router_bias is None else router_bias
    base = _shared_base(h2, residual, shared_w13, shared_w2, shared_gate_weight, shared_mode,
                        swiglu_limit)
    outputs = _forward_op(
        h2, base, router_weight, w13, w2, bias, int(top_k), str(routing_mode), int(n_group),
        int(topk_group), float(routed_scaling), list(normalized),
        current_route_weight_precision(), weight_gradient_dtype(),
        None if swiglu_limit is None else float(swiglu_limit), [],
    )
    return outputs[:4]


def _components(weight):
    parts = block_parts(weight)
    if parts is not None:
        return parts
    data, scale = kernels.quantize_weight_blocks(weight)
    return data, scale


def forward(
    h2, residual, router_weight, w13_experts, w2_experts, *, top_k, routing_mode,
    router_bias=None, n_group=1, topk_group=1, routed_scaling=1.0, lengths=None,
    weight_precision="float32", swiglu_implementation=None, swiglu_limit=None,
):
    """Explicit surface: the 11-tuple ``(output, aux, counts, probability_sum,
    logits, route_weights, route_ids, order, offsets, slots, h13)``; ``h13`` is
    this provider's interleaved gate/up pre-activation."""
    del weight_precision, swiglu_implementation
    return forward_routed(
        h2, residual, router_weight, _components(w13_experts), _components(w2_experts),
        top_k=top_k, routing_mode=routing_mode, router_bias=router_bias, n_group=n_group,
        topk_group=topk_group, routed_scaling=routed_scaling, lengths=lengths,
        swiglu_limit=swiglu_limit,
    )


def backward(
    grad_output, grad_aux, grad_probability_sum, h2, router_weight, w13_experts, w2_experts,
    logits, route_weights, route_ids, order, offsets, slots, h13, *, top_k, routing_mode,
    lengths, swiglu_implementation=None, swiglu_limit=None, weight_grad_dtype=None,
):
    """Explicit surface: ``(d_h2, d_residual, d_router, d_w13, d_w2)``."""
    del swiglu_implementation
    grad_dtype = weight_gradient_dtype() if weight_grad_dtype is None else weight_grad_dtype
    return backward_routed(
        grad_output, grad_aux, grad_probability_sum, h2, router_weight,
        _components(w13_experts), _components(w2_experts), logits, route_weights, route_ids,
        order, offsets, slots, h13, top_k=top_k, routing_mode=routing_mode, lengths=lengths,
        weight_grad_dtype=grad_dtype, swiglu_limit=swiglu_limit,
    )


def estimate(h2, residual, router_weight, w13_experts, w2_experts, *, top_k,
             entrypoint="forward", **_kwargs):
    """Physical GEMM FLOPs (block-FP8 MFMA) and the compulsory HBM bytes of the
    permute / quantize / combine passes of this implementation."""
    from ...dispatch.costs import CostHints

    rows = h2.numel() // h2.shape[-1]
    width, inter = h2.shape[-1], w2_experts.shape[2]
    a = rows * int(top_k)
    gemm = 6 * a * width * inter * (1 if entrypoint == "forward" else 2)
    traffic = (2 * rows * width + a * width + 4 * a * width // 128  # permute_quantize
               + 2 * a * 2 * inter * 2 + a * inter                # h write/read, act
               + 2 * a * width + 2 * rows * width * 2)            # y + combine
    return CostHints(implementation_flops=gemm, implementation_bytes_accessed=traffic)


IMPLEMENTATION = register_implementation(
    Implementation(
        operation="moe",
        implementation_id=IMPLEMENTATION_ID,
        provider="mi355x",
        priority=PRIORITY,
        deterministic=True,
        supports=supports,
        apply=apply,
        forward=forward,
        backward=backward,
        estimate=estimate,
    )
)

__all__ = [
    "GATHER_MIN_TOP_K",
    "routed_rows_gemm",
    "IMPLEMENTATION",
    "apply",
    "backward",
    "backward_routed",
    "forward",
    "forward_routed",
    "routing_backward",
    "supports",
    "transposed_data",
    "input_gradient_gemm",
    "available_transposed",
]
