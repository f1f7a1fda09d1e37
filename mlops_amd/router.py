"""The router GEMM and its gradients at the reference's precisions.

Semantics of ``src/mlops/kernels/router.py:54-113`` on the GPU:

* logits: bf16 operands (the router weight taken to the activation dtype),
  fp32 sums, fp32 result (``aten.mm.dtype``);
* input gradient: ``grad_logits`` taken to bf16, times the bf16 weight,
  added in place into the bf16 hidden gradient;
* weight gradient: the cotangent split ``hi = bf16(g)``, ``mid = bf16(g - hi)``,
  each multiplied against the bf16 activation with fp32 sums (fp32-quality
  gradient for an fp32 master), then written at the requested dtype.

These small GEMMs ([T,H]x[H,E]) run on hipBLASLt through torch; the MoE
provider's own kernels take over from the fp32 logits.
"""

from __future__ import annotations

import torch

OPERAND_DTYPES = (torch.bfloat16, torch.float16)
SPLIT_K = 8  # token chunks of the router weight gradient's product


def operand_dtype(hidden: torch.Tensor) -> torch.dtype:
    return hidden.dtype if hidden.is_cuda and hidden.dtype in OPERAND_DTYPES else torch.float32


def _product_fp32(left: torch.Tensor, right: torch.Tensor) -> torch.Tensor:
    if left.is_cuda and left.dtype in OPERAND_DTYPES and left.dtype == right.dtype:
        return torch.ops.aten.mm.dtype(left, right, torch.float32)
    return left.float() @ right.float()


def router_logits(hidden: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """fp32 ``[rows, E]`` logits of ``hidden [rows, D]`` through ``weight [E, D]``."""
    dtype = operand_dtype(hidden)
    return _product_fp32(hidden.to(dtype), weight.to(dtype).t())


def add_router_input_gradient_(grad_hidden, grad_logits, weight):
    """``grad_hidden += grad_logits @ weight`` in place, operands at its dtype."""
    dtype = operand_dtype(grad_hidden)
    if dtype == grad_hidden.dtype:
        grad_hidden.addmm_(grad_logits.to(dtype), weight.to(dtype))
    else:
        grad_hidden.add_((grad_logits.float() @ weight.float()).to(grad_hidden.dtype))
    return grad_hidden


def split_k_product(left: torch.Tensor, right: torch.Tensor) -> torch.Tensor:
    """``left^T @ right`` with fp32 sums and output, for token-major operands
    ``left [T, M]`` and ``right [T, N]`` (bf16/fp16 on the GPU) with a long
    token dimension and small M: split over the tokens into SPLIT_K batched
    products whose fp32 partials are summed. Each batch operand is a view (the
    left one transposed), so nothing is copied. hipBLASLt runs this form ~2x
    faster than the single long-K product on MI355X."""
    tokens = left.shape[0]
    split = SPLIT_K if tokens % SPLIT_K == 0 and tokens >= SPLIT_K * 512 else 1
    if split > 1 and left.is_cuda:
        chunk = tokens // split
        return torch.bmm(left.view(split, chunk, left.shape[1]).transpose(1, 2),
                         right.view(split, chunk, right.shape[1]),
                         out_dtype=torch.float32).sum(0)
    return _product_fp32(left.t(), right)


def router_weight_gradient_from_pieces(pieces, hidden, dtype) -> torch.Tensor:
    """:func:`router_weight_gradient` from the cotangent already split into
    its bf16 ``[hi | mid]`` pieces ``[T, 2E]`` (the router backward kernel
    writes them): ``hi^T x + mid^T x`` with fp32 sums. On the MI355X kernel
    (``mi355x_router_weight_grad``, 128-expert tiles) when E is a multiple of
    8 from 64 up and H a multiple of 256; fewer experts would leave most of
    its tile idle, and those and other widths use the split-K product on
    hipBLASLt."""
    experts = pieces.shape[1] // 2
    hidden = hidden.reshape(-1, hidden.shape[-1])
    if (pieces.is_cuda and hidden.dtype == torch.bfloat16 and experts % 8 == 0
            and experts >= 64 and hidden.shape[1] % 256 == 0):
        from . import kernels

        return kernels.router_weight_grad(pieces, hidden).to(dtype)
    both = split_k_product(pieces, hidden)
    return both[:experts].add_(both[experts:]).to(dtype)


def add_router_input_gradient_from_pieces_(grad_hidden, pieces, weight):
    """``grad_hidden += hi @ weight`` in place, ``hi = bf16(g)`` the first half
    of the pieces (the same operand as ``grad_logits.to(bf16)``)."""
    experts = pieces.shape[1] // 2
    grad_hidden.addmm_(pieces[:, :experts], weight.to(grad_hidden.dtype))
    return grad_hidden


def router_weight_gradient(grad_logits, hidden, dtype) -> torch.Tensor:
    """``grad_logits.T @ hidden`` with fp32 sums, the cotangent in two bf16 pieces."""
    operands = operand_dtype(hidden)
    if operands is torch.float32:
        return (grad_logits.float().t() @ hidden.float()).to(dtype)
    rows = hidden.to(operands)
    tokens, experts = grad_logits.shape
    # Both pieces side by side in one token-major buffer [T, 2E] (hi in the
    # first E columns, mid in the last), so one product [hi | mid]^T @ rows
    # (M = 2E) gives both, and each operand is a transposed view of a
    # contiguous block (no transposing copy). The product is split over the
    # token (K) dimension into SPLIT_K batched products whose fp32 partials
    # are summed: K = T is long and M x N small, and hipBLASLt runs the split
    # form ~2x faster on MI355X.
    pieces = torch.empty((tokens, 2 * experts), dtype=operands, device=grad_logits.device)
    high = pieces[:, :experts]
    high.copy_(grad_logits)
    torch.sub(grad_logits, high.float(), out=pieces[:, experts:])
    both = split_k_product(pieces, rows)
    gradient = both[:experts].add_(both[experts:])
    return gradient.to(dtype)


__all__ = [
    "add_router_input_gradient_",
    "add_router_input_gradient_from_pieces_",
    "router_weight_gradient_from_pieces",
    "split_k_product",
    "operand_dtype",
    "router_logits",
    "router_weight_gradient",
]
