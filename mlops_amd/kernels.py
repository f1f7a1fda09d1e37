"""Typed wrappers over the C-ABI kernels of ``libmlops_mi355x.so``.

Each wrapper validates shapes, dtypes and devices on the host, allocates its
outputs with torch on the input's device, and enqueues the kernel on torch's
current stream. None of them synchronizes or reads device memory.

Layouts: routed rows ``A = tokens * top_k`` are in expert-sorted order;
1x128 activation scales are stored K-block major (``scales[kb, row]``);
128x128 weight scales are ``[E, ceil(out/128), ceil(in/128)]``.
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _native

FP8 = torch.float8_e4m3fn
ROUTING_MODES = {"topk_then_softmax": 0, "softmax_then_topk": 1, "sigmoid_noaux_tc": 2}
STATS_CHUNK = 64
MAX_EXPERTS = 512
MAX_TOP_K = 32


class _HipEvents:
    """HIP events created with ``hipEventDisableSystemFence``, through the HIP
    runtime this process already loaded (torch's). A default event's record
    ends with a system-scope fence, a cache writeback that a timed interval
    would count; these events only take timestamps."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self):
        paths = [line.split()[-1] for line in open("/proc/self/maps") if "libamdhip64" in line]
        if not paths:
            raise RuntimeError("the HIP runtime is not loaded in this process")
        lib = ctypes.CDLL(paths[0])
        lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                            ctypes.c_void_p]
        lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib = lib

    def _check(self, status, what):
        if status != 0:
            raise RuntimeError(f"{what} failed with HIP error {status}")

    def record(self, stream) -> ctypes.c_void_p:
        event = ctypes.c_void_p()
        self._check(self.lib.hipEventCreateWithFlags(ctypes.byref(event), self.DISABLE_SYSTEM_FENCE),
                    "hipEventCreateWithFlags")
        self._check(self.lib.hipEventRecord(event, stream), "hipEventRecord")
        return event

    def elapsed_ms(self, start, end) -> float:
        ms = ctypes.c_float()
        self._check(self.lib.hipEventElapsedTime(ctypes.byref(ms), start, end),
                    "hipEventElapsedTime")
        return ms.value

    def destroy(self, event) -> None:
        self.lib.hipEventDestroy(event)


class LaunchTimer:
    """Records a pair of device events around each timed kernel launch, on the
    stream the kernel is enqueued on, with the launch's algorithmic work.
    Install with ``set_launch_timer``; read ``summary()`` after a sync."""

    def __init__(self):
        self.records = []  # (name, start, end, flops, bytes)
        self.events = _HipEvents()

    def start(self, device):
        return self.events.record(_stream(device))

    def stop(self, name, device, start, flops=0, nbytes=0):
        self.records.append((name, start, self.events.record(_stream(device)), flops, nbytes))

    def summary(self):
        """``{name: dict(launches, ms_total, ms_avg, flops, bytes)}``; the
        events are released."""
        out = {}
        for name, start, end, flops, nbytes in self.records:
            entry = out.setdefault(name, dict(launches=0, ms_total=0.0, flops=0, bytes=0))
            entry["launches"] += 1
            entry["ms_total"] += self.events.elapsed_ms(start, end)
            entry["flops"] += flops
            entry["bytes"] += nbytes
            self.events.destroy(start)
            self.events.destroy(end)
        self.records = []
        for entry in out.values():
            entry["ms_avg"] = entry["ms_total"] / entry["launches"]
        return out


_TIMER: LaunchTimer | None = None


def set_launch_timer(timer: LaunchTimer | None) -> None:
    global _TIMER
    _TIMER = timer


def _timed(name, device, flops, nbytes, fn, *args):
    if _TIMER is None:
        _native.call(fn, *args)
        return
    start = _TIMER.start(device)
    _native.call(fn, *args)
    _TIMER.stop(name, device, start, flops, nbytes)


_CU_COUNTS: dict[int, int] = {}


def _cu_count(device: torch.device) -> int:
    """Compute units of the device (cached; a host-side property query)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _CU_COUNTS:
        _CU_COUNTS[index] = torch.cuda.get_device_properties(index).multi_processor_count
    return _CU_COUNTS[index]


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _stream(device: torch.device):
    return torch.cuda.current_stream(device).cuda_stream


def _on_gpu(*tensors: torch.Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("the MI355X kernels take GPU tensors only")
        if not t.is_contiguous():
            raise ValueError("the MI355X kernels take contiguous tensors")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("all tensors of one kernel call must be on one device")
    return device


def _check(t: torch.Tensor, shape, dtype, name: str) -> None:
    if tuple(t.shape) != tuple(shape) or t.dtype != dtype:
        raise ValueError(f"{name}: expected {dtype} {tuple(shape)}, got {t.dtype} {tuple(t.shape)}")


def _limit(limit: float | None) -> float:
    return 0.0 if limit is None else float(limit)


# ------------------------------------------------------------------ router
def router_topk(
    logits: torch.Tensor,
    top_k: int,
    mode: str,
    *,
    bias: torch.Tensor | None = None,
    n_group: int = 1,
    topk_group: int = 1,
    routed_scaling: float = 1.0,
    forced_ids: torch.Tensor | None = None,
):
    """``(weights fp32 [T,k], ids int32 [T,k])`` of fp32 ``logits [T,E]``."""
    if mode not in ROUTING_MODES:
        raise ValueError(f"unsupported routing mode {mode!r}")
    if logits.dtype != torch.float32 or logits.ndim != 2:
        raise ValueError("router logits must be fp32 [tokens, experts]")
    tokens, experts = logits.shape
    if bias is not None:
        bias = bias.float().contiguous()
        if bias.shape != (experts,):
            raise ValueError("router bias must be [experts]")
    if forced_ids is not None:
        forced_ids = forced_ids.to(device=logits.device, dtype=torch.int32).contiguous()
        _check(forced_ids, (tokens, top_k), torch.int32, "forced_ids")
    device = _on_gpu(logits, bias, forced_ids)
    weights = torch.empty((tokens, top_k), dtype=torch.float32, device=device)
    ids = torch.empty((tokens, top_k), dtype=torch.int32, device=device)
    # logits read, weights and ids written (bias / forced ids are small)
    nbytes = 4 * tokens * experts + 8 * tokens * int(top_k)
    _timed(
        "router_topk", device, 0, nbytes,
        "mi355x_router_topk", _ptr(logits), tokens, experts, int(top_k), ROUTING_MODES[mode],
        _ptr(bias), int(n_group), int(topk_group), float(routed_scaling), _ptr(forced_ids),
        _ptr(weights), _ptr(ids), _stream(device),
    )
    return weights, ids


def segment_tables(lengths: Sequence[int], tokens: int, device):
    """``(seg_offsets, chunk_table, nchunks)`` for per-sequence statistics;
    ``(None, None, ceil(T/64))`` for one segment."""
    lengths = [int(x) for x in lengths]
    if len(lengths) <= 1:
        return None, None, (tokens + STATS_CHUNK - 1) // STATS_CHUNK
    offsets = [0]
    chunks = []
    for segment, length in enumerate(lengths):
        start = offsets[-1]
        for first in range(start, start + length, STATS_CHUNK):
            chunks.extend((first, segment))
        offsets.append(start + length)
    seg = torch.tensor(offsets, dtype=torch.int32).to(device, non_blocking=False)
    table = torch.tensor(chunks, dtype=torch.int32).to(device, non_blocking=False)
    return seg, table, len(chunks) // 2


def router_stats(logits, ids, top_k: int, mode: str, lengths: Sequence[int]):
    """``(aux fp32 [], prob_sum fp32 [E], seg_counts int32 [S,E], seg_offsets)``."""
    tokens, experts = logits.shape
    device = _on_gpu(logits, ids)
    seg_offsets, table, nchunks = segment_tables(lengths, tokens, device)
    segments = max(1, len(tuple(lengths)))
    aux = torch.empty((), dtype=torch.float32, device=device)
    prob_sum = torch.empty(experts, dtype=torch.float32, device=device)
    seg_counts = torch.empty((segments, experts), dtype=torch.int32, device=device)
    size = _native.query("mi355x_router_stats_workspace_size", nchunks, experts)
    workspace = torch.empty(size, dtype=torch.uint8, device=device)
    # logits and ids read once; per-expert outputs are negligible
    nbytes = 4 * tokens * experts + 4 * ids.numel()
    _timed(
        "router_stats", device, 0, nbytes,
        "mi355x_router_stats", _ptr(logits), _ptr(ids), tokens, experts, int(top_k),
        ROUTING_MODES[mode], segments, _ptr(seg_offsets), _ptr(table), nchunks, _ptr(aux),
        _ptr(prob_sum), _ptr(seg_counts), _ptr(workspace), size, _stream(device),
    )
    return aux, prob_sum, seg_counts, seg_offsets


def router_backward(
    logits, weights, ids, dscore, slots, mode: str, *, grad_aux=None, grad_prob_sum=None,
    offsets=None, seg_offsets=None, seg_counts=None, pieces=False,
):
    """fp32 ``grad_logits [T,E]`` (route weights' cotangent = ``dscore[slots]``).
    With ``pieces=True``, instead the bf16 ``[T, 2E]`` buffer ``[hi | mid]``,
    ``hi = bf16(g)``, ``mid = bf16(g - hi)`` (``mi355x_router_topk_bwd_split``)."""
    tokens, experts = logits.shape
    top_k = ids.shape[1]
    if grad_aux is not None:
        grad_aux = grad_aux.float().reshape(1).contiguous()
    if grad_prob_sum is not None:
        grad_prob_sum = grad_prob_sum.float().contiguous()
    device = _on_gpu(logits, weights, ids, dscore, slots, grad_aux, grad_prob_sum, offsets,
                     seg_offsets, seg_counts)
    segments = 1 if seg_counts is None else seg_counts.shape[0]
    if pieces:
        out = torch.empty((tokens, 2 * experts), dtype=torch.bfloat16, device=device)
        # logits read, both bf16 pieces written; weights, ids and dscore read
        _timed(
            "router_topk_bwd", device, 0, 8 * tokens * experts + 12 * tokens * top_k,
            "mi355x_router_topk_bwd_split", _ptr(logits), _ptr(weights), _ptr(ids), _ptr(dscore),
            _ptr(slots), tokens, experts, top_k, ROUTING_MODES[mode], _ptr(grad_aux),
            _ptr(grad_prob_sum), _ptr(offsets), segments, _ptr(seg_offsets), _ptr(seg_counts),
            None, _ptr(out), _stream(device),
        )
        return out
    grad = torch.empty((tokens, experts), dtype=torch.float32, device=device)
    # logits read and their gradient written; weights, ids and dscore read
    nbytes = 8 * tokens * experts + 12 * tokens * top_k
    _timed(
        "router_topk_bwd", device, 0, nbytes,
        "mi355x_router_topk_bwd", _ptr(logits), _ptr(weights), _ptr(ids), _ptr(dscore),
        _ptr(slots), tokens, experts, top_k, ROUTING_MODES[mode], _ptr(grad_aux),
        _ptr(grad_prob_sum), _ptr(offsets), segments, _ptr(seg_offsets), _ptr(seg_counts),
        _ptr(grad), _stream(device),
    )
    return grad


def router_weight_grad(pieces: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """fp32 ``[E, H]`` = ``hi^T x + mid^T x`` from the bf16 pieces ``[T, 2E]``
    (``hi | mid``) and the bf16 hidden state ``x [T, H]``."""
    if pieces.dtype != torch.bfloat16 or x.dtype != torch.bfloat16:
        raise ValueError("router_weight_grad takes bf16 pieces and hidden state")
    device = _on_gpu(pieces, x)
    tokens, hidden = x.shape
    experts = pieces.shape[1] // 2
    if pieces.shape != (tokens, 2 * experts):
        raise ValueError("pieces must be [T, 2E] beside x [T, H]")
    pieces, x = pieces.contiguous(), x.contiguous()
    out = torch.empty((experts, hidden), dtype=torch.float32, device=device)
    size = _native.query("mi355x_router_weight_grad_workspace_size", tokens, experts, hidden)
    ws = torch.empty(max(size, 4), dtype=torch.uint8, device=device)
    flops = 4 * tokens * experts * hidden
    # x and the pieces read once, the fp32 gradient written
    nbytes = 2 * tokens * hidden + 4 * tokens * experts + 4 * experts * hidden
    _timed("router_weight_grad", device, flops, nbytes, "mi355x_router_weight_grad",
           _ptr(pieces), _ptr(x), tokens, experts, hidden, _ptr(out), _ptr(ws), size,
           _stream(device))
    return out


# ----------------------------------------------------------------- permute
def permute_plan(ids: torch.Tensor, experts: int):
    """``(counts int64 [E], offsets int32 [E+1], order int32 [A], slots int32 [T,k])``."""
    if ids.dtype != torch.int32:
        raise ValueError("route ids must be int32")
    device = _on_gpu(ids)
    n = ids.numel()
    counts = torch.empty(experts, dtype=torch.int64, device=device)
    offsets = torch.empty(experts + 1, dtype=torch.int32, device=device)
    order = torch.empty(n, dtype=torch.int32, device=device)
    slots = torch.empty(ids.shape, dtype=torch.int32, device=device)
    size = _native.query("mi355x_permute_plan_workspace_size", n, experts)
    workspace = torch.empty(size, dtype=torch.uint8, device=device)
    # ids read, order and slots written (counts / offsets are per expert)
    _timed(
        "permute_plan", device, 0, 12 * n + 12 * experts,
        "mi355x_permute_plan", _ptr(ids), n, int(experts), _ptr(counts), _ptr(offsets),
        _ptr(order), _ptr(slots), _ptr(workspace), size, _stream(device),
    )
    return counts, offsets, order, slots


def permute_quantize(x: torch.Tensor, slots: torch.Tensor):
    """Each token of ``x bf16 [T,H]`` quantized once and written to its k
    routed rows: ``(q e4m3 [A,H], scales fp32 [H/128, A])``."""
    if x.dtype != torch.bfloat16 or x.ndim != 2:
        raise ValueError("permute_quantize takes bf16 [tokens, width]")
    tokens, width = x.shape
    top_k = slots.shape[1]
    _check(slots, (tokens, top_k), torch.int32, "slots")
    device = _on_gpu(x, slots)
    rows = tokens * top_k
    q = torch.empty((rows, width), dtype=FP8, device=device)
    scales = torch.empty((width // 128, rows), dtype=torch.float32, device=device)
    nbytes = 2 * tokens * width + rows * width + 4 * rows * (width // 128) + 4 * rows
    _timed("permute_quantize_fp8", device, 0, nbytes, "mi355x_permute_quantize_fp8", _ptr(x),
           tokens, width, top_k, _ptr(slots), _ptr(q), _ptr(scales), _stream(device))
    return q, scales


def quantize_rows(x: torch.Tensor, *, gate_up: bool = False):
    """Rows ``bf16 [R,W]`` -> ``(e4m3 [R,W], scales [W/128, R])``; ``gate_up``
    stores an interleaved gate/up row as gate columns then up columns."""
    if x.dtype != torch.bfloat16 or x.ndim != 2:
        raise ValueError("quantize_rows takes bf16 [rows, width]")
    rows, width = x.shape
    device = _on_gpu(x)
    q = torch.empty((rows, width), dtype=FP8, device=device)
    scales = torch.empty((width // 128, rows), dtype=torch.float32, device=device)
    nbytes = 2 * rows * width + rows * width + 4 * rows * (width // 128)
    _timed("quantize_rows_fp8", device, 0, nbytes, "mi355x_quantize_rows_fp8", _ptr(x), rows,
           width, width, int(gate_up), _ptr(q), _ptr(scales), _stream(device))
    return q, scales


def swiglu_quantize(h: torch.Tensor, limit: float | None = None, *, activation: bool = False):
    """``silu(gate) * up`` of interleaved ``h [R, 2I]`` as ``(e4m3 [R,I], scales [I/128, R])``,
    followed by the bf16 activation ``[R, I]`` itself when ``activation``."""
    if h.dtype != torch.bfloat16 or h.ndim != 2 or h.shape[1] % 2:
        raise ValueError("swiglu_quantize takes bf16 [rows, 2I]")
    rows, width = h.shape[0], h.shape[1] // 2
    device = _on_gpu(h)
    q = torch.empty((rows, width), dtype=FP8, device=device)
    scales = torch.empty((width // 128, rows), dtype=torch.float32, device=device)
    act = torch.empty((rows, width), dtype=torch.bfloat16, device=device) if activation else None
    nbytes = 4 * rows * width + rows * width + 4 * rows * (width // 128)
    if activation:
        nbytes += 2 * rows * width
    _timed("swiglu_quantize_fp8", device, 0, nbytes, "mi355x_swiglu_quantize_fp8", _ptr(h), rows,
           width, _limit(limit), _ptr(q), _ptr(scales), _ptr(act), _stream(device))
    return (q, scales, act) if activation else (q, scales)


def quantize_weight_blocks(w: torch.Tensor, *, transposed: bool = False):
    """``(data e4m3 [E,out,in], scale fp32 [E,ceil(out/128),ceil(in/128)][, data_t])``."""
    if w.ndim != 3 or w.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("quantize_weight_blocks takes bf16/fp32 [experts, out, in]")
    w = w.contiguous()
    device = _on_gpu(w)
    experts, out, inner = w.shape
    data = torch.empty(w.shape, dtype=FP8, device=device)
    scale = torch.empty((experts, -(-out // 128), -(-inner // 128)), dtype=torch.float32,
                        device=device)
    data_t = torch.empty((experts, inner, out), dtype=FP8, device=device) if transposed else None
    # the weight read once; e4m3 data (and its transpose) and the block scales written
    nbytes = w.numel() * w.element_size() + w.numel() * (2 if transposed else 1) + scale.numel() * 4
    _timed("quantize_weight_blocks", device, 0, nbytes, "mi355x_quantize_weight_blocks", _ptr(w),
           int(w.dtype == torch.float32), experts, out, inner, _ptr(data), _ptr(scale),
           _ptr(data_t), _stream(device))
    return (data, scale, data_t) if transposed else (data, scale)


def transpose_fp8(data: torch.Tensor) -> torch.Tensor:
    """e4m3 ``[E,R,C]`` -> ``[E,C,R]``."""
    if data.dtype != FP8 or data.ndim != 3:
        raise ValueError("transpose_fp8 takes e4m3 [E, R, C]")
    device = _on_gpu(data)
    experts, rows, cols = data.shape
    out = torch.empty((experts, cols, rows), dtype=FP8, device=device)
    _timed("transpose_fp8", device, 0, 2 * data.numel(), "mi355x_transpose_fp8", _ptr(data),
           experts, rows, cols, _ptr(out), _stream(device))
    return out


def wgrad_padded_rows(assignments: int, experts: int) -> int:
    return _native.query("mi355x_wgrad_padded_rows", int(assignments), int(experts))


def padded_row_blocks(offsets: torch.Tensor, padded: int) -> torch.Tensor:
    """int32 ``[padded/128, 2]``: (first sorted row, valid rows) of each padded
    128-row block of the weight-gradient layout."""
    experts = offsets.numel() - 1
    device = _on_gpu(offsets)
    blocks = torch.empty((padded // 128, 2), dtype=torch.int32, device=device)
    _native.call("mi355x_padded_row_blocks", _ptr(offsets), experts, int(padded), _ptr(blocks),
                 _stream(device))
    return blocks


def quantize_transpose(
    x: torch.Tensor, offsets: torch.Tensor, assignments: int, *, gather=None,
    gather_div: int = 1, gate_up: bool = False, padded: int | None = None, row_blocks=None,
):
    """Feature-major e4m3 wgrad operand of the routed rows of ``x``:
    ``(qt [W, P], scales [P/128, W], P)``, each expert's rows at its
    128-aligned padded offset (zeros between); the scales are powers of two.
    ``row_blocks`` (from :func:`padded_row_blocks`, same ``P``) may be passed
    to share it between calls."""
    if x.dtype != torch.bfloat16 or x.ndim != 2:
        raise ValueError("quantize_transpose takes bf16 [rows, width]")
    width = x.shape[1]
    experts = offsets.numel() - 1
    device = _on_gpu(x, offsets, gather)
    if padded is None:
        padded = wgrad_padded_rows(assignments, experts)
    if row_blocks is None:
        row_blocks = padded_row_blocks(offsets, padded)
    _check(row_blocks, (padded // 128, 2), torch.int32, "row_blocks")
    qt = torch.empty((width, padded), dtype=FP8, device=device)
    scales = torch.empty((padded // 128, width), dtype=torch.float32, device=device)
    if assignments > 0:
        # the routed bf16 rows read once (gathered or not), e4m3 [W, P] and the
        # per-(feature, 128-row block) scales written
        nbytes = 2 * assignments * width + width * padded + 4 * width * (padded // 128)
        _timed(
            "quantize_transpose_fp8", device, 0, nbytes,
            "mi355x_quantize_transpose_fp8", _ptr(x), x.stride(0), width, _ptr(gather),
            int(gather_div), int(gate_up), _ptr(row_blocks), int(padded), _ptr(qt), _ptr(scales),
            _stream(device),
        )
    return qt, scales, padded


def combine(y, slots, weights, residual):
    """``residual[t] + sum_j weights[t,j] * y[slots[t,j]]`` in fp32, rounded once."""
    tokens, top_k = slots.shape
    width = y.shape[1]
    _check(weights, (tokens, top_k), torch.float32, "route weights")
    _check(residual, (tokens, width), torch.bfloat16, "residual")
    device = _on_gpu(y, slots, weights, residual)
    out = torch.empty_like(residual)
    nbytes = 2 * tokens * top_k * width + 8 * tokens * top_k + 4 * tokens * width
    _timed("unpermute_combine", device, 0, nbytes, "mi355x_unpermute_combine", _ptr(y), _ptr(slots),
           _ptr(weights), _ptr(residual), tokens, top_k, width, _ptr(out), _stream(device))
    return out


def unpermute_sum(dx, slots):
    """``sum_j dx[slots[t,j]]`` per token, bf16."""
    tokens, top_k = slots.shape
    width = dx.shape[1]
    device = _on_gpu(dx, slots)
    out = torch.empty((tokens, width), dtype=dx.dtype, device=device)
    nbytes = 2 * tokens * top_k * width + 4 * tokens * top_k + 2 * tokens * width
    _timed("unpermute_sum", device, 0, nbytes, "mi355x_unpermute_sum", _ptr(dx), _ptr(slots),
           tokens, top_k, width, _ptr(out), _stream(device))
    return out


def routed_swiglu_backward(r, h, weights, order, limit=None, *, dh_out=None, a_prime=True):
    """``(dh [A,2I] interleaved, a' [A,I], dscore fp32 [A])``. ``dh`` is written
    into ``dh_out`` when given, which may be ``h`` itself (in place); with
    ``a_prime=False`` a' is not written and ``None`` is returned for it."""
    rows, width = r.shape
    _check(h, (rows, 2 * width), torch.bfloat16, "h")
    device = _on_gpu(r, h, weights, order, dh_out)
    if dh_out is not None:
        _check(dh_out, (rows, 2 * width), torch.bfloat16, "dh_out")
        if not dh_out.is_contiguous():
            raise ValueError("dh_out must be contiguous")
    dh = torch.empty_like(h) if dh_out is None else dh_out
    a_prime = torch.empty_like(r) if a_prime else None
    dscore = torch.empty(rows, dtype=torch.float32, device=device)
    # r and h read; dh, a' (when asked) and dscore written
    nbytes = (6 + 4 + (2 if a_prime is not None else 0)) * rows * width + 8 * rows
    _timed("routed_swiglu_bwd", device, 0, nbytes, "mi355x_routed_swiglu_bwd", _ptr(r), _ptr(h),
           _ptr(weights), _ptr(order), rows, width, _limit(limit), _ptr(dh), _ptr(a_prime),
           _ptr(dscore), _stream(device))
    return dh, a_prime, dscore


def routed_swiglu_backward_rows(r, h, weights, order, limit=None, *, a_prime=True):
    """``routed_swiglu_backward`` plus dh row-quantized gate-first from its
    bf16 values: ``(dh, a', dscore, dhq e4m3 [A, 2I], dh_scales [2I/128, A])``,
    the last two equal to ``quantize_rows(dh, gate_up=True)``; a' is ``None``
    (not written) with ``a_prime=False``."""
    rows, width = r.shape
    _check(h, (rows, 2 * width), torch.bfloat16, "h")
    device = _on_gpu(r, h, weights, order)
    dh = torch.empty_like(h)
    a_prime = torch.empty_like(r) if a_prime else None
    dscore = torch.empty(rows, dtype=torch.float32, device=device)
    dhq = torch.empty((rows, 2 * width), dtype=FP8, device=device)
    dhs = torch.empty((2 * width // 128, rows), dtype=torch.float32, device=device)
    # r and h read; dh, a', dscore, dhq and its scales written
    nbytes = ((12 + (2 if a_prime is not None else 0)) * rows * width + 8 * rows
              + 4 * rows * (2 * width // 128))
    _timed("routed_swiglu_bwd_rows", device, 0, nbytes, "mi355x_routed_swiglu_bwd_rows_fp8",
           _ptr(r), _ptr(h), _ptr(weights), _ptr(order), rows, width, _limit(limit), _ptr(dh),
           _ptr(a_prime), _ptr(dscore), _ptr(dhq), _ptr(dhs), _stream(device))
    return dh, a_prime, dscore, dhq, dhs


def swiglu_bwd_quantize(r, h, weights, order, offsets, *, padded=None, limit=None,
                        transposed_dh=True, transposed_ap=True, row_blocks=None):
    """Fused routed SwiGLU backward + quantizers (see the C header):
    ``(dhq [A,2I] e4m3 gate-first, dh_scales [2I/128, A], dh_t [2I, P] | None,
    dh_t_scales [P/128, 2I] | None, ap_t [I, P] | None, ap_t_scales [P/128, I]
    | None, dscore fp32 [A], P)``."""
    rows, width = r.shape
    _check(h, (rows, 2 * width), torch.bfloat16, "h")
    experts = offsets.numel() - 1
    device = _on_gpu(r, h, weights, order, offsets)
    if padded is None:
        padded = wgrad_padded_rows(rows, experts)
    if row_blocks is None:
        row_blocks = padded_row_blocks(offsets, padded)
    _check(row_blocks, (padded // 128, 2), torch.int32, "row_blocks")
    dhq = torch.empty((rows, 2 * width), dtype=FP8, device=device)
    dhs = torch.empty((2 * width // 128, rows), dtype=torch.float32, device=device)
    dht = dhts = apt = apts = None
    if transposed_dh:
        dht = torch.empty((2 * width, padded), dtype=FP8, device=device)
        dhts = torch.empty((padded // 128, 2 * width), dtype=torch.float32, device=device)
    if transposed_ap:
        apt = torch.empty((width, padded), dtype=FP8, device=device)
        apts = torch.empty((padded // 128, width), dtype=torch.float32, device=device)
    dscore = torch.empty(rows, dtype=torch.float32, device=device)
    nbytes = _native.query("mi355x_swiglu_bwd_quantize_workspace_size", rows, width)
    work = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    traffic = 6 * rows * width + 2 * rows * width + (3 * width * padded if rows else 0)
    _timed("swiglu_bwd_quantize", device, 0, traffic, "mi355x_swiglu_bwd_quantize", _ptr(r),
           _ptr(h), _ptr(weights), _ptr(order), _ptr(row_blocks), rows, width, int(padded),
           _limit(limit), _ptr(dhq), _ptr(dhs), _ptr(dht), _ptr(dhts), _ptr(apt), _ptr(apts),
           _ptr(dscore), _ptr(work), nbytes, _stream(device))
    return dhq, dhs, dht, dhts, apt, apts, dscore, padded


def swiglu_bwd_bf16(r, h, weights, order, offsets, *, padded, row_blocks, limit=None,
                    transposed_dh=True, transposed_ap=True):
    """The fused routed SwiGLU backward with bf16 ``dh [A, 2I]`` (h's
    interleaved order) and the transposed operands of the weight gradients
    (``mi355x_swiglu_bwd_bf16``): ``(dh, dh_t [2I, P], dh_t_scales [P/128, 2I],
    ap_t [I, P], ap_t_scales [P/128, I], dscore fp32 [A])``; ``dh_t`` (for
    dW13) and ``ap_t`` (for dW2) are skipped, and None, when not asked for."""
    rows, width = r.shape
    _check(h, (rows, 2 * width), torch.bfloat16, "h")
    device = _on_gpu(r, h, weights, order, offsets)
    _check(row_blocks, (padded // 128, 2), torch.int32, "row_blocks")
    dh = torch.empty((rows, 2 * width), dtype=torch.bfloat16, device=device)
    dht = dhts = apt = apts = None
    if transposed_dh:
        dht = torch.empty((2 * width, padded), dtype=FP8, device=device)
        dhts = torch.empty((padded // 128, 2 * width), dtype=torch.float32, device=device)
    if transposed_ap:
        apt = torch.empty((width, padded), dtype=FP8, device=device)
        apts = torch.empty((padded // 128, width), dtype=torch.float32, device=device)
    dscore = torch.empty(rows, dtype=torch.float32, device=device)
    nbytes = _native.query("mi355x_swiglu_bwd_quantize_workspace_size", rows, width)
    work = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    written_t = (2 * transposed_dh + transposed_ap) * width * padded if rows else 0
    traffic = 6 * rows * width + 4 * rows * width + written_t
    _timed("swiglu_bwd_bf16", device, 0, traffic, "mi355x_swiglu_bwd_bf16", _ptr(r), _ptr(h),
           _ptr(weights), _ptr(order), _ptr(row_blocks), rows, width, int(padded), _limit(limit),
           _ptr(dh), _ptr(dht), _ptr(dhts), _ptr(apt), _ptr(apts), _ptr(dscore), _ptr(work),
           nbytes, _stream(device))
    return dh, dht, dhts, apt, apts, dscore


# ------------------------------------------------------------------- GEMMs
def gemm(a, a_scale, w, w_scale, offsets, *, transposed_scale=False, interleave=False,
         addend=None, lora=None):
    """Grouped block-FP8 GEMM: bf16 ``[A, N]`` (see the C header for the math).
    ``lora = (z bf16 [A, R], b bf16 [E, N, R])``, R a multiple of 16: the
    rank-R term ``z b[e]^T`` joins the accumulators (``mi355x_gemm_fp8_block_lora``)."""
    if lora is not None:
        return _gemm_lora(a, a_scale, w, w_scale, offsets, transposed_scale, interleave, *lora)
    rows, k = a.shape
    experts, n, wk = w.shape
    if a.dtype != FP8 or w.dtype != FP8 or wk != k:
        raise ValueError("gemm takes e4m3 rows [A,K] and e4m3 weights [E,N,K]")
    _check(a_scale, (k // 128, rows), torch.float32, "row scales")
    expected = (experts, k // 128, n // 128) if transposed_scale else (experts, n // 128, k // 128)
    _check(w_scale, expected, torch.float32, "weight scales")
    _check(offsets, (experts + 1,), torch.int32, "offsets")
    if addend is not None:
        _check(addend, (rows, n), torch.bfloat16, "addend")
    device = _on_gpu(a, a_scale, w, w_scale, offsets, addend)
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=device)
    _timed(
        "gemm_fp8_block", device, 2 * rows * n * k, rows * k + experts * n * k + 2 * rows * n,
        "mi355x_gemm_fp8_block", _ptr(a), _ptr(a_scale), rows, _ptr(w), _ptr(w_scale),
        int(transposed_scale), experts, n, k, _ptr(offsets), int(interleave), _ptr(addend),
        _ptr(out), _stream(device),
    )
    return out


def gemm_kmajor(a, a_scale, w, w_scale, offsets):
    """Input-gradient GEMM on a weight as stored: ``a [A, K] @ w[e]`` for
    e4m3 ``w [E, K, N]`` with its own scales ``[E, K/128, N/128]``, bf16
    ``[A, N]`` (``mi355x_gemm_fp8_block_kmajor``); bitwise the same as
    :func:`gemm` on the transposed copy with ``transposed_scale=True``."""
    rows, k = a.shape
    experts, wk, n = w.shape
    if a.dtype != FP8 or w.dtype != FP8 or wk != k:
        raise ValueError("gemm_kmajor takes e4m3 rows [A,K] and an e4m3 weight [E,K,N]")
    _check(a_scale, (k // 128, rows), torch.float32, "row scales")
    _check(w_scale, (experts, k // 128, n // 128), torch.float32, "weight scales")
    _check(offsets, (experts + 1,), torch.int32, "offsets")
    if not w.is_contiguous():
        raise ValueError("gemm_kmajor: the weight must be contiguous")
    device = _on_gpu(a, a_scale, w, w_scale, offsets)
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=device)
    _timed(
        "gemm_fp8_block", device, 2 * rows * n * k, rows * k + experts * n * k + 2 * rows * n,
        "mi355x_gemm_fp8_block_kmajor", _ptr(a), _ptr(a_scale), rows, _ptr(w), _ptr(w_scale),
        experts, n, k, _ptr(offsets), _ptr(out), _stream(device),
    )
    return out


def quantize_token_rows(x: torch.Tensor):
    """Token rows ``bf16 [T, W]`` -> ``(e4m3 [T, W], scales [T, W/128])`` for
    :func:`gemm_gathered`: :func:`quantize_rows`' values, scales row-major."""
    if x.dtype != torch.bfloat16 or x.ndim != 2:
        raise ValueError("quantize_token_rows takes bf16 [rows, width]")
    x = x.contiguous()
    rows, width = x.shape
    device = _on_gpu(x)
    q = torch.empty((rows, width), dtype=FP8, device=device)
    scales = torch.empty((rows, width // 128), dtype=torch.float32, device=device)
    nbytes = 2 * rows * width + rows * width + 4 * rows * (width // 128)
    _timed("quantize_rows_fp8", device, 0, nbytes, "mi355x_quantize_token_rows_fp8", _ptr(x), rows,
           width, _ptr(q), _ptr(scales), _stream(device))
    return q, scales


def gemm_gathered(a, a_scale, a_rows, w, w_scale, offsets, *, interleave=False, kmajor=False,
                  rows_div=1):
    """:func:`gemm` (``kmajor=False``, ``w [E, N, K]`` with scales ``[E, N/128,
    K/128]``) or :func:`gemm_kmajor` (``w [E, K, N]``) whose GEMM row r is row
    ``a_rows[r] // rows_div`` of ``a [T, K]`` (``rows_div = top_k`` reads the
    plan's sorted slot order directly), token-major scales ``a_scale [T, K/128]``
    (:func:`quantize_token_rows`): the
    activation quantized once per token and read by each of its routed rows
    (``mi355x_gemm_fp8_block_gathered`` / ``_kmajor_gathered``). Bitwise the
    same as the routed-row forms on the permuted copy."""
    tokens, k = a.shape
    rows = a_rows.shape[0]
    if kmajor:
        experts, wk, n = w.shape
        wscale = (experts, k // 128, n // 128)
    else:
        experts, n, wk = w.shape
        wscale = (experts, n // 128, k // 128)
    if a.dtype != FP8 or w.dtype != FP8 or wk != k:
        raise ValueError("gemm_gathered takes e4m3 token rows [T,K] and an e4m3 weight")
    _check(a_scale, (tokens, k // 128), torch.float32, "token row scales")
    _check(a_rows, (rows,), torch.int32, "a_rows")
    _check(w_scale, wscale, torch.float32, "weight scales")
    _check(offsets, (experts + 1,), torch.int32, "offsets")
    if not w.is_contiguous():
        raise ValueError("gemm_gathered: the weight must be contiguous")
    device = _on_gpu(a, a_scale, a_rows, w, w_scale, offsets)
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=device)
    if kmajor:
        _timed("gemm_fp8_block", device, 2 * rows * n * k, rows * k + experts * n * k + 2 * rows * n,
               "mi355x_gemm_fp8_block_kmajor_gathered", _ptr(a), _ptr(a_scale), tokens,
               _ptr(a_rows), int(rows_div), rows, _ptr(w), _ptr(w_scale), experts, n, k, _ptr(offsets),
               _ptr(out), _stream(device))
    else:
        _timed("gemm_fp8_block", device, 2 * rows * n * k, rows * k + experts * n * k + 2 * rows * n,
               "mi355x_gemm_fp8_block_gathered", _ptr(a), _ptr(a_scale), tokens, _ptr(a_rows),
               int(rows_div), rows, _ptr(w), _ptr(w_scale), experts, n, k, _ptr(offsets), int(interleave),
               _ptr(out), _stream(device))
    return out


def rank_product(a, bt, offsets, *, splits=None):
    """``out[r] = a[r] @ bt[e]^T`` for the rows of each expert: bf16 ``[rows, R]``
    from bf16 ``a [rows, K]`` and ``bt [E, R, K]`` (``mi355x_rank_product``).
    ``splits`` divides K over several blocks per 32-row block (fp32 partials
    added in order; ``mi355x_rank_product_split``); by default enough splits
    for ~4 blocks per CU."""
    rows, k = a.shape
    experts, rank, bk = bt.shape
    if a.dtype != torch.bfloat16 or bt.dtype != torch.bfloat16 or bk != k:
        raise ValueError("rank_product takes bf16 a [rows, K] and bt [E, R, K]")
    _check(offsets, (experts + 1,), torch.int32, "offsets")
    device = _on_gpu(a, bt, offsets)
    out = torch.empty((rows, rank), dtype=torch.bfloat16, device=device)
    nbytes = 2 * rows * k + 2 * rows * rank
    if splits is None:
        blocks = -(-rows // 64)  # 64-row blocks of the staged kernel
        splits = 1
        if k % 128 == 0 and blocks:
            splits = max(1, min(k // 128, 8, -(-4 * _cu_count(device) // blocks)))
    if splits == 1:
        _timed("rank_product", device, 0, nbytes, "mi355x_rank_product", _ptr(a), rows, k,
               _ptr(bt), rank, _ptr(offsets), experts, _ptr(out), _stream(device))
        return out
    size = _native.query("mi355x_rank_product_workspace_size", rows, rank, splits)
    workspace = torch.empty(size, dtype=torch.uint8, device=device)
    _timed("rank_product", device, 0, nbytes, "mi355x_rank_product_split", _ptr(a), rows, k,
           _ptr(bt), rank, _ptr(offsets), experts, int(splits), _ptr(out), _ptr(workspace), size,
           _stream(device))
    return out


def rank_grad(big, small, offsets, *, transposed=False, chunk=None, gather=None, gather_div=1,
              weight=None, weight_index=None, alpha=1.0):
    """Per expert ``sum_j big[j]^T small[j]`` over its rows: fp32 ``[E, M, R]``
    (``[E, R, M]`` when ``transposed``) from bf16 ``big [rows, M]`` and ``small
    [rows, R]`` (``mi355x_rank_grad``; R a multiple of 16, at most 64).

    With ``gather`` (int32 ``[rows]``), row j of ``big [tokens, M]`` is
    ``big[gather[j] // gather_div]``; with ``weight`` (fp32), row j of
    ``small`` is ``bf16(small[j] * (weight[i] * alpha))``, i = ``weight_index[j]``
    (or j) (``mi355x_rank_grad_gather``)."""
    big_rows, m = big.shape
    rows, rank = small.shape
    experts = offsets.numel() - 1
    if big.dtype != torch.bfloat16 or small.dtype != torch.bfloat16:
        raise ValueError("rank_grad takes bf16 operands")
    plain = gather is None and weight is None
    if gather is None:
        _check(small, (big_rows, rank), torch.bfloat16, "rank operand")
    else:
        _check(gather, (rows,), torch.int32, "gather index")
    if weight is not None and (weight.dtype != torch.float32 or not weight.is_contiguous()):
        raise ValueError("rank_grad: the row weight must be contiguous fp32")
    if weight_index is not None:
        _check(weight_index, (rows,), torch.int32, "weight index")
    if not plain and (not big.is_contiguous() or not small.is_contiguous()):
        raise ValueError("rank_grad: operands must be contiguous")
    _check(offsets, (experts + 1,), torch.int32, "offsets")
    device = _on_gpu(big, small, offsets,
                     *(t for t in (gather, weight, weight_index) if t is not None))
    if chunk is None:
        # Enough (chunk x 256-column) blocks to fill the chip twice over.
        blocks_per_chunk = -(-m // 256) * (rank // 16)
        chunk = 256
        while chunk < 4096 and (rows // (2 * chunk)) * blocks_per_chunk >= 512:
            chunk *= 2
    out_shape = (experts, rank, m) if transposed else (experts, m, rank)
    out = torch.empty(out_shape, dtype=torch.float32, device=device)
    size = _native.query("mi355x_rank_grad_workspace_size", rows, experts, m, rank, chunk)
    workspace = torch.empty(size, dtype=torch.uint8, device=device)
    # HBM-bound: big is streamed once; the products are on the bf16 MFMA
    nbytes = 2 * rows * (m + rank) + 4 * experts * m * rank
    if plain:
        _timed("rank_grad", device, 0, nbytes, "mi355x_rank_grad", _ptr(big), rows, m,
               _ptr(small), rank, _ptr(offsets), experts, chunk, int(transposed), _ptr(out),
               _ptr(workspace), size, _stream(device))
    else:
        _timed("rank_grad", device, 0, nbytes + 4 * rows, "mi355x_rank_grad_gather", _ptr(big),
               big_rows, m, _ptr(small), rows, rank, _ptr(offsets), experts, chunk,
               _ptr(gather), int(gather_div), _ptr(weight), _ptr(weight_index), float(alpha),
               int(transposed), _ptr(out), _ptr(workspace), size, _stream(device))
    return out


def _gemm_lora(a, a_scale, w, w_scale, offsets, transposed_scale, interleave, z, b):
    rows, k = a.shape
    experts, n, wk = w.shape
    if a.dtype != FP8 or w.dtype != FP8 or wk != k:
        raise ValueError("gemm takes e4m3 rows [A,K] and e4m3 weights [E,N,K]")
    _check(a_scale, (k // 128, rows), torch.float32, "row scales")
    expected = (experts, k // 128, n // 128) if transposed_scale else (experts, n // 128, k // 128)
    _check(w_scale, expected, torch.float32, "weight scales")
    _check(offsets, (experts + 1,), torch.int32, "offsets")
    rank = z.shape[1] if z.ndim == 2 else -1
    _check(z, (rows, rank), torch.bfloat16, "LoRA z")
    _check(b, (experts, n, rank), torch.bfloat16, "LoRA b")
    device = _on_gpu(a, a_scale, w, w_scale, offsets, z, b)
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=device)
    _timed(
        "gemm_fp8_block", device, 2 * rows * n * k, rows * k + experts * n * k + 2 * rows * n,
        "mi355x_gemm_fp8_block_lora", _ptr(a), _ptr(a_scale), rows, _ptr(w), _ptr(w_scale),
        int(transposed_scale), experts, n, k, _ptr(offsets), int(interleave), _ptr(z), _ptr(b),
        rank, _ptr(out), _stream(device),
    )
    return out


def gemm_swiglu(a, a_scale, w, w_scale, offsets, *, limit=None, addend=None):
    """Up projection with SwiGLU fused: ``(h bf16 [A, 2I] interleaved, act e4m3
    [A, I], act_scales [I/128, A])``; ``act`` equals :func:`swiglu_quantize` of
    ``h`` bit for bit."""
    rows, k = a.shape
    experts, n, kw = w.shape
    if kw != k:
        raise ValueError(f"weight K {kw} != activation K {k}")
    _check(a_scale, (k // 128, rows), torch.float32, "activation scales")
    device = _on_gpu(a, a_scale, w, w_scale, offsets, addend)
    h = torch.empty((rows, n), dtype=torch.bfloat16, device=device)
    act = torch.empty((rows, n // 2), dtype=FP8, device=device)
    act_scales = torch.empty((n // 256, rows), dtype=torch.float32, device=device)
    _timed(
        "gemm_fp8_block", device, 2 * rows * n * k, rows * k + experts * n * k + 2 * rows * n,
        "mi355x_gemm_fp8_block_swiglu", _ptr(a), _ptr(a_scale), rows, _ptr(w), _ptr(w_scale),
        experts, n, k, _ptr(offsets), _ptr(addend), _limit(limit), _ptr(h), _ptr(act),
        _ptr(act_scales), _stream(device),
    )
    return h, act, act_scales


# ---------------------------------------------------------------- fp8_current
def quantize_rows_current(x: torch.Tensor, *, gather=None, gather_div: int = 1):
    """Per-row e4m3 ``(q [R, W], scales fp32 [R])`` of bf16 ``x`` rows, or of
    the rows ``x[gather[r] // gather_div]`` when ``gather`` is given
    (``mi355x_quantize_rows_current_fp8``)."""
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("quantize_rows_current takes bf16 [rows, width] with unit column stride")
    rows = x.shape[0] if gather is None else gather.numel()
    width = x.shape[1]
    if gather is not None and gather.dtype != torch.int32:
        raise ValueError("gather must be int32")
    device = _on_gpu(x, gather)
    q = torch.empty((rows, width), dtype=FP8, device=device)
    scales = torch.empty(rows, dtype=torch.float32, device=device)
    _native.call("mi355x_quantize_rows_current_fp8", _ptr(x), rows, width, x.stride(0),
                 _ptr(gather), int(gather_div), _ptr(q), _ptr(scales), _stream(device))
    return q, scales


def permute_quantize_current(x: torch.Tensor, slots: torch.Tensor):
    """Per-row e4m3 of the routed copies of token rows: ``(q [T*k, W], scales
    [T*k])`` with row ``slots[t, j]`` = token ``t`` quantized
    (``mi355x_permute_quantize_current_fp8``)."""
    if x.dtype != torch.bfloat16 or x.ndim != 2 or not x.is_contiguous():
        raise ValueError("permute_quantize_current takes contiguous bf16 [tokens, width]")
    tokens, width = x.shape
    if slots.ndim != 2 or slots.shape[0] != tokens or slots.dtype != torch.int32:
        raise ValueError("slots must be int32 [tokens, top_k]")
    top_k = slots.shape[1]
    device = _on_gpu(x, slots)
    q = torch.empty((tokens * top_k, width), dtype=FP8, device=device)
    scales = torch.empty(tokens * top_k, dtype=torch.float32, device=device)
    _native.call("mi355x_permute_quantize_current_fp8", _ptr(x), tokens, width, top_k,
                 _ptr(slots), _ptr(q), _ptr(scales), _stream(device))
    return q, scales


def swiglu_quantize_rows_current(h: torch.Tensor, limit: float | None = None, *,
                                 activation: bool = False):
    """SwiGLU of interleaved bf16 ``h [R, 2I]`` quantized per row:
    ``(q [R, I], scales fp32 [R])``, plus the bf16 activation ``[R, I]`` when
    ``activation`` (``mi355x_swiglu_quantize_rows_current_fp8``)."""
    if h.dtype != torch.bfloat16 or h.ndim != 2 or not h.is_contiguous():
        raise ValueError("swiglu_quantize_rows_current takes contiguous bf16 [rows, 2I]")
    rows, width = h.shape[0], h.shape[1] // 2
    device = _on_gpu(h)
    q = torch.empty((rows, width), dtype=FP8, device=device)
    scales = torch.empty(rows, dtype=torch.float32, device=device)
    act = torch.empty((rows, width), dtype=torch.bfloat16, device=device) if activation else None
    _native.call("mi355x_swiglu_quantize_rows_current_fp8", _ptr(h), rows, width, _limit(limit),
                 _ptr(q), _ptr(scales), _ptr(act), _stream(device))
    return (q, scales, act) if activation else (q, scales)


def quantize_weights_current(w: torch.Tensor, *, interleaved: bool = False):
    """Both orientations of bf16/fp32 ``w [E, out, in]``, per-row scaled:
    ``(data [E,out,in], transposed [E,in,out], scale [E,out], transposed_scale
    [E,in])``, rows gate/up-adjacent when ``interleaved``
    (``mi355x_quantize_weights_current_fp8``)."""
    if w.ndim != 3 or w.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("quantize_weights_current takes bf16/fp32 [experts, out, in]")
    w = w.contiguous()
    device = _on_gpu(w)
    experts, out, inner = w.shape
    data = torch.empty(w.shape, dtype=FP8, device=device)
    transposed = torch.empty((experts, inner, out), dtype=FP8, device=device)
    scale = torch.empty((experts, out), dtype=torch.float32, device=device)
    transposed_scale = torch.empty((experts, inner), dtype=torch.float32, device=device)
    size = _native.query("mi355x_quantize_weights_current_workspace_size", experts, out, inner)
    workspace = torch.empty(size, dtype=torch.uint8, device=device)
    _native.call("mi355x_quantize_weights_current_fp8", _ptr(w), int(w.dtype == torch.float32),
                 experts, out, inner, int(interleaved), _ptr(data), _ptr(scale),
                 _ptr(transposed), _ptr(transposed_scale), _ptr(workspace), size,
                 _stream(device))
    return data, transposed, scale, transposed_scale


def gemm_rowwise(a, a_scale, w, w_scale, offsets, *, lora=None):
    """Row-scaled grouped e4m3 GEMM: bf16 ``out[r] = (a[r] @ w[e]^T) * a_scale[r]
    * w_scale[e]`` per expert (``mi355x_gemm_fp8_rowwise``). ``lora = (z bf16
    [A, R], b bf16 [E, N, R])``, R a multiple of 16, adds ``z b[e]^T``
    (``mi355x_gemm_fp8_rowwise_lora``)."""
    if lora is not None:
        return _gemm_rowwise_lora(a, a_scale, w, w_scale, offsets, *lora)
    rows, k = a.shape
    experts, n, wk = w.shape
    if a.dtype != FP8 or w.dtype != FP8 or wk != k:
        raise ValueError("gemm_rowwise takes e4m3 rows [A,K] and e4m3 weights [E,N,K]")
    _check(a_scale, (rows,), torch.float32, "row scales")
    _check(w_scale, (experts, n), torch.float32, "weight row scales")
    _check(offsets, (experts + 1,), torch.int32, "offsets")
    device = _on_gpu(a, a_scale, w, w_scale, offsets)
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=device)
    _timed(
        "gemm_fp8_rowwise", device, 2 * rows * n * k, rows * k + experts * n * k + 2 * rows * n,
        "mi355x_gemm_fp8_rowwise", _ptr(a), _ptr(a_scale), rows, _ptr(w), _ptr(w_scale),
        experts, n, k, _ptr(offsets), _ptr(out), _stream(device),
    )
    return out


def gemm_rowwise_gathered(a, a_scale, a_rows, w, w_scale, offsets, *, rows_div=1):
    """:func:`gemm_rowwise` whose row r is row ``a_rows[r] // rows_div`` of per-token
    ``a [T, K]`` with descales ``a_scale [T]`` (:func:`quantize_rows_current`
    on the token rows; ``mi355x_gemm_fp8_rowwise_gathered``). Bitwise the
    same as on the permuted copy."""
    tokens, k = a.shape
    rows = a_rows.shape[0]
    experts, n, wk = w.shape
    if a.dtype != FP8 or w.dtype != FP8 or wk != k:
        raise ValueError("gemm_rowwise_gathered takes e4m3 token rows [T,K] and weights [E,N,K]")
    _check(a_scale, (tokens,), torch.float32, "token row scales")
    _check(a_rows, (rows,), torch.int32, "a_rows")
    _check(w_scale, (experts, n), torch.float32, "weight row scales")
    _check(offsets, (experts + 1,), torch.int32, "offsets")
    device = _on_gpu(a, a_scale, a_rows, w, w_scale, offsets)
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=device)
    _timed(
        "gemm_fp8_rowwise", device, 2 * rows * n * k, rows * k + experts * n * k + 2 * rows * n,
        "mi355x_gemm_fp8_rowwise_gathered", _ptr(a), _ptr(a_scale), tokens, _ptr(a_rows),
        int(rows_div), rows,
        _ptr(w), _ptr(w_scale), experts, n, k, _ptr(offsets), _ptr(out), _stream(device),
    )
    return out


def _gemm_rowwise_lora(a, a_scale, w, w_scale, offsets, z, b):
    rows, k = a.shape
    experts, n, wk = w.shape
    rank = z.shape[1] if z.ndim == 2 else -1
    if a.dtype != FP8 or w.dtype != FP8 or wk != k:
        raise ValueError("gemm_rowwise takes e4m3 rows [A,K] and e4m3 weights [E,N,K]")
    _check(a_scale, (rows,), torch.float32, "row scales")
    _check(w_scale, (experts, n), torch.float32, "weight row scales")
    _check(offsets, (experts + 1,), torch.int32, "offsets")
    _check(z, (rows, rank), torch.bfloat16, "lora z")
    _check(b, (experts, n, rank), torch.bfloat16, "lora b")
    if not (z.is_contiguous() and b.is_contiguous()):
        raise ValueError("lora factors must be contiguous")
    device = _on_gpu(a, a_scale, w, w_scale, offsets, z, b)
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=device)
    _timed(
        "gemm_fp8_rowwise", device, 2 * rows * n * (k + rank),
        rows * k + experts * n * k + 2 * rows * n,
        "mi355x_gemm_fp8_rowwise_lora", _ptr(a), _ptr(a_scale), rows, _ptr(w), _ptr(w_scale),
        experts, n, k, _ptr(offsets), _ptr(z), _ptr(b), rank, _ptr(out), _stream(device),
    )
    return out


def wgrad(p, p_scale, q, q_scale, offsets, *, out_dtype=torch.bfloat16, rows=None):
    """``out[e] = sum over expert e's rows of p[:, row] q[:, row]^T`` -> ``[E, M, N]``.
    ``rows`` (the routed row count, for the launch timer's FLOP count) is optional."""
    m, padded = p.shape
    n = q.shape[0]
    experts = offsets.numel() - 1
    _check(q, (n, padded), FP8, "q")
    _check(p_scale, (padded // 128, m), torch.float32, "p scales")
    _check(q_scale, (padded // 128, n), torch.float32, "q scales")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("wgrad writes bf16 or fp32")
    device = _on_gpu(p, p_scale, q, q_scale, offsets)
    out = torch.empty((experts, m, n), dtype=out_dtype, device=device)
    flops = 2 * m * n * (padded if rows is None else int(rows))
    _timed(
        "gemm_fp8_block_wgrad", device, flops, (m + n) * padded + experts * m * n * out.element_size(),
        "mi355x_gemm_fp8_block_wgrad", _ptr(p), _ptr(p_scale), m, _ptr(q), _ptr(q_scale), n,
        padded, _ptr(offsets), experts, _ptr(out), int(out_dtype == torch.float32),
        _stream(device),
    )
    return out
