"""The allocation-free permute plan (``mi355x_permute_plan_noalloc``).

It keeps its histogram in a fixed per-GPU device array instead of a caller
workspace. Called through the C ABI, it must give the same counts, offsets,
order and slots as ``mi355x_permute_plan`` (bit-exact, integer work), on two
calls in a row whose second input is smaller (the array keeps the first
call's contents), and refuse sizes beyond the array with a clear error.
"""

import pytest
import torch

from mlops_amd import _native

pytestmark = pytest.mark.gpu


def _ptr(t):
    return t.data_ptr()


def _outputs(n, shape, experts, device):
    return (torch.full((experts,), -7, dtype=torch.int64, device=device),
            torch.full((experts + 1,), -7, dtype=torch.int32, device=device),
            torch.full((n,), -7, dtype=torch.int32, device=device),
            torch.full(shape, -7, dtype=torch.int32, device=device))


def _with_workspace(ids, experts, device, stream):
    n = ids.numel()
    counts, offsets, order, slots = _outputs(n, ids.shape, experts, device)
    size = _native.query("mi355x_permute_plan_workspace_size", n, experts)
    workspace = torch.empty(size, dtype=torch.uint8, device=device)
    _native.call("mi355x_permute_plan", _ptr(ids), n, experts, _ptr(counts), _ptr(offsets),
                 _ptr(order), _ptr(slots), _ptr(workspace), size, stream)
    return counts, offsets, order, slots


def _noalloc(ids, experts, device, stream):
    n = ids.numel()
    counts, offsets, order, slots = _outputs(n, ids.shape, experts, device)
    _native.call("mi355x_permute_plan_noalloc", _ptr(ids), n, experts, _ptr(counts),
                 _ptr(offsets), _ptr(order), _ptr(slots), stream)
    return counts, offsets, order, slots


@pytest.mark.parametrize("sizes", [((16384, 8, 128), (1000, 8, 128)),
                                   ((4096, 2, 8), (37, 2, 8)),
                                   ((20000, 6, 300), (5, 6, 300))])
def test_noalloc_plan_equals_workspace_plan(device, sizes):
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator().manual_seed(sum(s[0] for s in sizes))
    for tokens, top_k, experts in sizes:  # second call smaller than the first
        logits = torch.randn(tokens, experts, generator=g)
        logits[:, 0] += 1.5  # an overloaded expert, as skewed routing gives
        ids = logits.topk(top_k, dim=1).indices.to(torch.int32).to(device)
        want = _with_workspace(ids, experts, device, stream)
        got = _noalloc(ids, experts, device, stream)
        torch.cuda.synchronize(device)
        for name, a, b in zip(("counts", "offsets", "order", "slots"), got, want):
            assert torch.equal(a.cpu(), b.cpu()), (name, tokens, top_k, experts)
        assert int(got[0].sum()) == tokens * top_k


def test_noalloc_plan_refuses_oversize(device):
    stream = torch.cuda.current_stream(device).cuda_stream
    experts = 1024
    limit = _native.query("mi355x_permute_plan_noalloc_max_assignments", experts)
    assert limit > 0
    ids = torch.zeros(1, dtype=torch.int32, device=device)
    with pytest.raises(_native.NativeError, match="scratch"):
        # the size check runs before any pointer is touched
        _native.call("mi355x_permute_plan_noalloc", _ptr(ids), limit + 1, experts,
                     None, None, None, None, stream)
