"""The C-ABI library (CPU checks, no GPU compute): it loads, exports every
function ``include/mlops_mi355x.h`` declares with the binding's signature,
and its argument validation rejects bad shapes with a message before any
kernel is launched."""

import ctypes
import re
from pathlib import Path

import pytest

from mlops_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "mlops_mi355x.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(mi355x_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_and_binding_agree():
    declared = _declared()
    assert declared == sorted(_native.SIGNATURES), set(declared) ^ set(_native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _native.library()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.mi355x_abi_version() == 1


def test_argument_counts_match_header():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, (_, argtypes) in _native.SIGNATURES.items():
        match = re.search(rf"\b{name}\s*\(([^)]*)\)", text)
        params = [p for p in match.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(argtypes), name


@pytest.mark.parametrize("name,args,message", [
    ("mi355x_gemm_fp8_block", (None, None, 10, None, None, 0, 4, 100, 256, None, 0, None, None, None),
     "N must be a multiple of 128"),
    ("mi355x_gemm_fp8_block", (None, None, 10, None, None, 0, 4, 256, 200, None, 0, None, None, None),
     "K must be a multiple of 128"),
    ("mi355x_router_topk", (None, 10, 1000, 2, 0, None, 1, 1, 1.0, None, None, None, None),
     "experts"),
    ("mi355x_permute_plan", (None, 10, 2000, None, None, None, None, None, 0, None), "experts"),
    ("mi355x_quantize_rows_fp8", (None, 4, 100, 100, 0, None, None, None), "multiple of 128"),
])
def test_validation_errors(name, args, message):
    with pytest.raises(_native.NativeError, match=message):
        _native.call(name, *args)


def test_sizes_are_queries():
    assert _native.query("mi355x_wgrad_padded_rows", 1000, 8) % 128 == 0
    assert _native.query("mi355x_wgrad_padded_rows", 1000, 8) >= 1000 + 8 * 127
    assert _native.query("mi355x_permute_plan_workspace_size", 131072, 128) >= 32 * 128 * 4
