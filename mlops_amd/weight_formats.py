"""Recognising FP8 expert-weight containers by what they carry, not by class.

The MoE operators accept any tensor subclass that exposes the reference's
container protocol: a ``components()`` method returning the stored tensors in
a fixed order (``src/mlops/block_fp8.py:81-82`` for block FP8;
``src/mlops/expert_parallel/quack/parameters/fp8.py:21`` for the per-row
form). So the reference's own ``mlops.block_fp8.BlockFP8Weight`` is served
exactly like this package's, without conversion and with its autograd graph
intact.

* block FP8: ``(data e4m3 [E, out, in], scale fp32 [E, ceil(out/128),
  ceil(in/128)])``;
* row FP8 (fp8_current): ``(data e4m3 [E, out, in], transposed e4m3 [E, in,
  out], scale fp32 [E, out], transposed_scale fp32 [E, in])`` plus an
  ``interleaved`` flag (attribute ``interleaved`` or ``_interleaved``).

A custom operator only sees a container's components if a torch-dispatch
rule is registered for the container's class; `route_containers` registers
the operator's rule for each new class the first time one is passed.
"""

from __future__ import annotations

import threading

import torch

E4M3 = torch.float8_e4m3fn


def _parts(weight):
    if not isinstance(weight, torch.Tensor) or type(weight) is torch.Tensor:
        return None
    method = getattr(type(weight), "components", None)
    if not callable(method):
        return None
    try:
        parts = tuple(weight.components())
    except Exception:  # a subclass whose components() is something else
        return None
    if not all(isinstance(p, torch.Tensor) for p in parts):
        return None
    return parts


def block_parts(weight):
    """``(data, scale)`` if ``weight`` carries the block-FP8 protocol, else None."""
    parts = _parts(weight)
    if parts is None or len(parts) != 2:
        return None
    data, scale = parts
    if data.dtype != E4M3 or data.ndim != 3 or tuple(data.shape) != tuple(weight.shape):
        return None
    experts, out, inner = data.shape
    if scale.dtype != torch.float32 or tuple(scale.shape) != (
            experts, -(-out // 128), -(-inner // 128)):
        return None
    return data, scale


def row_parts(weight):
    """``(data, transposed, scale, transposed_scale)`` if ``weight`` carries the
    row-FP8 protocol, else None."""
    parts = _parts(weight)
    if parts is None or len(parts) != 4:
        return None
    data, transposed, scale, transposed_scale = parts
    if data.dtype != E4M3 or data.ndim != 3 or tuple(data.shape) != tuple(weight.shape):
        return None
    experts, out, inner = data.shape
    if transposed.dtype != E4M3 or tuple(transposed.shape) != (experts, inner, out):
        return None
    if tuple(scale.shape) != (experts, out) or tuple(transposed_scale.shape) != (experts, inner):
        return None
    return parts


def is_block_fp8(weight) -> bool:
    return block_parts(weight) is not None


def is_row_fp8(weight) -> bool:
    return row_parts(weight) is not None


def row_interleaved(weight) -> bool:
    """Whether a row-FP8 container stores gate/up rows adjacent."""
    flag = getattr(weight, "interleaved", None)
    if flag is None:
        flag = getattr(weight, "_interleaved", False)
    return bool(flag)


_registered: dict[int, set] = {}
_lock = threading.Lock()


def register_container_class(operators, rule, cls) -> None:
    """Make ``rule`` the torch-dispatch rule of every operator in ``operators``
    for containers of class ``cls`` (idempotent)."""
    seen = _registered.setdefault(id(operators), set())
    if cls in seen:
        return
    with _lock:
        if cls not in seen:
            for op in operators:
                op.register_torch_dispatch(cls, rule)
            seen.add(cls)


def route_containers(operators, rule, *weights) -> None:
    """`register_container_class` for the class of every container among
    ``weights`` (tensors without components are skipped)."""
    for weight in weights:
        if _parts(weight) is not None:
            register_container_class(operators, rule, type(weight))


__all__ = ["block_parts", "is_block_fp8", "is_row_fp8", "register_container_class",
           "route_containers", "row_interleaved", "row_parts"]
