"""A weight stored as quantized parts: the base of the FP8 expert containers.

A container is a wrapper tensor: its shape and dtype are those of the logical
weight (the dtype its gradients arrive at), while its storage is a fixed,
named tuple of component tensors (e4m3 values and fp32 descales). Autograd
sees the container like any tensor; the container itself answers only the
handful of aten operations that parameter handling needs (detach, clone,
device/dtype copies, in-place publication, factory "likes"). Everything else
is refused, so that no kernel silently computes on the quantized storage.

Subclasses name their components and say how to rebuild themselves from new
components (`_rebuild`), how to expand to the logical value (`_expand`) and
how to quantize a master weight into their own layout (`_encode`).
"""

from __future__ import annotations

from typing import Callable

import torch
from torch.utils._python_dispatch import return_and_correct_aliasing


class _StraightThrough(torch.autograd.Function):
    """``transform(value)`` whose gradient is passed to ``value`` unchanged:
    quantizing a master into a container and expanding a container back are
    both identities as far as the training signal is concerned."""

    @staticmethod
    def forward(ctx, transform, value):
        return transform(value.detach())

    @staticmethod
    def backward(ctx, grad):
        return None, grad


def straight_through(transform: Callable, value: torch.Tensor) -> torch.Tensor:
    return _StraightThrough.apply(transform, value)


class QuantizedWeight(torch.Tensor):
    """Wrapper tensor over named quantized components (see the module doc)."""

    component_names: tuple[str, ...] = ()
    label = "quantized"  # how error messages name the format

    @classmethod
    def _wrap(cls, logical_like: torch.Tensor, dtype: torch.dtype, parts, **attributes):
        value = torch.Tensor._make_wrapper_subclass(
            cls, tuple(logical_like.shape), device=logical_like.device, dtype=dtype)
        for name, part in zip(cls.component_names, parts, strict=True):
            setattr(value, name, part)
        for name, attribute in attributes.items():
            setattr(value, name, attribute)
        return value

    # ---- subclass hooks
    def _rebuild(self, parts):
        raise NotImplementedError

    def _expand(self, dtype: torch.dtype) -> torch.Tensor:
        raise NotImplementedError

    def _encode(self, master: torch.Tensor):
        raise NotImplementedError

    def _flatten_metadata(self):
        return (self.dtype,)

    def _accepts_parts_of(self, other: "QuantizedWeight") -> None:
        """Raise when ``other``'s components cannot be copied into this one."""

    # ---- public surface shared by the containers
    def components(self):
        return tuple(getattr(self, name) for name in self.component_names)

    def __tensor_flatten__(self):
        return list(self.component_names), self._flatten_metadata()

    def _dequantize(self, dtype):
        return self._expand(self.dtype if dtype is None else dtype)

    def dequantize(self, *, dtype=None):
        """The weight the components represent, at the logical dtype or
        ``dtype``; differentiable straight through when the container is."""
        if torch.is_grad_enabled() and self.requires_grad:
            return straight_through(lambda c: c._dequantize(dtype), self)
        return self._dequantize(dtype)

    # ---- the aten operations a container answers
    def _op_detach(self, func, args, kwargs):
        out = self._rebuild([part.detach() for part in self.components()])
        return return_and_correct_aliasing(func, args, kwargs, out)

    def _op_clone(self, func, args, kwargs):
        return self._rebuild([part.clone(**kwargs) for part in self.components()])

    def _op_copy(self, func, args, kwargs):
        target, source = args[:2]
        if not isinstance(target, QuantizedWeight):
            # Expanding a container into a plain tensor.
            return target.copy_(source._dequantize(target.dtype), **kwargs)
        if isinstance(source, QuantizedWeight):
            target._accepts_parts_of(source)
            parts = source.components()
        else:
            # Publication from a master weight (e.g. after an optimizer step):
            # re-quantized the way the container was made.
            parts = target._encode(source)
        for mine, new in zip(target.components(), parts, strict=True):
            mine.copy_(new)
        return target

    def _op_to_copy(self, func, args, kwargs):
        if kwargs.get("dtype", self.dtype) != self.dtype:
            return self._dequantize(None).to(**kwargs)
        placement = {key: value for key, value in kwargs.items() if key != "dtype"}
        return self._rebuild([func(part, **placement) for part in self.components()])

    def _op_like(self, func, args, kwargs):
        # Factories "like" a container make a plain tensor of its logical
        # shape and dtype, on its device.
        options = dict(kwargs)
        options.setdefault("dtype", self.dtype)
        return func(self.components()[0], *args[1:], **options)

    _DISPATCH: dict | None = None

    @classmethod
    def _dispatch_table(cls):
        if QuantizedWeight._DISPATCH is None:
            aten = torch.ops.aten
            QuantizedWeight._DISPATCH = {
                aten.detach.default: QuantizedWeight._op_detach,
                aten.clone.default: QuantizedWeight._op_clone,
                aten.copy_.default: QuantizedWeight._op_copy,
                aten._to_copy.default: QuantizedWeight._op_to_copy,
                aten.empty_like.default: QuantizedWeight._op_like,
                aten.zeros_like.default: QuantizedWeight._op_like,
                aten.ones_like.default: QuantizedWeight._op_like,
                aten.new_empty_strided.default: QuantizedWeight._op_like,
            }
        return QuantizedWeight._DISPATCH

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func is torch.ops.aten._assert_tensor_metadata.default:
            with torch._C._DisableTorchDispatch():
                return func(*args, **kwargs)
        handler = cls._dispatch_table().get(func)
        if handler is None:
            raise NotImplementedError(
                f"{cls.__name__} does not compute {func}: pass it to an operator that takes "
                f"{cls.label} weights, or dequantize() it first")
        owner = args[0] if isinstance(args[0], QuantizedWeight) else args[1]
        return handler(owner, func, args, kwargs)


__all__ = ["QuantizedWeight", "straight_through"]
