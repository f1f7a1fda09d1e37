"""Expert weights as e4m3 with one descale per row, in both orientations:
`RowFP8Weight`, the weight format of ``compute_precision="fp8_current"``.

Contract of the reference container ``QuackFP8Weight``
(``src/mlops/expert_parallel/quack/parameters/fp8.py:20-214``), also exported
under that name. It is a tensor subclass whose logical shape is the weight
``[E, out, in]`` (nn.Linear rows; a gate/up weight holds gate rows then up
rows) and whose logical dtype is that of the gradients it receives. It
carries four components, in this order:

* ``_data`` e4m3 ``[E, out, in]``: the rows the forward GEMM reads;
* ``_transposed`` e4m3 ``[E, in, out]``: the K-major copy the input-gradient
  GEMM reads;
* ``_scale`` fp32 ``[E, out]``: one descale per row of ``_data``;
* ``_transposed_scale`` fp32 ``[E, in]``: one per row of ``_transposed``.

With ``interleaved=True`` both orientations store the rows gate/up-adjacent
(stored row 2j = gate row j, 2j + 1 = up row j). The up projection then
writes ``h`` interleaved without reordering. Each orientation is quantized
independently: ``scale = max(amax * (1/448), 1e-12)``, ``q = e4m3(clip(x /
scale, +-448))``. That is the reference's GPU path
(``kernels/quack_moe/quantize_transpose.py:316-339``), here
``mi355x_quantize_weights_current_fp8``. `quantize` and `dequantize`
differentiate straight through.
"""

from __future__ import annotations

import torch
from torch.utils._python_dispatch import return_and_correct_aliasing

COMPONENTS = ("_data", "_transposed", "_scale", "_transposed_scale")


def _logical_rows(value: torch.Tensor) -> torch.Tensor:
    """``[E, out, in]`` from gate/up-adjacent rows back to gate-then-up rows."""
    experts, out, inner = value.shape
    return value.view(experts, out // 2, 2, inner).transpose(1, 2).reshape(value.shape)


def quantize_components(weight: torch.Tensor, interleaved: bool):
    """``(data, transposed, scale, transposed_scale)`` of a bf16/fp32 GPU weight."""
    if weight.ndim != 3:
        raise ValueError("Expected an [experts, out, in] weight")
    if not weight.is_cuda:
        raise ValueError(
            "RowFP8Weight quantization runs on the MI355X; build the container from "
            "existing components on other devices"
        )
    from .kernels import quantize_weights_current

    return quantize_weights_current(weight.detach(), interleaved=interleaved)


class _Quantize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, weight, dtype, interleaved):
        return RowFP8Weight(*quantize_components(weight, interleaved),
                            dtype=weight.dtype if dtype is None else dtype,
                            interleaved=interleaved)

    @staticmethod
    def backward(ctx, grad):
        return grad, None, None


class _Dequantize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, weight, dtype):
        return weight.detach()._dequantize(dtype)

    @staticmethod
    def backward(ctx, grad):
        return grad, None


class RowFP8Weight(torch.Tensor):
    """A ``[E, out, in]`` expert weight as per-row scaled e4m3, both orientations."""

    @staticmethod
    def __new__(cls, data, transposed, scale, transposed_scale, *, dtype=torch.float32,
                interleaved=False):
        if data.ndim != 3 or data.dtype != torch.float8_e4m3fn:
            raise ValueError("Expected E4M3 data [experts, out, in]")
        experts, out, inner = data.shape
        if tuple(transposed.shape) != (experts, inner, out) or transposed.dtype != data.dtype:
            raise ValueError("Expected the E4M3 transpose [experts, in, out]")
        if tuple(scale.shape) != (experts, out) or tuple(transposed_scale.shape) != (experts, inner):
            raise ValueError("Expected FP32 descales [experts, out] and [experts, in]")
        value = torch.Tensor._make_wrapper_subclass(cls, tuple(data.shape), device=data.device,
                                                    dtype=dtype)
        for name, tensor in zip(COMPONENTS, (data, transposed, scale, transposed_scale)):
            setattr(value, name, tensor)
        value._interleaved = bool(interleaved)
        return value

    def __repr__(self):
        layout = ", interleaved" if self._interleaved else ""
        return (f"RowFP8Weight(shape={tuple(self.shape)}, logical_dtype={self.dtype}, "
                f"device={self.device}{layout})")

    @classmethod
    def quantize(cls, weight, *, dtype=None, interleaved=False):
        """Container of ``weight [E, out, in]`` (bf16 or fp32): both
        orientations quantized, rows gate/up-adjacent when ``interleaved``;
        ``dtype`` is the logical dtype (the weight's own when None). Its
        gradient is the weight's."""
        if weight.ndim != 3:
            raise ValueError("Expected an [experts, out, in] weight")
        if interleaved and weight.shape[1] % 2:
            raise ValueError("Interleaving gate and up rows needs an even row count")
        return _Quantize.apply(weight, dtype, interleaved)

    @property
    def interleaved(self):
        return self._interleaved

    def components(self):
        return tuple(getattr(self, name) for name in COMPONENTS)

    def __tensor_flatten__(self):
        return list(COMPONENTS), (self.dtype, self._interleaved)

    @staticmethod
    def __tensor_unflatten__(inner_tensors, metadata, outer_size, outer_stride):
        dtype, interleaved = metadata
        return RowFP8Weight(*(inner_tensors[n] for n in COMPONENTS), dtype=dtype,
                            interleaved=interleaved)

    def _dequantize(self, dtype):
        value = self._data.float() * self._scale[..., None]
        if self._interleaved:
            value = _logical_rows(value)
        return value.to(self.dtype if dtype is None else dtype)

    def dequantize(self, *, dtype=None):
        """The weight the rows represent, in nn.Linear row order (diagnostics);
        differentiable straight through."""
        if torch.is_grad_enabled() and self.requires_grad:
            return _Dequantize.apply(self, dtype)
        return self._dequantize(dtype)

    def _like(self, components):
        return type(self)(*components, dtype=self.dtype, interleaved=self._interleaved)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        aten, first = torch.ops.aten, args[0]
        if func is aten._assert_tensor_metadata.default:
            with torch._C._DisableTorchDispatch():
                return func(*args, **kwargs)
        if func is aten.detach.default:
            out = first._like([v.detach() for v in first.components()])
            return return_and_correct_aliasing(func, args, kwargs, out)
        if func is aten.clone.default:
            return first._like([v.clone(**kwargs) for v in first.components()])
        if func is aten.copy_.default:
            destination, source = args[:2]
            if isinstance(destination, cls):
                if isinstance(source, cls):
                    if source._interleaved != destination._interleaved:
                        raise ValueError("FP8 weights of different row orders")
                    parts = source.components()
                else:
                    # Publication from a master: both orientations quantized
                    # as at initialization, in the destination's row order.
                    parts = quantize_components(source, destination._interleaved)
                for target, part in zip(destination.components(), parts):
                    target.copy_(part)
                return destination
            return destination.copy_(source._dequantize(destination.dtype), **kwargs)
        if func is aten._to_copy.default:
            if kwargs.get("dtype", first.dtype) != first.dtype:
                return first._dequantize(None).to(**kwargs)
            options = {k: v for k, v in kwargs.items() if k != "dtype"}
            return first._like([aten._to_copy.default(v, **options) for v in first.components()])
        if func in (aten.empty_like.default, aten.zeros_like.default, aten.ones_like.default):
            return func(first._data, **dict(kwargs, dtype=kwargs.get("dtype", first.dtype)))
        if func is aten.new_empty_strided.default:
            return func(first._data, *args[1:],
                        **dict(kwargs, dtype=kwargs.get("dtype", first.dtype)))
        raise NotImplementedError(
            f"{func}: use the row FP8 components or dequantize for diagnostics")


QuackFP8Weight = RowFP8Weight  # the reference's name for this container

__all__ = ["COMPONENTS", "QuackFP8Weight", "RowFP8Weight", "quantize_components"]
