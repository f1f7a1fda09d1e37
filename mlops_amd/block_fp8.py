"""Expert weights stored once as block-scaled e4m3: `BlockFP8Weight`.

Contract of the reference container (``src/mlops/block_fp8.py:49-153``): a
tensor subclass whose logical shape is the weight ``[E, out, in]`` (rows in
nn.Linear order; a gate/up weight holds gate rows then up rows) and whose
logical dtype is that of the gradients it receives. It carries two
components: e4m3 ``_data [E, out, in]`` and fp32 ``_scale [E, ceil(out/128),
ceil(in/128)]`` with ``value ~ data * scale`` per 128x128 block, the layout
of DeepSeek-style FP8 checkpoints. `quantize` and `dequantize` differentiate
straight through.

Quantization runs on the GPU through ``mi355x_quantize_weight_blocks``; a
container can also be built directly from existing components on any device.
"""

from __future__ import annotations

import torch
from torch.utils._python_dispatch import return_and_correct_aliasing

BLOCK = 128
COMPONENTS = ("_data", "_scale")


def scale_shape(experts: int, out: int, inner: int) -> tuple[int, int, int]:
    return experts, -(-out // BLOCK), -(-inner // BLOCK)


def quantize_blocks(weight: torch.Tensor):
    """``(data e4m3, scale fp32)`` of a bf16/fp32 ``[E, out, in]`` GPU weight:
    ``scale = max(amax / 448, 1e-12)`` per 128x128 block (true division),
    ``data = e4m3(clip(weight / scale, +-448))``."""
    if weight.ndim != 3:
        raise ValueError("Expected an [experts, out, in] weight")
    if not weight.is_cuda:
        raise ValueError(
            "BlockFP8Weight quantization runs on the MI355X; build the container "
            "from existing (data, scale) components on other devices"
        )
    from .kernels import quantize_weight_blocks

    return quantize_weight_blocks(weight.detach())


def dequantize_blocks(data: torch.Tensor, scale: torch.Tensor, *, dtype=torch.float32):
    """``data * scale`` per block as ``[E, out, in]`` at ``dtype`` (diagnostics)."""
    _, out, inner = data.shape
    expanded = scale.float().repeat_interleave(BLOCK, 1).repeat_interleave(BLOCK, 2)
    return (data.float() * expanded[:, :out, :inner]).to(dtype)


class _Quantize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, weight, dtype):
        data, scale = quantize_blocks(weight)
        return BlockFP8Weight(data, scale, dtype=weight.dtype if dtype is None else dtype)

    @staticmethod
    def backward(ctx, grad):
        return grad, None


class _Dequantize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, weight, dtype):
        return weight.detach()._dequantize(dtype)

    @staticmethod
    def backward(ctx, grad):
        return grad, None


class BlockFP8Weight(torch.Tensor):
    """A ``[E, out, in]`` expert weight as e4m3 data plus 128x128 block scales."""

    @staticmethod
    def __new__(cls, data, scale, *, dtype=torch.bfloat16):
        if data.ndim != 3 or data.dtype != torch.float8_e4m3fn:
            raise ValueError("Expected E4M3 data [experts, out, in]")
        expected = scale_shape(*data.shape)
        if tuple(scale.shape) != expected or scale.dtype != torch.float32:
            raise ValueError(f"Expected FP32 block scales {expected}")
        value = torch.Tensor._make_wrapper_subclass(
            cls, tuple(data.shape), device=data.device, dtype=dtype
        )
        value._data = data
        value._scale = scale
        return value

    def __repr__(self):
        return (
            f"BlockFP8Weight(shape={tuple(self.shape)}, logical_dtype={self.dtype}, "
            f"device={self.device})"
        )

    @classmethod
    def quantize(cls, weight, *, dtype=None):
        """Container of ``weight [E, out, in]``; its gradient is the weight's."""
        if weight.ndim != 3:
            raise ValueError("Expected an [experts, out, in] weight")
        return _Quantize.apply(weight, dtype)

    def components(self):
        return self._data, self._scale

    def __tensor_flatten__(self):
        return list(COMPONENTS), (self.dtype,)

    @staticmethod
    def __tensor_unflatten__(inner_tensors, metadata, outer_size, outer_stride):
        (dtype,) = metadata
        return BlockFP8Weight(inner_tensors["_data"], inner_tensors["_scale"], dtype=dtype)

    def _dequantize(self, dtype):
        return dequantize_blocks(self._data, self._scale, dtype=self.dtype if dtype is None else dtype)

    def dequantize(self, *, dtype=None):
        """The represented weight (diagnostics); differentiable straight through."""
        if torch.is_grad_enabled() and self.requires_grad:
            return _Dequantize.apply(self, dtype)
        return self._dequantize(dtype)

    def _rebuilt(self, parts):
        data, scale = parts
        return type(self)(data, scale, dtype=self.dtype)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        aten = torch.ops.aten
        first = args[0]
        if func is aten._assert_tensor_metadata.default:
            with torch._C._DisableTorchDispatch():
                return func(*args, **kwargs)
        if func is aten.detach.default:
            out = first._rebuilt([t.detach() for t in first.components()])
            return return_and_correct_aliasing(func, args, kwargs, out)
        if func is aten.clone.default:
            return first._rebuilt([t.clone(**kwargs) for t in first.components()])
        if func is aten.copy_.default:
            dst, src = args[:2]
            if isinstance(dst, cls):
                # From another container: its components; from a master weight:
                # re-quantized as at initialization.
                parts = src.components() if isinstance(src, cls) else quantize_blocks(src)
                for target, part in zip(dst.components(), parts):
                    target.copy_(part)
                return dst
            return dst.copy_(src._dequantize(dst.dtype), **kwargs)
        if func is aten._to_copy.default:
            if kwargs.get("dtype", first.dtype) != first.dtype:
                return first._dequantize(None).to(**kwargs)
            options = {k: v for k, v in kwargs.items() if k != "dtype"}
            return first._rebuilt([aten._to_copy.default(t, **options) for t in first.components()])
        if func in (aten.empty_like.default, aten.zeros_like.default, aten.ones_like.default):
            return func(first._data, **dict(kwargs, dtype=kwargs.get("dtype", first.dtype)))
        if func is aten.new_empty_strided.default:
            return func(first._data, *args[1:], **dict(kwargs, dtype=kwargs.get("dtype", first.dtype)))
        raise NotImplementedError(
            f"{func}: use the block FP8 components or dequantize for diagnostics"
        )


__all__ = ["BLOCK", "BlockFP8Weight", "dequantize_blocks", "quantize_blocks", "scale_shape"]
