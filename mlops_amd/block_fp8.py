"""`BlockFP8Weight`: expert weights as e4m3 with one fp32 descale per 128x128 block.

This is the data format of the reference's container (``src/mlops/block_fp8.py``
:49-153) and of DeepSeek-style FP8 checkpoints: the logical weight is
``[E, out, in]`` in nn.Linear row order (a gate/up weight holds its gate rows,
then its up rows), stored as

* ``_data`` e4m3 ``[E, out, in]``, and
* ``_scale`` fp32 ``[E, ceil(out/128), ceil(in/128)]``,

with ``weight ~= data * scale`` over each 128x128 block. The container's
dtype is the logical one, the dtype its gradients come back at.

Quantization runs on the MI355X (``mi355x_quantize_weight_blocks``):
``scale = max(amax / 448, 1e-12)`` with a true division, ``data =
e4m3(clip(weight / scale, +-448))``. On other devices a container is built
from existing components.
"""

from __future__ import annotations

import torch

from ._quantized import QuantizedWeight, straight_through

BLOCK = 128
COMPONENTS = ("_data", "_scale")
E4M3 = torch.float8_e4m3fn


def scale_shape(experts: int, out: int, inner: int) -> tuple[int, int, int]:
    """Shape of the block descales of an ``[experts, out, inner]`` weight."""
    return experts, (out + BLOCK - 1) // BLOCK, (inner + BLOCK - 1) // BLOCK


def quantize_blocks(weight: torch.Tensor):
    """``(data e4m3, scale fp32)`` of a bf16/fp32 ``[E, out, in]`` weight on the GPU."""
    if weight.ndim != 3:
        raise ValueError(f"a block-FP8 weight is [experts, out, in]; got {tuple(weight.shape)}")
    if not weight.is_cuda:
        raise ValueError("block-FP8 quantization is an MI355X kernel; on this device, "
                         "build BlockFP8Weight(data, scale) from existing components")
    from .kernels import quantize_weight_blocks

    return quantize_weight_blocks(weight.detach())


def dequantize_blocks(data: torch.Tensor, scale: torch.Tensor, *, dtype=torch.float32):
    """``data * scale`` expanded over each block, cut to ``[E, out, in]``."""
    experts, out, inner = data.shape
    rows = scale.float().repeat_interleave(BLOCK, dim=1)[:, :out]
    full = rows.repeat_interleave(BLOCK, dim=2)[:, :, :inner]
    return (data.float() * full).to(dtype)


class BlockFP8Weight(QuantizedWeight):
    """An ``[E, out, in]`` expert weight held as e4m3 values and 128x128 block descales."""

    component_names = COMPONENTS
    label = "block-FP8"

    def __new__(cls, data, scale, *, dtype=torch.bfloat16):
        if data.dtype != E4M3 or data.ndim != 3:
            raise ValueError(f"BlockFP8Weight data must be E4M3 [experts, out, in]; got "
                             f"{data.dtype} {tuple(data.shape)}")
        want = scale_shape(*data.shape)
        if scale.dtype != torch.float32 or tuple(scale.shape) != want:
            raise ValueError(f"BlockFP8Weight scales must be fp32 {want}; got "
                             f"{scale.dtype} {tuple(scale.shape)}")
        return cls._wrap(data, dtype, (data, scale))

    def __repr__(self):
        return (f"BlockFP8Weight(shape={tuple(self.shape)}, logical_dtype={self.dtype}, "
                f"device={self.device})")

    @classmethod
    def quantize(cls, weight, *, dtype=None):
        """The container of a bf16/fp32 ``weight [E, out, in]``; ``dtype`` is the
        logical dtype (the weight's own when None). Gradients reaching the
        container reach ``weight`` unchanged."""
        if weight.ndim != 3:
            raise ValueError(f"a block-FP8 weight is [experts, out, in]; got {tuple(weight.shape)}")
        logical = weight.dtype if dtype is None else dtype
        return straight_through(lambda w: cls(*quantize_blocks(w), dtype=logical), weight)

    @staticmethod
    def __tensor_unflatten__(inner_tensors, metadata, outer_size, outer_stride):
        return BlockFP8Weight(*(inner_tensors[name] for name in COMPONENTS), dtype=metadata[0])

    def _rebuild(self, parts):
        return BlockFP8Weight(*parts, dtype=self.dtype)

    def _expand(self, dtype):
        return dequantize_blocks(self._data, self._scale, dtype=dtype)

    def _encode(self, master):
        return quantize_blocks(master)


__all__ = ["BLOCK", "BlockFP8Weight", "dequantize_blocks", "quantize_blocks", "scale_shape"]
