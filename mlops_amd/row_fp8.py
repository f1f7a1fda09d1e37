"""`RowFP8Weight`: expert weights as e4m3 rows with one descale per row, kept in
both orientations -- the weight format of ``compute_precision="fp8_current"``.

It has the data format of the reference's ``QuackFP8Weight``
(``src/mlops/expert_parallel/quack/parameters/fp8.py:20-214``) and is exported
under that name too. The logical weight is ``[E, out, in]`` in nn.Linear row
order; the container stores, in this component order,

* ``_data`` e4m3 ``[E, out, in]``, the rows the forward product reads;
* ``_transposed`` e4m3 ``[E, in, out]``, the rows the input-gradient product reads;
* ``_scale`` fp32 ``[E, out]`` and ``_transposed_scale`` fp32 ``[E, in]``,
  one descale per stored row of each.

Each orientation is quantized on its own rows: ``scale = max(amax * (1/448),
1e-12)``, ``q = e4m3(clip(x / scale, +-448))`` -- the reference's GPU rule
(``kernels/quack_moe/quantize_transpose.py:316-339``), here
``mi355x_quantize_weights_current_fp8``. With ``interleaved=True`` a gate/up
weight is stored with gate row j and up row j adjacent (stored rows 2j and
2j + 1) in both orientations, so the up projection writes its output already
interleaved; the logical value and the gradients keep gate-then-up order.
"""

from __future__ import annotations

import torch

from ._quantized import QuantizedWeight, straight_through

COMPONENTS = ("_data", "_transposed", "_scale", "_transposed_scale")
E4M3 = torch.float8_e4m3fn


def _gate_then_up(stored: torch.Tensor) -> torch.Tensor:
    """Rows stored gate/up-adjacent (2j, 2j + 1) put back as all gates, then all ups."""
    experts, rows, cols = stored.shape
    pairs = stored.reshape(experts, rows // 2, 2, cols)
    return torch.cat((pairs[:, :, 0], pairs[:, :, 1]), dim=1)


def quantize_components(weight: torch.Tensor, interleaved: bool):
    """``(data, transposed, scale, transposed_scale)`` of a bf16/fp32 GPU weight."""
    if weight.ndim != 3:
        raise ValueError(f"a row-FP8 weight is [experts, out, in]; got {tuple(weight.shape)}")
    if not weight.is_cuda:
        raise ValueError("row-FP8 quantization is an MI355X kernel; on this device, "
                         "build RowFP8Weight from existing components")
    from .kernels import quantize_weights_current

    return quantize_weights_current(weight.detach(), interleaved=interleaved)


class RowFP8Weight(QuantizedWeight):
    """An ``[E, out, in]`` expert weight as per-row scaled e4m3 in both orientations."""

    component_names = COMPONENTS
    label = "row-FP8"

    def __new__(cls, data, transposed, scale, transposed_scale, *, dtype=torch.float32,
                interleaved=False):
        if data.dtype != E4M3 or data.ndim != 3:
            raise ValueError(f"RowFP8Weight data must be E4M3 [experts, out, in]; got "
                             f"{data.dtype} {tuple(data.shape)}")
        experts, out, inner = data.shape
        if transposed.dtype != E4M3 or tuple(transposed.shape) != (experts, inner, out):
            raise ValueError(f"RowFP8Weight needs the E4M3 transpose {(experts, inner, out)}; "
                             f"got {transposed.dtype} {tuple(transposed.shape)}")
        for name, part, rows in (("scale", scale, out), ("transposed_scale", transposed_scale,
                                                         inner)):
            if tuple(part.shape) != (experts, rows):
                raise ValueError(f"RowFP8Weight {name} must be fp32 {(experts, rows)}; got "
                                 f"{tuple(part.shape)}")
        return cls._wrap(data, dtype, (data, transposed, scale, transposed_scale),
                         _interleaved=bool(interleaved))

    def __repr__(self):
        order = ", interleaved" if self._interleaved else ""
        return (f"RowFP8Weight(shape={tuple(self.shape)}, logical_dtype={self.dtype}, "
                f"device={self.device}{order})")

    @classmethod
    def quantize(cls, weight, *, dtype=None, interleaved=False):
        """The container of a bf16/fp32 ``weight [E, out, in]``: both
        orientations quantized, gate/up rows adjacent when ``interleaved``;
        ``dtype`` is the logical dtype (the weight's own when None).
        Gradients reaching the container reach ``weight`` unchanged."""
        if weight.ndim != 3:
            raise ValueError(f"a row-FP8 weight is [experts, out, in]; got {tuple(weight.shape)}")
        if interleaved and weight.shape[1] % 2:
            raise ValueError("interleaving gate and up rows needs an even number of rows")
        logical = weight.dtype if dtype is None else dtype
        return straight_through(
            lambda w: cls(*quantize_components(w, interleaved), dtype=logical,
                          interleaved=interleaved), weight)

    @property
    def interleaved(self):
        return self._interleaved

    def _flatten_metadata(self):
        return (self.dtype, self._interleaved)

    @staticmethod
    def __tensor_unflatten__(inner_tensors, metadata, outer_size, outer_stride):
        dtype, interleaved = metadata
        return RowFP8Weight(*(inner_tensors[name] for name in COMPONENTS), dtype=dtype,
                            interleaved=interleaved)

    def _rebuild(self, parts):
        return RowFP8Weight(*parts, dtype=self.dtype, interleaved=self._interleaved)

    def _expand(self, dtype):
        value = self._data.float() * self._scale.float().unsqueeze(-1)
        return (_gate_then_up(value) if self._interleaved else value).to(dtype)

    def _encode(self, master):
        return quantize_components(master, self._interleaved)

    def _accepts_parts_of(self, other):
        if getattr(other, "_interleaved", False) != self._interleaved:
            raise ValueError("cannot copy between RowFP8Weight containers of different row "
                             "orders (interleaved vs gate-then-up)")


QuackFP8Weight = RowFP8Weight  # the reference's name for this container

__all__ = ["COMPONENTS", "QuackFP8Weight", "RowFP8Weight", "quantize_components"]
