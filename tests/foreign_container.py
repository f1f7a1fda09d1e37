"""A block-FP8 weight container that is not this package's class: a tensor
subclass written here with only the reference container's protocol (the
``_data`` / ``_scale`` components, ``components()``, and the parameter
operations a training loop uses), as ``mlops.block_fp8.BlockFP8Weight``
exposes it (src/mlops/block_fp8.py:49-153). Tests pass it to the MI355X
operators to show that the boundary recognises containers by protocol."""

import torch
from torch.utils._python_dispatch import return_and_correct_aliasing


class ProtocolBlockWeight(torch.Tensor):
    @staticmethod
    def __new__(cls, data, scale, *, dtype=torch.bfloat16):
        value = torch.Tensor._make_wrapper_subclass(cls, tuple(data.shape), device=data.device,
                                                    dtype=dtype)
        value._data, value._scale = data, scale
        return value

    def components(self):
        return self._data, self._scale

    def __tensor_flatten__(self):
        return ["_data", "_scale"], (self.dtype,)

    @staticmethod
    def __tensor_unflatten__(inner, meta, outer_size, outer_stride):
        return ProtocolBlockWeight(inner["_data"], inner["_scale"], dtype=meta[0])

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        aten = torch.ops.aten
        if func is aten._assert_tensor_metadata.default:
            with torch._C._DisableTorchDispatch():
                return func(*args, **kwargs)
        first = args[0]
        if func is aten.detach.default:
            out = ProtocolBlockWeight(first._data.detach(), first._scale.detach(),
                                      dtype=first.dtype)
            return return_and_correct_aliasing(func, args, kwargs, out)
        if func in (aten.empty_like.default, aten.zeros_like.default, aten.ones_like.default):
            return func(first._data, **dict(kwargs, dtype=kwargs.get("dtype", first.dtype)))
        if func is aten.new_empty_strided.default:
            return func(first._data, *args[1:],
                        **dict(kwargs, dtype=kwargs.get("dtype", first.dtype)))
        raise NotImplementedError(f"ProtocolBlockWeight does not compute {func}")
