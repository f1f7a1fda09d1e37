"""Explicit forward / VJP surfaces."""

from . import moe

__all__ = ["moe"]
