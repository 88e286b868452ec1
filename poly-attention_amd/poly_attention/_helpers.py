"""Small helpers the reference takes from einx / torch_einops_utils, restated in torch.

einx is not a dependency here: the four einx patterns the reference uses are written out
as broadcasts (`where_keys`, `where_queries`, `add_key_bias`).
"""

from __future__ import annotations

from typing import Callable

import torch
from torch import Tensor, is_tensor


def exists(val) -> bool:
    return val is not None


def default(val, d):
    return val if exists(val) else d


def first(t):
    return t[0]


def cast_tuple(t, length: int = 1):
    """poly_attention.py:37-38"""
    return (t,) * length if is_tensor(t) or not isinstance(t, tuple) else t


def divisible_by(num: int, den: int) -> bool:
    return (num % den) == 0


def softclamp(x: Tensor, clamp_value: float) -> Tensor:
    """poly_attention.py:43-44"""
    return clamp_value * torch.tanh(x / clamp_value)


def maybe(fn: Callable) -> Callable:
    """torch_einops_utils.maybe: apply fn unless the argument is None."""

    def inner(t, *args, **kwargs):
        if t is None:
            return None
        return fn(t, *args, **kwargs)

    return inner


def safe_cat(tensors, dim: int = 0):
    """torch_einops_utils.safe_cat: concatenate the tensors that are not None (None if none)."""
    tensors = [t for t in tensors if exists(t)]
    if len(tensors) == 0:
        return None
    if len(tensors) == 1:
        return tensors[0]
    return torch.cat(tensors, dim=dim)


def repeat_kv(t: Tensor | None, rep: int) -> Tensor | None:
    """einops.repeat(t, 'b g n d -> b (g r) n d', r = rep): head g*rep + i copies kv head g."""
    if t is None or rep == 1:
        return t
    return t.repeat_interleave(rep, dim=1)


def where_keys(mask: Tensor, sim: Tensor, value: float) -> Tensor:
    """einx.where('b j, b h i j, -> b h i j', mask, sim, value)"""
    return torch.where(mask[:, None, None, :], sim, value)


def where_queries(mask: Tensor, sim: Tensor, value: float) -> Tensor:
    """einx.where('b i, b h i j, -> b h i j', mask, sim, value)"""
    return torch.where(mask[:, None, :, None], sim, value)


def add_key_bias(bias: Tensor, sim: Tensor) -> Tensor:
    """einx.add('b h j, b h i j -> b h i j', bias, sim)"""
    return sim + bias[:, :, None, :]
