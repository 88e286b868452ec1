"""Growable KV-cache storage behind the reference's cache tuples.

The reference appends to every cached tensor with ``torch.cat`` (poly_attention.py:285-287,
360-361; n_poly_attention.py:206-207, 281-282, 301-302), copying the whole cache each step.
Here each cached tensor is a view ``buf[..., :n, ...]`` of a capacity buffer; appending to
the newest view of a buffer writes the new positions in place and returns a longer view.
Older views (e.g. a cache kept for branching) stay valid: appending to them copies into a
fresh buffer, as does appending to any tensor this module did not create.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

_MIN_CAPACITY = 64


class _Slab:
    """A capacity buffer and the length of its newest handed-out view."""

    __slots__ = ("buf", "length", "dim")

    def __init__(self, buf: Tensor, length: int, dim: int):
        self.buf, self.length, self.dim = buf, length, dim


def _tag(view: Tensor, slab: _Slab, length: int) -> Tensor:
    view._pa_slab = (slab, length)  # noqa: SLF001 - metadata travels with the view object
    return view


def _new_slab(like: Tensor, dim: int, length: int, capacity: int, dtype=None) -> _Slab:
    shape = list(like.shape)
    shape[dim] = capacity
    buf = torch.empty(shape, dtype=dtype or like.dtype, device=like.device)
    return _Slab(buf, length, dim)


def append(cache: Optional[Tensor], new: Tensor, dim: int, dtype=None) -> Tensor:
    """``torch.cat((cache, new), dim)`` with amortised O(len(new)) cost."""
    dim = dim % new.dim()
    k = new.shape[dim]
    if cache is None:
        slab = _new_slab(new, dim, k, max(_MIN_CAPACITY, 2 * k), dtype)
        slab.buf.narrow(dim, 0, k).copy_(new)
        return _tag(slab.buf.narrow(dim, 0, k), slab, k)
    n = cache.shape[dim]
    meta = getattr(cache, "_pa_slab", None)
    if meta is not None:
        slab, length = meta
        if (slab.length == length == n and slab.dim == dim and n + k <= slab.buf.shape[dim]
                and slab.buf.dtype == (dtype or cache.dtype)):
            slab.buf.narrow(dim, n, k).copy_(new)
            slab.length = n + k
            return _tag(slab.buf.narrow(dim, 0, n + k), slab, n + k)
    slab = _new_slab(cache, dim, n + k, max(_MIN_CAPACITY, 2 * (n + k)), dtype)
    slab.buf.narrow(dim, 0, n).copy_(cache)
    slab.buf.narrow(dim, n, k).copy_(new)
    return _tag(slab.buf.narrow(dim, 0, n + k), slab, n + k)


def reserve(cache: Optional[Tensor], like_step: Tensor, dim: int, dtype=None) -> Tensor:
    """Like ``append`` but the new positions are left for a kernel to fill."""
    dim = dim % like_step.dim()
    k = like_step.shape[dim]
    if cache is None:
        slab = _new_slab(like_step, dim, k, max(_MIN_CAPACITY, 2 * k), dtype)
        return _tag(slab.buf.narrow(dim, 0, k), slab, k)
    n = cache.shape[dim]
    meta = getattr(cache, "_pa_slab", None)
    if meta is not None:
        slab, length = meta
        if (slab.length == length == n and slab.dim == dim and n + k <= slab.buf.shape[dim]
                and slab.buf.dtype == (dtype or cache.dtype)):
            slab.length = n + k
            return _tag(slab.buf.narrow(dim, 0, n + k), slab, n + k)
    slab = _new_slab(cache, dim, n + k, max(_MIN_CAPACITY, 2 * (n + k)), dtype)
    slab.buf.narrow(dim, 0, n).copy_(cache)
    return _tag(slab.buf.narrow(dim, 0, n + k), slab, n + k)


def adopt(t: Tensor, dim: int, dtype=None) -> Tensor:
    """Copy a freshly computed full tensor into a capacity buffer (prefill -> cache)."""
    return append(None, t if dtype is None else t.to(dtype), dim)
