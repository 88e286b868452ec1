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


def _set_host_count(counter: Tensor, n: int) -> None:
    counter._pa_host_n = int(n)


def _advance_host_count(counter: Tensor) -> None:
    """Mirror a device count's advance on the host; a captured advance runs again at every
    replay without the host seeing it, so capture ends the mirror."""
    n = getattr(counter, "_pa_host_n", None)
    if n is None:
        return
    capturing = counter.is_cuda and torch.cuda.is_current_stream_capturing()
    counter._pa_host_n = None if capturing else n + 1


class StaticCache:
    """A fixed-capacity poly KV cache whose position count lives on the device.

    Holds the tensors of a module's cache tuple -- order 2: ``(q2, q3, v3, lse23, msg)``
    (poly_attention.py:283-287, 360-363); order n: ``(qs, vs, lses, msgs)``
    (n_poly_attention.py:206-207, 338) -- in buffers of ``capacity`` positions.  Passed as
    ``cache=`` to PolyAttention / NPolyAttention on the fused GPU path, a single-token step
    writes the new token in place (one prologue kernel: the q RMSNorms, the rotary embedding
    and the appends), runs the decode kernels with the position count read on the device,
    advances the count and returns this same object.  Every step then has the same shapes
    and addresses, so a whole decode step can be captured once into a HIP graph
    (``torch.cuda.CUDAGraph``) and replayed per token.

    A step past the capacity is refused with an error when the position count is known on
    the host (eager steps).  Inside captured graphs the count lives only on the device: such a
    step stays inside the buffers (the kernels clamp the count to the capacity, so its token
    is not appended and the last position's msg / lse are rewritten) and sets a device flag,
    which ``check_overflow()`` reads after the loop; the cache is not valid after it.  Size
    the cache for prompt + steps.

    ``counter``: an int32 device tensor [1] shared by the caches of one model's layers (all
    holding the same positions), which the caller advances once per decode step, after
    every layer ran (``StaticCache.advance_counter``): one device add per token instead of
    one per layer.  Without it each cache owns its count and advances it itself.

    With a module's own rotary embedding (``use_rotary_embed=True`` and no external
    ``rotary_pos_emb``) the module's tuple cache holds its keys unrotated and rotates the whole
    cache at every step (poly_attention.py:302-304); a StaticCache holds them rotated at their
    positions instead, each rotated once as it is appended, which gives the same scores.  The
    positions copied in from the tuple cache are rotated in place at the first such step
    (``rotate_prefix``), which must run eagerly, before any graph capture.
    """

    def __init__(self, cache, capacity: int, counter: Tensor | None = None):
        self.order2 = isinstance(cache[0], Tensor)
        if self.order2:
            q2, q3, v3, lse, msg = cache
            qs, vs, lses, msgs = (q2, q3), (v3,), (lse,), (msg,)
        else:
            qs, vs, lses, msgs = cache
        n = qs[0].shape[2]
        if capacity <= n:
            raise ValueError(f"capacity {capacity} must exceed the {n} cached positions")
        self.capacity = int(capacity)
        self.prefix = n                 # positions copied from the tuple cache
        self.keys_rotated = False       # those positions rotated by a module's own rotary

        def grow(t: Tensor) -> Tensor:
            shape = list(t.shape)
            shape[2] = self.capacity
            buf = torch.empty(shape, dtype=t.dtype, device=t.device)
            buf.narrow(2, 0, n).copy_(t)
            return buf

        self.qs = [grow(t) for t in qs]
        self.vs = [grow(t) for t in vs]
        self.lses = [grow(t) for t in lses]
        self.msgs = [grow(t) for t in msgs]
        dev = qs[0].device
        # the next step's n (positions held + 1): its new token goes to position n - 1
        self.shared = counter is not None
        if self.shared:
            if counter.dtype != torch.int32 or counter.numel() != 1 or counter.device != dev:
                raise ValueError("counter: an int32 tensor of one element on the cache's device")
            self.n_step = counter
        else:
            self.n_step = torch.full((1,), n + 1, dtype=torch.int32, device=dev)
            _set_host_count(self.n_step, n + 1)
        # set to 1 by the prologue kernel when a step's position is past the capacity
        self.overflow = torch.zeros(1, dtype=torch.int32, device=dev)

    def rotate_prefix(self, rotary) -> None:
        """Rotate the keys of the positions copied from the tuple cache in place, as the
        module's rotary rotates cached keys (rotate_queries_with_cached_keys: position j for
        key j), once."""
        if self.keys_rotated:
            return
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("StaticCache with the module's own rotary: run one eager step "
                               "before capturing decode steps (the cached prefix is rotated "
                               "once, in place, at the first step)")
        for q in self.qs:
            head = q.narrow(2, 0, self.prefix)
            head.copy_(rotary.rotate_queries_or_keys(head))
        self.keys_rotated = True

    def host_step(self):
        """The next step's n as the host knows it, or None once graph replays (or a counter
        not made by ``make_counter``) advance it on the device only."""
        return getattr(self.n_step, "_pa_host_n", None)

    def check_overflow(self) -> None:
        """Raise if a step ran past the capacity (reads the device flag: synchronises)."""
        if int(self.overflow.item()):
            raise RuntimeError(f"StaticCache overflow: a step ran past the capacity "
                               f"{self.capacity}; its token was not cached")

    @staticmethod
    def make_counter(cache, device=None) -> Tensor:
        """A shared step counter for caches holding the positions of ``cache`` (a module's
        cache tuple): the next step's n."""
        q = cache[0] if isinstance(cache[0], Tensor) else cache[0][0]
        c = torch.full((1,), q.shape[2] + 1, dtype=torch.int32, device=device or q.device)
        _set_host_count(c, q.shape[2] + 1)
        return c

    @staticmethod
    def advance_counter(counter: Tensor) -> None:
        """Count the token every layer of a step has just written (shared counter)."""
        counter.add_(1)
        _advance_host_count(counter)

    def advance(self) -> None:
        """Count the token a step has just written (stream-ordered, capturable); with a
        shared counter the caller advances it once per step instead."""
        if not self.shared:
            self.n_step.add_(1)
            _advance_host_count(self.n_step)

    def seq_len(self) -> int:
        """Cached positions (reads the device count: synchronises)."""
        return min(int(self.n_step.item()) - 1, self.capacity)

    def as_tuple(self):
        """The cache as the module's tuple of tensors (views of the first seq_len() positions)."""
        n = self.seq_len()
        cut = lambda ts: tuple(t.narrow(2, 0, n) for t in ts)  # noqa: E731
        if self.order2:
            return (*cut(self.qs), *cut(self.vs), *cut(self.lses), *cut(self.msgs))
        return cut(self.qs), cut(self.vs), cut(self.lses), cut(self.msgs)
