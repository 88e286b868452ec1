"""The fused poly-attention op: drop-in for ``flash_poly_attention`` /
``PolyFlashAttention`` (flash_poly_attention.py:319-456), on libpolyattn's HIP kernels.

``flash_poly_attention(q1, q2, q3, v3, mask=None, context_mask=None, softclamp_value=None,
is_causal=True)`` with q1..v3 of shape [batch, heads, n, dim] computes the order-2 poly
attention with q2 as both the pass-1 queries and the pass-2 keys.  As in the reference op, a
``mask`` [batch, n] masks the keys of both passes and no queries
(flash_poly_attention.py:109-112,261-264).  Masked scores take the eager path's finite fill
-finfo.max (poly_attention.py:68), so a row whose every key is masked is the uniform average
over its keys where the reference's Triton kernel, filling -inf, gives NaN.
"""

from __future__ import annotations

import torch

from . import _lib
from ._helpers import exists


class PolyFlashAttention(torch.autograd.Function):
    """``PolyFlashAttention.apply(q1, q2, q3, v3, mask, softclamp_value, is_causal)``
    (flash_poly_attention.py:319-446): the two forward passes, and in the backward the two
    pass backwards, on the HIP kernels."""

    @staticmethod
    def forward(ctx, q1, q2, q3, v3, mask=None, softclamp_value=None, is_causal=True):
        from . import _ops

        _lib.load()
        scale = q1.shape[-1] ** -0.5
        softclamp = float(softclamp_value or 0.0)
        out, lse, lse23, msg = _ops.order2_forward(q1, q2, q3, v3, mask, bool(is_causal),
                                                   softclamp, scale)
        ctx.save_for_backward(q1, q2, q3, v3, msg, lse23, out, lse, mask)
        ctx.cfg = (bool(is_causal), softclamp, scale)
        ctx.slots = [_ops.slot_ref(t) for t in (q1, q2, q3, v3)]
        return out

    @staticmethod
    def backward(ctx, dout):
        from . import _ops

        *saved, mask = ctx.saved_tensors
        grads = _ops.order2_backward(saved, mask, ctx.cfg, ctx.slots, dout)
        return (*grads, None, None, None)


def flash_poly_attention(q1, q2, q3, v3, mask=None, context_mask=None, softclamp_value=None,
                         is_causal=True):
    assert not exists(context_mask), "context_mask is not supported in flash_poly_attention"
    assert q1.is_cuda, "flash_poly_attention runs on GPU tensors"
    _lib.load()
    if torch.compiler.is_compiling():
        # traced: the per-pass custom ops (opaque to the compiler, with autograd)
        from . import _ops

        out, _, _ = _ops.poly_chain([q1, q2], [q2, q3], [v3], causal=is_causal,
                                    softclamp=softclamp_value, scale=q1.shape[-1] ** -0.5,
                                    key_masks=[mask, mask])
        return out
    return PolyFlashAttention.apply(q1, q2, q3, v3, mask, softclamp_value, is_causal)
