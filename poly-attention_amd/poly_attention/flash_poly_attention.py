"""The fused poly-attention op: drop-in for ``flash_poly_attention`` /
``PolyFlashAttention`` (flash_poly_attention.py:319-456), on libpolyattn's HIP kernels.

``flash_poly_attention(q1, q2, q3, v3, mask=None, context_mask=None, softclamp_value=None,
is_causal=True)`` with q1..v3 of shape [batch, heads, n, dim] computes the order-2 poly
attention with q2 as both the pass-1 queries and the pass-2 keys.  The semantics are the
eager reference's (reference_poly_attention(q1, q2, q2, q3, v3, ...)); a ``mask`` masks the
keys of both passes and the queries of pass 2, the way Order2PolyAttention applies it.
"""

from __future__ import annotations

from . import _lib
from ._helpers import exists


def flash_poly_attention(q1, q2, q3, v3, mask=None, context_mask=None, softclamp_value=None,
                         is_causal=True):
    assert not exists(context_mask), "context_mask is not supported in flash_poly_attention"
    assert q1.is_cuda, "flash_poly_attention runs on GPU tensors"
    _lib.load()
    from . import _ops

    out, _, _ = _ops.poly_chain([q1, q2], [q2, q3], [v3], causal=is_causal,
                                softclamp=softclamp_value, scale=q1.shape[-1] ** -0.5,
                                query_mask=mask, key_masks=[mask, mask])
    return out


class PolyFlashAttention:
    """``PolyFlashAttention.apply(q1, q2, q3, v3, mask, softclamp_value, is_causal)``."""

    @staticmethod
    def apply(q1, q2, q3, v3, mask=None, softclamp_value=None, is_causal=True):
        return flash_poly_attention(q1, q2, q3, v3, mask=mask, softclamp_value=softclamp_value,
                                    is_causal=is_causal)
