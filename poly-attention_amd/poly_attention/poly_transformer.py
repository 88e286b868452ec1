"""PolyTransformer: drop-in for ``poly_attention/poly_transformer.py`` (0.3.6).

A stack of blocks, each x <- x + PolyAttention(RMSNorm(x)) then x <- x + FF(x), whose
input to the next block is not the last block's output but a learned mix of every block output
so far ("attention residuals", poly_transformer.py:17-56): per learned pseudo-query p, the
weights over the L outputs h_1..h_L at every position are softmax_l(<p, RMSNorm(h_l)> / sqrt(dim))
and the mix is sum_l w_l h_l.  With ``deep_cross_attention`` each mixing layer but the last
has three pseudo-queries: the first mix is the next block's input, the other two its two
contexts (after their own RMSNorms).

What is forced by interchangeable state dicts and seeded initialisation: the attribute names,
``layers[i]`` = [pre-attention RMSNorm, the two context RMSNorms or None, PolyAttention,
feed-forward (RMSNorm, Linear, GELU, Linear)], ``attn_residuals[i]`` with ``norm_keys`` and
``pseudo_queries``, and the creation order.  Only the attention core runs on the HIP kernels.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn
from torch.nn import Module, ModuleList, RMSNorm

from .poly_attention import Order2PolyAttention


class AttentionResidual(Module):
    """Learned mix of a list of same-shaped hidden states (poly_transformer.py:17-56).

    Returns one mixed tensor for a single pseudo-query, else a tuple with one per query."""

    def __init__(self, dim, num_pseudo_queries=1):
        super().__init__()
        self.norm_keys = RMSNorm(dim)
        self.scale = dim ** -0.5
        self.pseudo_queries = nn.Parameter(torch.randn(num_pseudo_queries, dim) * 0.02)

    def forward(self, hiddens):
        h = torch.stack(list(hiddens)) if isinstance(hiddens, (list, tuple)) else hiddens
        # h: [L, ..., dim]; logits [L, ..., P] = <RMSNorm(h), p> / sqrt(dim), weights over L
        logits = torch.matmul(self.norm_keys(h), self.pseudo_queries.t()) * self.scale
        weights = logits.softmax(dim=0)
        mixed = torch.matmul(weights.movedim(0, -1), h.movedim(0, -2))  # [..., P, dim]
        mixed = mixed.movedim(-2, 0)                                      # [P, ..., dim]
        return mixed[0] if mixed.shape[0] == 1 else tuple(mixed.unbind(0))


def FeedForward(dim, mult=4) -> nn.Sequential:
    """RMSNorm -> Linear(dim, mult*dim) -> GELU -> Linear(mult*dim, dim)
    (poly_transformer.py:60-70)."""
    hidden = int(dim * mult)
    return nn.Sequential(RMSNorm(dim), nn.Linear(dim, hidden), nn.GELU(), nn.Linear(hidden, dim))


class PolyTransformer(Module):
    """Stack of poly-attention blocks with attention residuals (poly_transformer.py:74-150)."""

    def __init__(self, dim, depth, heads=8, dim_head=64, causal=False,
                 deep_cross_attention=False, norm_out=False):
        super().__init__()
        self.depth = depth
        self.deep_cross_attention = deep_cross_attention
        self.layers = ModuleList([])
        self.norm_out = RMSNorm(dim) if norm_out else nn.Identity()
        for _ in range(depth):
            context_norms = ModuleList([RMSNorm(dim), RMSNorm(dim)]) if deep_cross_attention else None
            self.layers.append(ModuleList([
                RMSNorm(dim), context_norms,
                Order2PolyAttention(dim=dim, heads=heads, dim_head=dim_head, causal=causal),
                FeedForward(dim=dim)]))
        # three mixes (input and two contexts) feed each next block under deep cross
        # attention; the last layer mixes only the output
        mixes = [3 if deep_cross_attention and i < depth - 1 else 1 for i in range(depth)]
        self.attn_residuals = ModuleList([AttentionResidual(dim, num_pseudo_queries=p)
                                          for p in mixes])

    def forward(self, x, mask=None, return_layer_hiddens=False):
        outputs: list[Tensor] = []
        contexts = None
        for i, (block, mix) in enumerate(zip(self.layers, self.attn_residuals)):
            pre_norm, context_norms, attn, ff = block
            kwargs = {}
            if contexts is not None:
                kwargs["context"] = tuple(norm(c) for norm, c in zip(context_norms, contexts))
            h = x + attn(pre_norm(x), mask=mask, **kwargs)
            h = h + ff(h)
            outputs.append(h)
            mixed = mix(outputs)
            if self.deep_cross_attention and i < self.depth - 1:
                x, contexts = mixed[0], tuple(mixed[1:])
            else:
                x = mixed
        out = self.norm_out(x)
        return (out, outputs) if return_layer_hiddens else out
