"""Order-n poly attention: drop-in for ``poly_attention/n_poly_attention.py`` (0.3.6).

Same constructor, forward signature, parameter names / creation order and cache tuple
``(qs_rest_cache, vs_cache, lses, msgs)`` as the reference.  On GPU tensors the chain of
attention passes runs in libpolyattn's HIP kernels (the reference is eager-only here).
"""

from __future__ import annotations

from functools import partial

import torch
from torch import Tensor, einsum, nn
from torch.nn import Module, RMSNorm

from einops.layers.torch import Rearrange

from . import _cache, _lib
from ._helpers import (
    add_key_bias,
    cast_tuple,
    default,
    divisible_by,
    exists,
    first,
    maybe,
    repeat_kv,
    safe_cat,
    softclamp,
    where_keys,
    where_queries,
)
from .poly_attention import (_DECODE_ROWS, _compute_dtype, _q_norms, _static_decode_step,
                             fused_available)
from .rotary import RotaryEmbedding, apply_rotary_emb

LinearNoBias = partial(nn.Linear, bias=False)


class NPolyAttention(Module):
    """Order-n poly attention module (n_poly_attention.py:42-340)."""

    def __init__(self, dim, order=3, heads=8, kv_heads=None, dim_head=64, causal=False,
                 shared_kv=False, softclamp_value=None, use_rotary_embed=False, prenorm=False,
                 separate_context_norms=False, multiply_root_value=False,
                 use_root_value_as_attn_gate=False, attn_gate=False, use_flash_kernel=None):
        super().__init__()
        assert order > 1, "order must be greater than 1"
        self.norm = RMSNorm(dim) if prenorm else nn.Identity()

        self.context_norms = None
        if separate_context_norms and prenorm:
            self.context_norms = nn.ModuleList([RMSNorm(dim) for _ in range(order)])

        # not in the reference's signature (it has no fused order-n path); None = automatic
        self.use_flash_kernel = default(use_flash_kernel, fused_available())
        assert not (self.use_flash_kernel and not fused_available()), \
            "fused poly attention is not available"

        self.scale = dim_head ** -0.5

        kv_heads = default(kv_heads, heads)
        assert divisible_by(heads, kv_heads), "heads must be divisible by kv_heads"

        self.heads = heads
        self.kv_heads = kv_heads

        dim_inner = dim_head * heads
        dim_inner_kv = dim_head * kv_heads

        self.causal = causal
        self.shared_kv = shared_kv
        self.softclamp_value = softclamp_value

        self.multiply_root_value = multiply_root_value
        self.use_root_value_as_attn_gate = use_root_value_as_attn_gate
        self.attn_gate = attn_gate

        self.is_gqa = heads != kv_heads

        assert not (use_root_value_as_attn_gate and (self.is_gqa or self.shared_kv)), \
            "cannot use root value as attention gate if using GQA or shared KV"

        q_split = 2 if attn_gate else 1
        self.split_q = Rearrange("b n (split h d) -> split b h n d", split=q_split, h=self.heads)

        self.has_root_v = multiply_root_value and not shared_kv
        kv1_split = 2 if self.has_root_v else 1
        self.split_kv1 = Rearrange("b n (split h d) -> split b h n d", split=kv1_split,
                                   h=self.kv_heads)

        kv_split = 1 if shared_kv else 2
        self.split_kv = Rearrange("b n (split h d) -> split b h n d", split=kv_split,
                                  h=self.kv_heads)

        self.merge_heads = Rearrange("b h n d -> b n (h d)")

        if self.is_gqa:
            self.num_rep = heads // kv_heads

        self.order = order

        self.to_q = LinearNoBias(dim, dim_inner * q_split)

        kv_mult = 1 if shared_kv else 2
        self.to_kvs = nn.ModuleList([
            LinearNoBias(dim, dim_inner_kv * kv1_split),
            *[LinearNoBias(dim, dim_inner_kv * kv_mult) for _ in range(order - 1)],
        ])

        self.q_norms = nn.ModuleList([RMSNorm(dim_head) for _ in range(order + 1)])

        self.rotary_emb = RotaryEmbedding(dim_head) if use_rotary_embed else None

        self.to_out = nn.Linear(dim_inner, dim)

    def _use_fused(self, t: Tensor) -> bool:
        if not self.use_flash_kernel or not t.is_cuda:
            return False
        _lib.load()
        return True

    def _proj(self, layer: nn.Linear, x: Tensor) -> Tensor:
        """A projection (the reference calls the nn.Linear directly); on the fused path
        decode-sized inputs stream the weight on pa_linear_small, larger ones take the split-K
        weight gradient in training."""
        if self._use_fused(x):
            from . import _ops

            if x.numel() <= _DECODE_ROWS * x.shape[-1]:
                return _ops.linear(layer, x)
            return _ops.layer_train(layer, x)
        return layer(x)

    def _projs(self, layers, xs):
        """[layer(x) for layer, x in zip(layers, xs)]; on the fused path decode-sized
        projections of one input share pa_linear_small launches."""
        x0 = xs[0]
        if x0.numel() <= _DECODE_ROWS * x0.shape[-1] and self._use_fused(x0):
            from . import _ops

            return _ops.linear_many(list(layers), list(xs))
        return [layer(x) for layer, x in zip(layers, xs)]

    def forward(self, x, context: Tensor | tuple[Tensor, ...] | None = None, mask=None,
                context_mask: Tensor | tuple[Tensor | None, ...] | None = None,
                rotary_pos_emb=None, cache=None, return_cache=False):
        seq_len, device = x.shape[-2], x.device

        has_cache = exists(cache)
        if has_cache:
            assert seq_len == 1, "sequence length must be 1 when using kv cache"

        orig_x = x
        x = self.norm(x)

        has_context = exists(context)
        context = default(context, orig_x)
        context = cast_tuple(context, self.order)
        assert len(context) == self.order

        if self.multiply_root_value:
            assert first(context).shape[-2] == seq_len, (
                "first context sequence length (context[0]) must match base sequence x when "
                "multiply_root_value is True")

        if exists(context_mask):
            context_mask = cast_tuple(context_mask, self.order)
            assert len(context_mask) == self.order
        elif not has_context and exists(mask):
            context_mask = (mask,) * self.order
        else:
            context_mask = (None,) * self.order

        if exists(self.context_norms):
            context = tuple(norm(c) for c, norm in zip(context, self.context_norms))
        else:
            context = context if has_context else ((x,) * self.order)

        # the projections (the reference computes to_q first; they are independent, and on the
        # fused decode path the ones of a shared input go out together)
        if x.dim() == 3 and x.numel() > _DECODE_ROWS * x.shape[-1] and self._use_fused(x):
            # fused path: one GEMM for the projections of a shared input, views for the heads
            from . import _ops

            q_and_maybe_gates, kv1, *kvs_rest = _ops.project_heads(
                [self.to_q, *self.to_kvs], [x, *context],
                [(2 if self.attn_gate else 1, self.heads),
                 (2 if self.has_root_v else 1, self.kv_heads),
                 *[(1 if self.shared_kv else 2, self.kv_heads)] * (self.order - 1)])
        else:
            q_proj, kv1_proj, *rest_proj = self._projs([self.to_q, *self.to_kvs], [x, *context])
            q_and_maybe_gates = self.split_q(q_proj)
            kv1 = self.split_kv1(kv1_proj)
            kvs_rest = [self.split_kv(p) for p in rest_proj]

        if self.attn_gate:
            q1, gates = q_and_maybe_gates
        else:
            q1 = first(q_and_maybe_gates)

        if self.shared_kv:
            qs_rest = (first(kv1), *[first(kv) for kv in kvs_rest])
            root_value = first(qs_rest)
            vs_for_aggregation = qs_rest[1:]
        else:
            qs_rest = (first(kv1), *[first(kv) for kv in kvs_rest])
            vs_for_aggregation = tuple(kv[1] for kv in kvs_rest)
            root_value = kv1[1] if self.has_root_v else None

        qs = (q1, *qs_rest)

        # the root-value / gate epilogue (n_poly_attention.py:315-326): fused into the final
        # pass on the HIP path's order-2 chain, else the torch element-wise tail below
        epilogue = (root_value if self.multiply_root_value else None,
                    gates if self.attn_gate else None, self.use_root_value_as_attn_gate)
        epilogue_done = False

        if isinstance(cache, _cache.StaticCache):
            # fixed-capacity cache: norms, rotary and appends fused into the decode step
            out = _static_decode_step(self, qs, vs_for_aggregation, mask, context_mask,
                                      rotary_pos_emb, cache)
            new_cache = cache
            if exists(root_value) and self.is_gqa:
                root_value = repeat_kv(root_value, self.num_rep)
        else:
            # the q norms and the external rotary (fused into one kernel on the GPU path)
            qs = _q_norms(self, self.q_norms, qs, rotary_pos_emb)

            q1 = first(qs)
            qs_rest = qs[1:]

            if self._use_fused(q1):
                out, new_cache = self._fused_core(q1, qs_rest, vs_for_aggregation, mask,
                                                  context_mask, rotary_pos_emb, cache,
                                                  return_cache, epilogue)
                epilogue_done = True
            else:
                out, new_cache, root_value = self._eager_core(q1, qs_rest, vs_for_aggregation,
                                                              root_value, mask, context_mask,
                                                              rotary_pos_emb, cache, device)

        if self.multiply_root_value and not epilogue_done:
            if self.use_root_value_as_attn_gate:
                root_value = root_value.sigmoid()
            out = root_value * out

        if self.attn_gate and not epilogue_done:
            out = out * gates.sigmoid()

        out = self._proj(self.to_out, self.merge_heads(out))

        if not return_cache:
            return out
        return out, new_cache

    # -------------------------------------------------------------------------------------

    def _eager_core(self, q1, qs_rest, vs_for_aggregation, root_value, mask, context_mask,
                    rotary_pos_emb, cache, device):
        """n_poly_attention.py:196-313 (eager path)."""
        has_cache = exists(cache)
        if has_cache:
            c_qs, c_vs, c_lses, c_msgs = cache
        else:
            c_qs = (None,) * self.order
            c_vs = (None,) * (self.order - 1)
            c_lses = (None,) * (self.order - 1)
            c_msgs = (None,) * (self.order - 1)

        qs_rest_cache = tuple(safe_cat((cq, q), dim=-2) for cq, q in zip(c_qs, qs_rest))
        vs_cache = tuple(safe_cat((cv, v), dim=-2) for cv, v in zip(c_vs, vs_for_aggregation))

        if self.is_gqa:
            match_kv = maybe(lambda t: repeat_kv(t, self.num_rep))
            qs_rest_left = tuple(match_kv(t) for t in qs_rest)
            qs_rest_right = tuple(match_kv(t) for t in qs_rest_cache)
            vs_full = tuple(match_kv(t) for t in vs_cache)
            if exists(root_value):
                root_value = match_kv(root_value)
        else:
            qs_rest_left = qs_rest
            qs_rest_right = qs_rest_cache
            vs_full = vs_cache

        q_left_list = [q1, *qs_rest_left[:-1]]
        q_right_list = list(qs_rest_right)

        if not exists(rotary_pos_emb) and exists(self.rotary_emb):
            rotated = [self.rotary_emb.rotate_queries_with_cached_keys(ql, qr)
                       for ql, qr in zip(q_left_list, q_right_list)]
            q_left_list, q_right_list = zip(*rotated)

        scores = []
        for idx, (ql, qr, cmask) in enumerate(zip(q_left_list, q_right_list, context_mask)):
            is_first = idx == 0
            score = einsum("b h i d, b h j d -> b h i j", ql, qr) * self.scale
            if exists(self.softclamp_value):
                score = softclamp(score, self.softclamp_value)
            mask_value = -torch.finfo(score.dtype).max
            if self.causal and not has_cache:
                i, j = score.shape[-2:]
                causal_mask = torch.ones((i, j), device=device, dtype=torch.bool).triu(1)
                score = score.masked_fill(causal_mask, mask_value)
            if exists(cmask):
                score = where_keys(cmask, score, mask_value)
            if is_first and exists(mask):
                score = where_queries(mask, score, mask_value)
            scores.append(score)

        out = vs_full[-1]
        current_scores_k = scores[-1]
        new_cache_lses = []
        new_cache_msgs = []

        for k in range(self.order - 1, 1, -1):
            lse_k_step = current_scores_k.logsumexp(dim=-1)
            attn_k = current_scores_k.softmax(dim=-1)
            msg_step = einsum("b h i j, b h j d -> b h i d", attn_k, out)
            idx = (self.order - 1) - k
            lse_k_full = safe_cat((c_lses[idx], lse_k_step), dim=-1)
            msg_full = safe_cat((c_msgs[idx], msg_step), dim=-2)
            new_cache_msgs.append(msg_full)
            new_cache_lses.append(lse_k_full)
            out = vs_full[k - 2] * msg_full.to(vs_full[k - 2].dtype)
            current_scores_k = add_key_bias(lse_k_full.to(scores[k - 1].dtype), scores[k - 1])

        lse_1_step = current_scores_k.logsumexp(dim=-1)
        attn_1 = current_scores_k.softmax(dim=-1)
        msg_1_step = einsum("b h i j, b h j d -> b h i d", attn_1, out)
        idx = self.order - 2
        lse_1_full = safe_cat((c_lses[idx], lse_1_step), dim=-1)
        msg_1_full = safe_cat((c_msgs[idx], msg_1_step), dim=-2)
        new_cache_msgs.append(msg_1_full)
        new_cache_lses.append(lse_1_full)

        scores12 = add_key_bias(lse_1_full.to(scores[0].dtype), scores[0])
        attn12 = scores12.softmax(dim=-1)
        out = einsum("b h i j, b h j d -> b h i d", attn12, msg_1_full.to(attn12.dtype))

        new_cache = (qs_rest_cache, vs_cache, tuple(new_cache_lses), tuple(new_cache_msgs))
        return out, new_cache, root_value

    def _fused_core(self, q1, qs_rest, vs, mask, context_mask, rotary_pos_emb, cache,
                    return_cache, epilogue):
        """The order-n chain on the HIP kernels (qs_rest / vs stay at kv_heads), with the
        module epilogue applied: fused into the final pass on the order-2 chain's path."""
        from . import _ops

        order = self.order
        rep = self.num_rep if self.is_gqa else 1
        dt = _compute_dtype(q1, *qs_rest, *vs)
        q1 = q1.to(dt)
        qs_rest = tuple(q.to(dt) for q in qs_rest)
        vs = tuple(v.to(dt) for v in vs)
        module_rotary = not exists(rotary_pos_emb) and exists(self.rotary_emb)

        if not exists(cache):
            q_left, q_right = [q1, *qs_rest[:-1]], list(qs_rest)
            if module_rotary:
                rotated = [self.rotary_emb.rotate_queries_with_cached_keys(ql, qr)
                           for ql, qr in zip(q_left, q_right)]
                q_left, q_right = (list(t) for t in zip(*rotated))
            out, lses, msgs = _ops.poly_chain(q_left, q_right, list(vs), causal=self.causal,
                                              softclamp=self.softclamp_value, scale=self.scale,
                                              query_mask=mask, key_masks=list(context_mask),
                                              epilogue=epilogue)
            new_cache = None
            if return_cache:
                new_cache = (
                    tuple(_cache.adopt(q, -2) for q in qs_rest),
                    tuple(_cache.adopt(v, -2) for v in vs),
                    tuple(_cache.adopt(repeat_kv(l[:, :, :, None], rep)[..., 0], -1) for l in lses),
                    tuple(_cache.adopt(repeat_kv(m, rep), -2) for m in msgs),
                )
            return out, new_cache

        c_qs, c_vs, c_lses, c_msgs = cache
        qs_cache = [_cache.append(cq, q.to(cq.dtype), -2) for cq, q in zip(c_qs, qs_rest)]
        vs_cache = [_cache.append(cv, v.to(cv.dtype), -2) for cv, v in zip(c_vs, vs)]
        q_left, q_right = [q1, *qs_rest[:-1]], list(qs_cache)
        if module_rotary:
            rotated = [self.rotary_emb.rotate_queries_with_cached_keys(ql, qr)
                       for ql, qr in zip(q_left, q_right)]
            q_left, q_right = (list(t) for t in zip(*rotated))

        needs_grad = torch.is_grad_enabled() and any(
            t.requires_grad for t in (q1, *qs_rest, *vs, *c_qs, *c_vs, *c_lses, *c_msgs))
        masked = exists(mask) or any(exists(m) for m in context_mask)
        if needs_grad or masked:
            out, new_cache = self._fused_step_autograd(q_left, q_right, vs_cache, c_lses, c_msgs,
                                                       rep, qs_cache, mask, context_mask)
            return _ops.apply_epilogue(out, epilogue), new_cache

        lses_full = [_cache.reserve(l, l[:, :, :1], -1) for l in c_lses]
        msgs_full = [_cache.reserve(m, m[:, :, :1], -2) for m in c_msgs]
        out = _ops.poly_decode_step(q_left, q_right, vs_cache, msgs_full, lses_full,
                                    kv_heads=self.kv_heads, heads=self.heads,
                                    softclamp=self.softclamp_value, scale=self.scale)
        return _ops.apply_epilogue(out, epilogue), (tuple(qs_cache), tuple(vs_cache),
                                                     tuple(lses_full), tuple(msgs_full))

    def _fused_step_autograd(self, q_left, q_right, vs_cache, c_lses, c_msgs, rep, qs_cache,
                             mask=None, context_mask=None):
        """A differentiable (or masked) cached step: the reference's level loop with HIP
        passes.  Level l's context mask masks the keys of its whole cache, ``mask`` the new
        query of the final level (n_poly_attention.py:253-259)."""
        context_mask = list(context_mask) if context_mask is not None else [None] * self.order
        from . import _ops

        order = self.order
        H = self.heads
        lses_full, msgs_full = [], []
        lse_next = msg_next = None
        out = None
        for lvl in range(order - 1, -1, -1):
            idx = order - 1 - lvl  # cache index of this level's msg / lse (deepest first)
            k = q_right[lvl]
            if lvl == order - 1:
                v, vmul, bias = vs_cache[-1], None, None
            elif lvl == 0:
                v, vmul, bias = msg_next, None, lse_next
            else:
                v, vmul, bias = repeat_kv(vs_cache[lvl - 1], rep), msg_next, lse_next
            q = q_left[lvl]
            if bias is not None:  # key-side tensors at H heads
                k = repeat_kv(k, rep)
                if q.shape[1] != H:
                    q = repeat_kv(q, rep)
            o, lse = _ops.attn_pass(q, k, v, vmul, bias, key_mask=context_mask[lvl],
                                    query_mask=mask if lvl == 0 else None,
                                    softclamp=self.softclamp_value, scale=self.scale,
                                    may_degenerate=True)
            if lvl > 0:
                o_h = repeat_kv(o, H // o.shape[1])
                l_h = repeat_kv(lse[:, :, :, None], H // lse.shape[1])[..., 0]
                msg_next = torch.cat((c_msgs[idx], o_h.to(c_msgs[idx].dtype)), dim=-2)
                lse_next = torch.cat((c_lses[idx], l_h.to(c_lses[idx].dtype)), dim=-1)
                msgs_full.append(msg_next)
                lses_full.append(lse_next)
            else:
                out = o
        return out, (tuple(qs_cache), tuple(vs_cache), tuple(lses_full), tuple(msgs_full))
