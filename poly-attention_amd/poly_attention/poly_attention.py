"""Order-2 poly attention (Chakrabarti et al., https://arxiv.org/abs/2602.02422).

Drop-in for ``poly_attention/poly_attention.py`` of lucidrains/poly-attention 0.3.6: same
``reference_poly_attention`` function, same ``Order2PolyAttention`` constructor, forward
signature, parameter names / creation order and KV-cache tuple.  On GPU tensors the
attention core runs in the HIP kernels of libpolyattn (fused forward and backward passes,
split-K decode); ``reference_poly_attention`` is the reference's eager formulation and
serves CPU tensors and ``use_flash_kernel=False``.
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
from .rotary import RotaryEmbedding, apply_rotary_emb

LinearNoBias = partial(nn.Linear, bias=False)

# inputs of at most this many rows (a decode step's batch) take pa_linear_small projections
_DECODE_ROWS = 16


def fused_available() -> bool:
    """The HIP path's plugin switch: libpolyattn.so loads (poly_attention.py:17-20)."""
    return _lib.available()


def _q_norms(module, norms, qs, rotary_pos_emb=None):
    """The per-head q/k RMSNorms (poly_attention.py:271, n_poly_attention.py:188), then the
    external rotary when given (:275-276, :190-191): on the fused GPU path through pa_rmsnorm
    (forward and backward, the rotation inside the same kernel), else torch.nn.RMSNorm and
    apply_rotary_emb.  Without gradients and rotary the norms of a layer go out in one launch
    (pa_rmsnorm_fwd_many)."""
    many = _q_norms_one_launch(module, norms, qs, rotary_pos_emb)
    if many is not None:
        return many
    out = []
    for norm, q in zip(norms, qs):
        if (module._use_fused(q) and isinstance(norm, RMSNorm)
                and tuple(norm.normalized_shape) == (q.shape[-1],)):
            from . import _ops

            if _ops.rms_supported(q, norm.weight, rotary_pos_emb):
                out.append(_ops.rms_norm(q, norm.weight, norm.eps, rotary_pos_emb))
                continue
            if _ops.rms_supported(q, norm.weight):
                q = _ops.rms_norm(q, norm.weight, norm.eps)
                out.append(apply_rotary_emb(rotary_pos_emb, q) if exists(rotary_pos_emb) else q)
                continue
        q = norm(q)
        out.append(apply_rotary_emb(rotary_pos_emb, q) if exists(rotary_pos_emb) else q)
    return tuple(out)


def _q_norms_one_launch(module, norms, qs, rotary_pos_emb):
    """The norms of ``qs`` in one pa_rmsnorm_fwd_many launch when that applies: the fused GPU
    path, no gradient, no rotary, not under torch.compile, every norm an RMSNorm over the
    head dim of a tensor pa_rmsnorm takes, one dtype and head dim.  Else None."""
    from . import _lib, _ops

    if exists(rotary_pos_emb) or not 1 <= len(qs) <= _lib.PA_RMS_MAX_ITEMS:
        return None
    if torch.compiler.is_compiling():
        return None
    weights = [getattr(n, "weight", None) for n in norms]
    if torch.is_grad_enabled() and (any(q.requires_grad for q in qs) or
                                    any(w is not None and w.requires_grad for w in weights)):
        return None
    q0 = qs[0]
    for norm, q in zip(norms, qs):
        if not (isinstance(norm, RMSNorm) and module._use_fused(q)
                and tuple(norm.normalized_shape) == (q.shape[-1],)):
            return None
        if q.dtype != q0.dtype or q.shape[-1] != q0.shape[-1] or q.device != q0.device:
            return None
        if not _ops.rms_supported(q, norm.weight):
            return None
    return tuple(_ops.rms_norm_many(qs, weights, [n.eps for n in norms]))


def _static_decode_step(module, qs, vs, mask, context_mask, rotary_pos_emb,
                        cache: _cache.StaticCache) -> Tensor:
    """A single-token step on a StaticCache, for both module orders.

    One prologue launch does the q RMSNorms (poly_attention.py:271, n_poly_attention.py:188),
    the external rotary (:275-276, :190-191) and the cache appends (:284-286, :206-207);
    the decode kernels then read the position count on the device, and the count advances.
    ``qs`` = (q1, ..., q_{order+1}) are the raw projections [B, h, 1, d], ``vs`` the
    aggregation values (v3, ...).  Returns the output [B, heads, 1, d]."""
    from . import _ops

    q1 = qs[0]
    order = len(qs) - 1
    if not (module.use_flash_kernel and q1.is_cuda):
        raise RuntimeError("a StaticCache needs the fused GPU path (libpolyattn)")
    _lib.load()
    if q1.shape[-2] != 1:
        raise ValueError("a StaticCache step takes exactly one new token")
    if exists(mask) or any(exists(m) for m in context_mask):
        raise NotImplementedError("masks are not supported with a StaticCache")
    module_rotary = not exists(rotary_pos_emb) and exists(module.rotary_emb)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (*qs, *vs)):
        raise RuntimeError("StaticCache decode is inference-only: run it under torch.no_grad()")
    if len(cache.qs) != order or len(cache.vs) != order - 1:
        raise ValueError(f"StaticCache of order {len(cache.qs)} passed to an order-{order} module")
    n_host = cache.host_step()
    if n_host is not None and n_host > cache.capacity:
        raise RuntimeError(f"StaticCache is full: a step needs position {n_host - 1}, the "
                           f"capacity is {cache.capacity}")
    dt = cache.qs[0].dtype
    if any(t.dtype != dt for t in (*qs, *vs)):
        raise TypeError("StaticCache: the projections and the cache must share one dtype")
    norms = list(module.q_norms)
    eps = {n.eps for n in norms}
    if len(eps) != 1:
        raise NotImplementedError("q norms with different eps")
    eps = eps.pop()
    if eps is None:  # torch's rms_norm default: epsilon of the op-math type (fp32)
        eps = torch.finfo(torch.float32).eps
    angles = None
    if exists(rotary_pos_emb):
        if rotary_pos_emb.dim() not in (1, 2):
            raise NotImplementedError("rotary_pos_emb must be [positions, dim] or [dim]")
        angles = rotary_pos_emb if rotary_pos_emb.dim() == 1 else rotary_pos_emb[-1]
    if module_rotary:
        # the module's own rotary (poly_attention.py:302-304, n_poly_attention.py:224-229)
        # rotates every cached key at its position on every step; the StaticCache keeps its
        # keys rotated instead, each once, as the prologue appends it
        cache.rotate_prefix(module.rotary_emb)
    q_left = [torch.empty(q.shape[0], q.shape[1], 1, q.shape[3], dtype=dt, device=q.device)
              for q in qs[:-1]]
    items = []
    for i, (q, norm) in enumerate(zip(qs, norms)):
        w = norm.weight if norm.weight is not None else torch.ones(q.shape[-1], device=q.device)
        items.append((q, w, angles is not None or module_rotary, q_left[i] if i < order else None,
                      cache.qs[i - 1] if i >= 1 else None))
    items += [(v, None, False, None, buf) for v, buf in zip(vs, cache.vs)]
    rot = module.rotary_emb if module_rotary else None
    _ops.decode_prologue(items, eps=eps, angles=angles, n_dev=cache.n_step,
                         capacity=cache.capacity, overflow=cache.overflow,
                         inv_freq=rot.freqs if rot is not None else None,
                         interp=rot.interpolate_factor if rot is not None else 1.0)
    out = _ops.poly_decode_step(q_left, cache.qs, cache.vs, cache.msgs, cache.lses,
                                kv_heads=module.kv_heads, heads=module.heads,
                                softclamp=module.softclamp_value, scale=module.scale,
                                n_dev=cache.n_step)
    cache.advance()
    return out


# attention


def reference_poly_attention(q1, q2_pass1, q2_pass2, q3, v3, mask=None, context_mask=None,
                             softclamp_value=None, causal=False, cache=None):
    """Eager order-2 poly attention, as poly_attention.py:48-116.

    Pass 1 (q2 attends to q3) gives lse23 and msg; pass 2 (q1 attends to q2) adds lse23 as a
    key bias and aggregates msg.  Masked scores take the finite value -finfo.max.
    Returns (out, lse23_step, msg_step).
    """
    scale = q1.shape[-1] ** -0.5
    has_cache = exists(cache)
    context_mask1, context_mask2 = context_mask if exists(context_mask) else (None, None)

    sim23 = einsum("b h i d, b h j d -> b h i j", q2_pass1, q3) * scale
    if exists(softclamp_value):
        sim23 = softclamp(sim23, softclamp_value)
    mask_value = -torch.finfo(sim23.dtype).max
    if causal and not has_cache:
        i, j = sim23.shape[-2:]
        causal_mask = torch.ones((i, j), device=sim23.device, dtype=torch.bool).triu(1)
        sim23 = sim23.masked_fill(causal_mask, mask_value)
    if exists(context_mask2):
        sim23 = where_keys(context_mask2, sim23, mask_value)

    lse23_step = sim23.logsumexp(dim=-1)
    attn23 = sim23.softmax(dim=-1)
    msg_step = einsum("b h i j, b h j d -> b h i d", attn23, v3)

    _, _, _, clse23, cmsg = cache if has_cache else (None, None, None, None, None)
    lse23 = safe_cat((clse23, lse23_step), dim=-1)
    msg = safe_cat((cmsg, msg_step), dim=-2)

    sim12 = einsum("b h i d, b h j d -> b h i j", q1, q2_pass2) * scale
    if exists(softclamp_value):
        sim12 = softclamp(sim12, softclamp_value)
    if causal and not has_cache:
        i, j = sim12.shape[-2:]
        causal_mask = torch.ones((i, j), device=sim12.device, dtype=torch.bool).triu(1)
        sim12 = sim12.masked_fill(causal_mask, mask_value)
    if exists(context_mask1):
        sim12 = where_keys(context_mask1, sim12, mask_value)
    if exists(mask):
        sim12 = where_queries(mask, sim12, mask_value)

    sim12 = add_key_bias(lse23.to(sim12.dtype), sim12)
    attn12 = sim12.softmax(dim=-1)
    out = einsum("b h i j, b h j d -> b h i d", attn12, msg.to(attn12.dtype))
    return out, lse23_step, msg_step


def _compute_dtype(*ts: Tensor) -> torch.dtype:
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    dt = ts[0].dtype
    for t in ts[1:]:
        dt = torch.promote_types(dt, t.dtype)
    return dt


# poly attention


class Order2PolyAttention(Module):
    """Order-2 poly attention module (poly_attention.py:120-365)."""

    def __init__(self, dim, heads=8, kv_heads=None, dim_head=64, causal=False, shared_kv=False,
                 softclamp_value=None, use_rotary_embed=False, prenorm=False,
                 separate_context_norms=False, multiply_root_value=False,
                 use_root_value_as_attn_gate=False, attn_gate=False, use_flash_kernel=None):
        super().__init__()
        self.norm = RMSNorm(dim) if prenorm else nn.Identity()

        self.context_norms = None
        if separate_context_norms and prenorm:
            self.context_norms = nn.ModuleList([RMSNorm(dim), RMSNorm(dim)])

        # use_flash_kernel: None = the HIP path whenever libpolyattn loads and the tensors are
        # on the GPU; True = demand it; False = always eager
        self._flash_requested = use_flash_kernel
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

        kv_split = 1 if self.shared_kv else 2
        self.split_kv = Rearrange("b n (split h d) -> split b h n d", split=kv_split,
                                  h=self.kv_heads)

        self.merge_heads = Rearrange("b h n d -> b n (h d)")

        if self.is_gqa:
            self.num_rep = heads // kv_heads

        self.to_q = LinearNoBias(dim, dim_inner * q_split)

        kv_mult = 1 if shared_kv else 2
        self.to_kvs = nn.ModuleList([
            LinearNoBias(dim, dim_inner_kv * kv1_split),
            LinearNoBias(dim, dim_inner_kv * kv_mult),
        ])

        self.q_norms = nn.ModuleList([RMSNorm(dim_head), RMSNorm(dim_head), RMSNorm(dim_head)])

        self.rotary_emb = RotaryEmbedding(dim_head) if use_rotary_embed else None

        self.to_out = nn.Linear(dim_inner, dim)

    # -------------------------------------------------------------------------------------

    def _use_fused(self, t: Tensor) -> bool:
        if not self.use_flash_kernel or not t.is_cuda:
            return False
        _lib.load()  # a GPU tensor with the fused path requested: a missing library is fatal
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

        # contexts

        has_context = exists(context)
        context = default(context, orig_x)
        context = cast_tuple(context, 2)
        assert len(context) == 2

        if self.multiply_root_value:
            assert first(context).shape[-2] == seq_len, (
                "first context sequence length (context[0]) must match base sequence x when "
                "multiply_root_value is True")

        explicit_context_mask = exists(context_mask)
        if exists(context_mask):
            context_mask = cast_tuple(context_mask, 2)
            assert len(context_mask) == 2
        elif not has_context and exists(mask):
            context_mask = (mask, mask)
        else:
            context_mask = (None, None)

        if exists(self.context_norms):
            ctx1, ctx2 = (norm(c) for c, norm in zip(context, self.context_norms))
        else:
            ctx1, ctx2 = context if has_context else (x, x)

        # the projections (the reference computes to_q first; they are independent, and on the
        # fused decode path the ones of a shared input go out together)
        if x.dim() == 3 and x.numel() > _DECODE_ROWS * x.shape[-1] and self._use_fused(x):
            # fused path: one GEMM for the projections of a shared input, views for the heads
            from . import _ops

            q_and_maybe_gates, kv1, kv2 = _ops.project_heads(
                [self.to_q, *self.to_kvs], [x, ctx1, ctx2],
                [(2 if self.attn_gate else 1, self.heads),
                 (2 if self.has_root_v else 1, self.kv_heads),
                 (1 if self.shared_kv else 2, self.kv_heads)])
        else:
            q_proj, kv1_proj, kv2_proj = self._projs([self.to_q, *self.to_kvs], [x, ctx1, ctx2])
            q_and_maybe_gates = self.split_q(q_proj)
            kv1 = self.split_kv1(kv1_proj)
            kv2 = self.split_kv(kv2_proj)

        if self.attn_gate:
            q1, gates = q_and_maybe_gates
        else:
            q1 = first(q_and_maybe_gates)

        if self.shared_kv:
            qs = (q1, first(kv1), first(kv2))
            v2, v3 = first(kv1), first(kv2)
        else:
            q2 = first(kv1)
            v2 = kv1[1] if self.has_root_v else None
            q3, v3 = kv2
            qs = (q1, q2, q3)

        # the root-value / gate epilogue (poly_attention.py:342-351): fused into the final
        # pass on the HIP path, else the torch element-wise tail below
        epilogue = (v2 if self.multiply_root_value else None,
                    gates if self.attn_gate else None, self.use_root_value_as_attn_gate)
        epilogue_done = False

        if isinstance(cache, _cache.StaticCache):
            # fixed-capacity cache: norms, rotary and appends fused into the decode step
            out = _static_decode_step(self, qs, (v3,), mask, context_mask, rotary_pos_emb,
                                      cache)
            new_cache = cache
            v2 = repeat_kv(v2, self.num_rep) if self.is_gqa and exists(v2) else v2
        else:
            # the q norms and the external rotary (fused into one kernel on the GPU path), or
            # the norms applied by the attention passes as they load q1 / q2 / q3
            norms_on_load = self._norms_on_load(qs, v3, mask, context_mask, rotary_pos_emb,
                                                cache, return_cache)
            if norms_on_load is None:
                qs = _q_norms(self, self.q_norms, qs, rotary_pos_emb)

            q1, q2, q3 = qs

            # dispatch: the HIP kernels take every case on the GPU (masks, contexts, GQA,
            # caches); an explicitly requested fused kernel still refuses an explicit
            # context_mask, as the reference does (poly_attention.py:310)
            if self._flash_requested is True and explicit_context_mask:
                assert not any(exists(m) for m in context_mask), \
                    "context_mask is not supported in flash poly attention"

            if self._use_fused(q1):
                out, new_cache = self._fused_core(q1, q2, q3, v3, mask, context_mask,
                                                  rotary_pos_emb, cache, return_cache, epilogue,
                                                  norms_on_load)
                epilogue_done = True
            else:
                out, new_cache, v2 = self._eager_core(q1, q2, q3, v2, v3, mask, context_mask,
                                                      rotary_pos_emb, cache, return_cache)

        # elementwise multiply root values

        if self.multiply_root_value and not epilogue_done:
            if self.use_root_value_as_attn_gate:
                v2 = v2.sigmoid()
            out = v2 * out

        if self.attn_gate and not epilogue_done:
            out = out * gates.sigmoid()

        out = self._proj(self.to_out, self.merge_heads(out))

        if not return_cache:
            return out
        return out, new_cache

    # -------------------------------------------------------------------------------------

    def _eager_core(self, q1, q2, q3, v2, v3, mask, context_mask, rotary_pos_emb, cache,
                    return_cache):
        """poly_attention.py:283-365 (eager path)."""
        has_cache = exists(cache)
        cq2, cq3, cv3, clse23, cmsg = cache if has_cache else (None, None, None, None, None)

        q2_cache = safe_cat((cq2, q2), dim=-2)
        q3_cache = safe_cat((cq3, q3), dim=-2)
        v3_cache = safe_cat((cv3, v3), dim=-2)

        if self.is_gqa:
            match_kv = maybe(lambda t: repeat_kv(t, self.num_rep))
            q2, q3, v2, v3 = map(match_kv, (q2, q3, v2, v3))
            q2_full, q3_full, v3_full = map(match_kv, (q2_cache, q3_cache, v3_cache))
        else:
            q2_full, q3_full, v3_full = q2_cache, q3_cache, v3_cache

        q2_left = q2
        q2_right = q2_full

        if not exists(rotary_pos_emb) and exists(self.rotary_emb):
            q1, q2_right = self.rotary_emb.rotate_queries_with_cached_keys(q1, q2_right)
            q2_left, q3_full = self.rotary_emb.rotate_queries_with_cached_keys(q2_left, q3_full)

        out, lse23_step, msg_step = reference_poly_attention(
            q1, q2_left, q2_right, q3_full, v3_full, mask=mask, context_mask=context_mask,
            softclamp_value=self.softclamp_value, causal=self.causal, cache=cache)

        new_cache = None
        if return_cache:
            lse23_full = safe_cat((clse23, lse23_step), dim=-1)
            msg_full = safe_cat((cmsg, msg_step), dim=-2)
            new_cache = (q2_cache, q3_cache, v3_cache, lse23_full, msg_full)
        return out, new_cache, v2

    def _norms_on_load(self, qs, v3, mask, context_mask, rotary_pos_emb, cache, return_cache):
        """The q norms (poly_attention.py:196-200,271) to be applied by the attention passes
        as they load q1 / q2 / q3 rather than by a norm kernel whose outputs they read back:
        no gradient, cache, rotary or mask, and the short-pass kernel's shapes (head dim 64,
        at most 64 positions, not causal: PolyViT's attention).  ((weight, eps) x 3) or None."""
        from . import _ops

        if exists(cache) or return_cache or exists(rotary_pos_emb) or exists(self.rotary_emb):
            return None
        if exists(mask) or any(exists(m) for m in context_mask):
            return None
        if torch.compiler.is_compiling() or not self._use_fused(qs[0]):
            return None
        norms = self.q_norms
        weights = [getattr(n, "weight", None) for n in norms]
        if not all(isinstance(n, RMSNorm) and tuple(n.normalized_shape) == (q.shape[-1],)
                   for n, q in zip(norms, qs)):
            return None
        if torch.is_grad_enabled() and (any(t.requires_grad for t in (*qs, v3)) or
                                        any(w is not None and w.requires_grad for w in weights)):
            return None
        if not _ops.qk_norms_fusable(*qs, v3, weights, self.causal):
            return None
        # torch's RMSNorm without eps uses the fp32 epsilon for 16-bit inputs
        return tuple((w, n.eps if n.eps is not None else torch.finfo(torch.float32).eps)
                     for w, n in zip(weights, norms))

    def _fused_core(self, q1, q2, q3, v3, mask, context_mask, rotary_pos_emb, cache,
                    return_cache, epilogue, qk_norms=None):
        """The attention core on the HIP kernels (q2 / q3 / v3 stay at kv_heads), with the
        module epilogue applied: fused into pass 2 on the order-2 chain's path.  ``qk_norms``:
        q1 / q2 / q3 are not normalised yet and the passes apply these norms on load."""
        from . import _ops

        rep = self.num_rep if self.is_gqa else 1
        dt = _compute_dtype(q1, q2, q3, v3)
        q1, q2, q3, v3 = (t.to(dt) for t in (q1, q2, q3, v3))
        module_rotary = not exists(rotary_pos_emb) and exists(self.rotary_emb)

        if not exists(cache):
            q1r, q2r_right, q2r_left, q3r = q1, q2, q2, q3
            if module_rotary:
                q1r, q2r_right = self.rotary_emb.rotate_queries_with_cached_keys(q1, q2)
                q2r_left, q3r = self.rotary_emb.rotate_queries_with_cached_keys(q2, q3)
            out, lses, msgs = _ops.poly_chain(
                [q1r, q2r_left], [q2r_right, q3r], [v3], causal=self.causal,
                softclamp=self.softclamp_value, scale=self.scale, query_mask=mask,
                key_masks=list(context_mask), epilogue=epilogue, qk_norms=qk_norms,
                keep_levels=return_cache)
            new_cache = None
            if return_cache:
                lse23 = repeat_kv(lses[0][:, :, :, None], rep)[..., 0]
                msg = repeat_kv(msgs[0], rep)
                new_cache = (_cache.adopt(q2, -2), _cache.adopt(q3, -2), _cache.adopt(v3, -2),
                             _cache.adopt(lse23, -1), _cache.adopt(msg, -2))
            return out, new_cache

        # cached single-token step (poly_attention.py:283-287, 331-338, 360-365)
        cq2, cq3, cv3, clse23, cmsg = cache
        q2_cache = _cache.append(cq2, q2.to(cq2.dtype), -2)
        q3_cache = _cache.append(cq3, q3.to(cq3.dtype), -2)
        v3_cache = _cache.append(cv3, v3.to(cv3.dtype), -2)
        q1r, q2_left, q2_right, q3_full = q1, q2, q2_cache, q3_cache
        if module_rotary:
            q1r, q2_right = self.rotary_emb.rotate_queries_with_cached_keys(q1, q2_cache)
            q2_left, q3_full = self.rotary_emb.rotate_queries_with_cached_keys(q2, q3_cache)

        needs_grad = torch.is_grad_enabled() and any(
            t.requires_grad for t in (q1, q2, q3, v3, cq2, cq3, cv3, clse23, cmsg))
        key_mask1, key_mask2 = context_mask
        masked = exists(mask) or exists(key_mask1) or exists(key_mask2)
        if needs_grad or masked:
            # differentiable or masked step: the two passes as pass ops (the reference's math:
            # the context masks mask the keys of the whole cache, `mask` the new query of
            # pass 2; poly_attention.py:75-76,101-105)
            msg_step, lse_step = _ops.attn_pass(q2_left, q3_full, v3_cache, key_mask=key_mask2,
                                                softclamp=self.softclamp_value,
                                                scale=self.scale, may_degenerate=masked)
            lse_step_h = repeat_kv(lse_step[:, :, :, None], rep)[..., 0]
            lse23_full = torch.cat((clse23, lse_step_h.to(clse23.dtype)), dim=-1)
            msg_full = torch.cat((cmsg, repeat_kv(msg_step, rep).to(cmsg.dtype)), dim=-2)
            out, _ = _ops.attn_pass(q1r, repeat_kv(q2_right, rep), msg_full, bias=lse23_full,
                                    key_mask=key_mask1, query_mask=mask,
                                    softclamp=self.softclamp_value, scale=self.scale,
                                    may_degenerate=True)
            out = _ops.apply_epilogue(out, epilogue)
            return out, (q2_cache, q3_cache, v3_cache, lse23_full, msg_full)

        lse23_full = _cache.reserve(clse23, clse23[:, :, :1], -1)
        msg_full = _cache.reserve(cmsg, cmsg[:, :, :1], -2)
        out = _ops.poly_decode_step(
            [q1r, q2_left], [q2_right, q3_full], [v3_cache], [msg_full], [lse23_full],
            kv_heads=self.kv_heads, heads=self.heads, softclamp=self.softclamp_value,
            scale=self.scale)
        return _ops.apply_epilogue(out, epilogue), (q2_cache, q3_cache, v3_cache, lse23_full,
                                                     msg_full)
