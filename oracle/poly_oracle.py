"""CPU oracle for the poly-attention hot path -- TEST INFRASTRUCTURE ONLY.

A restatement of lucidrains/poly-attention 0.3.6's eager PyTorch math, op for op, on the CPU.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker (or the timed CPU baseline); the product path
(``poly-attention_amd/poly_attention``) never does.

Contents and what pins each function (see tests/test_oracle.py):
  reference_poly_attention   poly_attention.py:48-116  -- brute_order2 (pair-softmax closed
                             form, fp64), per-pass SDPA with a float bias, gradcheck
  order2_rows                the same for chosen query rows of one long slice (chunked pass 1)
                             -- equal to reference_poly_attention and its autograd dq1
  attn_pass                  one level: n_poly_attention.py:237-261 + :272-275 -- SDPA,
                             brute force, the finite-fill class semantics of masked rows
  n_poly_core                n_poly_attention.py:233-313 -- brute_order3 / brute_order_n
                             (path-sum closed forms), order-2 == reference_poly_attention
  order2_forward             poly_attention.py:206-365 (module forward, functional)
  npoly_forward              n_poly_attention.py:122-340 (module forward, functional)
  polyvit_forward            poly_vit.py:19-101 (PolyViT forward, functional) -- the position
                             table and the patch order pinned by closed forms / direct pixel
                             indexing, the composition by the drop-in module on the CPU
  attention_residual         poly_transformer.py:17-56 -- closed forms (one layer: identity,
                             zero query: layer mean, a dominant query: one-hot selection)
  polytransformer_forward    poly_transformer.py:60-150 (PolyTransformer forward, functional)
                             -- the composition by the drop-in module on the CPU in float64
  rotary_*                   rotary-embedding-torch's RoPE (absent here; parity unpinned for
                             the pair layout, pinned by rotation properties)
  brute_* / masked_pass_classes   independent float64 closed forms used as pins
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor, einsum

# ---------------------------------------------------------------------------------------
# small restated helpers (einx / torch_einops_utils patterns)


def exists(v):
    return v is not None


def softclamp(x: Tensor, c: float) -> Tensor:
    """poly_attention.py:43-44"""
    return c * torch.tanh(x / c)


def safe_cat(ts, dim):
    ts = [t for t in ts if t is not None]
    if not ts:
        return None
    return ts[0] if len(ts) == 1 else torch.cat(ts, dim=dim)


def where_keys(mask, sim, value):  # einx.where('b j, b h i j, -> b h i j')
    return torch.where(mask[:, None, None, :], sim, value)


def where_queries(mask, sim, value):  # einx.where('b i, b h i j, -> b h i j')
    return torch.where(mask[:, None, :, None], sim, value)


def add_key_bias(bias, sim):  # einx.add('b h j, b h i j -> b h i j')
    return sim + bias[:, :, None, :]


def repeat_kv(t, r):  # einops.repeat('b g n d -> b (g r) n d')
    return None if t is None else (t if r == 1 else t.repeat_interleave(r, dim=1))


# ---------------------------------------------------------------------------------------
# the order-2 core


def reference_poly_attention(q1, q2_pass1, q2_pass2, q3, v3, mask=None, context_mask=None,
                             softclamp_value=None, causal=False, cache=None):
    """poly_attention.py:48-116 -> (out, lse23_step, msg_step)."""
    scale = q1.shape[-1] ** -0.5
    has_cache = exists(cache)
    cm1, cm2 = context_mask if exists(context_mask) else (None, None)

    sim23 = einsum("b h i d, b h j d -> b h i j", q2_pass1, q3) * scale  # :63
    if exists(softclamp_value):
        sim23 = softclamp(sim23, softclamp_value)  # :65-66
    mask_value = -torch.finfo(sim23.dtype).max  # :68
    if causal and not has_cache:  # :70-73
        i, j = sim23.shape[-2:]
        sim23 = sim23.masked_fill(torch.ones((i, j), dtype=torch.bool).triu(1), mask_value)
    if exists(cm2):
        sim23 = where_keys(cm2, sim23, mask_value)  # :75-76
    lse23_step = sim23.logsumexp(dim=-1)  # :80
    attn23 = sim23.softmax(dim=-1)  # :81
    msg_step = einsum("b h i j, b h j d -> b h i d", attn23, v3)  # :82

    _, _, _, clse23, cmsg = cache if has_cache else (None,) * 5  # :84
    lse23 = safe_cat((clse23, lse23_step), dim=-1)  # :86
    msg = safe_cat((cmsg, msg_step), dim=-2)  # :87

    sim12 = einsum("b h i d, b h j d -> b h i j", q1, q2_pass2) * scale  # :91
    if exists(softclamp_value):
        sim12 = softclamp(sim12, softclamp_value)  # :93-94
    if causal and not has_cache:  # :96-99
        i, j = sim12.shape[-2:]
        sim12 = sim12.masked_fill(torch.ones((i, j), dtype=torch.bool).triu(1), mask_value)
    if exists(cm1):
        sim12 = where_keys(cm1, sim12, mask_value)  # :101-102
    if exists(mask):
        sim12 = where_queries(mask, sim12, mask_value)  # :104-105
    sim12 = add_key_bias(lse23, sim12)  # :109
    attn12 = sim12.softmax(dim=-1)  # :113
    out = einsum("b h i j, b h j d -> b h i d", attn12, msg)  # :114
    return out, lse23_step, msg_step


def attn_pass(q, k, v, vmul=None, bias=None, key_mask=None, query_mask=None, causal=False,
              softclamp_value=None, scale=None):
    """One level of the chain in the reference's arithmetic -> (out, lse).

    Scores as n_poly_attention.py:237-261 (scale, softclamp, causal / key / query masks filled
    with -finfo.max), the deeper level's lse added as a key bias (:288, :307), then
    logsumexp / softmax / aggregation (:272-275).  Head counts are expanded like the
    reference's repeat (poly_attention.py:290); vmul multiplies the values (:287).
    """
    H = max(t.shape[1] for t in (q, k, v, vmul, bias) if t is not None)
    q, k, v = (repeat_kv(t, H // t.shape[1]) for t in (q, k, v))
    if vmul is not None:
        v = v * repeat_kv(vmul, H // vmul.shape[1])
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    s = einsum("b h i d, b h j d -> b h i j", q, k) * scale
    if exists(softclamp_value):
        s = softclamp(s, softclamp_value)
    mv = -torch.finfo(s.dtype).max
    if causal:
        i, j = s.shape[-2:]
        s = s.masked_fill(torch.ones((i, j), dtype=torch.bool).triu(1), mv)
    if exists(key_mask):
        s = where_keys(key_mask, s, mv)
    if exists(query_mask):
        s = where_queries(query_mask, s, mv)
    if exists(bias):
        s = add_key_bias(repeat_kv(bias[:, :, :, None], H // bias.shape[1])[..., 0].to(s.dtype), s)
    lse = s.logsumexp(dim=-1)
    out = einsum("b h i j, b h j d -> b h i d", s.softmax(dim=-1), v)
    return out, lse


def n_poly_core(q_left: Sequence[Tensor], q_right: Sequence[Tensor], vs_full: Sequence[Tensor],
                context_mask=None, mask=None, causal=False, has_cache=False,
                softclamp_value=None, scale=None, c_lses=None, c_msgs=None):
    """n_poly_attention.py:233-313 (scores, right-to-left aggregation) -> (out, lses, msgs),
    lses / msgs deepest level first (the reference's cache order)."""
    order = len(q_left)
    scale = q_left[0].shape[-1] ** -0.5 if scale is None else scale
    context_mask = context_mask if exists(context_mask) else (None,) * order
    c_lses = c_lses if exists(c_lses) else (None,) * (order - 1)
    c_msgs = c_msgs if exists(c_msgs) else (None,) * (order - 1)

    scores = []
    for idx, (ql, qr, cmask) in enumerate(zip(q_left, q_right, context_mask)):
        score = einsum("b h i d, b h j d -> b h i j", ql, qr) * scale  # :237
        if exists(softclamp_value):
            score = softclamp(score, softclamp_value)  # :239-240
        mv = -torch.finfo(score.dtype).max  # :242
        if causal and not has_cache:  # :246-249
            i, j = score.shape[-2:]
            score = score.masked_fill(torch.ones((i, j), dtype=torch.bool).triu(1), mv)
        if exists(cmask):
            score = where_keys(cmask, score, mv)  # :253-254
        if idx == 0 and exists(mask):
            score = where_queries(mask, score, mv)  # :258-259
        scores.append(score)

    out = vs_full[-1]  # :265
    cur = scores[-1]
    lses, msgs = [], []
    for k in range(order - 1, 1, -1):  # :271-288
        lse_step = cur.logsumexp(dim=-1)
        msg_step = einsum("b h i j, b h j d -> b h i d", cur.softmax(dim=-1), out)
        idx = (order - 1) - k
        lse_full = safe_cat((c_lses[idx], lse_step), dim=-1)
        msg_full = safe_cat((c_msgs[idx], msg_step), dim=-2)
        msgs.append(msg_full)
        lses.append(lse_full)
        out = vs_full[k - 2] * msg_full
        cur = add_key_bias(lse_full, scores[k - 1])
    lse_step = cur.logsumexp(dim=-1)  # :292-305
    msg_step = einsum("b h i j, b h j d -> b h i d", cur.softmax(dim=-1), out)
    idx = order - 2
    lse_full = safe_cat((c_lses[idx], lse_step), dim=-1)
    msg_full = safe_cat((c_msgs[idx], msg_step), dim=-2)
    msgs.append(msg_full)
    lses.append(lse_full)
    s12 = add_key_bias(lse_full, scores[0])  # :307
    out = einsum("b h i j, b h j d -> b h i d", s12.softmax(dim=-1), msg_full)  # :311-313
    return out, lses, msgs


def order2_rows(q1: Tensor, q2: Tensor, q3: Tensor, v3: Tensor, rows: Tensor,
                dout_rows: Optional[Tensor] = None, causal: bool = True,
                softclamp_value: Optional[float] = None, chunk: int = 1024,
                key_keep: Optional[Tensor] = None):
    """reference_poly_attention (poly_attention.py:48-116, no cache) for one (batch, head)
    slice at lengths where the N x N score matrix does not fit: pass 1 runs over every pass-1
    row in chunks of ``chunk`` rows (its msg / lse23 feed every pass-2 key), pass 2 only for the
    query rows ``rows``.  q* / v3: [N, d].  ``key_keep`` ([N] bool): a key mask of both passes,
    as the context masks (poly_attention.py:75-76, 101-102) and the flash op's key mask
    (flash_poly_attention.py:109-112) apply it.  Returns (out[rows], msg, lse23) and, with the
    upstream gradient of those rows, also dq1[rows] (the pass-2 score gradient, which involves
    only the row itself: dS = P (dP - rowsum(dO * O)), dq1 = scale * dS q2 through the
    softclamp's derivative)."""
    n, d = q1.shape
    scale = d ** -0.5
    mask_value = -torch.finfo(q1.dtype).max
    msg = torch.empty_like(v3)
    lse23 = torch.empty(n, dtype=q1.dtype)
    for i0 in range(0, n, chunk):
        i1 = min(n, i0 + chunk)
        kend = i1 if causal else n
        sim = (q2[i0:i1] @ q3[:kend].T) * scale
        if exists(softclamp_value):
            sim = softclamp(sim, softclamp_value)
        if causal:
            later = torch.arange(kend)[None, :] > torch.arange(i0, i1)[:, None]
            sim = sim.masked_fill(later, mask_value)
        if key_keep is not None:
            sim = sim.masked_fill(~key_keep[None, :kend], mask_value)
        lse23[i0:i1] = sim.logsumexp(dim=-1)
        msg[i0:i1] = sim.softmax(dim=-1) @ v3[:kend]
    raw = (q1[rows] @ q2.T) * scale
    sim = softclamp(raw, softclamp_value) if exists(softclamp_value) else raw
    if causal:
        sim = sim.masked_fill(torch.arange(n)[None, :] > rows[:, None], mask_value)
    if key_keep is not None:
        sim = sim.masked_fill(~key_keep[None, :], mask_value)
    sim = sim + lse23[None, :]
    attn = sim.softmax(dim=-1)
    out = attn @ msg
    if dout_rows is None:
        return out, msg, lse23
    dsim = attn * (dout_rows @ msg.T - (dout_rows * out).sum(-1, keepdim=True))
    if exists(softclamp_value):
        dsim = dsim * (1 - torch.tanh(raw / softclamp_value) ** 2)
    if causal:
        dsim = dsim.masked_fill(torch.arange(n)[None, :] > rows[:, None], 0.0)
    if key_keep is not None:
        dsim = dsim.masked_fill(~key_keep[None, :], 0.0)
    dq1 = (dsim @ q2) * scale
    return out, msg, lse23, dq1


# ---------------------------------------------------------------------------------------
# rotary (rotary-embedding-torch >= 0.8.9, as used at poly_attention.py:14,202,277,303-304)


def rotary_freqs(dim: int, positions: Tensor, theta: float = 10000.0) -> Tensor:
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2)[: dim // 2].float() / dim))
    f = positions.float()[:, None] * inv
    return f.repeat_interleave(2, dim=-1)


def rotate_half(x: Tensor) -> Tensor:
    x = x.unflatten(-1, (-1, 2))
    x1, x2 = x.unbind(-1)
    return torch.stack((-x2, x1), dim=-1).flatten(-2)


def apply_rotary(freqs: Tensor, t: Tensor) -> Tensor:
    freqs = freqs[-t.shape[-2]:]
    rot = freqs.shape[-1]
    tm, tr = t[..., :rot], t[..., rot:]
    tm = tm * freqs.cos() + rotate_half(tm) * freqs.sin()
    return torch.cat((tm, tr), dim=-1).type(t.dtype)


def rotate_queries_with_cached_keys(dim: int, q: Tensor, k: Tensor):
    # positions are built in the activation dtype, then offset (get_seq_pos of the package)
    qn, kn = q.shape[-2], k.shape[-2]
    fq = rotary_freqs(dim, torch.arange(qn, dtype=q.dtype) + (kn - qn))
    fk = rotary_freqs(dim, torch.arange(kn, dtype=k.dtype))
    return apply_rotary(fq, q), apply_rotary(fk, k)


# ---------------------------------------------------------------------------------------
# module forwards (functional restatements; params = the module's state_dict)


def _rms(x, w):
    return F.rms_norm(x, (x.shape[-1],), w, None)


def _split(t, split, h):  # 'b n (split h d) -> split b h n d'
    b, n, _ = t.shape
    return t.reshape(b, n, split, h, -1).permute(2, 0, 3, 1, 4)


def order2_forward(p: dict, cfg: dict, x, context=None, mask=None, context_mask=None,
                   rotary_pos_emb=None, cache=None, return_cache=False):
    """Order2PolyAttention.forward, poly_attention.py:206-365 (eager branch)."""
    heads, kv_heads = cfg["heads"], cfg.get("kv_heads") or cfg["heads"]
    shared_kv, attn_gate = cfg.get("shared_kv", False), cfg.get("attn_gate", False)
    mrv, rv_gate = cfg.get("multiply_root_value", False), cfg.get("use_root_value_as_attn_gate", False)
    has_root_v = mrv and not shared_kv
    rep = heads // kv_heads
    seq_len = x.shape[-2]
    has_cache = exists(cache)
    orig_x = x
    if cfg.get("prenorm", False):
        x = _rms(x, p["norm.weight"])
    qg = _split(F.linear(x, p["to_q.weight"]), 2 if attn_gate else 1, heads)
    q1 = qg[0]
    gates = qg[1] if attn_gate else None
    has_context = exists(context)
    context = orig_x if context is None else context
    context = (context,) * 2 if torch.is_tensor(context) else context
    if exists(context_mask):
        context_mask = (context_mask,) * 2 if torch.is_tensor(context_mask) else context_mask
    elif not has_context and exists(mask):
        context_mask = (mask, mask)
    else:
        context_mask = (None, None)
    if "context_norms.0.weight" in p:
        ctx1, ctx2 = _rms(context[0], p["context_norms.0.weight"]), _rms(context[1], p["context_norms.1.weight"])
    else:
        ctx1, ctx2 = context if has_context else (x, x)
    kv1 = _split(F.linear(ctx1, p["to_kvs.0.weight"]), 2 if has_root_v else 1, kv_heads)
    kv2 = _split(F.linear(ctx2, p["to_kvs.1.weight"]), 1 if shared_kv else 2, kv_heads)
    if shared_kv:
        qs = (q1, kv1[0], kv2[0])
        v2, v3 = kv1[0], kv2[0]
    else:
        q2, v2 = kv1[0], (kv1[1] if has_root_v else None)
        q3, v3 = kv2[0], kv2[1]
        qs = (q1, q2, q3)
    qs = tuple(_rms(q, p[f"q_norms.{i}.weight"]) for i, q in enumerate(qs))
    if exists(rotary_pos_emb):
        qs = tuple(apply_rotary(rotary_pos_emb, q) for q in qs)
    q1, q2, q3 = qs
    cq2, cq3, cv3, clse23, cmsg = cache if has_cache else (None,) * 5
    q2_cache = safe_cat((cq2, q2), -2)
    q3_cache = safe_cat((cq3, q3), -2)
    v3_cache = safe_cat((cv3, v3), -2)
    q2, q3, v2, v3 = (repeat_kv(t, rep) for t in (q2, q3, v2, v3))
    q2_full, q3_full, v3_full = (repeat_kv(t, rep) for t in (q2_cache, q3_cache, v3_cache))
    q2_left, q2_right = q2, q2_full
    if not exists(rotary_pos_emb) and cfg.get("use_rotary_embed", False):
        d = q1.shape[-1]
        q1, q2_right = rotate_queries_with_cached_keys(d, q1, q2_right)
        q2_left, q3_full = rotate_queries_with_cached_keys(d, q2_left, q3_full)
    out, lse_step, msg_step = reference_poly_attention(
        q1, q2_left, q2_right, q3_full, v3_full, mask=mask, context_mask=context_mask,
        softclamp_value=cfg.get("softclamp_value"), causal=cfg.get("causal", False), cache=cache)
    if mrv:
        out = (v2.sigmoid() if rv_gate else v2) * out
    if attn_gate:
        out = out * gates.sigmoid()
    b, h, n, d = out.shape
    out = F.linear(out.permute(0, 2, 1, 3).reshape(b, n, h * d), p["to_out.weight"], p["to_out.bias"])
    if not return_cache:
        return out
    return out, (q2_cache, q3_cache, v3_cache, safe_cat((clse23, lse_step), -1),
                 safe_cat((cmsg, msg_step), -2))


def npoly_forward(p: dict, cfg: dict, x, context=None, mask=None, context_mask=None,
                  rotary_pos_emb=None, cache=None, return_cache=False):
    """NPolyAttention.forward, n_poly_attention.py:122-340."""
    order = cfg["order"]
    heads, kv_heads = cfg["heads"], cfg.get("kv_heads") or cfg["heads"]
    shared_kv, attn_gate = cfg.get("shared_kv", False), cfg.get("attn_gate", False)
    mrv, rv_gate = cfg.get("multiply_root_value", False), cfg.get("use_root_value_as_attn_gate", False)
    has_root_v = mrv and not shared_kv
    rep = heads // kv_heads
    has_cache = exists(cache)
    orig_x = x
    if cfg.get("prenorm", False):
        x = _rms(x, p["norm.weight"])
    qg = _split(F.linear(x, p["to_q.weight"]), 2 if attn_gate else 1, heads)
    q1, gates = qg[0], (qg[1] if attn_gate else None)
    has_context = exists(context)
    context = orig_x if context is None else context
    context = (context,) * order if torch.is_tensor(context) else context
    if exists(context_mask):
        context_mask = (context_mask,) * order if torch.is_tensor(context_mask) else context_mask
    elif not has_context and exists(mask):
        context_mask = (mask,) * order
    else:
        context_mask = (None,) * order
    if "context_norms.0.weight" in p:
        context = tuple(_rms(c, p[f"context_norms.{i}.weight"]) for i, c in enumerate(context))
    else:
        context = context if has_context else (x,) * order
    kv1 = _split(F.linear(context[0], p["to_kvs.0.weight"]), 2 if has_root_v else 1, kv_heads)
    kvs_rest = [_split(F.linear(c, p[f"to_kvs.{i + 1}.weight"]), 1 if shared_kv else 2, kv_heads)
                for i, c in enumerate(context[1:])]
    qs_rest = (kv1[0], *[kv[0] for kv in kvs_rest])
    if shared_kv:
        root_value, vs = qs_rest[0], qs_rest[1:]
    else:
        vs = tuple(kv[1] for kv in kvs_rest)
        root_value = kv1[1] if has_root_v else None
    qs = (q1, *qs_rest)
    qs = tuple(_rms(q, p[f"q_norms.{i}.weight"]) for i, q in enumerate(qs))
    if exists(rotary_pos_emb):
        qs = tuple(apply_rotary(rotary_pos_emb, q) for q in qs)
    q1, qs_rest = qs[0], qs[1:]
    if has_cache:
        c_qs, c_vs, c_lses, c_msgs = cache
    else:
        c_qs, c_vs = (None,) * order, (None,) * (order - 1)
        c_lses, c_msgs = (None,) * (order - 1), (None,) * (order - 1)
    qs_rest_cache = tuple(safe_cat((cq, q), -2) for cq, q in zip(c_qs, qs_rest))
    vs_cache = tuple(safe_cat((cv, v), -2) for cv, v in zip(c_vs, vs))
    qs_left = tuple(repeat_kv(t, rep) for t in qs_rest)
    qs_right = tuple(repeat_kv(t, rep) for t in qs_rest_cache)
    vs_full = tuple(repeat_kv(t, rep) for t in vs_cache)
    root_value = repeat_kv(root_value, rep)
    q_left, q_right = [q1, *qs_left[:-1]], list(qs_right)
    if not exists(rotary_pos_emb) and cfg.get("use_rotary_embed", False):
        d = q1.shape[-1]
        rot = [rotate_queries_with_cached_keys(d, a, b) for a, b in zip(q_left, q_right)]
        q_left, q_right = [r[0] for r in rot], [r[1] for r in rot]
    out, lses, msgs = n_poly_core(q_left, q_right, vs_full, context_mask, mask,
                                  cfg.get("causal", False), has_cache,
                                  cfg.get("softclamp_value"), None, c_lses, c_msgs)
    if mrv:
        out = (root_value.sigmoid() if rv_gate else root_value) * out
    if attn_gate:
        out = out * gates.sigmoid()
    b, h, n, d = out.shape
    out = F.linear(out.permute(0, 2, 1, 3).reshape(b, n, h * d), p["to_out.weight"], p["to_out.bias"])
    if not return_cache:
        return out
    return out, (qs_rest_cache, vs_cache, tuple(lses), tuple(msgs))


# ---------------------------------------------------------------------------------------
# PolyViT (poly_vit.py:13-101), functional


def posemb_sincos_2d(h: int, w: int, dim: int, temperature: int = 10000) -> Tensor:
    """poly_vit.py:19-30: frequencies 1 / T^(k / (dim/4 - 1)); per patch of a row-major h x w
    grid the features [sin(col f), cos(col f), sin(row f), cos(row f)] in fp32."""
    omega = torch.arange(dim // 4) / (dim // 4 - 1)
    omega = 1.0 / (temperature ** omega)
    y, x = torch.meshgrid(torch.arange(h), torch.arange(w), indexing="ij")
    y = y.reshape(-1, 1) * omega
    x = x.reshape(-1, 1) * omega
    return torch.cat((x.sin(), x.cos(), y.sin(), y.cos()), dim=-1)


def patchify(img: Tensor, ph: int, pw: int) -> Tensor:
    """'b c (h p1) (w p2) -> b (h w) (p1 p2 c)' (poly_vit.py:76)."""
    b, c, H, W = img.shape
    t = img.reshape(b, c, H // ph, ph, W // pw, pw)
    return t.permute(0, 2, 4, 3, 5, 1).reshape(b, (H // ph) * (W // pw), ph * pw * c)


def _sub(p: dict, prefix: str) -> dict:
    return {k[len(prefix):]: v for k, v in p.items() if k.startswith(prefix)}


def polyvit_forward(p: dict, cfg: dict, img: Tensor) -> Tensor:
    """PolyViT.forward (poly_vit.py:92-101) with the Transformer of :42-63; ``p`` the
    module's state_dict, ``cfg`` its constructor arguments."""
    ph, pw = (cfg["patch_size"],) * 2 if not isinstance(cfg["patch_size"], tuple) else cfg["patch_size"]
    ih, iw = (cfg["image_size"],) * 2 if not isinstance(cfg["image_size"], tuple) else cfg["image_size"]
    dim, order = cfg["dim"], cfg.get("order", 2)
    x = patchify(img, ph, pw)
    x = F.layer_norm(x, (x.shape[-1],), p["to_patch_embedding.1.weight"], p["to_patch_embedding.1.bias"])
    x = F.linear(x, p["to_patch_embedding.2.weight"], p["to_patch_embedding.2.bias"])
    x = F.layer_norm(x, (dim,), p["to_patch_embedding.3.weight"], p["to_patch_embedding.3.bias"])
    x = x + posemb_sincos_2d(ih // ph, iw // pw, dim).to(x.device, dtype=x.dtype)
    acfg = dict(heads=cfg["heads"], dim_head=cfg.get("dim_head", 64), causal=False, prenorm=True)
    for i in range(cfg["depth"]):
        pa = _sub(p, f"transformer.layers.{i}.0.")
        if order == 2:
            a = order2_forward(pa, acfg, x)
        else:
            a = npoly_forward(pa, dict(acfg, order=order), x)
        x = a + x
        pf = _sub(p, f"transformer.layers.{i}.1.")
        h = F.layer_norm(x, (dim,), pf["0.weight"], pf["0.bias"])
        h = F.gelu(F.linear(h, pf["1.weight"], pf["1.bias"]))
        x = F.linear(h, pf["3.weight"], pf["3.bias"]) + x
    x = F.layer_norm(x, (dim,), p["transformer.norm.weight"], p["transformer.norm.bias"])
    return F.linear(x.mean(dim=1), p["linear_head.weight"])


def attention_residual(p: dict, outputs: Sequence[Tensor]) -> list[Tensor]:
    """AttentionResidual.forward (poly_transformer.py:29-56): for each pseudo-query q_j (a row
    of ``p['pseudo_queries']``) the mix sum_l w_jl h_l of the block outputs h_1..h_L, with
    w_j. = softmax over l of <q_j, RMSNorm(h_l)> / sqrt(dim) at every position; written as
    explicit sums over the layer list."""
    dim = outputs[0].shape[-1]
    keys = [_rms(h, p["norm_keys.weight"]) for h in outputs]
    mixes = []
    for q in p["pseudo_queries"]:
        logits = torch.stack([(k * q).sum(-1) * dim ** -0.5 for k in keys])  # [L, ...]
        w = torch.softmax(logits, dim=0)
        mixes.append(sum(w[l][..., None] * h for l, h in enumerate(outputs)))
    return mixes


def polytransformer_forward(p: dict, cfg: dict, x: Tensor, mask=None) -> Tensor:
    """PolyTransformer.forward (poly_transformer.py:106-150) with FeedForward (:60-70) and
    the block layout of :91-104; ``p`` the module's state_dict, ``cfg`` its constructor
    arguments. Returns the output and the list of block outputs."""
    depth, deep = cfg["depth"], cfg.get("deep_cross_attention", False)
    acfg = dict(heads=cfg.get("heads", 8), dim_head=cfg.get("dim_head", 64),
                causal=cfg.get("causal", False))
    outputs, contexts = [], None
    for i in range(depth):
        pl = _sub(p, f"layers.{i}.")
        ctx = None
        if contexts is not None:
            ctx = tuple(_rms(c, pl[f"1.{j}.weight"]) for j, c in enumerate(contexts))
        x = order2_forward(_sub(pl, "2."), acfg, _rms(x, pl["0.weight"]), context=ctx,
                           mask=mask) + x
        h = F.gelu(F.linear(_rms(x, pl["3.0.weight"]), pl["3.1.weight"], pl["3.1.bias"]))
        x = F.linear(h, pl["3.3.weight"], pl["3.3.bias"]) + x
        outputs.append(x)
        mixes = attention_residual(_sub(p, f"attn_residuals.{i}."), outputs)
        if deep and i < depth - 1:
            x, contexts = mixes[0], tuple(mixes[1:])
        else:
            x = mixes[0]
    if cfg.get("norm_out", False):
        x = _rms(x, p["norm_out.weight"])
    return x, outputs


# ---------------------------------------------------------------------------------------
# independent pins: closed forms in float64 (numpy)


def _np64(t):
    return t.detach().to(torch.float64).cpu().numpy()


def brute_order2(q1, q2, q3, v3, causal=False, softclamp_value=None, scale=None):
    """out[i] = sum_{j,k} e^{S12[i,j] + S23[j,k]} v3[k] / sum_{j,k} e^{...}: the order-2 poly
    score as one softmax over (j, k) pairs (the paper's definition), causal: k <= j <= i."""
    q1, q2, q3, v3 = map(_np64, (q1, q2, q3, v3))
    d = q1.shape[-1]
    s = d ** -0.5 if scale is None else scale
    sc = (lambda x: softclamp_value * np.tanh(x / softclamp_value)) if softclamp_value else (lambda x: x)
    s12 = sc(np.einsum("bhid,bhjd->bhij", q1, q2) * s)
    s23 = sc(np.einsum("bhjd,bhkd->bhjk", q2, q3) * s)
    tot = s12[..., :, :, None] + s23[..., None, :, :]  # [b, h, i, j, k]
    if causal:
        n = q1.shape[-2]
        ii, jj, kk = np.meshgrid(np.arange(n), np.arange(n), np.arange(n), indexing="ij")
        tot = np.where((jj <= ii) & (kk <= jj), tot, -np.inf)
    m = tot.max(axis=(-1, -2), keepdims=True)
    w = np.exp(tot - m)
    num = np.einsum("bhijk,bhkd->bhid", w, v3)
    return num / w.sum(axis=(-1, -2))[..., None]


def brute_order3(q1, q2, q3, q4, v3, v4, causal=False, scale=None):
    """out[i] = sum_{j,k,l} e^{S12+S23+S34} (v3[k] * v4[l]) / sum e^{...} (path sum)."""
    q1, q2, q3, q4, v3, v4 = map(_np64, (q1, q2, q3, q4, v3, v4))
    d = q1.shape[-1]
    s = d ** -0.5 if scale is None else scale
    s12 = np.einsum("bhid,bhjd->bhij", q1, q2) * s
    s23 = np.einsum("bhjd,bhkd->bhjk", q2, q3) * s
    s34 = np.einsum("bhkd,bhld->bhkl", q3, q4) * s
    tot = s12[..., :, :, None, None] + s23[..., None, :, :, None] + s34[..., None, None, :, :]
    if causal:
        n = q1.shape[-2]
        i, j, k, l = np.meshgrid(*(np.arange(n),) * 4, indexing="ij")
        tot = np.where((j <= i) & (k <= j) & (l <= k), tot, -np.inf)
    m = tot.max(axis=(-1, -2, -3), keepdims=True)
    w = np.exp(tot - m)
    num = np.einsum("bhijkl,bhkd,bhld->bhid", w, v3, v4)
    return num / w.sum(axis=(-1, -2, -3))[..., None]


def brute_order_n(qs: Sequence[Tensor], vs: Sequence[Tensor], causal=False, scale=None):
    """Recursive path sum for any order: Z_l(j) = sum_k e^{S_l[j,k]} (v_{l+2}[k] *) Z_{l+1}(k)
    evaluated as explicit nested sums over paths (exponential, for tiny shapes)."""
    qs = [_np64(q) for q in qs]
    vs = [_np64(v) for v in vs]
    order = len(qs) - 1
    d = qs[0].shape[-1]
    s = d ** -0.5 if scale is None else scale
    S = [np.einsum("bhid,bhjd->bhij", qs[l], qs[l + 1]) * s for l in range(order)]
    B, H, n, _ = qs[0].shape
    out = np.zeros((B, H, n, d))
    for b in range(B):
        for h in range(H):
            for i in range(n):
                num = np.zeros(d)
                den = 0.0
                # enumerate paths (j_1 .. j_order)
                def rec(level, prev, acc_s, acc_v):
                    nonlocal num, den
                    if level == order:
                        w = math.exp(acc_s)
                        den += w
                        num += w * acc_v
                        return
                    for j in range(n):
                        if causal and j > prev:
                            continue
                        v_mult = acc_v
                        if level >= 1:  # value of the key at level >= 1 is v_{level+2}
                            v_mult = acc_v * vs[level - 1][b, h, j]
                        rec(level + 1, j, acc_s + S[level][b, h, prev, j], v_mult)
                rec(0, i, 0.0, np.ones(d))
                out[b, h, i] = num / den
    return out


def masked_pass_classes(q, k, v, bias=None, key_mask=None, query_mask=None, causal=False,
                        scale=None):
    """Float64 re-derivation of one masked pass in the reference's finite-fill arithmetic.

    Entry class = [own score masked] + [bias == -finfo.max] (+2 for a -inf bias), capped at
    2.  A row with a class-0 entry is an ordinary softmax over its class-0 entries; otherwise
    it is the uniform average over its class-1 entries (lse = -finfo.max); otherwise NaN.
    """
    q, k, v = map(_np64, (q, k, v))
    B, H, nq, d = q.shape
    nk = k.shape[2]
    s = d ** -0.5 if scale is None else scale
    S = np.einsum("bhid,bhjd->bhij", q, k) * s
    own = np.zeros((B, 1, nq, nk), dtype=bool)
    if causal:
        own |= np.triu(np.ones((nq, nk), dtype=bool), 1)[None, None]
    if key_mask is not None:
        own |= ~key_mask.numpy()[:, None, None, :]
    if query_mask is not None:
        own |= ~query_mask.numpy()[:, None, :, None]
    cls = own.astype(np.int64) + np.zeros((B, H, nq, nk), dtype=np.int64)
    bv = np.zeros((B, H, 1, nk))
    if bias is not None:
        bb = bias.detach().to(torch.float64).numpy()
        bcls = np.where(np.isneginf(bb), 2, np.where(bb <= -1e30, 1, 0))
        cls = cls + bcls[:, :, None, :]
        bv = np.where(bcls == 0, bb, 0.0)[:, :, None, :]
    cls = np.minimum(cls, 2)
    out = np.full((B, H, nq, d), np.nan)
    lse = np.full((B, H, nq), -np.inf)
    for b in range(B):
        for h in range(H):
            for i in range(nq):
                c0 = cls[b, h, i] == 0
                c1 = cls[b, h, i] == 1
                if c0.any():
                    x = (S[b, h, i] + bv[b, h, 0])[c0]
                    m = x.max()
                    w = np.exp(x - m)
                    out[b, h, i] = (w[:, None] * v[b, h][c0]).sum(0) / w.sum()
                    lse[b, h, i] = m + math.log(w.sum())
                elif c1.any():
                    out[b, h, i] = v[b, h][c1].mean(0)
                    lse[b, h, i] = -np.finfo(np.float32).max
    return out, lse
