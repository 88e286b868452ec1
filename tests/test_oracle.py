"""Pins of the CPU oracle (oracle/poly_oracle.py) against closed forms and library routines.

Each check is chosen so that a plausible slip in the oracle (a dropped bias, a transposed
operand, a wrong causal offset, a missing value product) fails it:
  * brute force: the order-2 / order-3 / order-n poly score as one softmax over key paths,
  * torch's scaled_dot_product_attention (a library routine) with a float bias for each pass,
  * torch.autograd.gradcheck in float64,
  * an independent float64 derivation of the reference's finite-fill masked rows,
  * rotation properties of RoPE (parity of its pair layout is unpinned: the package it comes
    from, rotary-embedding-torch, is absent here).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.poly_oracle as O

param = pytest.mark.parametrize


def rnd(*shape, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


@param("causal", (False, True))
@param("softclamp", (None, 2.0))
@param("n", (1, 5, 9))
def test_order2_matches_pair_softmax(causal, softclamp, n):
    q1, q2, q3, v3 = (rnd(2, 3, n, 8, seed=s) for s in range(4))
    out, _, _ = O.reference_poly_attention(q1, q2, q2, q3, v3, causal=causal,
                                           softclamp_value=softclamp)
    ref = O.brute_order2(q1, q2, q3, v3, causal=causal, softclamp_value=softclamp)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-10, atol=1e-10)


@param("causal", (False, True))
@param("softclamp", (None, 3.0))
def test_order2_rows_equals_full_core_and_its_dq1(causal, softclamp):
    """The chunked row-restricted form used at long lengths: out, msg, lse23 and dq1 of chosen
    rows equal reference_poly_attention and its autograd (chunks that do not divide N), and
    the brute-force pair softmax."""
    n, d = 37, 8
    q1, q2, q3, v3 = (rnd(n, d, seed=40 + s) for s in range(4))
    rows = torch.tensor([0, 5, 17, 36])
    dout = rnd(len(rows), d, seed=45)
    out, msg, lse23, dq1 = O.order2_rows(q1, q2, q3, v3, rows, dout_rows=dout, causal=causal,
                                         softclamp_value=softclamp, chunk=10)
    q = [t[None, None].clone().requires_grad_() for t in (q1, q2, q3, v3)]
    ref, lse_r, msg_r = O.reference_poly_attention(q[0], q[1], q[1], q[2], q[3], causal=causal,
                                                   softclamp_value=softclamp)
    g = torch.zeros_like(ref)
    g[0, 0, rows] = dout
    ref.backward(g)
    torch.testing.assert_close(out, ref[0, 0, rows].detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(msg, msg_r[0, 0].detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse23, lse_r[0, 0].detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dq1, q[0].grad[0, 0, rows], rtol=1e-10, atol=1e-10)
    brute = O.brute_order2(q1[None, None], q2[None, None], q3[None, None], v3[None, None],
                           causal=causal, softclamp_value=softclamp)
    np.testing.assert_allclose(out.numpy(), brute[0, 0, rows.numpy()], rtol=1e-10, atol=1e-10)


@param("causal", (False, True))
def test_order2_rows_with_a_key_mask(causal):
    """order2_rows with a key mask of both passes: out, msg, lse23 and dq1 of rows that keep
    a key equal reference_poly_attention with that mask as both context masks (and its
    autograd); without causality also the brute-force pair softmax over the kept keys alone
    (q2, q3, v3 restricted to them), and a mask applied to pass 2 only fails that pin."""
    n, d = 41, 8
    q1, q2, q3, v3 = (rnd(n, d, seed=60 + s) for s in range(4))
    keep = torch.ones(n, dtype=torch.bool)
    keep[:6] = False
    keep[20:27] = False
    keep[33] = False
    rows = torch.tensor([6, 7, 19, 30, 40])  # each keeps at least one key (causal too)
    dout = rnd(len(rows), d, seed=65)
    out, msg, lse23, dq1 = O.order2_rows(q1, q2, q3, v3, rows, dout_rows=dout, causal=causal,
                                         chunk=9, key_keep=keep)
    q = [t[None, None].clone().requires_grad_() for t in (q1, q2, q3, v3)]
    km = keep[None]
    ref, lse_r, msg_r = O.reference_poly_attention(q[0], q[1], q[1], q[2], q[3], causal=causal,
                                                   context_mask=(km, km))
    g = torch.zeros_like(ref)
    g[0, 0, rows] = dout
    ref.backward(g)
    torch.testing.assert_close(out, ref[0, 0, rows].detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(msg[keep], msg_r[0, 0, keep].detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse23[keep], lse_r[0, 0, keep].detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dq1, q[0].grad[0, 0, rows], rtol=1e-10, atol=1e-10)
    if not causal:
        sub = [t[keep][None, None] for t in (q2, q3, v3)]
        brute = O.brute_order2(q1[None, None], *sub)
        np.testing.assert_allclose(out.numpy(), brute[0, 0, rows.numpy()], rtol=1e-10,
                                   atol=1e-10)
        wrong, _, _ = O.reference_poly_attention(q1[None, None], q2[None, None], q2[None, None],
                                                 q3[None, None], v3[None, None],
                                                 context_mask=(km, None))
        assert np.abs(wrong[0, 0, rows].numpy() - brute[0, 0, rows.numpy()]).max() > 1e-3


def test_order2_brute_force_detects_dropped_bias():
    # planting a mistake in the oracle (no lse bias in pass 2) must break the pin
    q1, q2, q3, v3 = (rnd(1, 2, 6, 8, seed=10 + s) for s in range(4))
    ref = O.brute_order2(q1, q2, q3, v3)
    s = 8 ** -0.5
    msg = torch.softmax(q2 @ q3.transpose(-1, -2) * s, -1) @ v3
    wrong = torch.softmax(q1 @ q2.transpose(-1, -2) * s, -1) @ msg
    assert not np.allclose(wrong.numpy(), ref, atol=1e-6)


@param("causal", (False, True))
def test_passes_match_sdpa(causal):
    q1, q2, q3, v3 = (rnd(2, 2, 7, 16, seed=20 + s) for s in range(4))
    out, lse23, msg = O.reference_poly_attention(q1, q2, q2, q3, v3, causal=causal)
    n = q1.shape[2]
    cm = torch.ones(n, n, dtype=torch.bool).tril() if causal else None
    msg_ref = F.scaled_dot_product_attention(q2, q3, v3, attn_mask=cm)
    s = 16 ** -0.5
    sim = q2 @ q3.transpose(-1, -2) * s
    if causal:
        sim = sim.masked_fill(~cm, -math.inf)
    torch.testing.assert_close(msg, msg_ref, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(lse23, torch.logsumexp(sim, -1), rtol=1e-10, atol=1e-10)
    bias = lse23[:, :, None, :].expand(-1, -1, n, -1)
    if causal:
        bias = bias.masked_fill(~cm, -math.inf)
    out_ref = F.scaled_dot_product_attention(q1, q2, msg, attn_mask=bias)
    torch.testing.assert_close(out, out_ref, rtol=1e-10, atol=1e-10)


@param("causal", (False, True))
def test_order3_matches_path_sum(causal):
    qs = [rnd(1, 2, 5, 8, seed=30 + s) for s in range(4)]
    v3, v4 = rnd(1, 2, 5, 8, seed=40), rnd(1, 2, 5, 8, seed=41)
    out, lses, msgs = O.n_poly_core(qs[:3], qs[1:], [v3, v4], causal=causal)
    ref = O.brute_order3(*qs, v3, v4, causal=causal)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-10, atol=1e-10)
    assert len(lses) == len(msgs) == 2


@param("order", (2, 3, 4))
@param("causal", (False, True))
def test_order_n_matches_recursive_path_sum(order, causal):
    n = 4
    qs = [rnd(1, 1, n, 4, seed=50 + s) for s in range(order + 1)]
    vs = [rnd(1, 1, n, 4, seed=60 + s) for s in range(order - 1)]
    out, _, _ = O.n_poly_core(qs[:-1], qs[1:], vs, causal=causal)
    ref = O.brute_order_n(qs, vs, causal=causal)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-10, atol=1e-10)


@param("causal", (False, True))
def test_order2_core_equals_n_core(causal):
    q1, q2, q3, v3 = (rnd(2, 2, 6, 8, seed=70 + s) for s in range(4))
    a, lse_a, msg_a = O.reference_poly_attention(q1, q2, q2, q3, v3, causal=causal)
    b, lses, msgs = O.n_poly_core([q1, q2], [q2, q3], [v3], causal=causal)
    torch.testing.assert_close(a, b, rtol=0, atol=1e-12)
    torch.testing.assert_close(lse_a, lses[0], rtol=0, atol=1e-12)


def test_order2_gradcheck():
    q1, q2, q3, v3 = (rnd(1, 2, 5, 4, seed=80 + s).requires_grad_() for s in range(4))

    def f(a, b, c, d):
        return O.reference_poly_attention(a, b, b, c, d, causal=True, softclamp_value=3.0)[0]

    assert torch.autograd.gradcheck(f, (q1, q2, q3, v3))


@param("causal", (False, True))
def test_masked_rows_follow_finite_fill_classes(causal):
    """Fully-masked query rows are the uniform average over -finfo.max entries."""
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 2, 8, 16, generator=g) for _ in range(3))
    km = torch.ones(2, 8, dtype=torch.bool)
    km[:, 5:] = False
    km[1, 0] = False  # row 0 of batch 1 loses its only causal key
    qm = torch.ones(2, 8, dtype=torch.bool)
    qm[0, 6:] = False
    bias = torch.randn(2, 2, 8, generator=g)
    bias[1, 0, 3] = -torch.finfo(torch.float32).max  # a class-1 bias entry
    out, lse = O.attn_pass(q, k, v, bias=bias, key_mask=km, query_mask=qm, causal=causal)
    ref_out, ref_lse = O.masked_pass_classes(q, k, v, bias=bias, key_mask=km, query_mask=qm,
                                             causal=causal)
    np.testing.assert_allclose(out.numpy(), ref_out, rtol=1e-5, atol=1e-5)
    ok = np.isfinite(ref_lse) & (ref_lse > -1e30)
    np.testing.assert_allclose(lse.numpy()[ok], ref_lse[ok], rtol=1e-5, atol=1e-5)
    assert np.all(lse.numpy()[~ok] <= -1e30)


def test_padding_invariance_of_key_masks():
    """tests/test_poly_attention.py:516-539 in oracle form: padded+masked == unpadded."""
    q1 = rnd(2, 2, 6, 8, seed=90, dtype=torch.float32)
    q2u, q3u, v3u = (rnd(2, 2, n, 8, seed=91 + i, dtype=torch.float32)
                     for i, n in enumerate((5, 7, 7)))
    pad = lambda t, n: torch.cat((t, torch.zeros(2, 2, n, 8)), dim=2)  # noqa: E731
    q2p, q3p, v3p = pad(q2u, 3), pad(q3u, 4), pad(v3u, 4)
    m1 = torch.zeros(2, 8, dtype=torch.bool)
    m1[:, :5] = True
    m2 = torch.zeros(2, 11, dtype=torch.bool)
    m2[:, :7] = True
    a, _, _ = O.reference_poly_attention(q1, q2u, q2u, q3u, v3u)
    b, _, _ = O.reference_poly_attention(q1, q2p, q2p, q3p, v3p, context_mask=(m1, m2))
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_rotary_properties():
    d = 16
    q, k = rnd(1, 1, 9, d, seed=100, dtype=torch.float32), rnd(1, 1, 9, d, seed=101, dtype=torch.float32)
    qr, kr = O.rotate_queries_with_cached_keys(d, q, k)
    # rotations preserve norms
    torch.testing.assert_close(qr.norm(dim=-1), q.norm(dim=-1), rtol=1e-5, atol=1e-5)
    # scores depend only on relative positions: shift both by 3
    f = O.rotary_freqs(d, torch.arange(12))
    a = O.apply_rotary(f[:9], q) @ O.apply_rotary(f[:9], k).transpose(-1, -2)
    b = O.apply_rotary(f[3:12], q) @ O.apply_rotary(f[3:12], k).transpose(-1, -2)
    torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-4)
    # position 0 is the identity; the first pair at position 1 turns by 1 radian
    torch.testing.assert_close(qr[..., 0, :], q[..., 0, :])
    x = torch.zeros(1, 1, 2, d)
    x[..., 1, 0] = 1.0
    y = O.apply_rotary(O.rotary_freqs(d, torch.arange(2)), x)
    torch.testing.assert_close(y[0, 0, 1, :2], torch.tensor([math.cos(1.0), math.sin(1.0)]))


def test_polyvit_position_table_closed_form():
    """The oracle's sincos table against its closed form evaluated in float64: patch
    p = r*w + c of an h x w grid has [sin(c f_k), cos(c f_k), sin(r f_k), cos(r f_k)] with
    f_k = 10000^(-k / (q - 1)), q = dim / 4 (so f_0 = 1, f_{q-1} = 1e-4); a swapped row / column
    or sin / cos quarter fails."""
    h, w, dim = 3, 5, 16
    q = dim // 4
    pe = O.posemb_sincos_2d(h, w, dim)
    assert pe.shape == (h * w, dim) and pe.dtype == torch.float32
    for r in range(h):
        for c in range(w):
            p = r * w + c
            for k in range(q):
                f = 10000.0 ** (-k / (q - 1))
                want = (math.sin(c * f), math.cos(c * f), math.sin(r * f), math.cos(r * f))
                got = [pe[p, j * q + k].item() for j in range(4)]
                assert max(abs(a - b) for a, b in zip(got, want)) < 1e-6, (r, c, k)


def test_polyvit_patch_order_by_pixel_indexing():
    """The oracle's patch cut ('b c (h p1) (w p2) -> b (h w) (p1 p2 c)') checked pixel by
    pixel: token r*gw + c, feature (i*pw + j)*C + ch holds img[b, ch, r*ph + i, c*pw + j]."""
    g = torch.Generator().manual_seed(7)
    b, C, ph, pw, gh, gw = 2, 3, 2, 4, 3, 2
    img = torch.randn(b, C, gh * ph, gw * pw, generator=g)
    tok = O.patchify(img, ph, pw)
    assert tok.shape == (b, gh * gw, ph * pw * C)
    for bi in range(b):
        for r in range(gh):
            for c in range(gw):
                for i in range(ph):
                    for j in range(pw):
                        for ch in range(C):
                            assert tok[bi, r * gw + c, (i * pw + j) * C + ch] == \
                                img[bi, ch, r * ph + i, c * pw + j]


@pytest.mark.parametrize("order", (2, 3))
def test_polyvit_oracle_matches_module_on_cpu(order):
    """The oracle's PolyViT forward against the drop-in module's CPU (eager) path in float64
    on the same state dict."""
    from poly_attention import PolyViT

    cfg = dict(image_size=32, patch_size=8, num_classes=7, dim=64, depth=2, heads=4,
               mlp_dim=96, dim_head=16, order=order)
    torch.manual_seed(3)
    m = PolyViT(use_flash_kernel=False, **cfg).double().eval()
    img = torch.randn(2, 3, 32, 32, dtype=torch.float64)
    with torch.no_grad():
        want = m(img)
        got = O.polyvit_forward(m.state_dict(), cfg, img)
    torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)


def test_attention_residual_closed_forms():
    """The layer mix against what its formula fixes: one layer -> that layer (weights 1); a
    zero pseudo-query -> the plain mean over layers; a pseudo-query far along one layer's
    normalised direction -> that layer alone (the softmax saturates), the others not."""
    torch.manual_seed(8)
    dim = 32
    hs = [torch.randn(2, 5, dim, dtype=torch.float64) for _ in range(3)]
    w = 1 + 0.2 * torch.randn(dim, dtype=torch.float64)
    p = {"norm_keys.weight": w, "pseudo_queries": torch.zeros(2, dim, dtype=torch.float64)}
    assert torch.allclose(O.attention_residual(p, hs[:1])[0], hs[0], atol=1e-14)
    mean = (hs[0] + hs[1] + hs[2]) / 3
    for m in O.attention_residual(p, hs):
        assert torch.allclose(m, mean, atol=1e-14)
    # one position, a query aligned with layer 1's normalised key: weight -> 1 on layer 1
    one = [h[:1, :1] for h in hs]
    k1 = F.rms_norm(one[1], (dim,), w, None)[0, 0]
    p["pseudo_queries"] = torch.stack([k1 * 400.0, -k1 * 400.0])
    sel, anti = O.attention_residual(p, one)
    assert torch.allclose(sel, one[1], atol=1e-9)
    assert not torch.allclose(anti, one[1], atol=1e-3)


@pytest.mark.parametrize("deep_cross_attention", (False, True))
@pytest.mark.parametrize("causal", (False, True))
def test_polytransformer_oracle_matches_module_on_cpu(deep_cross_attention, causal):
    """The oracle's PolyTransformer forward against the drop-in module's CPU (eager) path in
    float64 on the same state dict, with a query mask (the reference test's shapes,
    poly-attention tests:405-424), the block outputs included."""
    from poly_attention import PolyTransformer

    cfg = dict(dim=64, depth=3, heads=4, dim_head=16, causal=causal,
               deep_cross_attention=deep_cross_attention, norm_out=True)
    torch.manual_seed(4)
    m = PolyTransformer(**cfg).double().eval()
    with torch.no_grad():
        for n, t in m.named_parameters():
            if n.endswith("norm_keys.weight") or n.endswith("pseudo_queries"):
                t.copy_(torch.randn_like(t) * 0.5 + (1.0 if n.endswith("weight") else 0.0))
    x = torch.randn(2, 16, 64, dtype=torch.float64)
    mask = torch.ones(2, 16, dtype=torch.bool)
    mask[:, 8:] = False
    for mk in (None, mask):
        with torch.no_grad():
            want, want_h = m(x, mask=mk, return_layer_hiddens=True)
            got, got_h = O.polytransformer_forward(m.state_dict(), cfg, x, mask=mk)
        torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)
        for a, b in zip(got_h, want_h):
            torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-10)
