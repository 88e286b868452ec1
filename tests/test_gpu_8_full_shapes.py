"""GPU parity at the BASELINE configurations' full shapes, against the CPU oracle.

* PolyAttention(dim=512, heads=8, dim_head=64, causal=False) fp32 forward on
  x [1, 1024, 512] -- the whole module;
* the order-2 causal core at B=4, N=4096, H=16, d=64 in bf16 on the module's own
  normed q1/q2/q3/v3, forward and all four gradients over the full problem, checked on two of
  the 64 (batch, head) slices (every slice is independent: kv_heads = heads);
* PolyViT(image 256, patch 32, dim 1024, depth 6, 16 heads, mlp 2048, 1000
  classes) bf16 forward on 4 images (the batch of 64 shrunk for the CPU oracle);
* the order-2 GQA decode step (32 query / 8 KV heads, d = 128, batch 32, 8192
  cached positions + the new one) over the full cache, checked on two (batch, KV group)
  slices -- output, and the msg / lse slots the step writes.

Bound as the other GPU suites (tests/parity.py); every check prints its raw max-abs error.
"""

import pytest
import torch

import oracle.poly_oracle as O
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu


def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda")


def test_config1_module_fp32_forward():
    from poly_attention import PolyAttention

    d = dev()
    torch.manual_seed(0)
    m = PolyAttention(dim=512, heads=8, dim_head=64, causal=False)
    x = torch.randn(1, 1024, 512, generator=torch.Generator().manual_seed(1))
    params = {k: v.detach().clone() for k, v in m.state_dict().items()}
    ref = O.order2_forward(params, dict(heads=8, dim_head=64, causal=False), x)
    with torch.no_grad():
        out = m.to(d)(x.to(d))
    torch.cuda.synchronize()
    assert_parity(out, ref, torch.float32, "config 1 module fp32 (1, 1024, 512)")


def test_config2_full_length_core_slices():
    """Forward + gradients of the config-2 core over all 64 (batch, head) units; two units
    (first and last) against the oracle at N = 4096."""
    from poly_attention import PolyAttention
    from poly_attention.flash_poly_attention import flash_poly_attention

    d = dev()
    B, N, DIM, H, DH = 4, 4096, 1024, 16, 64
    torch.manual_seed(0)
    m = PolyAttention(dim=DIM, heads=H, dim_head=DH, causal=True).to(d, torch.bfloat16)
    x = torch.randn(B, N, DIM, generator=torch.Generator().manual_seed(1)).to(d, torch.bfloat16)
    with torch.no_grad():
        q1 = m.split_q(m.to_q(x))[0]
        q2 = m.split_kv1(m.to_kvs[0](x))[0]
        q3, v3 = m.split_kv(m.to_kvs[1](x))
        qs = [norm(q) for norm, q in zip(m.q_norms, (q1, q2, q3))] + [v3]
    g_in = [t.contiguous().requires_grad_() for t in qs]
    dout = torch.randn(B, H, N, DH, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    out = flash_poly_attention(*g_in, is_causal=True)
    out.backward(dout.to(d))
    torch.cuda.synchronize()
    for b, h in ((0, 0), (B - 1, H - 1)):
        o_in = [t.detach()[b:b + 1, h:h + 1].float().cpu().requires_grad_() for t in g_in]
        ref, _, _ = O.reference_poly_attention(o_in[0], o_in[1], o_in[1], o_in[2], o_in[3],
                                               causal=True)
        ref.backward(dout[b:b + 1, h:h + 1].float())
        lp_in = [t.detach()[b:b + 1, h:h + 1].cpu().requires_grad_() for t in g_in]  # bf16 oracle
        lp, _, _ = O.reference_poly_attention(lp_in[0], lp_in[1], lp_in[1], lp_in[2], lp_in[3],
                                              causal=True)
        lp.backward(dout[b:b + 1, h:h + 1])
        what = f"config 2 N={N} slice (b={b}, h={h})"
        assert_parity(out[b:b + 1, h:h + 1], ref, torch.bfloat16, f"{what} out")
        for name, a, r, c in zip(("dq1", "dq2", "dq3", "dv3"), g_in, o_in, lp_in):
            assert_parity(a.grad[b:b + 1, h:h + 1], r.grad, torch.bfloat16, f"{what} {name}",
                          grad=True, ref_lp=c.grad)


def test_config3_polyvit_bf16_forward():
    from poly_attention import PolyViT

    d = dev()
    cfg = dict(image_size=256, patch_size=32, num_classes=1000, dim=1024, depth=6, heads=16,
               mlp_dim=2048)
    torch.manual_seed(0)
    vit = PolyViT(**cfg).to(d, torch.bfloat16).eval()
    img = torch.randn(4, 3, 256, 256, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    with torch.no_grad():
        out = vit(img.to(d))
    torch.cuda.synchronize()
    params = {k: v.float().cpu() for k, v in vit.state_dict().items()}
    with torch.no_grad():
        ref = O.polyvit_forward(params, dict(cfg, dim_head=64, order=2), img.float())
    assert_parity(out, ref, torch.bfloat16, "config 3 PolyViT bf16 logits (4 images)")


def test_config5_full_cache_decode_slices():
    from poly_attention import _ops

    d = dev()
    Bd, Hq, G, n_old, dh = 32, 32, 8, 8192, 128
    n, r = n_old + 1, Hq // G
    gen = torch.Generator(device=d).manual_seed(3)

    def rnd(*shape):
        return torch.randn(*shape, generator=gen, device=d).to(torch.bfloat16)

    q2c, q3c, v3c = rnd(Bd, G, n, dh), rnd(Bd, G, n, dh), rnd(Bd, G, n, dh)
    msg = rnd(Bd, Hq, n, dh)
    lse = torch.log(torch.arange(1, n + 1, device=d, dtype=torch.float32)) + \
        torch.randn(Bd, Hq, n, generator=gen, device=d)
    q1 = rnd(Bd, Hq, 1, dh)
    q2n = q2c[:, :, -1:].contiguous()
    msg_old = {bg: msg[bg[0], bg[1] * r:(bg[1] + 1) * r, :n_old].float().cpu() for bg in ((0, 0), (Bd - 1, G - 1))}
    lse_old = {bg: lse[bg[0], bg[1] * r:(bg[1] + 1) * r, :n_old].cpu() for bg in msg_old}
    out = _ops.poly_decode_step([q1, q2n], [q2c, q3c], [v3c], [msg], [lse], kv_heads=G,
                                heads=Hq, softclamp=None, scale=dh ** -0.5)
    torch.cuda.synchronize()
    for b, g in msg_old:
        hs = slice(g * r, (g + 1) * r)
        rep = lambda t: t[b:b + 1, g:g + 1].float().cpu().repeat_interleave(r, dim=1)  # noqa: E731
        cache = (None, None, None, lse_old[(b, g)][None], msg_old[(b, g)][None])
        ref, lse_step, msg_step = O.reference_poly_attention(
            q1[b:b + 1, hs].float().cpu(), rep(q2n), rep(q2c), rep(q3c), rep(v3c), cache=cache)
        what = f"config 5 n={n} slice (b={b}, group={g})"
        assert_parity(out[b:b + 1, hs], ref, torch.bfloat16, f"{what} out")
        assert_parity(msg[b:b + 1, hs, -1:], msg_step, torch.bfloat16, f"{what} msg slot")
        assert_parity(lse[b:b + 1, hs, -1], lse_step[..., 0], torch.float32, f"{what} lse slot",
                      tol=TOL[torch.bfloat16])
        # the cached positions are untouched
        assert torch.equal(msg[b, hs, :n_old].float().cpu(), msg_old[(b, g)])
