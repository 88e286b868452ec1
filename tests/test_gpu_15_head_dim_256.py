"""GPU parity of passes at head dims above 128 (libpolyattn through its C ABI) vs the CPU oracle.

The reference's Triton kernels take the head dim as BLOCK_DMODEL = dim (flash_poly_attention.py:
357,375,420,440; autotuned per value, :12-20), any power of two.  Here, 16-bit passes of head dim 256 run on the register-staged MFMA kernels
(k_mfma_fwd, k_mfma_bwd_dq, k_mfma_bwd_dkv at D = 256), and head dims 129..255 are zero-padded
to 256 by the host layer, masked passes included (the key mask folded into the key term, the
fully-masked rows finished by the fix-ups); fp32 passes of these head dims run on the generic
kernels.  Bound as tests/parity.py states it (fp32 1e-4; bf16 / f16 2e-2 plus one rounding of
the result's storage type).  The kernel profile shows which kernels ran.
"""

import pytest
import torch

import oracle.poly_oracle as O
from parity import assert_drift, assert_parity
from test_gpu_1_pass import check, dev, randn, run_pass

pytestmark = pytest.mark.gpu
param = pytest.mark.parametrize

MFMA = ("mfma_fwd", "mfma_bwd_dq", "mfma_bwd_dkv")
GENERIC = ("simt_fwd", "simt_bwd_dq", "simt_bwd_dkv")


def _profiled(q, k, v, **kw):
    from poly_attention import _lib

    dev()
    with _lib.KernelProfile() as prof:
        res = run_pass(q, k, v, **kw)
    return res, set(prof.times)


@param("dtype", (torch.bfloat16, torch.float16))
@param("d", (256, 160, 200))
@param("n", (40, 300))
@param("causal", (False, True))
def test_pass_head_dim_256_on_mfma(dtype, d, n, causal):
    """Forward and gradients at head dim 256 (160 and 200 padded to it): one partial key tile
    (n = 40) and ten 32-key forward tiles with a ragged end (n = 300, three query blocks)."""
    q, k, v = (randn((2, 2, n, d), dtype, s) for s in (201, 202, 203))
    res, ran = _profiled(q, k, v, causal=causal)
    check(res, dtype, f"head dim {d} {dtype} n={n} causal={causal}")
    for name in MFMA:
        assert name in ran, f"{name} did not run (kernels: {sorted(ran)})"
    assert not ran & set(GENERIC), sorted(ran)


@param("causal", (False, True))
@param("softclamp", (None, 10.0))
def test_pass_head_dim_256_gqa_bias_vmul(causal, softclamp):
    """A middle level of the chain at head dim 256: 8 query heads over 2 KV heads, key bias, value
    multiplier (the register-staged kernels' paths), softclamp on and off."""
    dtype = torch.bfloat16
    q = randn((1, 8, 150, 256), dtype, 211)
    k, v, vmul = (randn((1, 2, 150, 256), dtype, s) for s in (212, 213, 214))
    bias = randn((1, 2, 150), torch.float32, 215, scale=2.0)
    res, ran = _profiled(q, k, v, vmul=vmul, bias=bias, causal=causal, softclamp=softclamp)
    check(res, dtype, f"head dim 256 gqa+bias+vmul causal={causal} sc={softclamp}")
    for name in MFMA:
        assert name in ran, f"{name} did not run (kernels: {sorted(ran)})"


@param("dtype", (torch.bfloat16, torch.float16, torch.float32))
@param("d", (256, 192))
@param("causal", (False, True))
def test_pass_head_dim_256_masked(dtype, d, causal):
    """Key / query masks with fully-masked rows at head dims above 128: 16-bit passes on the
    register-staged MFMA kernels with the key mask folded into the key term and the fix-ups
    finishing the fully-masked rows; fp32 passes on the generic kernels."""
    q, k, v = (randn((2, 2, 24, d), dtype, s) for s in (221, 222, 223))
    km = torch.ones(2, 24, dtype=torch.bool)
    km[:, 17:] = False
    km[1, 0] = False
    qm = torch.ones(2, 24, dtype=torch.bool)
    qm[0, 20:] = False
    res, ran = _profiled(q, k, v, key_mask=km, query_mask=qm, causal=causal)
    check(res, dtype, f"masked head dim {d} {dtype} causal={causal}")
    if dtype == torch.float32:
        for name in GENERIC:
            assert name in ran, f"{name} did not run (kernels: {sorted(ran)})"
    else:
        for name in MFMA + ("fwd_fixup", "key_terms", "fix_rows", "fix_keys"):
            assert name in ran, f"{name} did not run (kernels: {sorted(ran)})"
        assert not ran & set(GENERIC), sorted(ran)


@param("n", (150, 256))
@param("causal", (False, True))
@param("gqa", (False, True))
def test_pass_head_dim_256_masked_bias_classes(n, causal, gqa):
    """The masked cases of the head-dim-64/128 test at head dim 256 in bf16: leading keys
    masked (causal rows 0-2 fully masked), batch 1's keys 3-5 biased to -finfo.max (bias class
    1: fully-masked rows with unmasked class-1 keys, finished by the part B fix-ups), a -inf
    bias entry, query-masked rows; gqa: 4 query heads over 2 key heads with a value
    multiplier."""
    dtype, d = torch.bfloat16, 256
    B, H, HK = 2, 4, (2 if gqa else 4)
    q = randn((B, H, n, d), dtype, 251)
    k, v = (randn((B, HK, n, d), dtype, s) for s in (252, 253))
    vmul = randn((B, HK, n, d), dtype, 254) if gqa else None
    bias = torch.log(torch.arange(1, n + 1).float())[None, None].repeat(B, HK, 1)
    bias = bias + randn((B, HK, n), torch.float32, 255)
    fmax = torch.finfo(torch.float32).max
    km = torch.ones(B, n, dtype=torch.bool)
    qm = torch.ones(B, n, dtype=torch.bool)
    km[:, :3] = False
    km[0, n // 2:n // 2 + 20] = False
    bias[1, :, 3:6] = -fmax
    bias[0, 0, 10] = -float("inf")
    qm[0, -7:] = False
    if not causal:
        km[1, 6:] = False
    res, ran = _profiled(q, k, v, vmul=vmul, bias=bias, key_mask=km, query_mask=qm,
                         causal=causal)
    check(res, dtype, f"masked head dim 256 n={n} causal={causal} gqa={gqa}")
    for name in MFMA + ("fix_rows", "fix_keys", "fix_part_b"):
        assert name in ran, f"{name} did not run (kernels: {sorted(ran)})"
    assert not ran & set(GENERIC), sorted(ran)


def test_pass_head_dim_256_fp32_generic():
    q, k, v = (randn((1, 2, 70, 256), torch.float32, s) for s in (231, 232, 233))
    res, ran = _profiled(q, k, v, causal=True)
    check(res, torch.float32, "head dim 256 fp32")
    assert "simt_fwd" in ran, sorted(ran)


@param("causal", (False, True))
def test_flash_poly_attention_head_dim_256(causal):
    """The order-2 chain (flash_poly_attention.py:334-396) at head dim 256 in bf16: both passes
    and the chain's backward (pass 1's dQ of q2 accumulated into pass 2's dK) on the MFMA
    kernels, against the fp32 oracle of poly_attention.py:48-116."""
    from poly_attention import _lib
    from poly_attention.flash_poly_attention import flash_poly_attention

    d = dev()
    g = torch.Generator().manual_seed(241)
    shape = (1, 2, 200, 256)
    ts = [torch.randn(shape, generator=g).to(torch.bfloat16) for _ in range(4)]
    gt = [t.to(d).requires_grad_() for t in ts]
    ot = [t.float().requires_grad_() for t in ts]
    with _lib.KernelProfile() as prof:
        out = flash_poly_attention(*gt, is_causal=causal)
        dout = torch.randn(out.shape, generator=g).to(torch.bfloat16)
        out.backward(dout.to(d))
        torch.cuda.synchronize()
    ref, _, _ = O.reference_poly_attention(ot[0], ot[1], ot[1], ot[2], ot[3], causal=causal)
    ref.backward(dout.float())
    # the oracle in bf16: the reference's own drift at that precision bounds the gradients
    lt = [t.clone().requires_grad_() for t in ts]
    lp, _, _ = O.reference_poly_attention(lt[0], lt[1], lt[1], lt[2], lt[3], causal=causal)
    lp.backward(dout)
    assert_parity(out, ref, torch.bfloat16, f"chain d=256 causal={causal} out")
    for i, (a, b, c) in enumerate(zip(gt, ot, lt)):
        assert_parity(a.grad, b.grad, torch.bfloat16, f"chain d=256 causal={causal} grad {i}",
                      grad=True, ref_lp=c.grad)
    ran = set(prof.times)
    for name in MFMA:
        assert name in ran, f"{name} did not run (kernels: {sorted(ran)})"
    assert not ran & set(GENERIC), sorted(ran)


@param("masked", (False, True))
def test_module_head_dim_256_bf16_training(masked):
    """PolyAttention (poly_attention.py:120-365) at dim_head = 256 trained in bf16: forward and
    backward through the fused projections, q/k norms, both passes on the head-dim-256 MFMA
    kernels (with a key-padding mask: the key term and fix-ups) and the output projection.  As in
    the config-2 module test, each result is held to the drift of the reference's own bf16
    arithmetic (tests/parity.py, assert_drift)."""
    from poly_attention import PolyAttention

    d = dev()
    B, N, DIM, H, DH = 2, 160, 512, 4, 256
    cfg = dict(heads=H, dim_head=DH, causal=True)
    torch.manual_seed(3)
    m = PolyAttention(dim=DIM, **cfg).to(d, torch.bfloat16)
    x = torch.randn(B, N, DIM, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    dout = torch.randn(B, N, DIM, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    mask = None
    if masked:  # right-padded batch row 1, left-padded batch row 0
        mask = torch.ones(B, N, dtype=torch.bool)
        mask[1, 120:] = False
        mask[0, :17] = False

    xg = x.to(d).requires_grad_()
    out = m(xg, mask=mask.to(d) if masked else None)
    out.backward(dout.to(d))
    torch.cuda.synchronize()

    sd = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    p32 = {k: v.float().requires_grad_(v.is_floating_point()) for k, v in sd.items()}
    x32 = x.float().requires_grad_()
    ref = O.order2_forward(p32, cfg, x32, mask=mask)
    ref.backward(dout.float())
    p16 = {k: v.clone().requires_grad_(v.is_floating_point()) for k, v in sd.items()}
    x16 = x.clone().requires_grad_()
    lp = O.order2_forward(p16, cfg, x16, mask=mask)
    lp.backward(dout)

    what = f"module dim_head=256 bf16 masked={masked}"
    assert_drift(out, ref, lp, f"{what} out")
    assert_drift(xg.grad, x32.grad, x16.grad, f"{what} dx")
    for name, p in m.named_parameters():
        assert p.grad is not None and p32[name].grad is not None, name
        assert_drift(p.grad, p32[name].grad, p16[name].grad, f"{what} d{name}")


@param("order", (2, 3))
def test_cache_stepwise_head_dim_256_bf16(order):
    """Prefill at dim_head = 256 in bf16 (the MFMA passes) with return_cache, then single-token
    steps through the decode kernel: the concatenated outputs against the oracle's parallel
    causal forward (reference tests:103-179), 2 KV heads under 4 query heads; held to the drift
    of the reference's own bf16 arithmetic, as the module test above."""
    from poly_attention import NPolyAttention, Order2PolyAttention

    d = dev()
    torch.manual_seed(13)
    cfg = dict(heads=4, kv_heads=2, dim_head=256, causal=True)
    if order == 2:
        m = Order2PolyAttention(dim=128, **cfg)
        fwd = O.order2_forward
    else:
        m = NPolyAttention(dim=128, order=order, **cfg)
        fwd = O.npoly_forward
        cfg = dict(cfg, order=order)
    m = m.to(d, torch.bfloat16)
    x = torch.randn(2, 70, 128).to(torch.bfloat16)
    sd = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    ref = fwd({k: v.float() for k, v in sd.items()}, cfg, x.float())
    lp = fwd(sd, cfg, x)  # the reference's own bf16 arithmetic: the drift bound
    with torch.no_grad():
        out0, cache = m(x[:, :64].to(d), return_cache=True)
        outs = [out0]
        for i in range(64, 70):
            o, cache = m(x[:, i:i + 1].to(d), cache=cache, return_cache=True)
            outs.append(o)
    assert_drift(torch.cat(outs, dim=1), ref, lp, f"stepwise dim_head=256 order={order} bf16")
