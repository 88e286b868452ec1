"""GPU: the per-head q/k RMSNorm, alone and with the rotary embedding in the same kernel
(pa_rmsnorm_fwd / pa_rmsnorm_bwd through the ``polyattn::rms_norm`` custom op) against
torch.nn.RMSNorm and apply_rotary_emb, and the modules' gradients with the fused norms against
the CPU oracle.

Tolerances: forward fp32 max-abs <= 1e-5, bf16 within one bf16 ulp; gradients as the other
GPU suites (tests/parity.py): fp32 max-abs <= 1e-4, bf16 <= 2e-2 plus one bf16 rounding.
"""

import pytest
import torch

import oracle.poly_oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu
param = pytest.mark.parametrize


def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda")


def split_heads(t, heads, d):
    """[B, N, 2*heads*d] -> the first of two [B, heads, N, d] strided views (module layout)."""
    B, N, _ = t.shape
    return t.reshape(B, N, 2, heads, d).permute(2, 0, 3, 1, 4)[0]


@param("dtype", (torch.float32, torch.bfloat16))
@param("d", (32, 64, 128))
@param("affine", (True, False))
def test_rmsnorm_forward_matches_torch(dtype, d, affine):
    from poly_attention import _ops

    dv = dev()
    torch.manual_seed(0)
    H = 3
    x = split_heads(torch.randn(2, 37, 2 * H * d, device=dv).to(dtype), H, d)
    norm = torch.nn.RMSNorm(d, elementwise_affine=affine).to(dv, dtype)
    if affine:
        with torch.no_grad():
            norm.weight.copy_(1 + 0.3 * torch.randn(d, device=dv))
    assert _ops.rms_supported(x, norm.weight)
    with torch.no_grad():
        ref = norm(x)
        got = _ops.rms_norm(x, norm.weight, norm.eps)
    if dtype == torch.float32:
        assert_parity(got, ref, dtype, f"rmsnorm fwd d={d} affine={affine}", tol=1e-5)
    else:
        diff = (got.float() - ref.float()).abs()
        ulp = ref.float().abs().clamp_min(1e-30) * 2.0 ** -7
        assert bool((diff <= ulp).all()), diff.max().item()


@param("dtype", (torch.float32, torch.bfloat16))
@param("d", (64, 128))
def test_rmsnorm_backward_matches_fp32_reference(dtype, d):
    from poly_attention import _ops

    dv = dev()
    torch.manual_seed(1)
    H = 4
    base = torch.randn(2, 50, 2 * H * d, device=dv).to(dtype)
    w = (1 + 0.3 * torch.randn(d, device=dv)).to(dtype)
    dy = torch.randn(2, H, 50, d, device=dv).to(dtype)
    # fp32 reference on the same rounded inputs
    xr = split_heads(base.float(), H, d).detach().requires_grad_()
    wr = w.float().detach().requires_grad_()
    torch.nn.functional.rms_norm(xr, (d,), wr, torch.finfo(torch.float32).eps).backward(dy.float())
    # torch's norm in the inputs' own dtype on the CPU (the reference's arithmetic at that
    # precision), whose drift bounds the low-precision gradients
    xl = split_heads(base.cpu(), H, d).detach().requires_grad_()
    wl = w.cpu().detach().requires_grad_()
    torch.nn.functional.rms_norm(xl, (d,), wl, torch.finfo(torch.float32).eps).backward(dy.cpu())
    x = split_heads(base, H, d).detach().requires_grad_()
    wg = w.detach().requires_grad_()
    _ops.rms_norm(x, wg, None).backward(dy)
    assert_parity(x.grad, xr.grad, dtype, f"rmsnorm dx d={d} {dtype}", grad=True, ref_lp=xl.grad)
    assert_parity(wg.grad, wr.grad, dtype, f"rmsnorm dw d={d} {dtype}", grad=True, ref_lp=wl.grad)
    assert wg.grad.dtype == dtype


def _angles(rot, positions, two_d, device):
    from poly_attention.rotary import RotaryEmbedding

    freqs = RotaryEmbedding(rot)(torch.arange(positions).float()).to(device)
    return freqs if two_d else freqs[-1]


@param("dtype", (torch.float32, torch.bfloat16))
@param("d,rot", ((64, 64), (64, 32), (128, 64)))
@param("two_d", (True, False))
def test_rmsnorm_rope_forward_matches_torch_ops(dtype, d, rot, two_d):
    """norm -> apply_rotary_emb in one kernel equals the two torch ops (rotation in fp32 on the
    rounded norm output, one rounding), angles as [positions >= N, rot] (the last N rows) or
    one [rot] row for every position."""
    from poly_attention import _ops
    from poly_attention.rotary import apply_rotary_emb

    dv = dev()
    torch.manual_seed(4)
    H = 3
    x = split_heads(torch.randn(2, 37, 2 * H * d, device=dv).to(dtype), H, d)
    norm = torch.nn.RMSNorm(d).to(dv, dtype)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.3 * torch.randn(d, device=dv))
    ang = _angles(rot, 45, two_d, dv)
    assert _ops.rms_supported(x, norm.weight, ang)
    with torch.no_grad():
        ref = apply_rotary_emb(ang, norm(x))
        got = _ops.rms_norm(x, norm.weight, norm.eps, ang)
    if dtype == torch.float32:
        assert_parity(got, ref, dtype, f"rmsnorm+rope fwd d={d} rot={rot}", tol=1e-5)
    else:
        diff = (got.float() - ref.float()).abs()
        ulp = ref.float().abs().clamp_min(1e-30) * 2.0 ** -7
        assert bool((diff <= ulp).all()), diff.max().item()


@param("dtype", (torch.float32, torch.bfloat16))
@param("rot", (64, 32))
def test_rmsnorm_rope_backward_matches_fp32_reference(dtype, rot):
    from poly_attention import _ops
    from poly_attention.rotary import apply_rotary_emb

    dv = dev()
    torch.manual_seed(5)
    H, d = 4, 64
    base = torch.randn(2, 50, 2 * H * d, device=dv).to(dtype)
    w = (1 + 0.3 * torch.randn(d, device=dv)).to(dtype)
    dy = torch.randn(2, H, 50, d, device=dv).to(dtype)
    ang = _angles(rot, 60, True, dv)
    xr = split_heads(base.float(), H, d).detach().requires_grad_()
    wr = w.float().detach().requires_grad_()
    yr = apply_rotary_emb(ang, torch.nn.functional.rms_norm(xr, (d,), wr, torch.finfo(torch.float32).eps))
    yr.backward(dy.float())
    xl = split_heads(base.cpu(), H, d).detach().requires_grad_()  # the same in dtype, on the CPU
    wl = w.cpu().detach().requires_grad_()
    apply_rotary_emb(ang.cpu(), torch.nn.functional.rms_norm(
        xl, (d,), wl, torch.finfo(torch.float32).eps)).backward(dy.cpu())
    x = split_heads(base, H, d).detach().requires_grad_()
    wg = w.detach().requires_grad_()
    _ops.rms_norm(x, wg, None, ang).backward(dy)
    assert_parity(x.grad, xr.grad, dtype, f"rmsnorm+rope dx rot={rot} {dtype}", grad=True,
                  ref_lp=xl.grad)
    assert_parity(wg.grad, wr.grad, dtype, f"rmsnorm+rope dw rot={rot} {dtype}", grad=True,
                  ref_lp=wl.grad)


def test_rmsnorm_weight_grad_is_deterministic():
    from poly_attention import _ops

    dv = dev()
    torch.manual_seed(2)
    x = torch.randn(4, 16, 1000, 64, device=dv, dtype=torch.bfloat16)
    w = torch.ones(64, device=dv, dtype=torch.bfloat16, requires_grad=True)
    dy = torch.randn_like(x)
    grads = []
    for _ in range(2):
        w.grad = None
        _ops.rms_norm(x, w, None).backward(dy)
        grads.append(w.grad.clone())
    assert torch.equal(grads[0], grads[1])


@param("order", (2, 3))
@param("rotary", (False, True))
def test_module_grads_with_fused_norms(order, rotary):
    """Module forward + backward on the GPU (fused core and fused q/k norms, with the external
    rotary inside the norm kernel) against the CPU oracle's autograd: input and parameter
    gradients, including the q-norm weights."""
    from poly_attention import NPolyAttention, Order2PolyAttention

    dv = dev()
    torch.manual_seed(3)
    cfg = dict(heads=4, dim_head=64, causal=True)
    if order == 2:
        m = Order2PolyAttention(dim=64, **cfg)
        fwd = O.order2_forward
    else:
        m = NPolyAttention(dim=64, order=3, **cfg)
        fwd = O.npoly_forward
        cfg = dict(cfg, order=3)
    with torch.no_grad():
        for n in m.q_norms:
            n.weight.copy_(1 + 0.3 * torch.randn_like(n.weight))
    x = torch.randn(2, 40, 64)
    g = torch.randn(2, 40, 64)
    freqs = O.rotary_freqs(64, torch.arange(40)) if rotary else None
    params = {k: v.detach().clone().requires_grad_() for k, v in m.state_dict().items()}
    xr = x.clone().requires_grad_()
    fwd(params, cfg, xr, rotary_pos_emb=freqs).backward(g)
    m = m.to(dv)
    xg = x.to(dv).requires_grad_()
    m(xg, rotary_pos_emb=freqs.to(dv) if rotary else None).backward(g.to(dv))
    what = f"module with fused norms order={order} rotary={rotary}"
    assert_parity(xg.grad, xr.grad, torch.float32, f"{what} dx")
    for name, p in m.named_parameters():
        assert_parity(p.grad, params[name].grad, torch.float32, f"{what} d{name}")


@param("dtype", (torch.bfloat16, torch.float32))
def test_rmsnorm_many_one_launch(dtype):
    """pa_rmsnorm_fwd_many: the q/k norms of a layer in one launch, without autograd (three
    head-split views of one projection, different weights and eps, and a contiguous tensor
    of another shape): each output bit-identical to pa_rmsnorm_fwd's, and torch.nn.RMSNorm's
    within one rounding."""
    from poly_attention import _ops

    d = dev()
    g = torch.Generator().manual_seed(31)
    proj = (torch.randn(2, 65, 3 * 16 * 64, generator=g) * 3).to(dtype).to(d)
    heads = proj.view(2, 65, 3, 16, 64).permute(2, 0, 3, 1, 4)  # 3 x [B, H, N, d] views
    xs = [heads[0], heads[1], heads[2], (torch.randn(1, 4, 7, 64, generator=g)).to(dtype).to(d)]
    ws = [(torch.rand(64, generator=g) + 0.5).to(dtype).to(d) for _ in xs]
    eps = [None, 1e-6, 1e-5, None]
    with torch.no_grad():
        ys = _ops.rms_norm_many(xs, ws, eps)
        for x, w, e, y in zip(xs, ws, eps, ys):
            one = _ops.rms_norm(x, w, e)
            assert torch.equal(y, one)
            ref = torch.nn.functional.rms_norm(x, (64,), w, e)
            if dtype == torch.float32:
                assert_parity(y, ref, dtype, "rms_norm_many fp32", tol=1e-5)
            else:  # one rounding apart at most
                diff = (y.float() - ref.float()).abs()
                ulp = ref.float().abs().clamp_min(1e-30) * 2.0 ** -7
                assert bool((diff <= ulp).all()), diff.max().item()
