"""GPU: the q / k RMSNorms applied by the short-pass kernel as it loads queries and keys
(pa_qk_norm), against the same chain on tensors normalised by pa_rmsnorm_fwd first.

Bound: bit-identical.  The kernel reproduces pa_rmsnorm_fwd's arithmetic and summation order,
so the normalised operands, and with them every output, are the same bits.  The module path
is checked the same way, and at PolyViT's full shape against the oracle in
tests/test_gpu_8_full_shapes.py.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu
param = pytest.mark.parametrize


def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda")


def _views(B, H, Hkv, n, dtype, g):
    """q1 [B, H, n, 64] and q2 / q3 / v3 [B, Hkv, n, 64] as head-split views of projections."""
    d = dev()
    p1 = (torch.randn(B, n, 2 * H * 64, generator=g) * 2).to(dtype).to(d)
    p2 = (torch.randn(B, n, 3 * Hkv * 64, generator=g) * 2).to(dtype).to(d)
    q1 = p1.view(B, n, 2, H, 64).permute(2, 0, 3, 1, 4)[0]
    q2, q3, v3 = p2.view(B, n, 3, Hkv, 64).permute(2, 0, 3, 1, 4)
    return q1, q2, q3, v3


@param("dtype", (torch.bfloat16, torch.float16))
@param("H,Hkv", ((4, 4), (8, 2)))
@param("n", (64, 37))
@param("softclamp", (None, 5.0))
def test_chain_norms_on_load_equal_norm_kernel(dtype, H, Hkv, n, softclamp):
    from poly_attention import _ops

    d = dev()
    g = torch.Generator().manual_seed(7)
    q1, q2, q3, v3 = _views(3, H, Hkv, n, dtype, g)
    ws = [(1 + 0.3 * torch.randn(64, generator=g)).to(dtype).to(d) for _ in range(3)]
    eps = [1e-6, torch.finfo(torch.float32).eps, 1e-5]
    assert _ops.qk_norms_fusable(q1, q2, q3, v3, ws, False)
    with torch.no_grad():
        n1, n2, n3 = _ops.rms_norm_many([q1, q2, q3], ws, eps)
        ref, ref_lses, ref_msgs = _ops.poly_chain([n1, n2], [n2, n3], [v3], causal=False,
                                                  softclamp=softclamp, scale=64 ** -0.5)
        got, lses, msgs = _ops.poly_chain([q1, q2], [q2, q3], [v3], causal=False,
                                          softclamp=softclamp, scale=64 ** -0.5,
                                          qk_norms=tuple(zip(ws, eps)))
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(msgs[0], ref_msgs[0]) and torch.equal(lses[0], ref_lses[0])


@param("gates", (False, True))
def test_module_norms_on_load_equal_separate_norms(gates):
    """PolyAttention in bf16 inference at a PolyViT-like shape (64 positions, head dim 64):
    the passes normalising q1 / q2 / q3 on load give the bits of the norm-kernel path."""
    from poly_attention import PolyAttention

    d = dev()
    torch.manual_seed(3)
    m = PolyAttention(dim=256, heads=4, dim_head=64, causal=False, attn_gate=gates,
                      multiply_root_value=gates).to(d, torch.bfloat16).eval()
    with torch.no_grad():
        for n in m.q_norms:
            n.weight.copy_(1 + 0.3 * torch.randn_like(n.weight))
    x = torch.randn(5, 64, 256, device=d).to(torch.bfloat16)
    qs_seen = []
    orig = type(m)._norms_on_load

    def spy(self, *a, **k):
        r = orig(self, *a, **k)
        qs_seen.append(r is not None)
        return r

    with torch.no_grad():
        type(m)._norms_on_load = spy
        try:
            got = m(x)
            type(m)._norms_on_load = lambda self, *a, **k: None
            ref = m(x)
        finally:
            type(m)._norms_on_load = orig
    torch.cuda.synchronize()
    assert qs_seen == [True], "the fused norms were not taken"
    assert torch.equal(got, ref)


def test_norms_on_load_refused_outside_the_short_kernel():
    """The library refuses q / k norms where the short-pass kernel does not run (causal here)
    instead of ignoring them."""
    from poly_attention import _lib, _ops

    d = dev()
    g = torch.Generator().manual_seed(1)
    q1, q2, q3, v3 = _views(2, 4, 4, 64, torch.bfloat16, g)
    w = torch.ones(64, device=d, dtype=torch.bfloat16)
    assert not _ops.qk_norms_fusable(q1, q2, q3, v3, [w, w, w], True)
    with pytest.raises(_lib.PolyAttnError) as e:
        _ops.pass_fwd_raw(q2, q3, v3, None, None, None, None, True, None, 0.125, False,
                          qk_norm=((w, 1e-6), (w, 1e-6)))
    assert e.value.status == _lib.PA_EUNSUPPORTED
