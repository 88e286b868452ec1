"""GPU: both forward passes of an order-2 chain in one launch (pa_poly_order2_fwd at the
short-pass shape: PolyViT's attention), against the two pa_attn_pass_fwd calls it replaces.

Bound: bit-identical (out, lse, lse23, msg and the epilogue's y).  The fused kernel runs each
32-query block with the same arithmetic as the short-pass kernel and hands pass 1's rounded
output and its lse to pass 2 unchanged.  The chain itself is checked against the oracle
through the modules (tests/test_gpu_2_modules.py; PolyViT at its full shape in
tests/test_gpu_8_full_shapes.py), which now run on this launch.
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


def _two_calls(q1, q2, q3, v3, softclamp, scale, epilogue, norms):
    from poly_attention import _ops

    n1, n2, n3 = norms if norms is not None else (None, None, None)
    msg, lse23 = _ops.pass_fwd_raw(q2, q3, v3, None, None, None, None, False, softclamp, scale,
                                   False, qk_norm=(n2, n3) if norms is not None else None)
    res = _ops.pass_fwd_raw(q1, q2, msg, None, lse23, None, None, False, softclamp, scale,
                            False, epilogue, qk_norm=(n1, n2) if norms is not None else None)
    return (res[0], res[1], lse23, msg) + tuple(res[2:])


@param("dtype", (torch.bfloat16, torch.float16))
@param("B,H,Hkv", ((3, 5, 5), (2, 8, 2)))
@param("n", (64, 37, 20))
@param("softclamp", (None, 5.0))
@param("norms", (False, True))
def test_order2_one_launch_equals_two_passes(dtype, B, H, Hkv, n, softclamp, norms):
    """(3, 5, 5): 15 units, an odd count (one padding unit in the last workgroup); n = 20 leaves
    the second 32-row block empty.  (2, 8, 2) is GQA: the library makes the two pass calls."""
    from poly_attention import _lib, _ops

    d = dev()
    g = torch.Generator().manual_seed(11)
    q1, q2, q3, v3 = _views(B, H, Hkv, n, dtype, g)
    nw = None
    if norms:
        ws = [(1 + 0.3 * torch.randn(64, generator=g)).to(dtype).to(d) for _ in range(3)]
        nw = tuple(zip(ws, (1e-6, torch.finfo(torch.float32).eps, 1e-5)))
    with torch.no_grad():
        ref = _two_calls(q1, q2, q3, v3, softclamp, 0.125, None, nw)
        with _lib.KernelProfile() as prof:
            got = _ops.order2_forward(q1, q2, q3, v3, None, False, softclamp, 0.125, norms=nw)
    torch.cuda.synchronize()
    fused = prof.times.get("mfma_order2_short", (0, 0.0))[0]
    assert fused == (1 if H == Hkv else 0), prof.times
    for name, a, b in zip(("out", "lse", "lse23", "msg"), got, ref):
        assert torch.equal(a, b), f"{name}: max diff {(a.float() - b.float()).abs().max().item()}"


@param("root_sigmoid", (False, True))
def test_order2_one_launch_with_epilogue(root_sigmoid):
    """The modules' root-value / gate epilogue on the second pass (y written beside out)."""
    from poly_attention import _ops

    d = dev()
    g = torch.Generator().manual_seed(12)
    B, H, n, dtype = 4, 6, 64, torch.bfloat16
    q1, q2, q3, v3 = _views(B, H, H, n, dtype, g)
    root = torch.randn(B, H, n, 64, generator=g).to(dtype).to(d)
    gate = torch.randn(B, H, n, 64, generator=g).to(dtype).to(d)
    epi = (root, gate, root_sigmoid)
    with torch.no_grad():
        ref = _two_calls(q1, q2, q3, v3, None, 0.125, epi, None)
        got = _ops.order2_forward(q1, q2, q3, v3, None, False, None, 0.125, epi)
    torch.cuda.synchronize()
    assert len(got) == len(ref) == 5
    for name, a, b in zip(("out", "lse", "lse23", "msg", "y"), got, ref):
        assert torch.equal(a, b), f"{name}: max diff {(a.float() - b.float()).abs().max().item()}"


def test_order2_one_launch_discarding_the_inner_level():
    """PA_FLAG_DISCARD_OUT on the first pass (the modules' inference path, which reads only
    out): the one launch skips writing msg and lse23, and out / lse keep their bits."""
    from poly_attention import _lib, _ops

    d = dev()
    g = torch.Generator().manual_seed(13)
    q1, q2, q3, v3 = _views(3, 5, 5, 64, torch.bfloat16, g)
    ws = [(1 + 0.3 * torch.randn(64, generator=g)).to(torch.bfloat16).to(d) for _ in range(3)]
    nw = tuple(zip(ws, (1e-6, 1e-6, 1e-6)))
    with torch.no_grad():
        ref = _two_calls(q1, q2, q3, v3, None, 0.125, None, nw)
        with _lib.KernelProfile() as prof:
            got = _ops.order2_forward(q1, q2, q3, v3, None, False, None, 0.125, norms=nw,
                                      keep_inner=False)
    torch.cuda.synchronize()
    assert prof.times.get("mfma_order2_short", (0, 0.0))[0] == 1, prof.times
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
