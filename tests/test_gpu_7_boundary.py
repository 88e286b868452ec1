"""GPU: the drop-in boundary's remaining behaviours against the CPU oracle.

* cached single-token steps with context masks (tuple caches): the reference masks the keys
  of the whole cache in every level (poly_attention.py:75-76,101-102;
  n_poly_attention.py:253-259);
* ``flash_poly_attention(mask=...)``: a key mask of both passes and no query mask, as the
  reference op (flash_poly_attention.py:109-112,261-264), forward and all gradients;
* StaticCache past its capacity: refused on the host for eager steps, flagged on the device
  for captured graph replays;
* torch.compile + autocast through the HIP path (the reference's tests:275-289), compared
  with the fp32 oracle.

Bound as the other GPU suites (tests/parity.py).
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


# ---------------------------------------------------------------------------------------
# cached decode with context masks


@param("order", (2, 3))
@param("kv_heads", (2, 4))
def test_cached_steps_with_context_masks(order, kv_heads):
    """Prefill 5 tokens with context masks and return_cache, then single-token steps whose
    context masks cover the whole cache: every step's output and the returned cache equal the
    oracle's own cached steps (the reference's eager cache branch)."""
    from poly_attention import NPolyAttention, Order2PolyAttention

    d = dev()
    torch.manual_seed(21)
    cfg = dict(heads=4, kv_heads=kv_heads, dim_head=64, causal=True)
    if order == 2:
        m = Order2PolyAttention(dim=64, **cfg).to(d)
        fwd = O.order2_forward
    else:
        m = NPolyAttention(dim=64, order=order, **cfg).to(d)
        fwd = O.npoly_forward
        cfg = dict(cfg, order=order)
    n, n0 = 11, 5
    x = torch.randn(2, n, 64)
    keep = torch.ones(2, n, dtype=torch.bool)
    keep[0, [2, 6, 9]] = False
    keep[1, [1, 7]] = False
    params = {k: v.cpu() for k, v in m.state_dict().items()}

    def masks(upto):
        return tuple(keep[:, :upto] for _ in range(order))

    with torch.no_grad():
        ref0, rcache = fwd(params, cfg, x[:, :n0], context_mask=masks(n0), return_cache=True)
        out0, cache = m(x[:, :n0].to(d), context_mask=tuple(t.to(d) for t in masks(n0)),
                        return_cache=True)
        assert_parity(out0, ref0, torch.float32, f"masked prefill order={order} kv={kv_heads}")
        for i in range(n0, n):
            ref, rcache = fwd(params, cfg, x[:, i:i + 1], context_mask=masks(i + 1),
                              cache=rcache, return_cache=True)
            out, cache = m(x[:, i:i + 1].to(d), context_mask=tuple(t.to(d) for t in masks(i + 1)),
                           cache=cache, return_cache=True)
            assert_parity(out, ref, torch.float32,
                          f"masked cached step {i} order={order} kv={kv_heads}")
    flat = lambda c: [t for x in c for t in (x if isinstance(x, tuple) else (x,))]  # noqa: E731
    for a, b in zip(flat(cache), flat(rcache)):
        assert_parity(a, b, torch.float32, f"masked cache contents order={order}")


# ---------------------------------------------------------------------------------------
# the op's mask: keys of both passes only


@param("dtype", (torch.float32, torch.bfloat16))
@param("causal", (False, True))
def test_flash_op_mask_masks_keys_of_both_passes(dtype, causal):
    from poly_attention.flash_poly_attention import PolyFlashAttention, flash_poly_attention

    d = dev()
    torch.manual_seed(22)
    n = 45
    ts = [torch.randn(2, 4, n, 64).to(dtype) for _ in range(4)]
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[0, 30:] = False
    mask[1, ::7] = False  # key 0 too: the first causal rows are fully masked
    g = [t.to(d).requires_grad_() for t in ts]
    o = [t.float().requires_grad_() for t in ts]
    out = flash_poly_attention(*g, mask=mask.to(d), is_causal=causal)
    assert isinstance(out.grad_fn, PolyFlashAttention._backward_cls)
    ref, _, _ = O.reference_poly_attention(o[0], o[1], o[1], o[2], o[3], causal=causal,
                                           context_mask=(mask, mask))
    dout = torch.randn(ref.shape).to(dtype)
    out.backward(dout.to(d))
    ref.backward(dout.float())
    lp_t = [t.clone().requires_grad_() for t in ts]  # the oracle in the inputs' dtype
    if dtype != torch.float32:
        lp, _, _ = O.reference_poly_attention(lp_t[0], lp_t[1], lp_t[1], lp_t[2], lp_t[3],
                                              causal=causal, context_mask=(mask, mask))
        lp.backward(dout)
    what = f"flash op key mask {dtype} causal={causal}"
    assert_parity(out, ref, dtype, f"{what} out")
    for i, (a, b, c) in enumerate(zip(g, o, lp_t)):
        assert_parity(a.grad, b.grad, dtype, f"{what} grad {i}", grad=True, ref_lp=c.grad)


# ---------------------------------------------------------------------------------------
# StaticCache capacity


def test_static_cache_overflow_raises_eager_and_flags_graph_replays():
    from poly_attention import NPolyAttention, StaticCache

    d = dev()
    torch.manual_seed(23)
    m = NPolyAttention(dim=64, order=3, heads=4, kv_heads=2, dim_head=64,
                       causal=True).to(d).eval()
    x = torch.randn(1, 8, 64, device=d)
    fd = O.rotary_freqs(64, torch.arange(8)).to(d)
    with torch.no_grad():
        _, cache = m(x[:, :4], rotary_pos_emb=fd[:4], return_cache=True)
        # eager: the host knows the count
        sc = StaticCache(cache, capacity=6)
        for i in (4, 5):
            m(x[:, i:i + 1], rotary_pos_emb=fd[:i + 1], cache=sc, return_cache=True)
        with pytest.raises(RuntimeError, match="StaticCache is full"):
            m(x[:, 6:7], rotary_pos_emb=fd[:7], cache=sc, return_cache=True)
        sc.check_overflow()  # nothing was written past the capacity
        # captured: only the device knows the count; the third replay overflows
        gsc = StaticCache(cache, capacity=6)
        xb, fb = x[:, 4:5].clone(), fd[4:5].clone()
        warm = StaticCache(cache, capacity=6)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            m(xb, rotary_pos_emb=fb, cache=warm, return_cache=True)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            m(xb, rotary_pos_emb=fb, cache=gsc, return_cache=True)
        assert gsc.host_step() is None
        for _ in range(2):
            graph.replay()
        torch.cuda.synchronize()
        gsc.check_overflow()
        graph.replay()
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="StaticCache overflow"):
            gsc.check_overflow()


# ---------------------------------------------------------------------------------------
# torch.compile + autocast


def test_compile_autocast_module_matches_oracle():
    """The reference's tests:275-289 -- PolyAttention(dim=128, heads=4,
    use_rotary_embed=True, use_flash_kernel=True) under torch.compile and autocast('cuda'),
    forward and backward -- with the output and the input gradient checked against the fp32
    oracle (autocast's float16 results: max-abs 2e-2 plus one float16 rounding)."""
    from torch.amp import autocast

    from poly_attention import PolyAttention

    d = dev()
    torch.manual_seed(24)
    attn = PolyAttention(dim=128, heads=4, use_rotary_embed=True, use_flash_kernel=True).to(d)
    params = {k: v.detach().cpu().clone() for k, v in attn.state_dict().items()}
    cfg = dict(heads=4, dim_head=64, use_rotary_embed=True)
    x = torch.randn(2, 64, 128)
    xg = x.to(d).requires_grad_()
    model = torch.compile(attn)
    with autocast("cuda"):
        out = model(xg)
        out.sum().backward()
    torch.cuda.synchronize()
    assert out.shape == (2, 64, 128)
    assert not torch.isnan(out).any()
    xo = x.clone().requires_grad_()
    ref = O.order2_forward(params, cfg, xo)
    ref.sum().backward()
    # the oracle with its weights and input in float16 (a bound at least as loose as
    # autocast's mixed float16 / fp32 arithmetic)
    x16 = x.half().requires_grad_()
    O.order2_forward({k: v.half() for k, v in params.items()}, cfg, x16).float().sum().backward()
    assert_parity(out, ref, torch.float16, "compile+autocast out")
    assert_parity(xg.grad, xo.grad, torch.float16, "compile+autocast dx", grad=True,
                  ref_lp=x16.grad)
