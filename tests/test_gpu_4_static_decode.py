"""GPU: the fixed-capacity decode path -- StaticCache, pa_decode_prologue (q RMSNorm + rotary
+ cache append in one launch) and pa_poly_decode with the position count on the device --
against torch's own ops, the CPU oracle's parallel forward, and replays of a HIP graph.

Bound as the other GPU suites (tests/parity.py): fp32 results max-abs <= 1e-4, bf16 results
max-abs <= 2e-2 plus one bf16 rounding of the value; the raw max-abs error is printed.
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
# the prologue kernel against torch's RMSNorm and apply_rotary_emb


@param("dtype", (torch.float32, torch.bfloat16))
@param("rotate", (False, True))
@param("heads,dim_head", ((4, 64), (2, 128), (3, 32)))
@param("adt", (torch.float32, torch.bfloat16))
def test_prologue_matches_torch_ops(dtype, rotate, heads, dim_head, adt):
    from poly_attention import _ops
    from poly_attention.rotary import RotaryEmbedding, apply_rotary_emb

    d = dev()
    torch.manual_seed(0)
    B, cap, pos = 3, 16, 5
    # a strided [B, heads, 1, dim_head] view, as the module's split of a projection gives
    proj = torch.randn(B, 1, 2 * heads * dim_head, device=d).to(dtype)
    src = proj.reshape(B, 1, 2, heads, dim_head).permute(2, 0, 3, 1, 4)[0]
    norm = torch.nn.RMSNorm(dim_head).to(d, dtype)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.5 * torch.randn(dim_head, device=d))
    # angles as the kernel receives them (bf16 angle rows are read as given, in fp32 math)
    freqs = RotaryEmbedding(dim_head).to(d)(torch.arange(pos + 1, device=d).float())
    freqs = freqs.to(adt).float()
    with torch.no_grad():
        ref = norm(src)
        if rotate:
            ref = apply_rotary_emb(freqs, ref)
    out = torch.empty(B, heads, 1, dim_head, device=d, dtype=dtype)
    cache = torch.full((B, heads, cap, dim_head), 7.0, device=d, dtype=dtype)
    vsrc = torch.randn(B, heads, 1, dim_head, device=d).to(dtype)
    vcache = torch.full((B, heads, cap, dim_head), 7.0, device=d, dtype=dtype)
    n_dev = torch.full((1,), pos + 1, dtype=torch.int32, device=d)  # the step's n
    _ops.decode_prologue([(src, norm.weight, rotate, out, cache),
                          (vsrc, None, False, None, vcache)],
                         eps=torch.finfo(torch.float32).eps,
                         angles=freqs[-1].to(adt) if rotate else None, n_dev=n_dev, capacity=cap)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert_parity(out, ref, torch.float32, "prologue fp32", tol=1e-5)
    else:
        # one rounding apart at most: within one bf16 ulp, and nearly all bit-identical
        diff = (out.float() - ref.float()).abs()
        ulp = ref.float().abs().clamp_min(1e-30) * 2.0 ** -7
        assert bool((diff <= ulp).all()), f"prologue bf16: max diff {diff.max().item():.3e}"
        assert (out == ref).float().mean().item() >= 0.97
    assert torch.equal(cache[:, :, pos:pos + 1], out)
    keep = torch.ones(cap, dtype=torch.bool)
    keep[pos] = False
    assert bool((cache[:, :, keep] == 7.0).all()), "cache positions other than pos changed"
    assert torch.equal(vcache[:, :, pos:pos + 1], vsrc)
    # a position outside the capacity writes nothing
    n_dev.fill_(cap + 1)
    vcache2 = torch.full_like(vcache, 7.0)
    _ops.decode_prologue([(vsrc, None, False, None, vcache2)], eps=1e-6, angles=None,
                         n_dev=n_dev, capacity=cap)
    torch.cuda.synchronize()
    assert bool((vcache2 == 7.0).all())


# ---------------------------------------------------------------------------------------
# modules: StaticCache steps equal the oracle's parallel causal forward


def _module(order, kv_heads, d, dtype):
    from poly_attention import NPolyAttention, Order2PolyAttention

    cfg = dict(heads=4, kv_heads=kv_heads, dim_head=64, causal=True)
    if order == 2:
        m = Order2PolyAttention(dim=64, **cfg)
        fwd = O.order2_forward
    else:
        m = NPolyAttention(dim=64, order=order, **cfg)
        fwd = O.npoly_forward
        cfg = dict(cfg, order=order)
    return m.to(d, dtype).eval(), fwd, cfg


@param("order", (2, 3))
@param("kv_heads", (1, 2, 4))
@param("dtype", (torch.float32, torch.bfloat16))
def test_static_cache_stepwise_equals_parallel(order, kv_heads, dtype):
    """Prefill with return_cache, move the cache into a StaticCache, then single-token steps
    with external rotary (train_enwik8.py:143,160-161): the outputs equal the oracle's
    parallel causal forward (reference tests:103-179 pattern)."""
    from poly_attention import StaticCache

    d = dev()
    torch.manual_seed(12)
    m, fwd, cfg = _module(order, kv_heads, d, dtype)
    n = 12
    x = torch.randn(2, n, 64).to(dtype)
    freqs = O.rotary_freqs(64, torch.arange(n))
    params = {k: v.float().cpu() for k, v in m.state_dict().items()}
    ref = fwd(params, cfg, x.float(), rotary_pos_emb=freqs)
    fd = freqs.to(d)
    with torch.no_grad():
        out0, cache = m(x[:, :5].to(d), rotary_pos_emb=fd[:5], return_cache=True)
        sc = StaticCache(cache, capacity=16)
        outs = [out0]
        for i in range(5, n):
            o, sc2 = m(x[:, i:i + 1].to(d), rotary_pos_emb=fd[:i + 1], cache=sc,
                       return_cache=True)
            assert sc2 is sc
            outs.append(o)
    assert_parity(torch.cat(outs, dim=1), ref, dtype,
                  f"static stepwise order={order} kv={kv_heads} {dtype}")
    assert sc.seq_len() == n
    tup = sc.as_tuple()
    q_cache = tup[0] if order == 2 else tup[0][0]
    assert q_cache.shape[2] == n


@param("order", (2, 3))
@param("dtype", (torch.float32, torch.bfloat16))
def test_static_cache_with_module_rotary(order, dtype):
    """The module's own rotary (use_rotary_embed=True, no external rotary_pos_emb): the tuple
    cache rotates every cached key each step (poly_attention.py:302-304); the StaticCache holds
    its keys rotated once, at the append (the prefix copied from the tuple cache rotated at the
    first step).  Steps equal the oracle's parallel forward and the tuple-cache steps; then one
    step captured into a HIP graph replays the eager steps of a twin cache."""
    from poly_attention import NPolyAttention, Order2PolyAttention, StaticCache

    d = dev()
    torch.manual_seed(16)
    cfg = dict(heads=4, kv_heads=2, dim_head=64, causal=True, use_rotary_embed=True)
    if order == 2:
        m, fwd = Order2PolyAttention(dim=64, **cfg), O.order2_forward
    else:
        cfg = dict(cfg, order=order)
        m, fwd = NPolyAttention(dim=64, **cfg), O.npoly_forward
    m = m.to(d, dtype).eval()
    n, n0 = 12, 5
    x = torch.randn(2, n + 4, 64).to(dtype)
    params = {k: v.float().cpu() for k, v in m.state_dict().items()}
    ref = fwd(params, cfg, x[:, :n].float())
    with torch.no_grad():
        out0, cache = m(x[:, :n0].to(d), return_cache=True)
        sc = StaticCache(cache, capacity=n + 6)
        twin = StaticCache(cache, capacity=n + 6)
        outs = [out0]
        for i in range(n0, n):
            xi = x[:, i:i + 1].to(d)
            o, _ = m(xi, cache=sc, return_cache=True)
            o_t, cache = m(xi, return_cache=True, cache=cache)
            m(xi, cache=twin, return_cache=True)
            assert_parity(o, o_t, dtype, f"module rotary static vs tuple step {i} order={order}")
            outs.append(o)
        assert_parity(torch.cat(outs, dim=1), ref, dtype,
                      f"module rotary static stepwise order={order} {dtype}")
        # capture one step (the prefix is already rotated) and replay it per token
        xb = x[:, n:n + 1].to(d).clone()
        graph_sc = StaticCache(cache, capacity=n + 6)
        m(xb, cache=graph_sc, return_cache=True)  # eager: rotates graph_sc's prefix
        _, cache = m(xb, return_cache=True, cache=cache)  # the tuple cache at the same step
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            warm = StaticCache(cache, capacity=n + 6)
            m(xb, cache=warm, return_cache=True)
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(graph):
            out_g, _ = m(xb, cache=graph_sc, return_cache=True)
        torch.cuda.synchronize()
        for i in range(n + 1, n + 4):
            xb.copy_(x[:, i:i + 1].to(d))
            graph.replay()
            torch.cuda.synchronize()
            o_t, cache = m(x[:, i:i + 1].to(d), return_cache=True, cache=cache)
            torch.cuda.synchronize()
            assert_parity(out_g, o_t, dtype, f"module rotary graph replay at {i} order={order}")


def test_prologue_module_rotary_positions_round_in_the_tensor_dtype():
    """The prologue's angles for a rotary module's own positions: rotary-embedding-torch builds
    the positions in the rotated tensor's dtype (get_seq_pos), so bf16 positions above 256 are
    rounded before the fp32 frequency product; the kernel matches the module's rotation of a
    query at those positions."""
    from poly_attention import _ops
    from poly_attention.rotary import RotaryEmbedding

    d = dev()
    rot = RotaryEmbedding(64).to(d)
    for pos in (3, 255, 257, 1001, 4097):
        src = torch.randn(2, 4, 1, 64, device=d).to(torch.bfloat16)
        out = torch.empty_like(src)
        n_dev = torch.full((1,), pos + 1, dtype=torch.int32, device=d)
        _ops.decode_prologue([(src, None, True, out, None)], eps=1e-6, angles=None, n_dev=n_dev,
                             capacity=pos + 1, inv_freq=rot.freqs, interp=1.0)
        ref = rot.rotate_queries_or_keys(src, offset=pos)
        torch.cuda.synchronize()
        diff = (out.float() - ref.float()).abs()
        ulp = ref.float().abs().clamp_min(1e-30) * 2.0 ** -7
        assert bool((diff <= ulp).all()), f"pos {pos}: max diff {diff.max().item():.3e}"
        assert (out == ref).float().mean().item() >= 0.97, f"pos {pos}"


def test_static_cache_matches_tuple_cache_steps():
    """The fixed-capacity path and the growing-tuple path give the same step outputs and the
    same cache contents (bf16, order 3, GQA)."""
    from poly_attention import StaticCache

    d = dev()
    torch.manual_seed(13)
    m, _, _ = _module(3, 2, d, torch.bfloat16)
    x = torch.randn(2, 10, 64, device=d).to(torch.bfloat16)
    fd = O.rotary_freqs(64, torch.arange(10)).to(d)
    with torch.no_grad():
        _, cache = m(x[:, :4], rotary_pos_emb=fd[:4], return_cache=True)
        sc = StaticCache(cache, capacity=12)
        for i in range(4, 10):
            o_t, cache = m(x[:, i:i + 1], rotary_pos_emb=fd[:i + 1], cache=cache,
                           return_cache=True)
            o_s, _ = m(x[:, i:i + 1], rotary_pos_emb=fd[:i + 1], cache=sc, return_cache=True)
            assert_parity(o_s, o_t, torch.bfloat16, f"static vs tuple step {i}")
    st = sc.as_tuple()
    for a, b in zip((*st[0], *st[1], *st[2], *st[3]), (*cache[0], *cache[1], *cache[2], *cache[3])):
        assert a.shape == b.shape
        assert_parity(a, b, a.dtype, "static vs tuple cache contents", tol=2e-2)


def test_static_caches_with_shared_counter_two_layers():
    """Two stacked order-3 layers whose StaticCaches share one step counter, advanced once
    per token after both layers: the steps equal the stack's parallel causal forward."""
    from poly_attention import StaticCache

    d = dev()
    torch.manual_seed(15)
    m1, _, _ = _module(3, 2, d, torch.float32)
    m2, _, _ = _module(3, 2, d, torch.float32)
    x = torch.randn(2, 9, 64, device=d)
    fd = O.rotary_freqs(64, torch.arange(9)).to(d)
    with torch.no_grad():
        ref = m2(m1(x, rotary_pos_emb=fd), rotary_pos_emb=fd)
        h, c1 = m1(x[:, :4], rotary_pos_emb=fd[:4], return_cache=True)
        out0, c2 = m2(h, rotary_pos_emb=fd[:4], return_cache=True)
        counter = StaticCache.make_counter(c1)
        s1 = StaticCache(c1, capacity=12, counter=counter)
        s2 = StaticCache(c2, capacity=12, counter=counter)
        outs = [out0]
        for i in range(4, 9):
            h, _ = m1(x[:, i:i + 1], rotary_pos_emb=fd[:i + 1], cache=s1, return_cache=True)
            o, _ = m2(h, rotary_pos_emb=fd[:i + 1], cache=s2, return_cache=True)
            StaticCache.advance_counter(counter)
            outs.append(o)
    assert_parity(torch.cat(outs, dim=1), ref, torch.float32, "two layers, shared counter")
    assert s1.seq_len() == s2.seq_len() == 9
    with pytest.raises(ValueError):
        StaticCache(c1, capacity=12, counter=torch.zeros(1, dtype=torch.int64, device=d))


def test_static_cache_errors():
    from poly_attention import StaticCache

    d = dev()
    m, _, _ = _module(2, 4, d, torch.float32)
    x = torch.randn(1, 4, 64, device=d)
    with torch.no_grad():
        _, cache = m(x, return_cache=True)
    with pytest.raises(ValueError):
        StaticCache(cache, capacity=4)
    sc = StaticCache(cache, capacity=8)
    with torch.no_grad(), pytest.raises(AssertionError):
        m(x[:, :2], cache=sc, return_cache=True)  # two tokens (the module's own assert)
    m3, _, _ = _module(3, 4, d, torch.float32)
    with torch.no_grad(), pytest.raises(ValueError):
        m3(x[:, :1], cache=sc, return_cache=True)  # order-2 cache in an order-3 module


# ---------------------------------------------------------------------------------------
# HIP graph: one captured decode step replayed per token


def test_static_decode_step_hip_graph_replays():
    """Capture one StaticCache step (projections, prologue, decode kernels, output
    projection) into a CUDAGraph and replay it per token, with the program's own eager
    steps and synchronisations between replays; every replay equals the eager step on a
    twin cache, and both caches end equal."""
    from poly_attention import StaticCache

    d = dev()
    torch.manual_seed(14)
    m, _, _ = _module(3, 2, d, torch.bfloat16)
    n0, steps = 8, 6
    x = torch.randn(2, n0 + steps, 64, device=d).to(torch.bfloat16)
    fd = O.rotary_freqs(64, torch.arange(n0 + steps)).to(d)
    with torch.no_grad():
        _, cache = m(x[:, :n0], rotary_pos_emb=fd[:n0], return_cache=True)
        eager_sc = StaticCache(cache, capacity=n0 + steps + 2)
        graph_sc = StaticCache(cache, capacity=n0 + steps + 2)
        warm_sc = StaticCache(cache, capacity=n0 + steps + 2)
        xb = x[:, n0:n0 + 1].clone()
        fb = fd[n0:n0 + 1].clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                m(xb, rotary_pos_emb=fb, cache=warm_sc, return_cache=True)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out_g, _ = m(xb, rotary_pos_emb=fb, cache=graph_sc, return_cache=True)
        torch.cuda.synchronize()
        assert graph_sc.seq_len() == n0, "capture must not execute the step"
        for i in range(n0, n0 + steps):
            xb.copy_(x[:, i:i + 1])
            fb.copy_(fd[i:i + 1])
            graph.replay()
            torch.cuda.synchronize()
            ref, _ = m(x[:, i:i + 1], rotary_pos_emb=fd[i:i + 1], cache=eager_sc,
                       return_cache=True)
            torch.cuda.synchronize()
            assert_parity(out_g, ref, torch.bfloat16, f"graph replay at position {i}", tol=1e-2)
    assert graph_sc.seq_len() == eager_sc.seq_len() == n0 + steps
    for a, b in zip(graph_sc.qs + graph_sc.vs + graph_sc.msgs + graph_sc.lses,
                    eager_sc.qs + eager_sc.vs + eager_sc.msgs + eager_sc.lses):
        assert_parity(a[:, :, :n0 + steps], b[:, :, :n0 + steps], a.dtype, "cache after replays",
                      tol=1e-2)
