"""GPU parity of the drop-in modules and ops (HIP path) vs the CPU oracle.

Bound (tests/parity.py): fp32 results max-abs <= 1e-4; bf16 results max-abs <= 2e-2 against
the fp32 oracle on the same bf16-rounded inputs and weights, plus one rounding of the result's
storage type per element; the raw max-abs error of every check is printed.
"""

import math

import pytest
import torch

import oracle.poly_oracle as O
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
param = pytest.mark.parametrize


def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda")


@param("dtype", (torch.float32, torch.bfloat16))
@param("causal", (False, True))
@param("softclamp_value", (None, 20.0))
@param("seq_len", (31, 32, 127, 128))
def test_flash_poly_attention(dtype, causal, softclamp_value, seq_len):
    """The reference's fused-op test (tests/test_poly_attention.py:213-240), fwd + 4 grads."""
    from poly_attention.flash_poly_attention import flash_poly_attention

    d = dev()
    torch.manual_seed(42)
    tensors = [torch.randn(2, 4, seq_len, 64).to(dtype) for _ in range(4)]
    g_t = [t.to(d).requires_grad_() for t in tensors]
    o_t = [t.float().requires_grad_() for t in tensors]
    q1, q2, q3, v3 = o_t
    out_ref, _, _ = O.reference_poly_attention(q1, q2, q2, q3, v3, softclamp_value=softclamp_value,
                                               causal=causal)
    dout = torch.randn_like(out_ref).to(dtype)
    out_ref.backward(dout.float())
    out = flash_poly_attention(*g_t, softclamp_value=softclamp_value, is_causal=causal)
    out.backward(dout.to(d))
    lp_t = [t.clone().requires_grad_() for t in tensors]  # the oracle in the inputs' dtype
    if dtype != torch.float32:
        lp, _, _ = O.reference_poly_attention(lp_t[0], lp_t[1], lp_t[1], lp_t[2], lp_t[3],
                                              softclamp_value=softclamp_value, causal=causal)
        lp.backward(dout)
    what = f"flash op {dtype} n={seq_len} causal={causal} sc={softclamp_value}"
    assert_parity(out, out_ref, dtype, f"{what} out")
    for i, (a, b, c) in enumerate(zip(g_t, o_t, lp_t)):
        assert_parity(a.grad, b.grad, dtype, f"{what} grad {i}", grad=True, ref_lp=c.grad)


def test_flash_poly_attention_context_mask_disallowed():  # reference tests:541-558
    from poly_attention.flash_poly_attention import flash_poly_attention

    d = dev()
    q = torch.randn(2, 4, 16, 32, device=d)
    cm = (torch.ones(2, 16, dtype=torch.bool), torch.ones(2, 16, dtype=torch.bool))
    with pytest.raises(AssertionError, match="context_mask is not supported"):
        flash_poly_attention(q, q, q, q, context_mask=cm)


ORDER2_CFGS = [
    dict(heads=4, dim_head=64, causal=False),
    dict(heads=4, dim_head=64, causal=True, softclamp_value=20.0),
    dict(heads=8, kv_heads=2, dim_head=64, causal=True),
    dict(heads=4, dim_head=32, causal=True, multiply_root_value=True, attn_gate=True,
         use_rotary_embed=True, prenorm=True),
    dict(heads=4, kv_heads=1, dim_head=64, causal=False, shared_kv=True),
    # the epilogue fused into pass 2 at the MFMA head dim: GQA root, sigmoid root, shared kv
    dict(heads=8, kv_heads=2, dim_head=64, causal=True, multiply_root_value=True, attn_gate=True),
    dict(heads=4, dim_head=64, causal=False, multiply_root_value=True,
         use_root_value_as_attn_gate=True, attn_gate=True),
    dict(heads=4, kv_heads=2, dim_head=64, causal=True, shared_kv=True, multiply_root_value=True),
]


def _grad_params(m):
    # the module's weights as CPU leaves for the oracle, so that it returns their gradients
    return {k: v.detach().cpu().clone().requires_grad_(v.is_floating_point())
            for k, v in m.state_dict().items()}


def _check_param_grads(m, params, what=""):
    """Every parameter gradient (projections through the fused head split and concatenated
    GEMM, q/k norm weights, output projection) against the oracle's."""
    for k, p in m.named_parameters():
        ref = params[k].grad
        assert (p.grad is None) == (ref is None), k
        if ref is not None:
            assert_parity(p.grad, ref, torch.float32, f"{what} d{k}")


@param("cfg", ORDER2_CFGS)
@param("masked", (False, True))
@param("seq_len", (31, 64))
def test_order2_module_e2e(cfg, masked, seq_len):
    """Module-level fwd + dx vs the oracle (reference tests:242-273 and :291-341)."""
    from poly_attention import Order2PolyAttention

    d = dev()
    torch.manual_seed(42)
    m = Order2PolyAttention(dim=64, use_flash_kernel=True, **cfg).to(d)
    x = torch.randn(2, seq_len, 64)
    mask = None
    if masked:
        mask = torch.ones(2, seq_len, dtype=torch.bool)
        mask[:, seq_len // 2:] = False
    xg = x.to(d).requires_grad_()
    out = m(xg, mask=mask.to(d) if masked else None)
    params = _grad_params(m)
    xo = x.clone().requires_grad_()
    ref = O.order2_forward(params, cfg, xo, mask=mask)
    dout = torch.randn_like(ref)
    out.backward(dout.to(d))
    ref.backward(dout)
    what = f"order2 module {cfg} masked={masked} n={seq_len}"
    assert_parity(out, ref, torch.float32, f"{what} out")
    assert_parity(xg.grad, xo.grad, torch.float32, f"{what} dx")
    _check_param_grads(m, params, what)


@param("order", (2, 3))
@param("gate_root", (False, True))
def test_npoly_module_epilogue_e2e(order, gate_root):
    """NPolyAttention's root value / gate (n_poly_attention.py:315-326): fused into the final
    pass at order 2, torch element-wise at order 3; fwd, dx and parameter gradients."""
    from poly_attention import NPolyAttention

    d = dev()
    torch.manual_seed(9)
    cfg = dict(heads=4, dim_head=64, causal=True, order=order, multiply_root_value=True,
               use_root_value_as_attn_gate=gate_root, attn_gate=True)
    m = NPolyAttention(dim=64, use_flash_kernel=True, **cfg).to(d)
    x = torch.randn(2, 40, 64)
    xg = x.to(d).requires_grad_()
    out = m(xg)
    params = _grad_params(m)
    xo = x.clone().requires_grad_()
    ref = O.npoly_forward(params, cfg, xo)
    dout = torch.randn_like(ref)
    out.backward(dout.to(d))
    ref.backward(dout)
    what = f"npoly epilogue order={order} sigmoid root={gate_root}"
    assert_parity(out, ref, torch.float32, f"{what} out")
    assert_parity(xg.grad, xo.grad, torch.float32, f"{what} dx")
    _check_param_grads(m, params, what)


@param("dtype", (torch.bfloat16, torch.float16, torch.float32))
@param("root_heads,root_sigmoid,gate", ((8, False, True), (2, False, True), (8, True, True),
                                        (8, False, False), (None, False, True)))
def test_fused_epilogue_equals_torch_tail(dtype, root_heads, root_sigmoid, gate):
    """The order-2 chain with the epilogue fused into pass 2 against the same chain followed
    by torch's element-wise tail (poly_attention.py:342-351) on the same kernels: y, and the
    gradients of q1..v3, root and gate.  An implementation-consistency check (the oracle
    parity of the epilogue is test_order2_module_e2e's and test_gpu_14's): both sides are
    results stored in bf16 / f16, each rounded on its own, so y is held to two storage
    roundings of the value (tol 0); the gradients to four roundings of their largest value,
    since torch's tail also rounds its intermediate products (dy * out, the sigmoid's
    derivative, a GQA root's per-head terms before their sum) where the fused epilogue keeps
    them in fp32.  fp32 allows for the sigmoid's last bit and the order of the GQA root's
    head sum (tol 1e-5)."""
    from poly_attention import _ops

    d = dev()
    B, H, N, D = 2, 8, 160, 64
    gen = torch.Generator().manual_seed(5)

    def rnd(*s):
        return torch.randn(*s, generator=gen).to(dtype).to(d)

    q1, q2, q3, v3 = (rnd(B, H, N, D) for _ in range(4))
    root = rnd(B, root_heads, N, D) if root_heads else None
    gt = rnd(B, H, N, D) if gate else None
    dy = rnd(B, H, N, D)
    leaves = [t.requires_grad_() for t in (q1, q2, q3, v3, root, gt) if t is not None]
    epi = (root, gt, root_sigmoid)
    y, _, _, _ = _ops._Order2Chain.apply(q1, q2, q3, v3, root, gt, True, 0.0, D ** -0.5,
                                         root_sigmoid)
    y.backward(dy)
    fused = [y.detach()] + [t.grad for t in leaves]
    for t in leaves:
        t.grad = None
    out, _, _, _ = _ops._Order2Chain.apply(q1, q2, q3, v3, None, None, True, 0.0, D ** -0.5,
                                           False)
    ref = _ops.apply_epilogue(out, epi)
    ref.backward(dy)
    torch.cuda.synchronize()
    names = ["y", "dq1", "dq2", "dq3", "dv3"] + (["droot"] if root is not None else []) + \
        (["dgate"] if gate else [])
    what = f"fused epilogue {dtype} root_heads={root_heads} sigmoid={root_sigmoid} gate={gate}"
    u = {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}[dtype]
    for name, a, b in zip(names, fused, [ref.detach()] + [t.grad for t in leaves]):
        b = b.float().cpu()
        if dtype == torch.float32:
            tol = 1e-5
        else:
            tol = 0.0 if name == "y" else 4 * u * b.abs().max().item()
        assert_parity(a, b, dtype, f"{what} {name}", tol=tol, grad=name != "y", roundings=2)


@param("order", (2, 3, 4))
@param("kv_heads", (2, 4))
@param("causal", (False, True))
def test_npoly_module_e2e(order, kv_heads, causal):
    from poly_attention import NPolyAttention

    d = dev()
    torch.manual_seed(7)
    cfg = dict(heads=4, kv_heads=kv_heads, dim_head=64, causal=causal, order=order)
    m = NPolyAttention(dim=64, **cfg).to(d)
    x = torch.randn(2, 40, 64)
    xg = x.to(d).requires_grad_()
    out = m(xg)
    params = _grad_params(m)
    xo = x.clone().requires_grad_()
    ref = O.npoly_forward(params, cfg, xo)
    dout = torch.randn_like(ref)
    out.backward(dout.to(d))
    ref.backward(dout)
    what = f"npoly module {cfg}"
    assert_parity(out, ref, torch.float32, f"{what} out")
    assert_parity(xg.grad, xo.grad, torch.float32, f"{what} dx")
    _check_param_grads(m, params, what)


def test_contexts_and_context_masks_e2e():
    """Variable context lengths with context masks (reference tests:426-514) on the GPU."""
    from poly_attention import Order2PolyAttention

    d = dev()
    torch.manual_seed(3)
    cfg = dict(heads=4, dim_head=64)
    m = Order2PolyAttention(dim=64, **cfg).to(d)
    x, c1, c2 = torch.randn(2, 16, 64), torch.randn(2, 20, 64), torch.randn(2, 24, 64)
    mx = torch.ones(2, 16, dtype=torch.bool)
    mx[:, 12:] = False
    m1 = torch.ones(2, 20, dtype=torch.bool)
    m1[:, 15:] = False
    m2 = torch.ones(2, 24, dtype=torch.bool)
    m2[:, 18:] = False
    out = m(x.to(d), context=(c1.to(d), c2.to(d)), mask=mx.to(d),
            context_mask=(m1.to(d), m2.to(d)))
    params = {k: v.cpu() for k, v in m.state_dict().items()}
    ref = O.order2_forward(params, cfg, x, context=(c1, c2), mask=mx, context_mask=(m1, m2))
    assert_parity(out.detach(), ref, torch.float32, "contexts + context masks out")


@param("order", (2, 3))
@param("kv_heads", (1, 2, 4))
@param("use_rotary_embed", (False, True))
def test_kv_cache_stepwise_equals_parallel(order, kv_heads, use_rotary_embed):
    """Prefill with return_cache, then single-token steps through the decode kernel; the
    concatenated outputs equal the oracle's parallel causal forward (reference tests:103-179)."""
    from poly_attention import NPolyAttention, Order2PolyAttention

    d = dev()
    torch.manual_seed(11)
    cfg = dict(heads=4, kv_heads=kv_heads, dim_head=64, causal=True,
               use_rotary_embed=use_rotary_embed)
    if order == 2:
        m = Order2PolyAttention(dim=64, **cfg).to(d)
        fwd = O.order2_forward
    else:
        m = NPolyAttention(dim=64, order=order, **cfg).to(d)
        fwd = O.npoly_forward
        cfg = dict(cfg, order=order)
    x = torch.randn(2, 12, 64)
    params = {k: v.cpu() for k, v in m.state_dict().items()}
    ref = fwd(params, cfg, x)
    with torch.no_grad():
        out0, cache = m(x[:, :5].to(d), return_cache=True)
        outs = [out0]
        for i in range(5, 12):
            o, cache = m(x[:, i:i + 1].to(d), cache=cache, return_cache=True)
            outs.append(o)
    assert_parity(torch.cat(outs, dim=1), ref, torch.float32,
                  f"stepwise order={order} kv={kv_heads} rotary={use_rotary_embed}")


@param("chunk,H,G,dh,sc", ((0, 8, 2, 128, None), (64, 8, 2, 128, None), (64, 64, 2, 128, None),
                           (0, 2, 2, 128, None), (64, 2, 2, 64, None), (64, 4, 2, 64, None),
                           (0, 4, 2, 32, 5.0), (64, 3, 3, 128, 5.0), (0, 2, 2, 256, None),
                           (64, 8, 4, 256, None)))
def test_decode_kernel_gqa_synthetic_cache(chunk, H, G, dh, sc):
    """Config-5 shape class (GQA) at a small cache, with a synthetic cache (q/k/v/msg ~ N(0,1),
    lse = log(j+1) + N(0,1)) against the oracle's cached branch; chunk=64 splits the 299 cached
    positions over five partial records (the merge path); 64 query heads on 2 KV heads (33
    level heads per group) exceed the combine kernel's LDS state budget, so some heads are
    merged in its second phase.  One or two heads per KV group take the streaming partial
    kernel, more the grouped one."""
    from poly_attention import _ops

    d = dev()
    g = torch.Generator().manual_seed(5)
    B, n = 2, 300
    r = H // G
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        q2c, q3c, v3c = (torch.randn(B, G, n, dh, generator=g).to(dtype) for _ in range(3))
        msg = torch.randn(B, H, n, dh, generator=g).to(dtype)
        lse = (torch.log(torch.arange(1, n + 1).float()) + torch.randn(B, H, n, generator=g))
        q1 = torch.randn(B, H, 1, dh, generator=g).to(dtype)
        q2n = q2c[:, :, -1:].clone()
        # oracle: the reference's cached step with the cache of the first n-1 positions
        f = lambda t: O.repeat_kv(t.float(), r)  # noqa: E731
        cache = (None, None, None, lse[:, :, :-1], msg[:, :, :-1].float())
        ref, lse_step, msg_step = O.reference_poly_attention(
            q1.float(), f(q2n), f(q2c), f(q3c), f(v3c), cache=cache, softclamp_value=sc)
        msg_d, lse_d = msg.to(d).clone(), lse.to(d).clone()
        out = _ops.poly_decode_step([q1.to(d), q2n.to(d)], [q2c.to(d), q3c.to(d)], [v3c.to(d)],
                                    [msg_d], [lse_d], kv_heads=G, heads=H, softclamp=sc,
                                    scale=dh ** -0.5, chunk=chunk)
        torch.cuda.synchronize()
        what = f"decode {dtype} chunk={chunk} H={H} G={G} d={dh} sc={sc}"
        assert_parity(out, ref, dtype, f"{what} out")
        assert_parity(msg_d[:, :, -1:], msg_step, dtype, f"{what} msg slot")
        assert_parity(lse_d[:, :, -1], lse_step[:, :, 0], torch.float32, f"{what} lse slot",
                      tol=TOL[dtype])
        # untouched cache positions
        assert torch.equal(msg_d[:, :, :-1].cpu(), msg[:, :, :-1])


def test_polyvit_forward_replays_from_hip_graph():
    """PolyViT's forward captured once into a HIP graph (the position table no longer moves
    host -> device per call) replays bit-identical to the eager forward, for new inputs
    copied into the captured buffer."""
    from poly_attention import PolyViT

    d = dev()
    torch.manual_seed(16)
    vit = PolyViT(image_size=32, patch_size=8, num_classes=10, dim=64, depth=2, heads=4,
                  mlp_dim=128).to(d, torch.bfloat16).eval()
    img = torch.randn(4, 3, 32, 32, device=d).to(torch.bfloat16)
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            vit(img)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = vit(img)
        for seed in range(3):
            new = torch.randn(4, 3, 32, 32, generator=torch.Generator().manual_seed(seed))
            img.copy_(new.to(d, torch.bfloat16))
            graph.replay()
            torch.cuda.synchronize()
            ref = vit(img)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"replay {seed}"
