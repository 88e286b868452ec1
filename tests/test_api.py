"""The drop-in API on CPU tensors (eager path), modelled on the reference's own tests
(tests/test_poly_attention.py of lucidrains/poly-attention 0.3.6): shapes, Order2 == order-n
equivalence, parallel == stepwise KV cache, context masks, error messages -- plus the
package's modules against the oracle's functional restatement with the same weights."""

import pytest
import torch

import oracle.poly_oracle as O
from poly_attention import NPolyAttention, Order2PolyAttention, PolyAttention, PolyViT
from poly_attention.poly_attention import reference_poly_attention
from poly_attention.poly_transformer import PolyTransformer
from poly_attention.rotary import RotaryEmbedding

param = pytest.mark.parametrize


def setup_function(_):
    torch.manual_seed(0)


@param("causal", (False, True))
@param("kv_heads", (1, 2, 4))
def test_poly_attention(causal, kv_heads):  # reference tests:11-23
    attn = PolyAttention(dim=128, heads=4, kv_heads=kv_heads, dim_head=32, causal=causal)
    x = torch.randn(2, 32, 128)
    rotary_pos_emb = RotaryEmbedding(32)(torch.arange(32))
    out = attn(x, rotary_pos_emb=rotary_pos_emb)
    assert out.shape == (2, 32, 128)
    assert not torch.isnan(out).any()


@param("kv_heads", (1, 2, 4))
def test_poly_attention_mask(kv_heads):  # reference tests:25-39
    attn = PolyAttention(dim=128, heads=4, kv_heads=kv_heads, dim_head=32)
    x = torch.randn(2, 32, 128)
    mask = torch.ones(2, 32).bool()
    mask[:, 16:] = False
    out = attn(x, mask=mask, rotary_pos_emb=RotaryEmbedding(32)(torch.arange(32)))
    assert out.shape == (2, 32, 128)
    assert not torch.isnan(out).any()


@param("causal", (False, True))
@param("kv_heads", (1, 2, 4))
@param("multiply_root_value", (False, True))
@param("use_root_value_as_attn_gate", (False, True))
@param("attn_gate", (False, True))
def test_generalized_poly_attention_equivalence(causal, kv_heads, multiply_root_value,
                                                use_root_value_as_attn_gate, attn_gate):
    # reference tests:41-85
    if use_root_value_as_attn_gate and kv_heads != 4:
        pytest.skip("cannot use root value as attention gate if using GQA")
    kw = dict(dim=128, heads=4, kv_heads=kv_heads, dim_head=32, causal=causal,
              softclamp_value=20.0, multiply_root_value=multiply_root_value,
              use_root_value_as_attn_gate=use_root_value_as_attn_gate, attn_gate=attn_gate)
    m2 = Order2PolyAttention(**kw)
    mn = NPolyAttention(order=2, **kw)
    mn.load_state_dict(m2.state_dict(), strict=False)
    x = torch.randn(2, 32, 128)
    rpe = RotaryEmbedding(32)(torch.arange(32))
    mask = torch.ones(2, 32).bool()
    mask[:, 16:] = False
    assert torch.allclose(m2(x, rotary_pos_emb=rpe), mn(x, rotary_pos_emb=rpe), atol=1e-5)
    assert torch.allclose(m2(x, mask=mask, rotary_pos_emb=rpe),
                          mn(x, mask=mask, rotary_pos_emb=rpe), atol=1e-5)


@param("causal", (False, True))
@param("kv_heads", (1, 2, 4))
@param("order", (2, 3, 4))
@param("shared_kv", (False, True))
def test_n_poly_attention(causal, kv_heads, order, shared_kv):  # reference tests:87-101
    attn = NPolyAttention(dim=128, order=order, heads=4, kv_heads=kv_heads, dim_head=32,
                          causal=causal, shared_kv=shared_kv)
    out = attn(torch.randn(2, 32, 128), rotary_pos_emb=RotaryEmbedding(32)(torch.arange(32)))
    assert out.shape == (2, 32, 128)
    assert not torch.isnan(out).any()


@param("use_rotary_embed", (False, True))
def test_poly_attention_kv_cache(use_rotary_embed):  # reference tests:103-137
    attn = PolyAttention(dim=128, heads=4, dim_head=32, causal=True,
                         use_rotary_embed=use_rotary_embed)
    x = torch.randn(2, 5, 128)
    out_parallel = attn(x)
    cache, outs = None, []
    for i in range(5):
        out, cache = attn(x[:, i:i + 1], cache=cache, return_cache=True)
        outs.append(out)
    assert torch.allclose(out_parallel, torch.cat(outs, dim=-2), atol=1e-5)


@param("order", (2, 3, 4))
@param("kv_heads", (2, 4))
@param("shared_kv", (False, True))
@param("use_rotary_embed", (False, True))
def test_n_poly_attention_kv_cache(order, kv_heads, shared_kv, use_rotary_embed):
    # reference tests:139-179
    attn = NPolyAttention(dim=128, order=order, heads=4, kv_heads=kv_heads, dim_head=32,
                          causal=True, shared_kv=shared_kv, use_rotary_embed=use_rotary_embed)
    x = torch.randn(2, 5, 128)
    out_parallel = attn(x)
    cache, outs = None, []
    for i in range(5):
        out, cache = attn(x[:, i:i + 1], cache=cache, return_cache=True)
        outs.append(out)
    assert torch.allclose(out_parallel, torch.cat(outs, dim=-2), atol=1e-5)


@param("order", (2, 3, 4))
def test_prenorm(order):  # reference tests:181-192
    attn = (PolyAttention(dim=128, heads=4, dim_head=32, prenorm=True) if order == 2 else
            NPolyAttention(dim=128, order=order, heads=4, dim_head=32, prenorm=True))
    out = attn(torch.randn(2, 32, 128))
    assert out.shape == (2, 32, 128) and not torch.isnan(out).any()


@param("order", (2, 3))
def test_poly_vit(order):  # reference tests:194-211
    vit = PolyViT(image_size=32, patch_size=8, num_classes=10, dim=64, depth=2, heads=4,
                  mlp_dim=128, order=order)
    preds = vit(torch.randn(2, 3, 32, 32))
    assert preds.shape == (2, 10) and not torch.isnan(preds).any()


def test_poly_vit_position_table_survives_casts():
    """The reference keeps the sin-cos table in fp32 and casts it per forward (poly_vit.py:96):
    module casts must leave the stored table exact (a half round trip would round it)."""
    from oracle.poly_oracle import posemb_sincos_2d

    vit = PolyViT(image_size=32, patch_size=8, num_classes=10, dim=64, depth=1, heads=4,
                  mlp_dim=128)
    exact = posemb_sincos_2d(h=4, w=4, dim=64)
    assert not torch.equal(exact.half().float(), exact)  # the cast would be visible
    vit = vit.half().float().to(torch.bfloat16)
    assert vit.pos_embedding.dtype == torch.float32
    assert torch.equal(vit.pos_embedding, exact)
    assert vit.linear_head.weight.dtype == torch.bfloat16  # the rest of the module was cast


def test_contexts():  # reference tests:343-370
    attn = PolyAttention(dim=64, heads=4)
    x, c1, c2, c3 = (torch.randn(2, 16, 64) for _ in range(4))
    assert attn(x, context=c1).shape == (2, 16, 64)
    assert attn(x, context=(c1, c2)).shape == (2, 16, 64)
    attn3 = NPolyAttention(dim=64, order=3, heads=4)
    assert attn3(x, context=c1).shape == (2, 16, 64)
    assert attn3(x, context=(c1, c2, c3)).shape == (2, 16, 64)


def test_context_equivalence():  # reference tests:372-403
    a2 = PolyAttention(dim=64, heads=4, use_flash_kernel=False)
    an = NPolyAttention(dim=64, order=2, heads=4)
    an.load_state_dict(a2.state_dict(), strict=False)
    x = torch.randn(2, 16, 64)
    assert torch.allclose(a2(x, context=x + 1.0), an(x, context=x + 1.0), atol=1e-3)
    assert torch.allclose(a2(x, context=(x + 1.0, x - 1.0)), an(x, context=(x + 1.0, x - 1.0)),
                          atol=1e-3)


@param("causal", (False, True))
@param("deep_cross_attention", (False, True))
def test_poly_transformer(deep_cross_attention, causal):  # reference tests:405-424
    model = PolyTransformer(dim=64, depth=3, heads=4, dim_head=16, causal=causal,
                            deep_cross_attention=deep_cross_attention)
    mask = torch.ones(2, 16, dtype=torch.bool)
    mask[:, 8:] = False
    assert model(torch.randn(2, 16, 64), mask=mask).shape == (2, 16, 64)


def test_variable_context_lengths_and_equivalence():  # reference tests:426-514
    m2 = PolyAttention(dim=64, heads=4, use_flash_kernel=False)
    mn = NPolyAttention(dim=64, order=2, heads=4)
    mn.load_state_dict(m2.state_dict(), strict=False)
    x, c1, c2 = torch.randn(2, 16, 64), torch.randn(2, 20, 64), torch.randn(2, 24, 64)
    mx = torch.ones(2, 16, dtype=torch.bool)
    mx[:, 12:] = False
    m1 = torch.ones(2, 20, dtype=torch.bool)
    m1[:, 15:] = False
    m2m = torch.ones(2, 24, dtype=torch.bool)
    m2m[:, 18:] = False
    a = m2(x, context=(c1, c2), mask=mx, context_mask=(m1, m2m))
    b = mn(x, context=(c1, c2), mask=mx, context_mask=(m1, m2m))
    assert not torch.isnan(a).any()
    assert torch.allclose(a, b, atol=1e-5)


@param("order", (2, 3, 4))
def test_n_poly_attention_variable_context_lengths(order):  # reference tests:454-475
    attn = NPolyAttention(dim=64, order=order, heads=4)
    ctxs = tuple(torch.randn(2, 10 + 5 * i, 64) for i in range(order))
    cms = tuple(torch.ones(2, 10 + 5 * i, dtype=torch.bool) for i in range(order))
    for i, cm in enumerate(cms):
        cm[:, (10 + 5 * i) // 2:] = False
    out = attn(torch.randn(2, 16, 64), context=ctxs, context_mask=cms)
    assert out.shape == (2, 16, 64) and not torch.isnan(out).any()


def test_context_mask_correctness():  # reference tests:516-539
    attn = PolyAttention(dim=64, heads=4, use_flash_kernel=False)
    x = torch.randn(2, 16, 64)
    c1u, c2u = torch.randn(2, 10, 64), torch.randn(2, 12, 64)
    c1p = torch.cat([c1u, torch.zeros(2, 10, 64)], dim=1)
    c2p = torch.cat([c2u, torch.zeros(2, 12, 64)], dim=1)
    m1 = torch.zeros(2, 20, dtype=torch.bool)
    m1[:, :10] = True
    m2 = torch.zeros(2, 24, dtype=torch.bool)
    m2[:, :12] = True
    assert torch.allclose(attn(x, context=(c1u, c2u)),
                          attn(x, context=(c1p, c2p), context_mask=(m1, m2)), atol=1e-5)


@param("order", (2, 3))
@param("shared_kv", (False, True))
def test_variable_context_shared_kv(order, shared_kv):  # reference tests:560-576
    attn = (PolyAttention(dim=64, heads=4, shared_kv=shared_kv) if order == 2 else
            NPolyAttention(dim=64, order=order, heads=4, shared_kv=shared_kv))
    ctxs = tuple(torch.randn(2, 10 + 5 * i, 64) for i in range(order))
    out = attn(torch.randn(2, 16, 64), context=ctxs)
    assert out.shape == (2, 16, 64) and not torch.isnan(out).any()


def test_error_messages():  # reference tests:578-586 and poly_attention.py:154,171,221
    attn = PolyAttention(dim=64, heads=4, multiply_root_value=True)
    with pytest.raises(AssertionError, match="first context sequence length"):
        attn(torch.randn(2, 16, 64), context=(torch.randn(2, 20, 64), torch.randn(2, 24, 64)))
    with pytest.raises(AssertionError, match="heads must be divisible by kv_heads"):
        PolyAttention(dim=64, heads=4, kv_heads=3)
    with pytest.raises(AssertionError, match="cannot use root value as attention gate"):
        PolyAttention(dim=64, heads=4, kv_heads=2, use_root_value_as_attn_gate=True)
    attn = PolyAttention(dim=64, heads=4, causal=True)
    _, cache = attn(torch.randn(1, 3, 64), return_cache=True)
    with pytest.raises(AssertionError, match="sequence length must be 1 when using kv cache"):
        attn(torch.randn(1, 2, 64), cache=cache)


def test_explicit_flash_refuses_context_mask():  # reference tests:554-558
    attn = PolyAttention(dim=64, heads=4, use_flash_kernel=True)
    cm = (torch.ones(2, 16, dtype=torch.bool), torch.ones(2, 16, dtype=torch.bool))
    with pytest.raises(AssertionError, match="context_mask is not supported"):
        attn(torch.randn(2, 16, 64), context_mask=cm)


def test_state_dict_keys_match_reference_layout():
    attn = PolyAttention(dim=64, heads=4, kv_heads=2, prenorm=True, separate_context_norms=True,
                         use_rotary_embed=True, multiply_root_value=True, attn_gate=True)
    keys = list(attn.state_dict().keys())
    assert keys == ["norm.weight", "context_norms.0.weight", "context_norms.1.weight",
                    "to_q.weight", "to_kvs.0.weight", "to_kvs.1.weight", "q_norms.0.weight",
                    "q_norms.1.weight", "q_norms.2.weight", "rotary_emb.freqs", "to_out.weight",
                    "to_out.bias"]
    assert attn.to_kvs[0].weight.shape == (2 * 2 * 64, 64)
    assert attn.to_q.weight.shape == (2 * 4 * 64, 64)


# ---- package modules vs the oracle's functional restatement (same weights) ---------------

CFGS = [
    dict(heads=4, dim_head=16, causal=False),
    dict(heads=4, dim_head=16, causal=True, kv_heads=2, softclamp_value=5.0),
    dict(heads=4, dim_head=16, causal=True, multiply_root_value=True, attn_gate=True,
         use_rotary_embed=True, prenorm=True),
    dict(heads=4, dim_head=16, causal=False, shared_kv=True, kv_heads=1),
]


@param("cfg", CFGS)
@param("masked", (False, True))
def test_order2_module_matches_oracle(cfg, masked):
    m = Order2PolyAttention(dim=32, use_flash_kernel=False, **cfg)
    x = torch.randn(2, 9, 32)
    mask = None
    if masked:
        mask = torch.ones(2, 9, dtype=torch.bool)
        mask[1, 6:] = False
    ref = O.order2_forward(m.state_dict(), cfg, x, mask=mask)
    torch.testing.assert_close(m(x, mask=mask), ref, rtol=1e-5, atol=1e-5)


@param("order", (2, 3, 4))
@param("cfg", CFGS)
def test_npoly_module_matches_oracle(order, cfg):
    m = NPolyAttention(dim=32, order=order, use_flash_kernel=False, **cfg)
    x = torch.randn(2, 7, 32)
    ref = O.npoly_forward(m.state_dict(), dict(cfg, order=order), x)
    torch.testing.assert_close(m(x), ref, rtol=1e-5, atol=1e-5)


def test_reference_poly_attention_matches_oracle():
    q1, q2, q3, v3 = (torch.randn(2, 3, 11, 16) for _ in range(4))
    mask = torch.ones(2, 11, dtype=torch.bool)
    mask[0, 7:] = False
    for causal in (False, True):
        a = reference_poly_attention(q1, q2, q2, q3, v3, mask=mask, context_mask=(mask, mask),
                                     causal=causal, softclamp_value=4.0)
        b = O.reference_poly_attention(q1, q2, q2, q3, v3, mask=mask, context_mask=(mask, mask),
                                       causal=causal, softclamp_value=4.0)
        for x, y in zip(a, b):
            torch.testing.assert_close(x, y, rtol=0, atol=0)


@param("shared", (True, False))
@param("splits", (((1, 4), (1, 4), (2, 4)), ((2, 4), (2, 2), (1, 2), (2, 2))))
def test_project_heads_matches_rearrange_split(shared, splits):
    """The fused path's projections + head splits (one GEMM over concatenated weights when the
    input is shared; views with a one-copy backward) against layer(x) + einops Rearrange, in
    values and in every gradient; one piece of a two-piece layer is left unused (its gradient
    is None)."""
    from einops.layers.torch import Rearrange

    from poly_attention import _ops

    d = 8
    layers = [torch.nn.Linear(32, p * h * d, bias=False).double() for p, h in splits]
    x = torch.randn(2, 5, 32, dtype=torch.float64, requires_grad=True)
    xs = [x] * len(layers) if shared else [
        torch.randn(2, 5, 32, dtype=torch.float64, requires_grad=True) for _ in layers]

    def run(fused):
        for t in (*xs, *(l.weight for l in layers)):
            t.grad = None
        if fused:
            groups = _ops.project_heads(layers, xs, list(splits))
        else:
            groups = [list(Rearrange("b n (s h d) -> s b h n d", s=p, h=h)(l(xi)))
                      for l, xi, (p, h) in zip(layers, xs, splits)]
        pieces = [t for g in groups for t in g]
        assert all(t.shape[1] == h for g, (_, h) in zip(groups, splits) for t in g)
        g = torch.Generator().manual_seed(3)
        loss = sum((t * torch.randn(t.shape, generator=g, dtype=t.dtype)).sum()
                   for t in pieces[:-1])  # the last piece unused
        loss.backward()
        return ([t.detach().clone() for t in pieces],
                [t.grad.clone() for t in (*dict.fromkeys(xs), *(l.weight for l in layers))])

    vals, grads = run(True)
    vals_ref, grads_ref = run(False)
    for a, b in zip(vals + grads, vals_ref + grads_ref):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_project_heads_keeps_hooked_layers():
    """A layer with a forward hook is called as a module (the hook fires), not folded into
    the concatenated GEMM."""
    from poly_attention import _ops

    layers = [torch.nn.Linear(16, 8, bias=False) for _ in range(2)]
    seen = []
    layers[1].register_forward_hook(lambda m, i, o: seen.append(o.shape))
    x = torch.randn(1, 3, 16)
    _ops.project_heads(layers, [x, x], [(1, 2), (1, 2)])
    assert seen == [torch.Size([1, 3, 8])]


class _Twice(torch.autograd.Function):
    """A consumer that, like the pass and RMSNorm backwards, writes its input gradient into
    the head-split projection's gradient buffer when its input is a piece of one."""

    @staticmethod
    def forward(ctx, x):
        from poly_attention import _ops

        ctx.slot = _ops.slot_ref(x)
        ctx.like = (x.shape, x.dtype)
        return 2 * x

    @staticmethod
    def backward(ctx, dy):
        from poly_attention import _ops

        out = _ops.claim_slot(ctx.slot, torch.empty(ctx.like[0], dtype=ctx.like[1]))
        if out is None:
            return 2 * dy
        torch.mul(dy, 2, out=out)
        return out


@param("retain", (False, True))
def test_project_heads_gradient_slots(retain):
    """Consumers that write their gradients into the projection's gradient buffer: a piece
    used once (written in place), a piece used by two such consumers (the second one's claim
    is refused; autograd's sum is copied in), a piece used by a plain op and an unused piece.
    A second backward over the retained graph gives the same gradients."""
    from poly_attention import _ops

    splits = [(2, 3), (2, 3)]
    layers = [torch.nn.Linear(24, p * h * 4, bias=False).double() for p, h in splits]
    x = torch.randn(2, 5, 24, dtype=torch.float64, requires_grad=True)
    g = [torch.randn(2, 3, 5, 4, dtype=torch.float64) for _ in range(4)]

    def loss_of(pieces, twice):
        a, b, c, _ = pieces
        return ((twice(a) * g[0]).sum() + (twice(b) * g[1]).sum() + (twice(b) * g[2]).sum()
                + (c.sin() * g[3]).sum())

    def grads(fused):
        for t in (x, *(l.weight for l in layers)):
            t.grad = None
        if fused:
            pieces = [t for grp in _ops.project_heads(layers, [x, x], splits) for t in grp]
            loss = loss_of(pieces, _Twice.apply)
        else:
            pieces = [t for l, (p, h) in zip(layers, splits)
                      for t in l(x).unflatten(-1, (p, h, 4)).permute(2, 0, 3, 1, 4).unbind(0)]
            loss = loss_of(pieces, lambda t: 2 * t)
        loss.backward(retain_graph=retain)
        first = [t.grad.clone() for t in (x, *(l.weight for l in layers))]
        if retain:
            for t in (x, *(l.weight for l in layers)):
                t.grad = None
            loss.backward()
            again = [t.grad for t in (x, *(l.weight for l in layers))]
            for a, b in zip(first, again):
                torch.testing.assert_close(a, b, rtol=0, atol=0)
        return first

    for a, b in zip(grads(True), grads(False)):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_weight_grad_split_choice():
    """The split-K weight gradient's batch count: 8 for outputs up to 2^20 elements, 4 up to
    2^22, else none; halved until every batch holds >= 2048 rows and divides the rows."""
    from poly_attention import _ops

    assert _ops._dw_splits(16384, 1024, 1024) == 8
    assert _ops._dw_splits(16384, 4096, 1024) == 4
    assert _ops._dw_splits(16384, 4096, 4096) == 1
    assert _ops._dw_splits(6144, 256, 512) == 2
    assert _ops._dw_splits(2048, 1024, 1024) == 1
    assert _ops._dw_splits(16383, 1024, 1024) == 1
    x = torch.randn(4, 8, 16, requires_grad=True)
    lin = torch.nn.Linear(16, 8)
    torch.testing.assert_close(_ops.layer_train(lin, x), lin(x))  # CPU: plain F.linear


def test_project_heads_follows_weight_updates():
    """The fused projection concatenates the current weights on every call: updates through
    ``.data`` (which do not bump the version counter), in-place optimizer steps, new weight
    tensors and an inference-mode warm-up followed by a forward with gradients all see the
    weights as they are."""
    from poly_attention import _ops

    layers = [torch.nn.Linear(16, n, bias=False) for n in (8, 16)]
    x = torch.randn(2, 3, 16)
    splits = [(1, 2), (2, 2)]

    def run(grad=False):
        with torch.set_grad_enabled(grad):
            return [t for g in _ops.project_heads(layers, [x, x], splits) for t in g]

    def ref():
        with torch.no_grad():
            return [t for l, (p, h) in zip(layers, splits)
                    for t in l(x).unflatten(-1, (p, h, 4)).permute(2, 0, 3, 1, 4).unbind(0)]

    def check(grad=False):
        for a, b in zip(run(grad), ref()):
            torch.testing.assert_close(a.detach(), b)

    check()
    layers[1].weight.data.copy_(torch.randn(16, 16))  # no version bump
    check()
    with torch.no_grad():
        layers[1].weight.mul_(2.0)
    check()
    layers[0].weight = torch.nn.Parameter(torch.randn(8, 16))
    check()
    with torch.inference_mode():
        run()
    outs = run(grad=True)
    sum(o.sum() for o in outs).backward()
    assert all(l.weight.grad is not None for l in layers)
    check()


def test_poly_flash_attention_is_an_autograd_function():
    """PolyFlashAttention subclasses torch.autograd.Function, as the reference's does
    (flash_poly_attention.py:319), with apply(q1, q2, q3, v3, mask, softclamp_value,
    is_causal)."""
    import inspect

    from poly_attention.flash_poly_attention import PolyFlashAttention

    assert issubclass(PolyFlashAttention, torch.autograd.Function)
    params = list(inspect.signature(PolyFlashAttention.forward).parameters)
    assert params == ["ctx", "q1", "q2", "q3", "v3", "mask", "softclamp_value", "is_causal"]


def test_static_cache_host_count_mirror():
    """The StaticCache's host mirror of the device count: set by construction and
    make_counter, advanced with the count outside capture."""
    from poly_attention import StaticCache
    from poly_attention._cache import _advance_host_count, _set_host_count

    c = torch.zeros(1, dtype=torch.int32)
    _set_host_count(c, 5)
    _advance_host_count(c)
    assert c._pa_host_n == 6
    cache = (torch.zeros(1, 2, 3, 4),) * 3 + (torch.zeros(1, 2, 3), torch.zeros(1, 2, 3, 4))
    counter = StaticCache.make_counter(cache)
    assert counter._pa_host_n == 4 and int(counter) == 4
    StaticCache.advance_counter(counter)
    assert counter._pa_host_n == 5 and int(counter) == 5


def test_norm_layout_check_traces_without_graph_breaks():
    """The q/k-norm dispatch check reads no data pointer, so torch.compile traces through it
    in one graph (a pointer read splits the module's graph, and the split graphs' aliased
    outputs were what torch's compiled-autograd cache failed to serialise)."""
    from poly_attention import _ops

    torch._dynamo.reset()
    w = torch.ones(64)

    def f(x):
        return x * 2 if _ops.rms_layout_supported(x, w) else x - 1

    x = torch.randn(2, 3, 5, 64)
    ex = torch._dynamo.explain(f)(x)
    assert ex.graph_break_count == 0 and ex.graph_count == 1
    # a misaligned base pointer is copied by the call itself, keeping the layout
    base = torch.randn(2 * 3 * 5 * 64 + 1)
    xm = base[1:].view(2, 3, 5, 64)
    assert xm.data_ptr() % 16 != 0
    xa = _ops._aligned16(xm)
    assert xa.data_ptr() % 16 == 0 and torch.equal(xa, xm) and xa.stride() == xm.stride()
