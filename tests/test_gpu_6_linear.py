"""GPU: pa_linear_small (the projections of a decode step) against an fp32 restatement of
torch.nn.functional.linear, and its use inside the modules and the decode harness.

Tolerances: max-abs fp32 1e-5, f16 2e-3, bf16 2e-2, each plus one rounding of the result's
dtype per element (tests/parity.py): the kernel accumulates in fp32 and rounds once, so it
sits within one output rounding of the fp32 sum.
"""

import pytest
import torch

from parity import assert_parity

pytestmark = pytest.mark.gpu
param = pytest.mark.parametrize

TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}


def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda")


def assert_close(got, ref, tol, what):
    """Max-abs error of the result (in its own dtype) within ``tol`` plus one rounding of that
    dtype per element (tests/parity.py)."""
    assert_parity(got, ref, got.dtype, what, tol=tol)


def fp32_linear(x, w, b):
    y = x.float().cpu() @ w.float().cpu().t()
    return y + b.float().cpu() if b is not None else y


@param("dtype", (torch.float32, torch.bfloat16, torch.float16))
@param("rows", (1, 3, 8, 16))
@param("k,n", ((1024, 1024), (1024, 4096), (4096, 1024), (64, 200), (512, 257), (2048, 2048)))
@param("with_bias", (False, True))
def test_linear_small_matches_fp32(dtype, rows, k, n, with_bias):
    from poly_attention import _ops

    d = dev()
    if rows * k * torch.tensor([], dtype=dtype).element_size() > 65536:
        pytest.skip("x exceeds the staging limit (linear_supported routes it to torch)")
    g = torch.Generator().manual_seed(rows * 7 + k + n)
    x = torch.randn(rows, k, generator=g).to(d, dtype)
    w = (torch.randn(n, k, generator=g) * k ** -0.5).to(d, dtype)
    b = torch.randn(n, generator=g).to(d, dtype) if with_bias else None
    assert _ops.linear_supported(x, w, b)
    y = _ops.linear_small(x, w, b)
    torch.cuda.synchronize()
    assert y.shape == (rows, n) and y.dtype == dtype
    assert_close(y, fp32_linear(x, w, b), TOL[dtype], f"{dtype} rows={rows} k={k} n={n}")


def test_linear_small_strided_and_batched_inputs():
    """x as a [B, 1, K] token batch and as a row-strided view (a column slice of a wider
    buffer); the output keeps x's leading shape."""
    from poly_attention import _ops

    d = dev()
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(384, 512, generator=g) * 0.05).to(d, torch.bfloat16)
    b = torch.randn(384, generator=g).to(d, torch.bfloat16)
    x3 = torch.randn(6, 1, 512, generator=g).to(d, torch.bfloat16)
    y3 = _ops.linear_small(x3, w, b)
    assert y3.shape == (6, 1, 384)
    assert_close(y3, fp32_linear(x3.reshape(6, 512), w, b).reshape(6, 1, 384), 2e-2, "batched")
    wide = torch.randn(5, 1024, generator=g).to(d, torch.bfloat16)
    xs = wide[:, 256:768]
    assert xs.stride(0) == 1024
    assert _ops.linear_supported(xs, w, b)
    assert_close(_ops.linear_small(xs, w, b), fp32_linear(xs, w, b), 2e-2, "row-strided x")
    torch.cuda.synchronize()


def test_linear_small_agrees_with_torch_linear():
    """Against torch's own GPU F.linear (hipBLASLt), the decode harness's former path: at
    most one output rounding apart, nearly all elements identical."""
    from poly_attention import _ops

    d = dev()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(8, 1024, generator=g).to(d, torch.bfloat16)
    w = (torch.randn(4096, 1024, generator=g) * 0.03).to(d, torch.bfloat16)
    b = torch.randn(4096, generator=g).to(d, torch.bfloat16)
    ours = _ops.linear_small(x, w, b).float()
    ref = torch.nn.functional.linear(x, w, b).float()
    ulp = ref.abs().clamp_min(1e-30) * 2.0 ** -7
    assert bool(((ours - ref).abs() <= ulp).all())
    assert (ours == ref).float().mean().item() >= 0.9


def test_linear_group_with_epilogues_matches_torch_ops():
    """Four outputs of one x in one launch -- plain, with bias, with GELU and with a residual
    -- each equal to the separate torch ops (F.linear, nn.GELU, +), which round after every
    step, in bf16 and fp32."""
    from poly_attention import _ops

    d = dev()
    for dtype, tol in ((torch.bfloat16, 0.0), (torch.float32, 1e-5)):
        g = torch.Generator().manual_seed(9)
        x = torch.randn(8, 1024, generator=g).to(d, dtype)
        ws = [(torch.randn(n, 1024, generator=g) * 0.03).to(d, dtype) for n in (1024, 2048, 4096, 512)]
        b1 = torch.randn(2048, generator=g).to(d, dtype)
        b2 = torch.randn(4096, generator=g).to(d, dtype)
        res = torch.randn(8, 512, generator=g).to(d, dtype)
        specs = [(ws[0], None, False, None), (ws[1], b1, False, None), (ws[2], b2, True, None),
                 (ws[3], None, False, res)]
        with torch.no_grad():
            outs = _ops.linear_small_group(x, specs)
            F = torch.nn.functional
            lins = [F.linear(x, ws[0]), F.linear(x, ws[1], b1), F.linear(x, ws[2], b2),
                    F.linear(x, ws[3])]
            refs = [lins[0], lins[1], F.gelu(lins[2]), res + lins[3]]
        torch.cuda.synchronize()
        for i, (o, r, li) in enumerate(zip(outs, refs, lins)):
            assert o.shape == r.shape
            if dtype == torch.bfloat16:
                # within one rounding of torch's bf16 chain (its GEMM sums in another order,
                # so the product may sit one rounding away before the epilogue)
                mag = torch.maximum(r.float().abs(), li.float().abs()).clamp_min(2.0 ** -20)
                assert bool(((o.float() - r.float()).abs() <= 2 * mag * 2.0 ** -7).all()), f"output {i}"
            else:
                assert_close(o, r, 1e-5, f"output {i} fp32")
        # against an fp32 restatement, independent of torch's GPU ops
        ref_gelu = fp32_linear(x, ws[2], b2)
        if dtype == torch.bfloat16:
            ref_gelu = ref_gelu.to(dtype).float()
        ref_gelu = torch.nn.functional.gelu(ref_gelu)
        assert_close(outs[2], ref_gelu, max(tol, 2e-2 if dtype == torch.bfloat16 else 1e-5), "gelu")


@param("dtype", (torch.bfloat16, torch.float32))
def test_linear_pre_add_and_norm_match_torch_ops(dtype):
    """x + x_add (also returned), RMSNorm, the product, GELU -- one launch -- against the
    separate torch ops of a pre-norm feed-forward block; the returned sum is bit-identical."""
    from poly_attention import _ops

    d = dev()
    torch.manual_seed(11)
    layer = torch.nn.Linear(1024, 2048).to(d, dtype)
    norm = torch.nn.RMSNorm(1024).to(d, dtype)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.3 * torch.randn(1024, device=d))
        x = torch.randn(8, 1, 1024, device=d).to(dtype)
        a = torch.randn(8, 1, 1024, device=d).to(dtype)
        y, xs = _ops.linear(layer, x, x_add=a, norm=norm, gelu=True, return_sum=True)
        ref_xs = x + a
        lin = layer(norm(ref_xs))
        ref = torch.nn.functional.gelu(lin)
        torch.cuda.synchronize()
    assert torch.equal(xs, ref_xs)
    assert y.shape == ref.shape
    if dtype == torch.bfloat16:
        # the norm output and the product may each sit one rounding from torch's
        mag = torch.maximum(ref.float().abs(), lin.float().abs()).clamp_min(2.0 ** -20)
        assert bool(((y.float() - ref.float()).abs() <= 4 * mag * 2.0 ** -7).all())
    else:
        assert_close(y, ref, 1e-5, "fp32")
    # the norm alone, without weight and without the add (the logits projection)
    plain = torch.nn.RMSNorm(1024, elementwise_affine=False).to(d)
    with torch.no_grad():
        y2 = _ops.linear(layer, x, norm=plain)
        ref2 = layer(plain(x))
    if dtype == torch.bfloat16:
        mag = ref2.float().abs().clamp_min(2.0 ** -20)
        assert bool(((y2.float() - ref2.float()).abs() <= 4 * mag * 2.0 ** -7 + 1e-3).all())
    else:
        assert_close(y2, ref2, 1e-5, "fp32 plain norm")


def test_linear_many_groups_shared_input():
    """linear_many: projections of one input go out four per launch and equal the layers."""
    from poly_attention import _lib, _ops

    d = dev()
    torch.manual_seed(10)
    layers = [torch.nn.Linear(256, n, bias=(i % 2 == 0)).to(d) for i, n in enumerate((256, 512, 128, 256, 64))]
    x = torch.randn(4, 1, 256, device=d)
    with torch.no_grad(), _lib.KernelProfile() as prof:
        outs = _ops.linear_many(layers, [x] * len(layers))
        torch.cuda.synchronize()
    assert prof.times["linear_small"][0] == 2  # 4 + 1 outputs
    with torch.no_grad():
        for layer, o in zip(layers, outs):
            assert_close(o, fp32_linear(x.reshape(4, 256), layer.weight, layer.bias).reshape(4, 1, -1),
                         1e-5, "linear_many")


@param("rows,n,k", ((16384, 1024, 1024), (8192, 4096, 1024), (6144, 256, 512)))
def test_linear_train_split_k_weight_grad(rows, n, k):
    """The training projections' split-K weight gradient (bf16 batches with fp32 partial
    sums) and the rest of its backward against fp32 references, bf16 tolerance."""
    from poly_attention import _ops

    d = dev()
    torch.manual_seed(5)
    assert _ops._dw_splits(rows, n, k) > 1
    lin = torch.nn.Linear(k, n).to(d, torch.bfloat16)
    x = torch.randn(2, rows // 2, k, device=d, dtype=torch.bfloat16, requires_grad=True)
    y = _ops.layer_train(lin, x)
    assert y.grad_fn is not None and "LinearTrain" in type(y.grad_fn).__name__
    dy = torch.randn_like(y)
    y.backward(dy)
    x32 = x.detach().float().reshape(rows, k)
    w32, dy32 = lin.weight.detach().float(), dy.float().reshape(rows, n)
    tol = TOL[torch.bfloat16]
    assert_close(y.reshape(rows, n), x32 @ w32.t() + lin.bias.detach().float(), tol, "y")
    assert_close(x.grad.reshape(rows, k), dy32 @ w32, tol, "dx")
    assert_close(lin.weight.grad, dy32.t() @ x32, tol, "dw")
    assert_close(lin.bias.grad, dy32.sum(0), tol, "db")


def test_linear_supported_routes_other_calls_to_torch():
    from poly_attention import _ops

    d = dev()
    w = torch.randn(64, 128, device=d)
    lin = torch.nn.Linear(128, 64).to(d)
    assert not _ops.linear_supported(torch.randn(17, 128, device=d), w)  # more than 16 rows
    assert not _ops.linear_supported(torch.randn(4, 128, device=d).half(), w)  # mixed dtypes
    xg = torch.randn(4, 128, device=d, requires_grad=True)
    assert not _ops.linear_supported(xg, w)  # autograd keeps torch's op
    y = _ops.linear(lin, xg)  # falls back to the layer itself
    y.sum().backward()
    assert xg.grad is not None
    with torch.no_grad():
        x = torch.randn(4, 128, device=d)
        assert_close(_ops.linear(lin, x), fp32_linear(x, lin.weight, lin.bias), 1e-5, "layer")


def test_decode_steps_with_streamed_projections_equal_parallel():
    """An order-3 module's single-token steps (projections on pa_linear_small) equal its
    parallel causal forward (projections on torch) -- the reference tests:103-179 pattern."""
    from poly_attention import NPolyAttention

    d = dev()
    torch.manual_seed(21)
    m = NPolyAttention(dim=256, order=3, heads=4, dim_head=64, causal=True).to(d).eval()
    x = torch.randn(3, 10, 256, device=d)
    with torch.no_grad():
        ref = m(x)
        out0, cache = m(x[:, :4], return_cache=True)
        outs = [out0]
        for i in range(4, 10):
            o, cache = m(x[:, i:i + 1], cache=cache, return_cache=True)
            outs.append(o)
    assert_close(torch.cat(outs, dim=1), ref, 1e-4, "stepwise")


@param("dtype", (torch.float32, torch.bfloat16, torch.float16))
@param("rows", (1, 5, 16))
@param("k", (64, 512, 2048))
def test_linear_fused_options_sweep(dtype, rows, k):
    """Every input/output option together (x_add + sum, RMSNorm with weight, two outputs: GELU
    with bias, residual) across dtypes, row counts and widths, against an fp32 restatement
    that rounds at the same steps."""
    from poly_attention import _ops

    d = dev()
    es = torch.tensor([], dtype=dtype).element_size()
    if rows * k * es > 65536:
        pytest.skip("x exceeds the staging limit")
    g = torch.Generator().manual_seed(rows * 31 + k)
    rnd = lambda *s: torch.randn(*s, generator=g).to(d, dtype)  # noqa: E731
    x, xa = rnd(rows, k), rnd(rows, k)
    norm = torch.nn.RMSNorm(k).to(d, dtype)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.25 * torch.randn(k, generator=g).to(d))
    w1, b1 = (rnd(96, k) * k ** -0.5), rnd(96)
    w2, res = (rnd(40, k) * k ** -0.5), rnd(rows, 40)
    with torch.no_grad():
        (y1, y2), xs = _ops.linear_small_group(x, [(w1, b1, True, None), (w2, None, False, res)],
                                               x_add=xa, norm=norm, return_sum=True)
    torch.cuda.synchronize()
    r = lambda t: t.to(dtype).float()  # noqa: E731  (one rounding to the dtype)
    xs_ref = r(x.float().cpu() + xa.float().cpu())
    assert torch.equal(xs.float().cpu(), xs_ref)
    rstd = torch.rsqrt(xs_ref.pow(2).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps)
    xn = r(xs_ref * rstd * norm.weight.float().cpu())
    y1_ref = r(torch.nn.functional.gelu(r(xn @ w1.float().cpu().t() + b1.float().cpu())))
    y2_ref = r(res.float().cpu() + r(xn @ w2.float().cpu().t()))
    tol = {torch.float32: 1e-5, torch.float16: 4e-3, torch.bfloat16: 3e-2}[dtype]
    assert_close(y1, y1_ref, tol, f"gelu output {dtype} rows={rows} k={k}")
    assert_close(y2, y2_ref, tol, f"residual output {dtype} rows={rows} k={k}")
