"""GPU parity of single attention passes (libpolyattn through its C ABI) vs the CPU oracle.

Bound (tests/parity.py): fp32 results max-abs <= 1e-4; bf16 / f16 results max-abs <= 2e-2
against the fp32 oracle on the same low-precision-rounded inputs, plus one rounding of the
result's storage type per element; the raw max-abs error of every check is printed.
"""

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


def randn(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def run_pass(q, k, v, vmul=None, bias=None, key_mask=None, query_mask=None, causal=False,
             softclamp=None, grads=True, seed=99):
    """Run the HIP pass (autograd custom op) and the oracle on the same inputs."""
    from poly_attention import _ops

    d = dev()
    inputs = [q, k, v, vmul, bias]
    g_in = [t.detach().to(d).requires_grad_(grads) if t is not None else None for t in inputs]
    o_in = [t.detach().float().clone().requires_grad_(grads) if t is not None else None
            for t in inputs]
    km = key_mask.to(d) if key_mask is not None else None
    qm = query_mask.to(d) if query_mask is not None else None
    out, lse = _ops.attn_pass(*g_in, key_mask=km, query_mask=qm, causal=causal,
                              softclamp=softclamp)
    ref_out, ref_lse = O.attn_pass(*o_in, key_mask=key_mask, query_mask=query_mask,
                                   causal=causal, softclamp_value=softclamp)
    res = dict(out=(out, ref_out, None), lse=(lse, ref_lse, None))
    if grads:
        do = randn(ref_out.shape, q.dtype, seed)
        dl = randn(ref_lse.shape, torch.float32, seed + 1)
        torch.autograd.backward((out, lse), (do.to(d), dl.to(d)))
        torch.autograd.backward((ref_out, ref_lse), (do.float(), dl))
        lp_in = [None] * len(inputs)
        if q.dtype != torch.float32:
            # the oracle in the inputs' own precision: the reference's arithmetic at that
            # precision, whose drift from the fp32 oracle bounds the low-precision gradients
            lp_in = [t.detach().clone().requires_grad_() if t is not None else None for t in inputs]
            lp_out, lp_lse = O.attn_pass(*lp_in, key_mask=key_mask, query_mask=query_mask,
                                         causal=causal, softclamp_value=softclamp)
            torch.autograd.backward((lp_out, lp_lse), (do, dl.to(lp_lse.dtype)))
        for name, a, b, c in zip(("dq", "dk", "dv", "dvmul", "dbias"), g_in, o_in, lp_in):
            if a is not None:
                res[name] = (a.grad, b.grad, c.grad if c is not None else None)
    torch.cuda.synchronize()
    return res


def check(res, dtype, what=""):
    for name, (got, ref, ref_lp) in res.items():
        if name == "lse":  # fp32 in both, from inputs rounded to dtype
            got = got.float().cpu()
            ok = ref.detach() > -1e30
            assert_parity(got[ok], ref.detach()[ok], torch.float32, f"{what} lse", tol=TOL[dtype])
            assert bool((got[~ok] <= -1e30).all()), "fully-masked rows must keep lse = -finfo.max"
            continue
        # gradients (dbias stored in fp32) are computed from inputs in dtype
        assert_parity(got, ref, dtype, f"{what} {name}", tol=TOL[dtype],
                      grad=name.startswith("d"), ref_lp=ref_lp)


@param("dtype", (torch.float32, torch.bfloat16, torch.float16))
@param("n", (31, 32, 127, 128))
@param("causal", (False, True))
@param("softclamp", (None, 20.0))
def test_pass_basic(dtype, n, causal, softclamp):
    """The reference's fused-op test grid (tests:213-240): N in {31,32,127,128}, d = 64."""
    shape = (2, 4, n, 64)
    q, k, v = (randn(shape, dtype, s) for s in (1, 2, 3))
    check(run_pass(q, k, v, causal=causal, softclamp=softclamp), dtype,
          f"basic {dtype} n={n} causal={causal} sc={softclamp}")


@param("dtype", (torch.float32, torch.bfloat16))
@param("d", (16, 32, 128))
def test_pass_head_dims(dtype, d):
    q, k, v = (randn((1, 2, 40, d), dtype, s) for s in (4, 5, 6))
    check(run_pass(q, k, v, causal=True), dtype, f"head dim {d} {dtype}")


@param("dtype", (torch.float32, torch.bfloat16))
@param("causal", (False, True))
def test_pass_gqa_bias_vmul(dtype, causal):
    """A middle level of the chain: queries at 8 heads over 2 KV heads, key bias (the deeper
    level's lse) and a value multiplier (the deeper level's msg)."""
    q = randn((2, 8, 50, 64), dtype, 7)
    k, v, vmul = (randn((2, 2, 50, 64), dtype, s) for s in (8, 9, 10))
    bias = randn((2, 2, 50), torch.float32, 11, scale=2.0)
    check(run_pass(q, k, v, vmul=vmul, bias=bias, causal=causal), dtype,
          f"gqa+bias+vmul {dtype} causal={causal}")


@param("dtype", (torch.float32, torch.bfloat16))
@param("causal", (False, True))
def test_pass_masks_and_degenerate_rows(dtype, causal):
    """Key / query masks with fully-masked rows (uniform over -finfo.max entries)."""
    q, k, v = (randn((2, 2, 24, 32), dtype, s) for s in (12, 13, 14))
    km = torch.ones(2, 24, dtype=torch.bool)
    km[:, 17:] = False
    km[1, 0] = False
    qm = torch.ones(2, 24, dtype=torch.bool)
    qm[0, 20:] = False
    bias = randn((2, 2, 24), torch.float32, 15)
    bias[1, 1, 5] = -torch.finfo(torch.float32).max
    check(run_pass(q, k, v, bias=bias, key_mask=km, query_mask=qm, causal=causal), dtype,
          f"masks {dtype} causal={causal}")


@param("dtype", (torch.bfloat16, torch.float16, torch.float32))
@param("d", (64, 128))
@param("n", (150, 256))
@param("causal", (False, True))
@param("gqa", (False, True))
def test_pass_masked_mfma_head_dims(dtype, d, n, causal, gqa):
    """Masked passes at the MFMA head dims (the backward's normal rows on the MFMA kernels, the
    fully-masked rows added by the fix-ups), forward and all gradients:
    * leading keys masked: causal rows 0-2 fully masked (class-1 keys all masked ones);
    * batch 1, keys 3-5 biased to -finfo.max (bias class 1): causal rows 3-5 fully masked with
      unmasked class-1 keys; non-causal, every other key of batch 1 masked as well, so every
      row of batch 1 is fully masked the same way;
    * a -inf bias entry (class 2) and query-masked rows (uniform over the bias-class-0 keys);
    * gqa: 4 query heads over 2 key heads with a value multiplier (a middle chain level).
    n = 150 leaves a key count that is not a multiple of 4 (row-padded key terms).  fp32 passes
    take the fp32 MFMA backward kernels and the same fix-ups (the kernel profile shows them)."""
    from poly_attention import _lib

    B, H, HK = 2, 4, (2 if gqa else 4)
    q = randn((B, H, n, d), dtype, 31)
    k, v = (randn((B, HK, n, d), dtype, s) for s in (32, 33))
    vmul = randn((B, HK, n, d), dtype, 34) if gqa else None
    bias = torch.log(torch.arange(1, n + 1).float())[None, None].repeat(B, HK, 1)
    bias = bias + randn((B, HK, n), torch.float32, 35)
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
    with _lib.KernelProfile() as prof:
        res = run_pass(q, k, v, vmul=vmul, bias=bias, key_mask=km, query_mask=qm, causal=causal)
    check(res, dtype, f"masked mfma {dtype} d={d} n={n} causal={causal} gqa={gqa}")
    ran = set(prof.times)
    if dtype == torch.float32:
        assert any(k.startswith("mfma_bwd_f32_dq") for k in ran), sorted(ran)
        assert any(k.startswith("mfma_bwd_f32_dkv") for k in ran), sorted(ran)
    assert "fix_rows" in ran and "fix_keys" in ran, sorted(ran)


@param("dtype", (torch.bfloat16, torch.float32))
@param("causal", (False, True))
@param("softclamp", (None, 5.0))
def test_pass_masked_mfma_cross_lengths_softclamp(dtype, causal, softclamp):
    """Masks at the MFMA head dim with 96 queries over 200 keys (contexts), softclamp on the
    scores, a key bias with -finfo.max entries and GQA: the key term, the fully-masked-row
    fix-ups and the causal limits with nq != nk."""
    nq, nk = 96, 200
    q = randn((2, 4, nq, 64), dtype, 61)
    k, v = (randn((2, 2, nk, 64), dtype, s) for s in (62, 63))
    bias = randn((2, 2, nk), torch.float32, 64) + 2.0
    bias[0, :, 2:4] = -torch.finfo(torch.float32).max
    km = torch.ones(2, nk, dtype=torch.bool)
    km[0, :2] = False
    km[1, 50:120] = False
    qm = torch.ones(2, nq, dtype=torch.bool)
    qm[1, :5] = False
    res = run_pass(q, k, v, bias=bias, key_mask=km, query_mask=qm, causal=causal,
                   softclamp=softclamp)
    check(res, dtype, f"masked cross {dtype} causal={causal} sc={softclamp}")


@param("causal", (False, True))
def test_pass_masked_mfma_key_mask_only(causal):
    """A key mask with no bias (the first pass of a masked chain): the key mask becomes the
    MFMA kernels' only key term; batch 1 masks every key (every row fully masked)."""
    dtype, n = torch.bfloat16, 200
    q, k, v = (randn((2, 4, n, 64), dtype, s) for s in (41, 42, 43))
    km = torch.ones(2, n, dtype=torch.bool)
    km[0, ::5] = False
    km[0, :2] = False
    km[1] = False
    check(run_pass(q, k, v, key_mask=km, causal=causal), dtype,
          f"masked mfma key mask only causal={causal}")


@param("dtype,gqa", ((torch.bfloat16, False), (torch.float16, False), (torch.bfloat16, True)))
@param("causal", (False, True))
@param("with_bias", (False, True))
def test_pass_padding_masks_skip_whole_tiles(dtype, gqa, causal, with_bias):
    """Padding masks that cover whole key tiles and whole key blocks: the MFMA kernels pass
    over a tile whose every key term is -inf (forward and dQ: 64-key tiles) and skip a
    workgroup's sweep when all 128 keys of its block are masked (dK/dV), which must give the
    eager result, forward and all gradients:
    * batch 0: left padding, keys 0-199 masked (causal rows 0-199 fully masked);
    * batch 1: right padding, keys 300-511 masked;
    * batch 2: keys 128-383 masked (dead tiles between live ones) and every fifth key;
    * batch 3: a key bias of -inf on keys 64-191 instead of a mask (with_bias), else unmasked.
    gqa: 4 query heads over 2 key heads (the dK/dV workgroups sum both query heads of a group;
    the key bias, at the key heads, is the key term's)."""
    B, H, n, d = 4, 4, 512, 64
    HK = 2 if gqa else H
    q = randn((B, H, n, d), dtype, 71)
    k, v = (randn((B, HK, n, d), dtype, s) for s in (72, 73))
    km = torch.ones(B, n, dtype=torch.bool)
    km[0, :200] = False
    km[1, 300:] = False
    km[2, 128:384] = False
    km[2, ::5] = False
    bias = None
    if with_bias:
        bias = randn((B, HK, n), torch.float32, 74)
        bias[3, :, 64:192] = -float("inf")
    res = run_pass(q, k, v, bias=bias, key_mask=km, causal=causal)
    check(res, dtype, f"padding masks {dtype} gqa={gqa} causal={causal} bias={with_bias}")


@param("gqa", (False, True))
def test_pass_padding_masks_units_spread_over_xcds(gqa):
    """Grids that divide over the 8 XCDs with heads a multiple of 8 (times the GQA group): each
    XCD then runs some heads of every batch row (instead of whole batch rows), so that padding
    of some rows spreads over all XCDs.  Left padding on batch 0 (keys 0-639 masked, causal
    rows 0-639 fully masked), right padding on batch 1 (keys 384- masked): forward and every
    gradient against the eager result.  gqa: 16 query heads over 8 key heads (group of 2)."""
    B, n, d = 2, 1024, 64
    H, HK = (16, 8) if gqa else (8, 8)
    q = randn((B, H, n, d), torch.bfloat16, 81)
    k, v = (randn((B, HK, n, d), torch.bfloat16, s) for s in (82, 83))
    km = torch.ones(B, n, dtype=torch.bool)
    km[0, :640] = False
    km[1, 384:] = False
    res = run_pass(q, k, v, key_mask=km, causal=True)
    check(res, torch.bfloat16, f"padding masks spread over XCDs gqa={gqa}")


@param("causal", (False, True))
def test_pass_padding_masks_ragged_length(causal):
    """A length that is not a multiple of the 64-key tile (1000) with padding that does not
    align to tiles: batch 0 left-padded (keys 0-332 masked), batch 1 right-padded (keys from
    777 on masked), 8 query heads over 4 key heads.  The live key range then starts and ends
    inside tiles, and its last tile is also the partial last tile of the keys."""
    B, H, HK, n, d = 2, 8, 4, 1000, 64
    q = randn((B, H, n, d), torch.bfloat16, 91)
    k, v = (randn((B, HK, n, d), torch.bfloat16, s) for s in (92, 93))
    km = torch.ones(B, n, dtype=torch.bool)
    km[0, :333] = False
    km[1, 777:] = False
    res = run_pass(q, k, v, key_mask=km, causal=causal)
    check(res, torch.bfloat16, f"padding masks ragged n={n} causal={causal}")


@param("causal", (False, True))
def test_pass_key_masked_forward_with_and_without_workspace(causal):
    """pa_attn_pass_fwd on a key-masked bf16 pass: with its optional workspace the key mask
    becomes a per-key term and the direct-to-LDS kernel runs; without it the register-staged
    kernel reads the mask.  The same outputs up to the two kernels' different rounding points
    (P enters its MFMA in bf16 in both, summed in a different order: 1e-2 here, below the
    oracle bound both meet) and lse (the direct-to-LDS kernel sums the rounded P, as its PV
    product uses them: 2e-3), fully-masked rows included."""
    import ctypes

    from poly_attention import _lib, _ops

    d = dev()
    lib = _lib.load()
    n = 256
    q, k, v = (randn((2, 4, n, 64), torch.bfloat16, s).to(d) for s in (51, 52, 53))
    bias = (randn((2, 4, n), torch.float32, 54) + 3.0).to(d)
    km = torch.ones(2, n, dtype=torch.bool)
    km[0, :3] = False
    km[1, n // 3:] = False
    km8 = km.to(d).to(torch.uint8)
    results = []
    for use_ws in (False, True):
        out = torch.empty_like(q)
        lse = torch.empty(2, 4, n, dtype=torch.float32, device=d)
        p = _ops._pass_struct(q, k, v, None, bias, km8, None, out, lse, causal, 0.0, 64 ** -0.5,
                              True)
        ws = None
        if use_ws:
            nbytes = lib.pa_attn_pass_fwd_workspace(ctypes.byref(p))
            assert nbytes > 0
            ws = torch.empty(nbytes, dtype=torch.uint8, device=d)
            p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
        _lib.check(lib.pa_attn_pass_fwd(ctypes.byref(p), torch.cuda.current_stream().cuda_stream),
                   "pa_attn_pass_fwd")
        torch.cuda.synchronize()
        results.append((out, lse))
    (o0, l0), (o1, l1) = results
    assert_parity(o1, o0.float(), torch.bfloat16, f"key-masked fwd, workspace vs none causal={causal}",
                  tol=1e-2)
    assert_parity(l1, l0, torch.float32, f"key-masked lse, workspace vs none causal={causal}",
                  tol=2e-3)


@param("dtype", (torch.bfloat16, torch.float16))
@param("nq,nk", ((64, 64), (17, 50), (64, 1), (33, 64)))
@param("softclamp", (None, 5.0))
def test_pass_short_sequences(dtype, nq, nk, softclamp):
    """Short non-causal passes at head dim 64 (nq, nk <= 64: the PolyViT shape, one unit per
    wave): a key bias with a -finfo.max entry, a query-masked row, GQA, forward and all
    gradients."""
    q = randn((2, 8, nq, 64), dtype, 71)
    k, v = (randn((2, 2, nk, 64), dtype, s) for s in (72, 73))
    bias = randn((2, 2, nk), torch.float32, 74) + 1.0
    bias[1, 0, 0] = -torch.finfo(torch.float32).max
    qm = torch.ones(2, nq, dtype=torch.bool)
    qm[0, nq // 2] = False
    check(run_pass(q, k, v, bias=bias, query_mask=qm, causal=False, softclamp=softclamp), dtype,
          f"short {dtype} nq={nq} nk={nk} sc={softclamp}")
    check(run_pass(q, k, v, causal=False, softclamp=softclamp), dtype,
          f"short {dtype} nq={nq} nk={nk} sc={softclamp} no bias")


@param("dtype", (torch.float32, torch.bfloat16))
def test_pass_cross_lengths(dtype):
    """Different query and key lengths (contexts), causal with a top-left aligned mask."""
    q = randn((2, 4, 20, 64), dtype, 16)
    k, v = (randn((2, 4, 33, 64), dtype, s) for s in (17, 18))
    check(run_pass(q, k, v, causal=True), dtype, f"cross lengths {dtype} causal")
    check(run_pass(q, k, v, causal=False), dtype, f"cross lengths {dtype}")


@param("heads,n,d", ((8, 1024, 64), (3, 1000, 64), (8, 512, 128)))
def test_pass_multi_block_causal_grids(heads, n, d):
    """Causal passes with many query / key blocks per head: the workgroup order that runs the
    heaviest blocks of all heads of an XCD first (8 heads: whole heads per XCD; 3 heads: the
    unit-by-unit fallback), forward and all gradients, with a key bias as in pass 2."""
    dtype = torch.bfloat16
    q, k, v = (randn((1, heads, n, d), dtype, s) for s in (21, 22, 23))
    bias = torch.log(torch.arange(1, n + 1).float())[None, None].repeat(1, heads, 1)
    bias = bias + randn((1, heads, n), torch.float32, 24)
    check(run_pass(q, k, v, causal=True), dtype, f"grid h={heads} n={n} d={d}")
    check(run_pass(q, k, v, bias=bias, causal=True), dtype, f"grid h={heads} n={n} d={d} bias")


@param("B,H", ((4, 8), (4, 16)))
@param("causal", (False, True))
def test_f32_forward_multiwave_workgroups(B, H, causal):
    """fp32 forwards whose grids take two (4 x 8 heads) and four (4 x 16) 32-query waves per
    workgroup sharing each key tile; smaller grids split the keys over the waves instead, and
    the other tests cover those."""
    q = randn((B, H, 1024, 64), torch.float32, 81)
    k = randn((B, H, 1024, 64), torch.float32, 82)
    v = randn((B, H, 1024, 64), torch.float32, 83)
    check(run_pass(q, k, v, causal=causal, grads=False), torch.float32,
          f"fp32 multi-wave B={B} H={H} causal={causal}")


def _run_profiled(q, k, v, **kw):
    from poly_attention import _lib

    with _lib.KernelProfile() as prof:
        res = run_pass(q, k, v, **kw)
    return res, prof.times


SPLIT_KERNELS = ("mfma_fwd_f32_split", "mfma_bwd_f32_dq_split", "mfma_bwd_f32_dkv_split")


@param("d", (64, 128))
@param("causal", (False, True))
def test_f32_split_kernels_head_dims(d, causal):
    """fp32 grids of fewer than 512 blocks of 32 rows take the split kernels: the forward's and
    dQ's key tiles, or dK/dV's query tiles, over four waves whose partial results are merged in
    wave order.  Head dims 64 and 128 at n = 160 (five tiles per block), against the oracle at
    1e-4; the kernel profile shows the three split kernels ran."""
    q, k, v = (randn((1, 3, 160, d), torch.float32, s) for s in (91, 92, 93))
    res, times = _run_profiled(q, k, v, causal=causal)
    check(res, torch.float32, f"fp32 split d={d} causal={causal}")
    for name in SPLIT_KERNELS:
        assert name in times, f"{name} did not run (kernels: {sorted(times)})"


@param("causal", (False, True))
def test_f32_split_kernels_gqa_bias_vmul(causal):
    """The split backward of a middle level: 8 query heads over 2 KV heads (dK/dV sums the four
    heads of a group over its waves), key bias, value multiplier, n = 128."""
    q = randn((1, 8, 128, 64), torch.float32, 94)
    k, v, vmul = (randn((1, 2, 128, 64), torch.float32, s) for s in (95, 96, 97))
    bias = randn((1, 2, 128), torch.float32, 98, scale=2.0)
    res, times = _run_profiled(q, k, v, vmul=vmul, bias=bias, causal=causal)
    check(res, torch.float32, f"fp32 split gqa+bias+vmul causal={causal}")
    for name in SPLIT_KERNELS:
        assert name in times, f"{name} did not run (kernels: {sorted(times)})"


def test_f32_split_kernels_causal_cross_lengths():
    """Causal with 96 queries over 200 keys (top-left aligned: later keys fully masked for every
    query) on the split kernels, d = 128, 4 query heads over 2 KV heads (so that dK/dV has the
    four query tiles per key block its split needs)."""
    q = randn((1, 4, 96, 128), torch.float32, 99)
    k, v = (randn((1, 2, 200, 128), torch.float32, s) for s in (100, 101))
    res, times = _run_profiled(q, k, v, causal=True)
    check(res, torch.float32, "fp32 split causal 96x200")
    for name in SPLIT_KERNELS:
        assert name in times, f"{name} did not run (kernels: {sorted(times)})"
