"""Write the golden fixtures under tests/golden/ (float64 inputs and expected outputs).

Every expected value comes from a closed form that does not share code with the oracle's
two-pass formulation:
  * order 2: one softmax over (j, k) pairs of S12[i,j] + S23[j,k] (the paper's definition of
    the order-2 poly score), gradients by autograd through that closed form;
  * order 3: one softmax over (j, k, l) paths, values v3[k] * v4[l];
  * one pass of the chain (lse / msg of pass 1): textbook softmax / logsumexp;
  * a masked pass: the finite-fill class semantics (entry class = [own score masked] +
    [bias == -finfo.max]; rows without a class-0 entry average their class-1 entries).
Before writing, each fixture is cross-checked against the oracle (oracle/poly_oracle.py) in
float64 and the script aborts on any disagreement above 1e-10.  The reference itself cannot
be imported here (einx, rotary_embedding_torch, torch_einops_utils are not installed), so no
reference-produced vectors exist; the reference ships none either.

Inputs are rounded to float32 before use, so an fp32 run of the HIP path sees exactly the
fixture's inputs.  Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle.poly_oracle as O  # noqa: E402

FLT_MAX = float(np.finfo(np.float32).max)


def _inputs(gen, *shapes, scale=1.0):
    return [(torch.randn(*s, generator=gen, dtype=torch.float64) * scale).float().double()
            for s in shapes]


def _causal(n, dims):
    """bool mask over paths (i, j, k, ...) with each index <= the previous one."""
    idx = torch.meshgrid(*(torch.arange(n),) * dims, indexing="ij")
    ok = torch.ones((n,) * dims, dtype=torch.bool)
    for a in range(dims - 1):
        ok &= idx[a + 1] <= idx[a]
    return ok


def pair_softmax_order2(q1, q2, q3, v3, causal, softclamp):
    s = q1.shape[-1] ** -0.5
    sc = (lambda x: softclamp * torch.tanh(x / softclamp)) if softclamp else (lambda x: x)
    s12 = sc(torch.einsum("bhid,bhjd->bhij", q1, q2) * s)
    s23 = sc(torch.einsum("bhjd,bhkd->bhjk", q2, q3) * s)
    tot = s12[..., :, :, None] + s23[..., None, :, :]
    if causal:
        tot = tot.masked_fill(~_causal(q1.shape[-2], 3), float("-inf"))
    w = torch.softmax(tot.flatten(-2), dim=-1).view_as(tot)
    return torch.einsum("bhijk,bhkd->bhid", w, v3)


def path_softmax_order3(q1, q2, q3, q4, v3, v4, causal):
    s = q1.shape[-1] ** -0.5
    s12 = torch.einsum("bhid,bhjd->bhij", q1, q2) * s
    s23 = torch.einsum("bhjd,bhkd->bhjk", q2, q3) * s
    s34 = torch.einsum("bhkd,bhld->bhkl", q3, q4) * s
    tot = s12[..., :, :, None, None] + s23[..., None, :, :, None] + s34[..., None, None, :, :]
    if causal:
        tot = tot.masked_fill(~_causal(q1.shape[-2], 4), float("-inf"))
    w = torch.softmax(tot.flatten(-3), dim=-1).view_as(tot)
    return torch.einsum("bhijkl,bhkd,bhld->bhid", w, v3, v4)


def _grads(fn, inputs, dout):
    leaves = [t.clone().requires_grad_(True) for t in inputs]
    out = fn(*leaves)
    grads = torch.autograd.grad(out, leaves, dout)
    return out.detach(), [g.detach() for g in grads]


def _close(a, b, what):
    a = torch.as_tensor(a, dtype=torch.float64)
    b = torch.as_tensor(b, dtype=torch.float64)
    err = (a - b).abs().max().item()
    if not err <= 1e-10:
        raise SystemExit(f"{what}: brute force and oracle disagree by {err}")


def _close_tol(a, b, tol, what):
    a = torch.as_tensor(a, dtype=torch.float64)
    b = torch.as_tensor(b, dtype=torch.float64)
    err = (a - b).abs().max().item()
    if not err <= tol:
        raise SystemExit(f"{what}: class form and float32 oracle disagree by {err}")


def _save(name, **arrays):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **{k: np.asarray(v.numpy() if torch.is_tensor(v) else v)
                                 for k, v in arrays.items()})
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


def order2_fixture(name, seed, B, H, N, d, causal, softclamp):
    gen = torch.Generator().manual_seed(seed)
    q1, q2, q3, v3, dout = _inputs(gen, *([(B, H, N, d)] * 5))
    fn = lambda a, b, c, v: pair_softmax_order2(a, b, c, v, causal, softclamp)  # noqa: E731
    out, (dq1, dq2, dq3, dv3) = _grads(fn, (q1, q2, q3, v3), dout)
    # cross-checks: the oracle (two passes, autograd) and the numpy brute force
    leaves = [t.clone().requires_grad_(True) for t in (q1, q2, q3, v3)]
    o_out, _, _ = O.reference_poly_attention(leaves[0], leaves[1], leaves[1], leaves[2],
                                             leaves[3], softclamp_value=softclamp,
                                             causal=causal)
    o_grads = torch.autograd.grad(o_out, leaves, dout)
    _close(out, o_out.detach(), f"{name} out")
    for g, og, nm in zip((dq1, dq2, dq3, dv3), o_grads, ("dq1", "dq2", "dq3", "dv3")):
        _close(g, og, f"{name} {nm}")
    _close(out, O.brute_order2(q1, q2, q3, v3, causal=causal, softclamp_value=softclamp),
           f"{name} numpy brute force")
    _save(name, q1=q1, q2=q2, q3=q3, v3=v3, dout=dout, out=out, dq1=dq1, dq2=dq2, dq3=dq3,
          dv3=dv3, causal=np.array(causal), softclamp=np.array(softclamp or 0.0))


def order3_fixture(name, seed, B, H, N, d, causal):
    gen = torch.Generator().manual_seed(seed)
    q1, q2, q3, q4, v3, v4, dout = _inputs(gen, *([(B, H, N, d)] * 7))
    fn = lambda a, b, c, e, v, w: path_softmax_order3(a, b, c, e, v, w, causal)  # noqa: E731
    out, grads = _grads(fn, (q1, q2, q3, q4, v3, v4), dout)
    leaves = [t.clone().requires_grad_(True) for t in (q1, q2, q3, q4, v3, v4)]
    o_out, _, _ = O.n_poly_core(leaves[:3], leaves[1:4], [leaves[4], leaves[5]], causal=causal)
    o_grads = torch.autograd.grad(o_out, leaves, dout)
    _close(out, o_out.detach(), f"{name} out")
    for g, og, nm in zip(grads, o_grads, ("dq1", "dq2", "dq3", "dq4", "dv3", "dv4")):
        _close(g, og, f"{name} {nm}")
    _close(out, O.brute_order3(q1, q2, q3, q4, v3, v4, causal=causal), f"{name} path sum")
    _save(name, q1=q1, q2=q2, q3=q3, q4=q4, v3=v3, v4=v4, dout=dout, out=out,
          dq1=grads[0], dq2=grads[1], dq3=grads[2], dq4=grads[3], dv3=grads[4], dv4=grads[5],
          causal=np.array(causal))


def gqa_decode_fixture(name, seed, B, H, Hkv, n, d):
    """Order-2 GQA over n positions: the causal output of every query, plus pass 1's
    lse23 / msg per position (at Hkv heads) -- the cache a decode step reads.  Its last row
    is what one decode step with n-1 cached positions must return."""
    gen = torch.Generator().manual_seed(seed)
    q1, = _inputs(gen, (B, H, n, d))
    q2, q3, v3 = _inputs(gen, *([(B, Hkv, n, d)] * 3))
    r = H // Hkv
    ex = lambda t: t.repeat_interleave(r, dim=1)  # noqa: E731  (einops 'b g n d -> b (g r) n d')
    out = pair_softmax_order2(q1, ex(q2), ex(q3), ex(v3), True, None)
    s = d ** -0.5
    s23 = torch.einsum("bhjd,bhkd->bhjk", q2, q3) * s
    s23 = s23.masked_fill(~_causal(n, 2), float("-inf"))
    lse23 = torch.logsumexp(s23, dim=-1)
    msg = torch.einsum("bhjk,bhkd->bhjd", torch.softmax(s23, dim=-1), v3)
    o_out, o_lse, o_msg = O.reference_poly_attention(q1, ex(q2), ex(q2), ex(q3), ex(v3),
                                                     causal=True)
    _close(out, o_out, f"{name} out")
    _close(ex(lse23), o_lse, f"{name} lse23")
    _close(ex(msg), o_msg, f"{name} msg")
    _save(name, q1=q1, q2=q2, q3=q3, v3=v3, out=out, lse23=lse23, msg=msg)


def masked_pass_fixture(name, seed, B, H, nq, nk, d):
    """One pass with a key mask, a query mask (one fully masked query row per batch) and a
    key bias holding -finfo.max entries; expected (out, lse) by the class semantics."""
    gen = torch.Generator().manual_seed(seed)
    q, = _inputs(gen, (B, H, nq, d))
    k, v = _inputs(gen, *([(B, H, nk, d)] * 2))
    bias, = _inputs(gen, (B, H, nk))
    bias[:, :, 1::5] = -FLT_MAX
    key_mask = torch.rand(B, nk, generator=gen) > 0.3
    key_mask[:, 0] = True
    query_mask = torch.ones(B, nq, dtype=torch.bool)
    query_mask[:, 2] = False
    out, lse = O.masked_pass_classes(q, k, v, bias=bias, key_mask=key_mask,
                                     query_mask=query_mask)
    # the finite fill is a float32 effect (-finfo.max + -finfo.max overflows to -inf only in
    # float32), so the oracle is run in float32 here, as the reference would run
    o_out, o_lse = O.attn_pass(q.float(), k.float(), v.float(), bias=bias.float(),
                               key_mask=key_mask, query_mask=query_mask)
    _close_tol(out, o_out, 1e-5, f"{name} out")
    _close_tol(lse, o_lse, 1e-5 * FLT_MAX, f"{name} lse (fully-masked rows)")
    ok = lse > -1e30
    _close_tol(lse[ok], o_lse.numpy()[ok], 1e-5, f"{name} lse")
    _save(name, q=q, k=k, v=v, bias=bias, key_mask=key_mask.numpy(),
          query_mask=query_mask.numpy(), out=out, lse=lse)


def main():
    torch.set_default_dtype(torch.float64)
    order2_fixture("order2_causal_softclamp.npz", 11, B=2, H=2, N=13, d=16, causal=True,
                   softclamp=2.0)
    order2_fixture("order2_noncausal.npz", 12, B=1, H=3, N=10, d=32, causal=False,
                   softclamp=None)
    order3_fixture("order3_causal.npz", 13, B=1, H=2, N=7, d=16, causal=True)
    gqa_decode_fixture("order2_gqa_decode.npz", 14, B=2, H=4, Hkv=2, n=12, d=64)
    masked_pass_fixture("masked_pass.npz", 15, B=2, H=2, nq=9, nk=11, d=16)


if __name__ == "__main__":
    main()
