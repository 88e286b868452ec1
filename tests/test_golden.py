"""The oracle against the committed golden fixtures (tests/golden/*.npz, float64).

The fixtures' expected values come from closed forms (pair / path softmax, textbook
logsumexp, the finite-fill class semantics) written by tests/golden/make_golden.py; this
file re-runs the oracle on the fixture inputs so that a later change to the oracle that
breaks it fails here even if the brute-force pins in test_oracle.py were changed with it.
"""

import os

import numpy as np
import pytest
import torch

import oracle.poly_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name)) as z:  # allow_pickle stays False
        return {k: torch.from_numpy(z[k].copy()) for k in z.files}


def close(a, b, tol, what):
    a = torch.as_tensor(a, dtype=torch.float64)
    b = torch.as_tensor(b, dtype=torch.float64)
    err = (a - b).abs().max().item()
    assert err <= tol, f"{what}: max-abs err {err:.3e}"


@pytest.mark.parametrize("name", ["order2_causal_softclamp.npz", "order2_noncausal.npz"])
def test_oracle_order2_matches_golden(name):
    g = load(name)
    causal = bool(g["causal"])
    sc = float(g["softclamp"]) or None
    leaves = [g[k].clone().requires_grad_(True) for k in ("q1", "q2", "q3", "v3")]
    out, _, _ = O.reference_poly_attention(leaves[0], leaves[1], leaves[1], leaves[2], leaves[3],
                                           softclamp_value=sc, causal=causal)
    close(out.detach(), g["out"], 1e-10, "out")
    grads = torch.autograd.grad(out, leaves, g["dout"])
    for gr, k in zip(grads, ("dq1", "dq2", "dq3", "dv3")):
        close(gr, g[k], 1e-10, k)


def test_oracle_order3_matches_golden():
    g = load("order3_causal.npz")
    names = ("q1", "q2", "q3", "q4", "v3", "v4")
    leaves = [g[k].clone().requires_grad_(True) for k in names]
    out, _, _ = O.n_poly_core(leaves[:3], leaves[1:4], leaves[4:], causal=bool(g["causal"]))
    close(out.detach(), g["out"], 1e-10, "out")
    grads = torch.autograd.grad(out, leaves, g["dout"])
    for gr, k in zip(grads, ("dq1", "dq2", "dq3", "dq4", "dv3", "dv4")):
        close(gr, g[k], 1e-10, k)


def test_oracle_gqa_and_cached_step_match_golden():
    g = load("order2_gqa_decode.npz")
    H, Hkv = g["q1"].shape[1], g["q2"].shape[1]
    ex = lambda t: O.repeat_kv(t, H // Hkv)  # noqa: E731
    out, lse, msg = O.reference_poly_attention(g["q1"], ex(g["q2"]), ex(g["q2"]), ex(g["q3"]),
                                               ex(g["v3"]), causal=True)
    close(out, g["out"], 1e-10, "out")
    close(lse, ex(g["lse23"][..., None])[..., 0], 1e-10, "lse23")
    close(msg, ex(g["msg"]), 1e-10, "msg")
    # the cached single-token step (poly_attention.py:84-87 with a cache of n-1 positions)
    q2 = ex(g["q2"])
    cache = (q2[:, :, :-1], ex(g["q3"])[:, :, :-1], ex(g["v3"])[:, :, :-1],
             ex(g["lse23"][..., None])[..., 0][:, :, :-1], ex(g["msg"])[:, :, :-1])
    step, _, _ = O.reference_poly_attention(g["q1"][:, :, -1:], q2[:, :, -1:], q2,
                                            ex(g["q3"]), ex(g["v3"]), causal=True, cache=cache)
    close(step, g["out"][:, :, -1:], 1e-10, "cached step")


def test_oracle_masked_pass_matches_golden():
    g = load("masked_pass.npz")
    out, lse = O.attn_pass(g["q"].float(), g["k"].float(), g["v"].float(), bias=g["bias"].float(),
                           key_mask=g["key_mask"], query_mask=g["query_mask"])
    close(out, g["out"], 1e-5, "out")
    ok = g["lse"] > -1e30
    close(lse[ok], g["lse"][ok], 1e-5, "lse")
    assert (lse[~ok] == -torch.finfo(torch.float32).max).all()
    # the fixture holds a fully masked query row and -finfo.max bias entries
    assert (~g["query_mask"]).any() and (g["bias"] <= -1e30).any()
