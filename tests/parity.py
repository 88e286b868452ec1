"""The parity bound of the GPU suites, shared by every test that compares the HIP path with
the CPU oracle.

The north star's bound is a max-abs error: 1e-4 for fp32 results, 2e-2 for bf16 / f16
results, against the fp32 oracle evaluated on the same low-precision-rounded inputs.

* fp32 results are held to the raw bound: max |got - ref| <= tol.
* A result stored in bf16 / f16 cannot be closer to the fp32 value than the rounding of its
  own storage type, which grows with the value: a bf16 number of magnitude M has a grid
  spacing of up to 2^-7 M, so above |M| ~ 5 one rounding alone exceeds 2e-2.  Such results
  are held element by element to |got - ref| <= tol + u |ref| with u = 2^-8 (bf16) or 2^-11
  (f16): the absolute bound plus one rounding of the stored value.  Outputs of attention
  (|ref| of order 1) are therefore held to ~2e-2; only large gradients use the second term.
* A gradient computed from bf16 / f16 inputs is a sum of many terms formed from rounded
  intermediates (P and dS enter the MFMAs in the input dtype, D = rowsum(dO * O) reads the
  stored, rounded O, a GQA key gradient sums the query heads of its group), so its rounding
  error scales with the size of its terms rather than with each element's value: gradients
  are held to |got - ref| <= tol + u (|ref| + max|ref|), u the rounding of the input dtype
  (also for gradients stored in fp32, such as a key bias's).  For fp32 inputs u = 0 and the
  bound is the raw 1e-4.

Every check prints the raw max-abs error, the largest |ref| and the bound's margin, and,
when the environment variable PA_PARITY_LOG names a file, appends them there as one JSON
line, so the raw figures of a run can be collected.
"""

from __future__ import annotations

import json
import os

import torch

TOL = {torch.float32: 1e-4, torch.float64: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}
ROUND = {torch.float32: 0.0, torch.float64: 0.0, torch.bfloat16: 2.0 ** -8,
         torch.float16: 2.0 ** -11}


def _bound_text(tol: float, u: float, grad: bool) -> str:
    if not u:
        return f"{tol:g}"
    return f"{tol:g} + {u:g}(|ref| + max|ref|)" if grad else f"{tol:g} + {u:g}|ref|"


def record(what: str, raw: float, ref_max: float, tol: float, u: float, excess: float,
           n: int, grad: bool = False) -> None:
    line = {"check": what, "raw_max_abs": raw, "ref_max_abs": ref_max, "tol": tol,
            "rounding": u, "gradient": grad, "worst_excess": excess, "elements": n}
    print(f"[parity] {what}: raw max-abs {raw:.3e} (max|ref| {ref_max:.3e}, bound "
          f"{_bound_text(tol, u, grad)})", flush=True)
    path = os.environ.get("PA_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(line) + "\n")


def assert_parity(got, ref, dtype, what: str, tol: float | None = None,
                  grad: bool = False) -> float:
    """Assert the north star's bound for a result computed in ``dtype`` (see the module
    docstring; ``grad``: a gradient, ``dtype`` then its inputs' dtype); ``tol`` overrides the
    dtype's bound.  Returns the raw max-abs error."""
    got = got.detach().double().cpu()
    ref = torch.as_tensor(ref).detach().double().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    tol = TOL[dtype] if tol is None else tol
    u = ROUND[dtype]
    nan = torch.isnan(ref)
    if bool(nan.any()):  # NaN where the reference is NaN (rows of -inf scores), else values
        assert bool(torch.isnan(got[nan]).all()), f"{what}: a value where the reference is NaN"
        got, ref = got[~nan], ref[~nan]
    if got.numel() == 0:
        return 0.0
    assert bool(torch.isfinite(got).all()), f"{what}: non-finite values"
    diff = (got - ref).abs()
    raw = diff.max().item()
    ref_max = ref.abs().max().item()
    bound = tol + u * ref.abs() + (u * ref_max if grad else 0.0)
    excess = (diff - bound).max().item()
    record(what, raw, ref_max, tol, u, excess, got.numel(), grad)
    assert excess <= 0.0, (f"{what}: raw max-abs err {raw:.3e} exceeds "
                           f"{_bound_text(tol, u, grad)} (max|ref| {ref_max:.3e})")
    return raw
