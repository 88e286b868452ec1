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
* A gradient computed from bf16 / f16 inputs is held to the same element-wise bound
  tol + u |ref|.  Where it is exceeded, the check needs ``ref_lp``: the oracle's result for
  the same inputs evaluated in the low-precision type itself (the reference's own arithmetic
  at that precision).  Such a gradient is a sum of many terms formed from rounded
  intermediates (P and dS enter the MFMAs in the input type, D = rowsum(dO * O) reads the
  stored, rounded O, a GQA key gradient sums the query heads of its group), so its error
  scales with its terms rather than with each element; it then passes only if its error is
  within the reference's own low-precision drift: RMS(got - ref) <= 1.25 RMS(ref_lp - ref)
  and max|got - ref| <= 1.5 max|ref_lp - ref|.  For fp32 inputs u = 0 and the bound is the
  raw 1e-4.

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


def _bound_text(tol: float, u: float) -> str:
    return f"{tol:g} + {u:g}|ref|" if u else f"{tol:g}"


def record(what: str, raw: float, ref_max: float, tol: float, u: float, excess: float,
           n: int, grad: bool = False, drift: dict | None = None) -> None:
    line = {"check": what, "raw_max_abs": raw, "ref_max_abs": ref_max, "tol": tol,
            "rounding": u, "gradient": grad, "worst_excess": excess, "elements": n}
    text = (f"[parity] {what}: raw max-abs {raw:.3e} (max|ref| {ref_max:.3e}, bound "
            f"{_bound_text(tol, u)})")
    if drift is not None:
        line.update(drift)
        text += (f"; RMS {drift['rms']:.3e}, the low-precision oracle's drift: RMS "
                 f"{drift['drift_rms']:.3e}, max {drift['drift_max']:.3e}"
                 + (" (element bound exceeded: held to the drift)" if excess > 0 else ""))
    print(text, flush=True)
    path = os.environ.get("PA_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(line) + "\n")


def assert_parity(got, ref, dtype, what: str, tol: float | None = None,
                  grad: bool = False, ref_lp=None, roundings: int = 1) -> float:
    """Assert the north star's bound for a result computed in ``dtype`` (see the module
    docstring; ``grad``: a gradient, ``dtype`` then its inputs' dtype; ``ref_lp``: for a
    low-precision gradient, the oracle's result in that precision); ``tol`` overrides the
    dtype's bound.  ``roundings``: storage roundings the element bound allows (2 where ``ref``
    is itself a result stored in ``dtype``, e.g. a second GPU path: two values rounded
    independently from one real value may sit one grid step, two roundings, apart).  Returns
    the raw max-abs error."""
    got = got.detach().double().cpu()
    ref = torch.as_tensor(ref).detach().double().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    tol = TOL[dtype] if tol is None else tol
    u = ROUND[dtype] * roundings
    lp = None if ref_lp is None else torch.as_tensor(ref_lp).detach().double().cpu()
    nan = torch.isnan(ref)
    if bool(nan.any()):  # NaN where the reference is NaN (rows of -inf scores), else values
        assert bool(torch.isnan(got[nan]).all()), f"{what}: a value where the reference is NaN"
        got, ref = got[~nan], ref[~nan]
        lp = None if lp is None else lp[~nan]
    if got.numel() == 0:
        return 0.0
    assert bool(torch.isfinite(got).all()), f"{what}: non-finite values"
    diff = (got - ref).abs()
    raw = diff.max().item()
    ref_max = ref.abs().max().item()
    excess = (diff - (tol + u * ref.abs())).max().item()
    if excess <= 0.0:
        record(what, raw, ref_max, tol, u, excess, got.numel(), grad)
        return raw
    assert grad and u > 0 and lp is not None, (
        f"{what}: raw max-abs err {raw:.3e} exceeds {_bound_text(tol, u)} (max|ref| {ref_max:.3e})")
    dr = (lp - ref).abs()
    drift = {"rms": diff.pow(2).mean().sqrt().item(), "drift_rms": dr.pow(2).mean().sqrt().item(),
             "drift_max": dr.max().item()}
    record(what, raw, ref_max, tol, u, excess, got.numel(), grad, drift)
    assert drift["rms"] <= 1.25 * drift["drift_rms"] and raw <= 1.5 * drift["drift_max"], (
        f"{what}: raw max-abs err {raw:.3e} (RMS {drift['rms']:.3e}) exceeds "
        f"{_bound_text(tol, u)} and the low-precision oracle's drift (max {drift['drift_max']:.3e},"
        f" RMS {drift['drift_rms']:.3e}; max|ref| {ref_max:.3e})")
    return raw


def assert_drift(got, ref, ref_lp, what: str, tol: float = 2e-2, u: float = 2.0 ** -8,
                 rms_factor: float = 1.25, max_factor: float = 1.5) -> float:
    """A low-precision result of a whole stack (many roundings outside the attention core, as
    the reference's own low-precision arithmetic has) against the fp32 oracle: within the
    element bound tol + u|ref| everywhere, or else within the drift of ``ref_lp`` (the oracle
    evaluated in the low-precision type on the same inputs): RMS distance <= rms_factor x
    that drift's RMS and max-abs distance <= max_factor x its max.  Returns the raw max-abs
    error."""
    got = got.detach().double().cpu()
    ref = torch.as_tensor(ref).detach().double().cpu()
    lp = torch.as_tensor(ref_lp).detach().double().cpu()
    assert got.shape == ref.shape == lp.shape, what
    assert bool(torch.isfinite(got).all()), f"{what}: non-finite values"
    diff, dr = (got - ref).abs(), (lp - ref).abs()
    raw = diff.max().item()
    excess = (diff - (tol + u * ref.abs())).max().item()
    drift = {"rms": diff.pow(2).mean().sqrt().item(), "drift_rms": dr.pow(2).mean().sqrt().item(),
             "drift_max": dr.max().item()}
    record(what, raw, ref.abs().max().item(), tol, u, excess, got.numel(), True, drift)
    if excess <= 0.0:
        return raw
    assert drift["rms"] <= rms_factor * drift["drift_rms"], (
        f"{what}: max-abs {raw:.3e} exceeds {_bound_text(tol, u)} and its RMS {drift['rms']:.3e} "
        f"> {rms_factor} x the low-precision oracle's {drift['drift_rms']:.3e}")
    assert raw <= max_factor * drift["drift_max"], (
        f"{what}: max-abs {raw:.3e} exceeds {_bound_text(tol, u)} and {max_factor} x the "
        f"low-precision oracle's {drift['drift_max']:.3e}")
    return raw
