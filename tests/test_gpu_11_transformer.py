"""GPU: PolyTransformer (the stack of poly-attention blocks mixed by attention residuals) on the
HIP attention core against the CPU oracle's functional restatement of the same state dict.

Tolerances: fp32 max-abs <= 1e-4 for outputs and gradients (tests/parity.py); bf16 outputs
against the drift of the reference's own arithmetic in bf16 (the bf16 test's docstring).
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


def _model(cfg, seed):
    from poly_attention import PolyTransformer

    torch.manual_seed(seed)
    m = PolyTransformer(**cfg)
    with torch.no_grad():  # non-trivial layer mixes (the seeded queries are ~0.02)
        for n, t in m.named_parameters():
            if n.endswith("pseudo_queries"):
                t.copy_(torch.randn_like(t) * 0.5)
    return m


@param("deep_cross_attention", (False, True))
@param("causal", (False, True))
@param("dim_head", (64, 16))
def test_polytransformer_fp32_forward_backward(deep_cross_attention, causal, dim_head):
    """Output, block outputs, input gradient and every parameter gradient with a query mask
    (the reference test's mask: the second half of every sequence dropped)."""
    d = dev()
    cfg = dict(dim=64, depth=3, heads=4, dim_head=dim_head, causal=causal,
               deep_cross_attention=deep_cross_attention, norm_out=True)
    m = _model(cfg, 11)
    x = torch.randn(2, 40, 64)
    g = torch.randn(2, 40, 64)
    mask = torch.ones(2, 40, dtype=torch.bool)
    mask[:, 20:] = False
    params = {k: v.detach().clone().requires_grad_() for k, v in m.state_dict().items()}
    xr = x.clone().requires_grad_()
    ref, ref_h = O.polytransformer_forward(params, cfg, xr, mask=mask)
    ref.backward(g)
    m = m.to(d)
    xg = x.to(d).requires_grad_()
    out, hs = m(xg, mask=mask.to(d), return_layer_hiddens=True)
    out.backward(g.to(d))
    what = f"PolyTransformer fp32 deep={deep_cross_attention} causal={causal} d={dim_head}"
    assert_parity(out, ref, torch.float32, f"{what} out")
    for i, (a, b) in enumerate(zip(hs, ref_h)):
        assert_parity(a, b, torch.float32, f"{what} block {i}")
    assert_parity(xg.grad, xr.grad, torch.float32, f"{what} dx")
    for name, p in m.named_parameters():
        if p.grad is None:  # the first block's context norms: no contexts yet
            assert params[name].grad is None, name
            continue
        assert_parity(p.grad, params[name].grad, torch.float32, f"{what} d{name}")


@param("deep_cross_attention", (False, True))
def test_polytransformer_bf16_forward(deep_cross_attention):
    """bf16 weights and activations at a longer sequence (causal, head dim 64) against the
    fp32 oracle on the bf16-rounded state dict and input.

    A whole stack in bf16 rounds after every linear layer, norm and residual add (torch's
    ops, outside the attention core), so its distance from the fp32 result exceeds the
    single-kernel bound: the oracle itself evaluated in bf16 (the reference's own arithmetic
    at this precision) lands 3.3e-2 - 3.6e-2 (max-abs) and 3.9e-3 (RMS) from it here, and
    which element drifts most depends on where the roundings fall.  The check holds the GPU
    model's RMS distance to at most 1.25 times the bf16 oracle's and its max-abs distance to
    the attention bound (2e-2 + one rounding) or at most 1.5 times the bf16 oracle's."""
    d = dev()
    cfg = dict(dim=256, depth=2, heads=4, dim_head=64, causal=True,
               deep_cross_attention=deep_cross_attention, norm_out=True)
    m = _model(cfg, 12).to(d, torch.bfloat16).eval()
    x = torch.randn(2, 300, 256, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    with torch.no_grad():
        out = m(x.to(d)).float().cpu()
    params16 = {k: v.cpu() for k, v in m.state_dict().items()}
    params = {k: v.float() for k, v in params16.items()}
    with torch.no_grad():
        ref, _ = O.polytransformer_forward(params, cfg, x.float())
        ref16, _ = O.polytransformer_forward(params16, cfg, x)
    drift = (ref16.float() - ref).abs()
    err = (out - ref).abs()
    rms, drift_rms = err.pow(2).mean().sqrt().item(), drift.pow(2).mean().sqrt().item()
    bound = 2e-2 + 2.0 ** -8 * ref.abs()
    what = f"PolyTransformer bf16 deep={deep_cross_attention}"
    print(f"[parity] {what}: raw max-abs {err.max().item():.3e}, RMS {rms:.3e} (max|ref| "
          f"{ref.abs().max().item():.3e}; the bf16 oracle's max-abs {drift.max().item():.3e}, "
          f"RMS {drift_rms:.3e})", flush=True)
    assert rms <= 1.25 * drift_rms, what
    assert bool((err <= bound).all()) or err.max().item() <= 1.5 * drift.max().item(), what
