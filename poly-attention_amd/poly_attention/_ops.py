"""Host side of the HIP poly-attention path: tensors -> ABI structs -> libpolyattn.

* ``polyattn::pass_fwd`` / ``polyattn::pass_bwd`` -- one attention pass (one level of the
  poly chain) as torch custom ops with fake (meta) kernels and autograd, so torch.compile
  and autocast see an opaque, differentiable op.  They are registered for CUDA (HIP)
  devices only: there is no CPU implementation, the product path fails loudly without the
  library.
* ``poly_chain`` -- the order-n forward of poly_attention.py:48-116 / n_poly_attention.py:
  233-313 as a right-to-left sequence of passes (each level's lse is the next level's key
  bias, each level's output its value, multiplied by that level's v in the middle levels).
* ``poly_decode_step`` -- the cached single-token step through ``pa_poly_decode``.
* ``decode_prologue`` -- the q norms, rotary and cache appends before a fixed-capacity
  (StaticCache) step, through ``pa_decode_prologue``.
* ``rms_norm`` -- the per-head q/k RMSNorm (``polyattn::rms_norm`` custom op with autograd)
  through ``pa_rmsnorm_fwd`` / ``pa_rmsnorm_bwd``.
"""

from __future__ import annotations

import contextlib
import ctypes
from typing import Optional, Sequence

import torch
from torch import Tensor

from . import _lib
from ._lib import (
    DTYPE_CODE,
    PA_EPI_ROOT_SIGMOID,
    PA_FLAG_DISCARD_OUT,
    PA_FLAG_MAY_DEGENERATE,
    PA_NORM_K,
    PA_NORM_Q,
    PaDecode,
    PaEpilogue,
    PaMask,
    PaPass,
    PaPassGrad,
    PaQkNorm,
    PaRmsNorm,
    PaView,
)

# ---------------------------------------------------------------------------------------
# marshalling


def _inner_contig(t: Tensor) -> Tensor:
    return t if t.stride(-1) == 1 or t.shape[-1] == 1 else t.contiguous()


def _view(t: Optional[Tensor]) -> PaView:
    v = PaView()
    if t is None:
        return v
    assert t.dim() in (3, 4), "expected a [batch, heads, n(, dim)] tensor"
    if t.dim() == 4:
        assert t.stride(-1) == 1 or t.shape[-1] == 1, "feature stride must be 1"
    v.ptr = t.data_ptr()
    v.sb, v.sh, v.sn = t.stride(0), t.stride(1), t.stride(2)
    v.heads = t.shape[1]
    v.dtype = DTYPE_CODE[t.dtype]
    return v


def _heads_inner(t: Tensor) -> bool:
    """A [B, H, N, d] view whose head stride is below its position stride: the layout of the
    modules' split projections ([B, N, H*d] seen per head)."""
    return t.dim() == 4 and t.shape[1] > 1 and t.shape[2] > 1 and t.stride(1) < t.stride(2)


def _empty_heads(shape, like: Tensor, dtype=None) -> Tensor:
    """A new [B, H, N, d] tensor in the layout of ``like``: heads-inner ([B, N, H, d] storage,
    so that merging the heads afterwards is a free view) when ``like`` is, else contiguous."""
    dtype = like.dtype if dtype is None else dtype
    B, H, N, d = shape
    if _heads_inner(like):
        return torch.empty(B, N, H, d, dtype=dtype, device=like.device).permute(0, 2, 1, 3)
    return torch.empty(B, H, N, d, dtype=dtype, device=like.device)


def _mask(m: Optional[Tensor]) -> PaMask:
    pm = PaMask()
    if m is None:
        return pm
    assert m.dtype == torch.uint8 and m.dim() == 2
    pm.ptr = m.data_ptr()
    pm.sb, pm.sn = m.stride(0), m.stride(1)
    return pm


def _mask_u8(m: Optional[Tensor]) -> Optional[Tensor]:
    if m is None:
        return None
    return m.to(torch.uint8)


def _device(t: Tensor):
    """The tensor's device as the current one (a no-op context when it already is)."""
    if t.device.index is None or t.device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(t.device)


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _epilogue_struct(epilogue, y) -> PaEpilogue:
    """epilogue = (root or None, gate or None, root_sigmoid); y its output buffer."""
    root, gate, root_sigmoid = epilogue
    e = PaEpilogue()
    e.root, e.gate, e.y = _view(root), _view(gate), _view(y)
    e.flags = PA_EPI_ROOT_SIGMOID if root_sigmoid else 0
    return e


def _qk_norm_struct(qk_norm) -> PaQkNorm:
    """qk_norm = (q norm, k norm), each (weight, eps) or None: RMSNorms applied on load."""
    qn, kn = qk_norm
    n = PaQkNorm()
    if qn is not None:
        n.q_weight, n.q_eps, n.flags = qn[0].data_ptr(), float(qn[1]), n.flags | PA_NORM_Q
    if kn is not None:
        n.k_weight, n.k_eps, n.flags = kn[0].data_ptr(), float(kn[1]), n.flags | PA_NORM_K
    return n


def qk_norms_fusable(q1: Tensor, q2: Tensor, q3: Tensor, v3: Tensor, weights, causal: bool) -> bool:
    """The order-2 chain can normalise its q1 / q2 / q3 as the passes load them (the short-pass
    kernel's q / k norms): 16-bit CUDA tensors of head dim 64 and at most 64 positions, not
    causal, every norm weight a contiguous, 16-byte aligned [64] tensor of that dtype, rows
    aligned for the MFMA kernels."""
    ts = (q1, q2, q3, v3)
    dt = q1.dtype
    if dt not in (torch.bfloat16, torch.float16) or causal:
        return False
    if any(not t.is_cuda or t.dtype != dt or t.dim() != 4 or t.shape[-1] != 64 or
           t.shape[2] > 64 or t.stride(-1) != 1 for t in ts):
        return False
    if any(t.data_ptr() % 16 or any(st % 8 for st in t.stride()[:3]) for t in ts):
        return False
    return all(w is not None and w.dtype == dt and w.is_contiguous() and w.numel() == 64
               and w.data_ptr() % 16 == 0 for w in weights)


def _pass_struct(q, k, v, vmul, bias, key_mask, query_mask, out, lse, causal, softclamp, scale,
                 may_degenerate, epi: Optional[PaEpilogue] = None) -> PaPass:
    p = PaPass()
    p.batch, p.heads, p.nq, p.dim = q.shape[0], out.shape[1], q.shape[2], q.shape[3]
    p.nk = k.shape[2]
    p.scale = float(scale)
    p.softclamp = float(softclamp) if softclamp else 0.0
    p.causal = int(bool(causal))
    p.flags = PA_FLAG_MAY_DEGENERATE if may_degenerate else 0
    p.q, p.k, p.v = _view(q), _view(k), _view(v)
    p.vmul, p.bias = _view(vmul), _view(bias)
    p.key_mask, p.query_mask = _mask(key_mask), _mask(query_mask)
    p.out, p.lse = _view(out), _view(lse)
    p.epi = ctypes.addressof(epi) if epi is not None else None
    return p


def _pass_heads(q, k, v, vmul, bias) -> int:
    return max(t.shape[1] for t in (q, k, v, vmul, bias) if t is not None)


def _check_pass_inputs(q, k, v, vmul, bias, key_mask, query_mask):
    assert q.dim() == k.dim() == v.dim() == 4, "q, k, v must be [batch, heads, n, dim]"
    assert q.dtype == k.dtype == v.dtype, "q, k, v must share one dtype"
    assert q.dtype in DTYPE_CODE, f"unsupported dtype {q.dtype}"
    assert k.shape[2] == v.shape[2], "k and v must have the same length"
    assert q.shape[-1] == k.shape[-1] == v.shape[-1], "q, k, v must share the head dim"
    if vmul is not None:
        assert vmul.dtype == v.dtype and vmul.shape[2] == v.shape[2]
    if bias is not None:
        assert bias.dim() == 3 and bias.shape[2] == k.shape[2]
    if key_mask is not None:
        assert key_mask.shape == (k.shape[0], k.shape[2])
    if query_mask is not None:
        assert query_mask.shape == (q.shape[0], q.shape[2])


# ---------------------------------------------------------------------------------------
# one pass: raw calls


def _padded_dim(q: Tensor) -> Optional[int]:
    """The MFMA head dim (64, 128, or 256 for 16-bit passes) a CUDA pass of another head dim
    up to 256 is run at, its features zero-padded: the padded features add nothing to any
    score, and the padded value features are zero (the scale stays the caller's), so out, lse
    and every gradient are the unpadded pass's.  None when the pass runs as it is."""
    d = q.shape[-1]
    if not q.is_cuda or d in (64, 128, 256) or d > 256:
        return None
    if d > 128:
        return 256 if q.dtype in (torch.bfloat16, torch.float16) else None
    return 64 if d < 64 else 128


def _pad(t: Optional[Tensor], dp: int) -> Optional[Tensor]:
    return None if t is None else torch.nn.functional.pad(t, (0, dp - t.shape[-1]))


def _unpad(t: Tensor, d: int, like: Tensor, buf: Optional[Tensor] = None) -> Tensor:
    """The first d features of t, in ``buf`` or in a new tensor laid out as an unpadded call
    lays out its result for an input like ``like``."""
    if buf is None:
        buf = _empty_heads((*t.shape[:3], d), _inner_contig(like))
    buf.copy_(t[..., :d])
    return buf


def _padded_epilogue(epilogue, dp):
    if epilogue is None:
        return None
    root, gate, root_sigmoid = epilogue
    return _pad(root, dp), _pad(gate, dp), root_sigmoid


def pass_fwd_raw(q, k, v, vmul, bias, key_mask, query_mask, causal, softclamp, scale,
                 may_degenerate, epilogue=None, qk_norm=None):
    """One pass forward: (out, lse), and with ``epilogue`` = (root, gate, root_sigmoid) the
    modules' gated output y as a third result (computed where the kernel stores out).
    ``qk_norm`` = (q norm, k norm), each (weight, eps) or None: RMSNorms of q and k applied
    as the kernel loads them (where the short-pass kernel runs, see qk_norms_fusable)."""
    dp = _padded_dim(q)
    if dp is not None:
        assert qk_norm is None, "q / k norms on load need head dim 64"

        d = q.shape[-1]
        res = pass_fwd_raw(_pad(q, dp), _pad(k, dp), _pad(v, dp), _pad(vmul, dp), bias,
                           key_mask, query_mask, causal, softclamp, scale, may_degenerate,
                           _padded_epilogue(epilogue, dp))
        return tuple(t if i == 1 else _unpad(t, d, q) for i, t in enumerate(res))
    p, res, _keep = _pass_prepare(q, k, v, vmul, bias, key_mask, query_mask, causal, softclamp,
                                  scale, may_degenerate, epilogue, qk_norm)
    with _device(q):
        _lib.check(_lib.load().pa_attn_pass_fwd(ctypes.byref(p), _stream(q)), "pa_attn_pass_fwd")
    return res


def _pass_prepare(q, k, v, vmul, bias, key_mask, query_mask, causal, softclamp, scale,
                  may_degenerate, epilogue=None, qk_norm=None):
    """The pa_pass of one forward pass over unpadded inputs with its outputs allocated:
    (struct, results, keep), results as pass_fwd_raw returns them and ``keep`` what the
    struct points at, to be held until the launch."""
    lib = _lib.load()
    q, k, v = _inner_contig(q), _inner_contig(k), _inner_contig(v)
    vmul = _inner_contig(vmul) if vmul is not None else None
    _check_pass_inputs(q, k, v, vmul, bias, key_mask, query_mask)
    km, qm = _mask_u8(key_mask), _mask_u8(query_mask)
    B, _, nq, d = q.shape
    H = _pass_heads(q, k, v, vmul, bias)
    out = _empty_heads((B, H, nq, d), q)
    lse = torch.empty(B, H, nq, dtype=torch.float32, device=q.device)
    y = epi = None
    if epilogue is not None:
        y = _empty_heads((B, H, nq, d), q)
        epi = _epilogue_struct(epilogue, y)
    p = _pass_struct(q, k, v, vmul, bias, km, qm, out, lse, causal, softclamp, scale,
                     may_degenerate or km is not None or qm is not None, epi)
    norm = None
    if qk_norm is not None:
        norm = _qk_norm_struct(qk_norm)
        p.norm = ctypes.addressof(norm)
    ws = None
    if km is not None:  # a key-masked pass takes the faster kernel with a workspace
        ws_bytes = lib.pa_attn_pass_fwd_workspace(ctypes.byref(p))
        if ws_bytes:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
            p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
    res = (out, lse) if epilogue is None else (out, lse, y)
    return p, res, (q, k, v, vmul, bias, km, qm, epi, norm, ws, epilogue)


def _out_buffer(buf: Optional[Tensor], like: Tensor) -> Tensor:
    if buf is None:
        return _empty_heads(like.shape, like)
    assert buf.shape == like.shape and buf.dtype == like.dtype and buf.stride(-1) == 1
    return buf


def pass_bwd_raw(dout, dlse, q, k, v, vmul, bias, key_mask, query_mask, out, lse, causal,
                 softclamp, scale, may_degenerate, dq_into: Optional[Tensor] = None,
                 dq_out: Optional[Tensor] = None, dk_out: Optional[Tensor] = None,
                 dv_out: Optional[Tensor] = None, epilogue=None):
    """One pass backward.  ``dq_into``: a gradient buffer of q's shape that the query gradient
    is added into (PA_ACC_DQ) instead of a new tensor.  ``dq_out`` / ``dk_out`` / ``dv_out``:
    buffers (any strided view of the right shape) that the gradients are written to instead
    of new tensors.  With ``epilogue`` (as in the forward) ``dout`` is the gradient of y and
    the gradients of root and gate follow the other five."""
    dp = _padded_dim(q)
    if dp is not None:
        d = q.shape[-1]
        res = pass_bwd_raw(_pad(_inner_contig(dout), dp), dlse, _pad(q, dp), _pad(k, dp),
                           _pad(v, dp), _pad(vmul, dp), bias, key_mask, query_mask,
                           _pad(out, dp), lse, causal, softclamp, scale, may_degenerate,
                           epilogue=_padded_epilogue(epilogue, dp))
        dq, dk, dv, dvmul, dbias = res[:5]
        if dq_into is not None:
            dq_into.add_(dq[..., :d])
            dq = dq_into
        else:  # at the pass head count when q has fewer heads (the caller sums them)
            dq = _unpad(dq, d, q, dq_out if dq.shape[1] == q.shape[1] else None)
        dk = _unpad(dk, d, k, dk_out)
        dv = _unpad(dv, d, v, dv_out)
        dvmul = _unpad(dvmul, d, vmul) if dvmul is not None else None
        extra = ()
        if epilogue is not None:
            droot, dgate = res[5:]
            extra = (_unpad(droot, d, epilogue[0]) if droot is not None else None,
                     _unpad(dgate, d, epilogue[1]) if dgate is not None else None)
        return (dq, dk, dv, dvmul, dbias) + extra
    lib = _lib.load()
    q, k, v = _inner_contig(q), _inner_contig(k), _inner_contig(v)
    vmul = _inner_contig(vmul) if vmul is not None else None
    dout = _inner_contig(dout).to(q.dtype)
    km, qm = _mask_u8(key_mask), _mask_u8(query_mask)
    H = out.shape[1]
    if q.shape[1] != H:
        # queries shared by several pass heads: the backward wants them per pass head (the
        # caller sums the per-head dq back)
        q = q.repeat_interleave(H // q.shape[1], dim=1)
        dq_out = None
    hk = k.shape[1]
    key_side = [t for t in (v, vmul, bias) if t is not None]
    assert all(t.shape[1] == hk for t in key_side), \
        "backward: k, v, vmul and bias must share one head count"
    accumulate = 0
    if dq_into is not None:
        assert dq_into.shape == q.shape and dq_into.dtype == q.dtype
        dq, accumulate = dq_into, _lib.PA_ACC_DQ
    else:
        dq = _out_buffer(dq_out, q)
    dk = _out_buffer(dk_out, k)
    dv = _out_buffer(dv_out, v)
    dvmul = _empty_heads(vmul.shape, vmul, v.dtype) if vmul is not None else None
    dbias = (torch.empty(bias.shape, dtype=torch.float32, device=q.device)
             if bias is not None else None)
    dlse32 = dlse.float() if dlse is not None else None
    g = PaPassGrad()
    g.fwd = _pass_struct(q, k, v, vmul, bias, km, qm, out, lse, causal, softclamp, scale,
                         may_degenerate or km is not None or qm is not None)
    g.dout, g.dlse = _view(dout), _view(dlse32)
    g.dq, g.dk, g.dv = _view(dq), _view(dk), _view(dv)
    g.dvmul, g.dbias = _view(dvmul), _view(dbias)
    g.accumulate = accumulate
    droot = dgate = epi = None
    if epilogue is not None:
        root, gate, _ = epilogue
        droot = _empty_heads(root.shape, root) if root is not None else None
        dgate = _empty_heads(gate.shape, gate) if gate is not None else None
        epi = _epilogue_struct(epilogue, out)  # y is not read by the backward
        g.fwd.epi = ctypes.addressof(epi)
        g.droot, g.dgate = _view(droot), _view(dgate)
    ws_bytes = lib.pa_attn_pass_bwd_workspace(ctypes.byref(g))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    g.workspace, g.workspace_bytes = ws.data_ptr(), ws_bytes
    with _device(q):
        _lib.check(lib.pa_attn_pass_bwd(ctypes.byref(g), _stream(q)), "pa_attn_pass_bwd")
    if dbias is not None and bias is not None and dbias.dtype != bias.dtype:
        dbias = dbias.to(bias.dtype)
    if epilogue is not None:
        return dq, dk, dv, dvmul, dbias, droot, dgate
    return dq, dk, dv, dvmul, dbias


# ---------------------------------------------------------------------------------------
# custom ops


@torch.library.custom_op("polyattn::pass_fwd", mutates_args=(), device_types="cuda")
def pass_fwd_op(q: Tensor, k: Tensor, v: Tensor, vmul: Optional[Tensor], bias: Optional[Tensor],
                key_mask: Optional[Tensor], query_mask: Optional[Tensor], causal: bool,
                softclamp: float, scale: float, may_degenerate: bool) -> tuple[Tensor, Tensor]:
    return pass_fwd_raw(q, k, v, vmul, bias, key_mask, query_mask, causal, softclamp, scale,
                        may_degenerate)


@pass_fwd_op.register_fake
def _(q, k, v, vmul, bias, key_mask, query_mask, causal, softclamp, scale, may_degenerate):
    # the layouts pass_fwd_raw allocates (heads-inner output for heads-inner queries)
    q = _inner_contig(q)
    B, _, nq, d = q.shape
    H = _pass_heads(q, k, v, vmul, bias)
    return (_empty_heads((B, H, nq, d), q), q.new_empty(B, H, nq, dtype=torch.float32))


@torch.library.custom_op("polyattn::pass_bwd", mutates_args=(), device_types="cuda")
def pass_bwd_op(dout: Tensor, dlse: Optional[Tensor], q: Tensor, k: Tensor, v: Tensor,
                vmul: Optional[Tensor], bias: Optional[Tensor], key_mask: Optional[Tensor],
                query_mask: Optional[Tensor], out: Tensor, lse: Tensor, causal: bool,
                softclamp: float, scale: float,
                may_degenerate: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    dq, dk, dv, dvmul, dbias = pass_bwd_raw(dout, dlse, q, k, v, vmul, bias, key_mask,
                                            query_mask, out, lse, causal, softclamp, scale,
                                            may_degenerate)
    if dvmul is None:
        dvmul = q.new_empty(0)
    if dbias is None:
        dbias = q.new_empty(0)
    return dq, dk, dv, dvmul, dbias


@pass_bwd_op.register_fake
def _(dout, dlse, q, k, v, vmul, bias, key_mask, query_mask, out, lse, causal, softclamp, scale,
      may_degenerate):
    # the layouts pass_bwd_raw allocates
    q, k, v = _inner_contig(q), _inner_contig(k), _inner_contig(v)
    H = out.shape[1]
    if q.shape[1] != H:
        dq = q.new_empty(q.shape[0], H, *q.shape[2:])
    else:
        dq = _empty_heads(q.shape, q)
    dvmul = _empty_heads(vmul.shape, vmul, v.dtype) if vmul is not None else q.new_empty(0)
    dbias = bias.new_empty(bias.shape) if bias is not None else q.new_empty(0)
    return dq, _empty_heads(k.shape, k), _empty_heads(v.shape, v), dvmul, dbias


def _pass_setup(ctx, inputs, output):
    q, k, v, vmul, bias, key_mask, query_mask, causal, softclamp, scale, may_degenerate = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, vmul, bias, key_mask, query_mask, out, lse)
    ctx.causal, ctx.softclamp, ctx.scale = causal, softclamp, scale
    ctx.may_degenerate = may_degenerate
    ctx.has_vmul, ctx.has_bias = vmul is not None, bias is not None
    ctx.slots = [slot_ref(t) for t in (q, k, v)]
    ctx.set_materialize_grads(False)


def _pass_backward(ctx, dout, dlse):
    q, k, v, vmul, bias, key_mask, query_mask, out, lse = ctx.saved_tensors
    if dout is None:
        dout = torch.zeros_like(out)
    # a q / k / v that is a piece of a head-split projection: its gradient goes straight into
    # the projection's gradient buffer (eager only; the op is opaque to tracing)
    outs = [claim_slot(r, t) for r, t in zip(ctx.slots, (q, k, v))]
    if q.shape[1] != out.shape[1]:
        outs[0] = None
    if any(o is not None for o in outs):
        dq, dk, dv, dvmul, dbias = pass_bwd_raw(dout, dlse, q, k, v, vmul, bias, key_mask,
                                                query_mask, out, lse, ctx.causal, ctx.softclamp,
                                                ctx.scale, ctx.may_degenerate, dq_out=outs[0],
                                                dk_out=outs[1], dv_out=outs[2])
        if dvmul is None:
            dvmul = q.new_empty(0)
        if dbias is None:
            dbias = q.new_empty(0)
    else:
        dq, dk, dv, dvmul, dbias = pass_bwd_op(dout, dlse, q, k, v, vmul, bias, key_mask,
                                               query_mask, out, lse, ctx.causal, ctx.softclamp,
                                               ctx.scale, ctx.may_degenerate)
    if dq.shape[1] != q.shape[1]:  # queries were shared across pass heads: sum their grads
        dq = dq.unflatten(1, (q.shape[1], -1)).sum(2)
    return (dq, dk, dv, dvmul if ctx.has_vmul else None, dbias if ctx.has_bias else None,
            None, None, None, None, None, None)


torch.library.register_autograd("polyattn::pass_fwd", _pass_backward, setup_context=_pass_setup)


def _needs_op(*ts) -> bool:
    """Whether a call must go through the registered custom op (autograd or torch.compile
    tracing); plain inference calls the library directly (less host overhead per launch)."""
    if torch.compiler.is_compiling():
        return True
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def attn_pass(q: Tensor, k: Tensor, v: Tensor, vmul: Optional[Tensor] = None,
              bias: Optional[Tensor] = None, key_mask: Optional[Tensor] = None,
              query_mask: Optional[Tensor] = None, causal: bool = False,
              softclamp: Optional[float] = None, scale: Optional[float] = None,
              may_degenerate: bool = False) -> tuple[Tensor, Tensor]:
    """One differentiable attention pass on the GPU: returns (out, lse[fp32])."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    if not _needs_op(q, k, v, vmul, bias):
        return pass_fwd_raw(q, k, v, vmul, bias, key_mask, query_mask, bool(causal),
                            float(softclamp or 0.0), float(scale), bool(may_degenerate))
    return pass_fwd_op(q, k, v, vmul, bias, key_mask, query_mask, bool(causal),
                       float(softclamp or 0.0), float(scale), bool(may_degenerate))


# ---------------------------------------------------------------------------------------
# per-head RMSNorm


def _rms_angles(x: Tensor, angles: Optional[Tensor]) -> Optional[Tensor]:
    """The rotary angle rows of x's positions as pa_rmsnorm reads them: a [rot_dim] row for
    every position, or the last N rows of [positions, rot_dim] (apply_rotary_emb's slicing)."""
    if angles is None:
        return None
    if angles.dim() == 2:
        angles = angles.narrow(0, angles.shape[0] - x.shape[2], x.shape[2])
    return angles


def _rms_struct(x: Tensor, weight: Optional[Tensor], eps: float,
                angles: Optional[Tensor] = None) -> PaRmsNorm:
    r = PaRmsNorm()
    r.batch, r.heads, r.n, r.dim = x.shape
    r.eps = float(eps)
    r.x = _view(x)
    if weight is not None:
        r.weight, r.weight_dtype = weight.data_ptr(), DTYPE_CODE[weight.dtype]
    a = _rms_angles(x, angles)
    if a is not None:
        r.angles, r.angles_dtype = a.data_ptr(), DTYPE_CODE[a.dtype]
        r.rot_dim = a.shape[-1]
        r.angles_stride = a.stride(0) if a.dim() == 2 else 0
    return r


def _aligned16(t: Tensor) -> Tensor:
    """t itself when its data starts on a 16-byte boundary, else a copy in the same layout
    (fresh storage is aligned)."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def rms_supported(x: Tensor, weight: Optional[Tensor], angles: Optional[Tensor] = None) -> bool:
    """Shapes and layouts pa_rmsnorm takes (on a CUDA tensor): ``rms_layout_supported``."""
    return x.is_cuda and rms_layout_supported(x, weight, angles)


def rms_layout_supported(x: Tensor, weight: Optional[Tensor],
                         angles: Optional[Tensor] = None) -> bool:
    """[B, H, N, d] with strides that keep rows 16-byte aligned (a misaligned base pointer is
    copied by the call itself, so that traced code never reads a pointer); rotary angles
    (optional) as apply_rotary_emb takes them for such an x: [rot_dim] or
    [positions >= N, rot_dim], rot_dim even and <= d, no gradient."""
    if x.dim() != 4 or x.dtype not in DTYPE_CODE:
        return False
    e = 4 if x.dtype == torch.float32 else 8
    d = x.shape[-1]
    if d % e or d > 512 or x.stride(-1) != 1 or x.numel() == 0:
        return False
    if any(st % e for st in x.stride()[:3]):
        return False
    if angles is not None:
        if angles.dim() not in (1, 2) or angles.dtype not in DTYPE_CODE or angles.requires_grad:
            return False
        if angles.device != x.device or angles.stride(-1) != 1:
            return False
        rot = angles.shape[-1]
        if rot % 2 or rot > d or (angles.dim() == 2 and angles.shape[0] < x.shape[2]):
            return False
    return weight is None or (weight.dim() == 1 and weight.numel() == d
                              and weight.dtype in DTYPE_CODE and weight.is_contiguous())


@torch.library.custom_op("polyattn::rms_norm", mutates_args=(), device_types="cuda")
def rms_norm_op(x: Tensor, weight: Optional[Tensor], eps: float,
                angles: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    return _rms_fwd_raw(x, weight, eps, angles)


def _rms_fwd_raw(x: Tensor, weight: Optional[Tensor], eps: float,
                 angles: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    lib = _lib.load()
    y = _empty_heads(x.shape, x)
    rstd = torch.empty(x.shape[:3], dtype=torch.float32, device=x.device)
    r = _rms_struct(_aligned16(x), weight, eps, angles)
    r.y, r.rstd = _view(y), rstd.data_ptr()
    with _device(x):
        _lib.check(lib.pa_rmsnorm_fwd(ctypes.byref(r), _stream(x)), "pa_rmsnorm_fwd")
    return y, rstd


@rms_norm_op.register_fake
def _(x, weight, eps, angles=None):
    return _empty_heads(x.shape, x), x.new_empty(x.shape[:3], dtype=torch.float32)


@torch.library.custom_op("polyattn::rms_norm_bwd", mutates_args=(), device_types="cuda")
def rms_norm_bwd_op(dy: Tensor, x: Tensor, weight: Optional[Tensor], rstd: Tensor,
                    eps: float, angles: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    return _rms_bwd_raw(dy, x, weight, rstd, eps, angles)


def _rms_bwd_raw(dy: Tensor, x: Tensor, weight: Optional[Tensor], rstd: Tensor, eps: float,
                 angles: Optional[Tensor] = None,
                 dx_out: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    lib = _lib.load()
    if dy.stride(-1) != 1 or any(st % (4 if dy.dtype == torch.float32 else 8)
                                 for st in dy.stride()[:3]):
        dy = dy.contiguous()
    dy = _aligned16(dy)
    dx = _empty_heads(x.shape, x) if dx_out is None else dx_out
    if dx_out is not None and (not rms_supported(dx_out, weight, angles) or dx_out.data_ptr() % 16):
        dx = _empty_heads(x.shape, x)
    r = _rms_struct(_aligned16(x), weight, eps, angles)
    r.rstd = rstd.data_ptr()
    r.dy, r.dx = _view(dy), _view(dx)
    dw32 = None
    if weight is not None:
        dw32 = torch.empty(x.shape[-1], dtype=torch.float32, device=x.device)
        r.dweight = dw32.data_ptr()
    ws_bytes = lib.pa_rmsnorm_bwd_workspace(ctypes.byref(r))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    r.workspace, r.workspace_bytes = ws.data_ptr(), ws_bytes
    with _device(x):
        _lib.check(lib.pa_rmsnorm_bwd(ctypes.byref(r), _stream(x)), "pa_rmsnorm_bwd")
    dw = dw32.to(weight.dtype) if weight is not None else x.new_empty(0)
    return dx, dw


@rms_norm_bwd_op.register_fake
def _(dy, x, weight, rstd, eps, angles=None):
    return _empty_heads(x.shape, x), (weight.new_empty(weight.shape) if weight is not None
                                      else x.new_empty(0))


def _rms_setup(ctx, inputs, output):
    x, weight, eps, angles = inputs
    _, rstd = output
    ctx.save_for_backward(x, weight, rstd, angles)
    ctx.eps = eps
    ctx.slot = slot_ref(x)
    ctx.set_materialize_grads(False)


def _rms_backward(ctx, dy, drstd):
    x, weight, rstd, angles = ctx.saved_tensors
    if dy is None:
        return None, None, None, None
    dx_out = claim_slot(ctx.slot, x)
    if dx_out is not None:  # eager: write dx into the split projection's gradient
        dx, dw = _rms_bwd_raw(dy, x, weight, rstd, ctx.eps, angles, dx_out)
    else:
        dx, dw = rms_norm_bwd_op(dy, x, weight, rstd, ctx.eps, angles)
    return dx, (dw if weight is not None else None), None, None


torch.library.register_autograd("polyattn::rms_norm", _rms_backward, setup_context=_rms_setup)


def rms_norm(x: Tensor, weight: Optional[Tensor], eps: Optional[float],
             angles: Optional[Tensor] = None) -> Tensor:
    """torch.nn.RMSNorm(d)(x) over the last dim of a [B, H, N, d] CUDA tensor on the HIP
    kernels, followed by apply_rotary_emb(angles, .) when angles are given (the caller checks
    rms_supported).  eps=None is torch's default, the epsilon of the fp32 op-math type."""
    if eps is None:
        eps = torch.finfo(torch.float32).eps
    if not _needs_op(x, weight):
        return _rms_fwd_raw(x, weight, float(eps), angles)[0]
    return rms_norm_op(x, weight, float(eps), angles)[0]


def rms_norm_many(xs: Sequence[Tensor], weights: Sequence[Optional[Tensor]],
                  eps: Sequence[Optional[float]]) -> list[Tensor]:
    """torch.nn.RMSNorm of up to PA_RMS_MAX_ITEMS [B, H, N, d] CUDA tensors of one dtype and d
    in one launch (pa_rmsnorm_fwd_many), without autograd: the q/k norms of a layer when no
    gradient is needed.  The caller checks rms_supported for each (no rotary angles)."""
    lib = _lib.load()
    n = len(xs)
    assert 1 <= n <= _lib.PA_RMS_MAX_ITEMS
    items = (PaRmsNorm * n)()
    ys, keep = [], []
    for k, (x, w, e) in enumerate(zip(xs, weights, eps)):
        x = _aligned16(x)
        y = _empty_heads(x.shape, x)
        r = _rms_struct(x, w, torch.finfo(torch.float32).eps if e is None else float(e))
        r.y = _view(y)  # no rstd: nothing runs backward through these norms
        items[k] = r
        ys.append(y)
        keep.append(x)
    with _device(xs[0]):
        _lib.check(lib.pa_rmsnorm_fwd_many(items, n, _stream(xs[0])), "pa_rmsnorm_fwd_many")
    return ys


# ---------------------------------------------------------------------------------------
# projections of a single-token decode step

LINEAR_MAX_ROWS = 16


def linear_supported(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None) -> bool:
    """Whether pa_linear_small takes F.linear(x, weight, bias): plain inference (no autograd,
    not under torch.compile) on CUDA tensors of one dtype, at most 16 rows of x (all leading
    dims), in_features a multiple of 8 (4 for fp32) with x fitting the 64 KiB staging."""
    k = x.shape[-1] if x.dim() >= 1 else 0
    if k == 0 or x.numel() > LINEAR_MAX_ROWS * k:  # the common, large case first
        return False
    if not (x.is_cuda and weight.is_cuda) or x.dtype not in DTYPE_CODE or weight.dtype != x.dtype:
        return False
    if weight.dim() != 2 or weight.device != x.device or weight.shape[1] != k:
        return False
    if torch.compiler.is_compiling() or _needs_op(x, weight, bias):
        return False
    rows = x.numel() // k
    e = 4 if x.dtype == torch.float32 else 8
    if not 1 <= rows <= LINEAR_MAX_ROWS or k % e or rows * k * x.element_size() > 65536:
        return False
    if weight.stride(-1) != 1 or weight.stride(0) % e or weight.data_ptr() % 16:
        return False
    if bias is not None and (bias.dtype != x.dtype or bias.dim() != 1 or bias.stride(0) != 1
                             or bias.shape[0] != weight.shape[0] or bias.device != x.device):
        return False
    return True


def _rows2d(t: Tensor, k: int, e: int) -> Tensor:
    t2 = t.reshape(-1, k)
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) % e):
        t2 = t2.contiguous()
    return _aligned16(t2)


def linear_small_group(x: Tensor, specs, *, x_add: Optional[Tensor] = None,
                       norm: Optional[torch.nn.Module] = None, return_sum: bool = False):
    """Up to four projections of one decode-sized x in one launch of pa_linear_small.
    ``specs``: (weight, bias, gelu, residual) per output -- F.linear(x, weight, bias), then
    GELU (erf form) when ``gelu``, then ``+ residual`` when given, rounded after each step as
    the separate torch ops.  Before the products x may take ``+ x_add`` and an RMSNorm
    (``norm``: a torch.nn.RMSNorm over the features); ``return_sum`` also returns x + x_add.
    The caller checks linear_supported for every (x, weight, bias)."""
    lib = _lib.load()
    assert 1 <= len(specs) <= _lib.PA_LINEAR_MAX_OUT
    k = x.shape[-1]
    e = 4 if x.dtype == torch.float32 else 8
    x2 = _rows2d(x, k, e)
    rows = x2.shape[0]
    lin = _lib.PaLinear()
    lin.rows, lin.in_features, lin.dtype, lin.count = rows, k, DTYPE_CODE[x.dtype], len(specs)
    lin.x, lin.x_stride = x2.data_ptr(), x2.stride(0)
    keep, xs = [x2], None
    if x_add is not None:
        a2 = _rows2d(x_add.to(x.dtype), k, e)
        keep.append(a2)
        lin.x_add, lin.x_add_stride = a2.data_ptr(), a2.stride(0)
        if return_sum:
            xs = torch.empty(rows, k, dtype=x.dtype, device=x.device)
            lin.x_sum, lin.x_sum_stride = xs.data_ptr(), xs.stride(0)
    if norm is not None:
        lin.norm = 1
        eps = norm.eps if norm.eps is not None else torch.finfo(torch.float32).eps
        lin.norm_eps = float(eps)
        if norm.weight is not None:
            w = norm.weight.detach().contiguous()
            keep.append(w)
            lin.norm_weight, lin.norm_dtype = w.data_ptr(), DTYPE_CODE[w.dtype]
    outs = []
    for o, (w, b, gelu, res) in zip(lin.out, specs):
        n = w.shape[0]
        y = torch.empty(rows, n, dtype=x.dtype, device=x.device)
        o.w, o.w_stride, o.out_features = w.data_ptr(), w.stride(0), n
        o.activation = _lib.PA_ACT_GELU if gelu else _lib.PA_ACT_NONE
        o.bias = b.data_ptr() if b is not None else None
        if res is not None:
            r2 = res.reshape(rows, n)
            if r2.stride(-1) != 1:
                r2 = r2.contiguous()
            keep.append(r2)
            o.residual, o.residual_stride = r2.data_ptr(), r2.stride(0)
        o.y, o.y_stride = y.data_ptr(), y.stride(0)
        outs.append(y.reshape(*x.shape[:-1], n))
    with _device(x):
        _lib.check(lib.pa_linear_small(ctypes.byref(lin), _stream(x)), "pa_linear_small")
    if return_sum:
        return outs, xs.reshape(x.shape)
    return outs


def linear_small(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None) -> Tensor:
    """torch.nn.functional.linear(x, weight, bias) on pa_linear_small: the weight streamed
    once by every CU for decode-sized x (the caller checks linear_supported)."""
    return linear_small_group(x, [(weight, bias, False, None)])[0]


def _norm_fusable(norm: Optional[torch.nn.Module], x: Tensor) -> bool:
    if norm is None:
        return True
    return (isinstance(norm, torch.nn.RMSNorm) and tuple(norm.normalized_shape) == (x.shape[-1],)
            and (norm.weight is None or (norm.weight.dtype in DTYPE_CODE and norm.weight.is_cuda)))


def linear(layer: torch.nn.Linear, x: Tensor, *, gelu: bool = False,
           residual: Optional[Tensor] = None, x_add: Optional[Tensor] = None,
           norm: Optional[torch.nn.Module] = None, return_sum: bool = False):
    """residual + gelu?(layer(norm?(x + x_add?))) with each part optional -- on one launch of
    pa_linear_small when linear_supported, else with the layer and torch ops.  With
    ``return_sum`` returns (y, x + x_add)."""
    n = layer.weight.shape[0]
    if x.is_cuda and linear_supported(x, layer.weight, layer.bias) and _norm_fusable(norm, x) and (
            residual is None or (residual.dtype == x.dtype and residual.device == x.device
                                 and residual.shape == (*x.shape[:-1], n))) and (
            x_add is None or (x_add.shape == x.shape and x_add.dtype == x.dtype
                              and x_add.device == x.device)):
        r = linear_small_group(x, [(layer.weight, layer.bias, gelu, residual)], x_add=x_add,
                               norm=norm, return_sum=return_sum and x_add is not None)
        if return_sum:
            return (r[0][0], r[1]) if x_add is not None else (r[0], x)
        return r[0]
    xs = x if x_add is None else x + x_add
    y = layer(norm(xs) if norm is not None else xs)
    if gelu:
        y = torch.nn.functional.gelu(y)
    if residual is not None:
        y = residual + y
    return (y, xs) if return_sum else y


def linear_many(layers, xs) -> list[Tensor]:
    """[layer(x) for layer, x in zip(layers, xs)], the projections of one input sharing
    launches of pa_linear_small (up to four per launch) when every call qualifies."""
    x = xs[0]
    if x.is_cuda and all(xi is x for xi in xs) and all(
            linear_supported(x, layer.weight, layer.bias) for layer in layers):
        outs = []
        for i in range(0, len(layers), _lib.PA_LINEAR_MAX_OUT):
            group = layers[i:i + _lib.PA_LINEAR_MAX_OUT]
            outs += linear_small_group(x, [(l.weight, l.bias, False, None) for l in group])
        return outs
    return [linear(layer, xi) for layer, xi in zip(layers, xs)]


# ---------------------------------------------------------------------------------------
# head split of the training / prefill projections


class _GradSlots:
    """The gradient buffer of a head-split projection ([B, N, F]), allocated on first use in the
    backward.  A backward that produces the gradient of a piece (the pass and RMSNorm
    backwards) may claim the piece's slot -- a [B, h, N, d] view of the buffer -- and write its
    result there, so that the split's backward finds the pieces already in place.  Each slot
    is handed out once per backward; a second consumer of the same piece allocates its own
    gradient (autograd sums the two, and the split copies the sum into the slot)."""

    def __init__(self, shape, dtype, device, heads, d):
        self.shape, self.dtype, self.device, self.heads, self.d = shape, dtype, device, heads, d
        self.offsets = [0]
        for h in heads:
            self.offsets.append(self.offsets[-1] + h * d)
        self.buf = None
        self.claimed = set()

    def view(self, i: int) -> Tensor:
        if self.buf is None:
            self.buf = torch.empty(self.shape, dtype=self.dtype, device=self.device)
        o, h = self.offsets[i], self.heads[i]
        return self.buf[..., o:o + h * self.d].unflatten(-1, (h, self.d)).transpose(1, 2)

    def claim(self, i: int) -> Optional[Tensor]:
        if i in self.claimed:
            return None
        self.claimed.add(i)
        return self.view(i)

    def take(self) -> Tensor:
        # the finished buffer leaves with the split's gradient: a later backward over the same
        # graph (retain_graph) starts over with a new buffer
        buf, self.buf, self.claimed = self.buf, None, set()
        return buf


def slot_ref(t: Optional[Tensor]):
    """At a consumer's forward: the gradient-slot reference of ``t`` when it is a piece of a
    head-split projection (``project_heads``), else None."""
    return getattr(t, "_pa_grad_slot", None) if t is not None else None


def claim_slot(ref, like: Tensor) -> Optional[Tensor]:
    """At the consumer's backward: the piece's gradient slot, claimed for writing, when it
    matches ``like`` (the gradient the consumer would allocate) in shape and dtype."""
    if ref is None:
        return None
    slots, i = ref
    if (tuple(like.shape) != (slots.shape[0], slots.heads[i], slots.shape[1], slots.d)
            or like.dtype != slots.dtype or like.device != slots.device):
        return None
    return slots.claim(i)


class _SplitHeads(torch.autograd.Function):
    """``rearrange(t, 'b n (p h d) -> p b h n d')`` of a [B, N, F] projection as one [B, h, N, d]
    view per piece (pieces may differ in head count).  The backward assembles the projection's
    gradient in a ``_GradSlots`` buffer: pieces whose consumers wrote their gradient into its
    slot cost nothing, the others are copied in (or zero-filled when unused).  (Through einops,
    autograd would zero-fill the selected slots, stack the pieces and copy the permuted stack
    back: three to five copies of the projection per step.)"""

    @staticmethod
    def forward(ctx, t, heads, d, slots):
        ctx.slots = slots
        ctx.set_materialize_grads(False)
        outs, off = [], 0
        for h in heads:
            outs.append(t[..., off:off + h * d].unflatten(-1, (h, d)).transpose(1, 2))
            off += h * d
        return tuple(outs)

    @staticmethod
    def backward(ctx, *grads):
        slots = ctx.slots
        B, N, _ = slots.shape
        if slots.buf is None:
            # no consumer wrote in place: one concatenation (a single piece is a free view,
            # the kernels' gradients being heads-inner)
            parts = [torch.zeros(B, N, h * slots.d, dtype=slots.dtype, device=slots.device)
                     if g is None else g.transpose(1, 2).reshape(B, N, h * slots.d)
                     for g, h in zip(grads, slots.heads)]
            slots.claimed = set()
            return (parts[0] if len(parts) == 1 else torch.cat(parts, dim=-1)), None, None, None
        for i, g in enumerate(grads):
            v = slots.view(i)
            if g is None:
                v.zero_()
            elif not (g.data_ptr() == v.data_ptr() and g.stride() == v.stride()):
                v.copy_(g)
        return slots.take(), None, None, None


def _plain_linear(layer) -> bool:
    # exactly nn.Linear with no hooks: bypassing layer(x) must not skip anything a caller added
    return (type(layer) is torch.nn.Linear and not layer._forward_hooks
            and not layer._forward_pre_hooks)


def _dw_splits(rows: int, out_features: int, in_features: int) -> int:
    """Batches of the split-K weight-gradient GEMM: a tall-skinny dy^T x (many rows, a small
    output) leaves most CUs idle as one GEMM (hipBLASLt tiles only the output); measured on
    MI355X at 16384 rows, 1024 x 1024 takes 108 us as one GEMM and 54 us in 8 batches,
    4096 x 1024 195 us and 159 us in 4."""
    outs = out_features * in_features
    s = 8 if outs <= 1 << 20 else 4 if outs <= 1 << 22 else 1
    while s > 1 and (rows % s or rows // s < 2048):
        s //= 2
    return s


def _weight_grad(dy2: Tensor, x2: Tensor) -> Tensor:
    """dy2^T @ x2 ([rows, out]^T [rows, in]) in the weights' dtype: split-K batches with fp32
    partial products summed in fp32 and rounded once, as one GEMM's fp32 accumulator is."""
    rows, n = dy2.shape
    k = x2.shape[1]
    s = _dw_splits(rows, n, k)
    if s == 1:
        return dy2.t() @ x2
    a = dy2.view(s, rows // s, n).transpose(1, 2)
    p = torch.bmm(a, x2.view(s, rows // s, k), out_dtype=torch.float32)
    return p.sum(0).to(dy2.dtype)


class _LinearTrain(torch.autograd.Function):
    """F.linear(x, weight, bias) whose backward takes the weight gradient as split-K batches
    (``_weight_grad``); dx and the bias gradient are the GEMM and sum torch's Linear backward
    computes."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return torch.nn.functional.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1])
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = (dy2 @ weight).view(x.shape)
        if ctx.needs_input_grad[1]:
            x2 = x.reshape(-1, x.shape[-1])
            dw = _weight_grad(dy2.contiguous(), x2.contiguous())
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = dy2.sum(0)
        return dx, dw, db


def linear_train(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None) -> Tensor:
    """F.linear for training-sized GPU inputs: with a weight gradient to compute and a shape
    that profits, the split-K weight gradient; otherwise F.linear itself."""
    rows = x.numel() // x.shape[-1] if x.dim() else 0
    if (x.is_cuda and torch.is_grad_enabled() and weight.requires_grad
            and x.dtype == weight.dtype and x.dtype in (torch.bfloat16, torch.float16)
            and (bias is None or bias.dtype == x.dtype)
            and not torch.is_autocast_enabled() and not torch.compiler.is_compiling()
            and _dw_splits(rows, weight.shape[0], weight.shape[1]) > 1):
        return _LinearTrain.apply(x, weight, bias)
    return torch.nn.functional.linear(x, weight, bias)


def layer_train(layer, x: Tensor) -> Tensor:
    """layer(x) for a training-sized input; a plain hook-free nn.Linear goes through
    ``linear_train``."""
    if _plain_linear(layer):
        return linear_train(x, layer.weight, layer.bias)
    return layer(x)


def _concat_weights(layers) -> Tensor:
    """torch.cat of the layers' weights, built on every call: a cached copy would miss
    in-place updates that bypass the version counter (``weight.data.copy_``), and a copy
    made under inference mode cannot be saved for a later backward.  Inside a captured HIP
    graph the concatenation is one of the captured kernels, so replays see the current
    weights."""
    return torch.cat([l.weight for l in layers])


def project_heads(layers, xs, splits):
    """The modules' projections followed by their head splits
    (poly_attention.py:258-266, 322-340; n_poly_attention.py:103-110, 177-196):
    ``[rearrange(layer(x), 'b n (p h d) -> p b h n d') for ...]`` with ``splits[i] = (p, h)``,
    each result a list of p views [B, h, N, d].  When every layer reads the same input and is
    a plain bias-free nn.Linear, the projections run as one GEMM over the concatenated
    weights (one dx GEMM and one weight-gradient GEMM in the backward instead of one per layer
    plus the adds of dx).  The head splits are views; the pass and RMSNorm backwards write
    their pieces' gradients straight into the projection's gradient buffer."""
    x = xs[0]
    d = []
    for layer, (p, h) in zip(layers, splits):
        assert layer.weight.shape[0] % (p * h) == 0
        d.append(layer.weight.shape[0] // (p * h))
    fuse = (len(layers) > 1 and all(xi is x for xi in xs) and x.dim() == 3
            and len(set(d)) == 1 and not torch.compiler.is_compiling()
            and not torch.nn.modules.module._global_forward_hooks
            and not torch.nn.modules.module._global_forward_pre_hooks
            and all(_plain_linear(l) and l.bias is None for l in layers)
            and len({l.weight.dtype for l in layers}) == 1)
    if fuse:
        w = _concat_weights(layers)
        heads = tuple(h for p, h in splits for _ in range(p))
        pieces = _split_heads(linear_train(x, w), heads, d[0])
        out, i = [], 0
        for p, _ in splits:
            out.append(list(pieces[i:i + p]))
            i += p
        return out
    out = []
    for layer, xi, (p, h), di in zip(layers, xs, splits, d):
        y = layer_train(layer, xi)
        assert y.dim() == 3, "expected a [batch, n, features] projection"
        out.append(list(_split_heads(y, (h,) * p, di)))
    return out


def _split_heads(t: Tensor, heads, d: int):
    if not (torch.is_grad_enabled() and t.requires_grad) or torch.compiler.is_compiling():
        # no gradient (or traced): plain views, without the gradient-slot autograd node
        outs, off = [], 0
        for h in heads:
            outs.append(t[..., off:off + h * d].unflatten(-1, (h, d)).transpose(1, 2))
            off += h * d
        return tuple(outs)
    slots = _GradSlots(t.shape, t.dtype, t.device, tuple(heads), d)
    pieces = _SplitHeads.apply(t, tuple(heads), d, slots)
    if t.requires_grad and not torch.compiler.is_compiling():
        for i, piece in enumerate(pieces):
            piece._pa_grad_slot = (slots, i)
    return pieces


# ---------------------------------------------------------------------------------------
# the order-n chain


def order2_forward(q1, q2, q3, v3, key_mask, causal, softclamp, scale, epilogue=None,
                   norms=None, keep_inner=True):
    """The two forward passes of the order-2 chain (poly_attention.py:48-116 with q2 as both
    the pass-1 queries and the pass-2 keys); ``key_mask`` masks the keys of both passes.
    Returns (out, lse, lse23, msg), and with ``epilogue`` = (root, gate, root_sigmoid) the
    modules' gated output y (computed in pass 2's store) as a fifth result.  ``norms`` =
    ((w1, eps1), (w2, eps2), (w3, eps3)): q1, q2, q3 are raw and the passes apply their
    RMSNorms on load (qk_norms_fusable; no gradient).  ``keep_inner=False``: the caller does
    not read lse23 and msg, which the one-launch path then leaves unwritten."""
    degenerate = key_mask is not None
    n1, n2, n3 = norms if norms is not None else (None, None, None)
    if key_mask is None and _padded_dim(q2) is None:
        # both passes through pa_poly_order2_fwd: one launch where both are short passes
        q2 = _inner_contig(q2)
        p1, (msg, lse23), keep1 = _pass_prepare(
            q2, q3, v3, None, None, None, None, causal, softclamp, scale, False,
            qk_norm=(n2, n3) if norms is not None else None)
        p2, res, keep2 = _pass_prepare(
            q1, q2, msg, None, lse23, None, None, causal, softclamp, scale, False, epilogue,
            qk_norm=(n1, n2) if norms is not None else None)
        if not keep_inner:
            p1.flags |= PA_FLAG_DISCARD_OUT
        with _device(q2):
            _lib.check(_lib.load().pa_poly_order2_fwd(ctypes.byref(p1), ctypes.byref(p2),
                                                      _stream(q2)), "pa_poly_order2_fwd")
        return (res[0], res[1], lse23, msg) + tuple(res[2:])
    msg, lse23 = pass_fwd_raw(q2, q3, v3, None, None, key_mask, None, causal, softclamp, scale,
                              degenerate, qk_norm=(n2, n3) if norms is not None else None)
    res = pass_fwd_raw(q1, q2, msg, None, lse23, key_mask, None, causal, softclamp, scale,
                       degenerate, epilogue, qk_norm=(n1, n2) if norms is not None else None)
    return (res[0], res[1], lse23, msg) + tuple(res[2:])


def order2_backward(saved, key_mask, cfg, slots, dout, dlse=None, dlse23_ext=None,
                    dmsg_ext=None, epilogue=None):
    """The two pass backwards of ``order2_forward``, back to back: pass 2's key gradient of
    q2 is the buffer that pass 1's query gradient of q2 is accumulated into (no separate
    add).  ``saved`` = (q1, q2, q3, v3, msg, lse23, out, lse); ``slots`` the head-split
    gradient slots of q1..v3 (or Nones).  Returns (dq1, dq2, dq3, dv3); with ``epilogue``
    (as in the forward) ``dout`` is the gradient of y and (droot, dgate) follow."""
    q1, q2, q3, v3, msg, lse23, out, lse = saved
    causal, softclamp, scale = cfg
    degenerate = key_mask is not None
    if dout is None:
        dout = torch.zeros_like(out)
    # inputs that are pieces of a head-split projection get their gradients written into
    # its gradient buffer
    dq1_out, dq2_out, dq3_out, dv3_out = (claim_slot(r, t) for r, t in
                                          zip(slots, (q1, q2, q3, v3)))
    res = pass_bwd_raw(dout, dlse, q1, q2, msg, None, lse23, key_mask, None, out, lse, causal,
                       softclamp, scale, degenerate, dq_out=dq1_out, dk_out=dq2_out,
                       epilogue=epilogue)
    dq1, dq2, dmsg, _, dlse23 = res[:5]
    if dmsg_ext is not None:
        dmsg = dmsg + dmsg_ext
    if dlse23_ext is not None:
        dlse23 = dlse23 + dlse23_ext
    _, dq3, dv3, _, _ = pass_bwd_raw(dmsg, dlse23, q2, q3, v3, None, None, key_mask, None, msg,
                                     lse23, causal, softclamp, scale, degenerate, dq_into=dq2,
                                     dk_out=dq3_out, dv_out=dv3_out)
    return (dq1, dq2, dq3, dv3) + tuple(res[5:])


class _Order2Chain(torch.autograd.Function):
    """The order-2 chain (poly_attention.py:48-116) as one autograd node
    (``order2_forward`` / ``order2_backward``), with the modules' root-value / gate epilogue
    (poly_attention.py:342-351) fused into pass 2 when root or gate is given: the first
    output is then the gated y."""

    @staticmethod
    def forward(ctx, q1, q2, q3, v3, root, gate, causal, softclamp, scale, root_sigmoid):
        epi = (root, gate, root_sigmoid) if root is not None or gate is not None else None
        res = order2_forward(q1, q2, q3, v3, None, causal, softclamp, scale, epi)
        out, lse, lse23, msg = res[:4]
        ctx.save_for_backward(q1, q2, q3, v3, msg, lse23, out, lse, root, gate)
        ctx.cfg = (causal, softclamp, scale)
        ctx.root_sigmoid = root_sigmoid
        ctx.slots = [slot_ref(t) for t in (q1, q2, q3, v3)]
        ctx.set_materialize_grads(False)
        return (res[4] if epi is not None else out), lse, lse23, msg

    @staticmethod
    def backward(ctx, dout, dlse, dlse23_ext, dmsg_ext):
        *saved, root, gate = ctx.saved_tensors
        epi = (root, gate, ctx.root_sigmoid) if root is not None or gate is not None else None
        grads = order2_backward(saved, None, ctx.cfg, ctx.slots, dout, dlse, dlse23_ext,
                                dmsg_ext, epi)
        droot, dgate = grads[4:] if epi is not None else (None, None)
        return (*grads[:4], droot, dgate, None, None, None, None)


def apply_epilogue(out: Tensor, epilogue) -> Tensor:
    """The modules' epilogue in torch (poly_attention.py:342-351, n_poly_attention.py:315-326),
    where it is not fused into the final pass; the root may be at fewer heads (repeated)."""
    root, gate, root_sigmoid = epilogue
    if root is not None:
        if root.shape[1] != out.shape[1]:
            root = root.repeat_interleave(out.shape[1] // root.shape[1], dim=1)
        out = (root.sigmoid() if root_sigmoid else root) * out
    if gate is not None:
        out = out * gate.sigmoid()
    return out


def _epilogue_fusable(epilogue, q1, heads) -> bool:
    root, gate, _ = epilogue
    shape = (q1.shape[0], heads, q1.shape[2], q1.shape[3])
    for t in (root, gate):
        if t is None:
            continue
        if t.dtype != q1.dtype or t.stride(-1) != 1 or t.device != q1.device:
            return False
        # the kernels move root / gate rows in 8-byte words
        if t.data_ptr() % 16 != 0 or any(st % 4 != 0 for st in t.stride()[:3]):
            return False
    if gate is not None and tuple(gate.shape) != shape:
        return False
    if root is not None:
        r = root.shape
        if (r[0], r[2], r[3]) != (shape[0], shape[2], shape[3]) or heads % r[1] != 0:
            return False
    return True


def _chain_fusable(q_left, q_right, vs, query_mask, key_masks, may_degenerate) -> bool:
    if len(q_left) != 2 or torch.compiler.is_compiling() or may_degenerate:
        return False
    if query_mask is not None or any(m is not None for m in key_masks):
        return False
    q1, q2 = q_left
    if q_right[0] is not q2 or q2.shape[1] != q_right[1].shape[1]:
        return False
    # pass 2 queries at the pass head count (no shared-query backward)
    if q1.shape[1] != max(q1.shape[1], q2.shape[1], vs[0].shape[1]):
        return False
    return _needs_op(q1, q2, q_right[1], vs[0])


def poly_chain(q_left: Sequence[Tensor], q_right: Sequence[Tensor], vs: Sequence[Tensor], *,
               causal: bool, softclamp: Optional[float], scale: float,
               query_mask: Optional[Tensor] = None,
               key_masks: Optional[Sequence[Optional[Tensor]]] = None,
               may_degenerate: bool = False, epilogue=None, qk_norms=None,
               keep_levels: bool = True):
    """Order-n poly attention through HIP passes.

    q_left[l] . q_right[l] are the scores of level l (l = 0 is q1 . q2); vs are the values
    v_3 .. v_{n+1}.  Returns (out, lses, msgs) with lses / msgs ordered deepest level first
    (the reference's cache order, n_poly_attention.py:268-305).  ``epilogue`` = (root, gate,
    root_sigmoid): the modules' root-value / gate epilogue applied to out (fused into the
    final pass on the order-2 chain's path, else in torch).  ``qk_norms`` = the (weight, eps)
    RMSNorms of q1, q2, q3 of an order-2 chain whose inputs are not normalised yet: applied as
    the passes load them (no gradient; the caller checks qk_norms_fusable); with them
    ``keep_levels=False`` says the caller reads only out: lses and msgs come back as None, and
    the one-launch path does not write the inner level.
    """
    n = len(q_left)
    assert len(q_right) == n and len(vs) == n - 1 and n >= 2
    key_masks = list(key_masks) if key_masks is not None else [None] * n
    if epilogue is not None and epilogue[0] is None and epilogue[1] is None:
        epilogue = None
    if qk_norms is not None:
        assert n == 2 and q_right[0] is q_left[1] and query_mask is None and not may_degenerate
        assert all(m is None for m in key_masks)
        fuse = epilogue is not None and _epilogue_fusable(epilogue, q_left[0], q_left[0].shape[1])
        res = order2_forward(q_left[0], q_left[1], q_right[1], vs[0], None, bool(causal),
                             softclamp, float(scale), epilogue if fuse else None, norms=qk_norms,
                             keep_inner=keep_levels)
        out = res[4] if fuse else res[0]
        if epilogue is not None and not fuse:
            out = apply_epilogue(out, epilogue)
        return out, ([res[2]] if keep_levels else None), ([res[3]] if keep_levels else None)
    if _chain_fusable(q_left, q_right, vs, query_mask, key_masks, may_degenerate):
        root = gate = None
        root_sigmoid = False
        fuse = epilogue is not None and _epilogue_fusable(epilogue, q_left[0], q_left[0].shape[1])
        if fuse:
            root, gate, root_sigmoid = epilogue
        out, _, lse23, msg = _Order2Chain.apply(q_left[0], q_left[1], q_right[1], vs[0], root,
                                                gate, bool(causal), float(softclamp or 0.0),
                                                float(scale), bool(root_sigmoid))
        if epilogue is not None and not fuse:
            out = apply_epilogue(out, epilogue)
        return out, [lse23], [msg]
    may_degenerate = may_degenerate or query_mask is not None or any(
        m is not None for m in key_masks)
    lses, msgs = [], []
    msg_next = lse_next = None
    out = None
    for lvl in range(n - 1, -1, -1):
        if lvl == n - 1:
            v, vmul, bias = vs[-1], None, None
        elif lvl == 0:
            v, vmul, bias = msg_next, None, lse_next
        else:
            v, vmul, bias = vs[lvl - 1], msg_next, lse_next
        o, lse = attn_pass(q_left[lvl], q_right[lvl], v, vmul, bias,
                           key_mask=key_masks[lvl],
                           query_mask=query_mask if lvl == 0 else None,
                           causal=causal, softclamp=softclamp, scale=scale,
                           may_degenerate=may_degenerate)
        if lvl > 0:
            msgs.append(o)
            lses.append(lse)
            msg_next, lse_next = o, lse
        else:
            out = o
    if epilogue is not None:
        out = apply_epilogue(out, epilogue)
    return out, lses, msgs


# ---------------------------------------------------------------------------------------
# decode


def poly_decode_step(q_new: Sequence[Tensor], k_caches: Sequence[Tensor],
                     v_caches: Sequence[Tensor], msg_caches: Sequence[Tensor],
                     lse_caches: Sequence[Tensor], *, kv_heads: int, heads: int,
                     softclamp: Optional[float], scale: float, chunk: int = 0,
                     n_dev: Optional[Tensor] = None, noalloc: bool = False,
                     out: Optional[Tensor] = None) -> Tensor:
    """One cached decode step through pa_poly_decode (no autograd).

    Level l (l = 0: q1 . q2) has query q_new[l] [B, h, 1, d] and keys k_caches[l]
    [B, kv_heads, n, d] whose position n-1 already holds the new token.  v_caches are the
    value caches v_3 .. v_{n+1}; msg_caches / lse_caches (deepest first, the reference's
    order) hold n positions whose slot n-1 this call fills.  Returns the output [B, heads, 1, d].

    With ``n_dev`` (a device int32 [1]) the caches are fixed-capacity buffers (n = their
    length is the bound) and the step's n is read on the device, so the launch is the same
    at every position (HIP-graph capturable).

    ``noalloc``: through pa_poly_decode_noalloc, whose split-K records use the library's static
    per-device scratch (no workspace tensor); with ``out`` given as well, the call allocates
    nothing on the device.
    """
    lib = _lib.load()
    order = len(q_new)
    assert len(k_caches) == order and len(v_caches) == order - 1
    assert len(msg_caches) == order - 1 and len(lse_caches) == order - 1
    B, _, n, d = k_caches[0].shape
    dt = q_new[0].dtype
    if out is None:
        out = torch.empty(B, heads, 1, d, dtype=dt, device=q_new[0].device)
    assert out.shape == (B, heads, 1, d) and out.dtype == dt and out.stride(-1) == 1
    D = PaDecode()
    D.batch, D.kv_heads, D.n, D.dim, D.order = B, kv_heads, n, d, order
    D.scale = float(scale)
    D.softclamp = float(softclamp) if softclamp else 0.0
    D.chunk = int(chunk)
    keep = []
    # pa_decode level t = chain level lvl = order - 1 - t (chain level lvl scores
    # q_{lvl+1} . q_{lvl+2}); the msg / lse caches list the deepest level first, so level
    # lvl >= 1 writes cache index order-1-lvl and level lvl <= order-2 reads index order-2-lvl
    for t in range(order):
        lvl = order - 1 - t
        L = D.levels[t]
        q = _inner_contig(q_new[lvl])
        keep.append(q)
        L.q, L.k = _view(q), _view(k_caches[lvl])
        if t == 0:
            L.v = _view(v_caches[-1])
            heads_t = max(q.shape[1], v_caches[-1].shape[1])
        else:
            src = order - 2 - lvl
            if lvl == 0:
                L.v = _view(msg_caches[src])
                heads_t = heads
            else:
                L.v = _view(v_caches[lvl - 1])
                L.vmul = _view(msg_caches[src])
                heads_t = max(q.shape[1], msg_caches[src].shape[1], lse_caches[src].shape[1])
            L.bias = _view(lse_caches[src])
        if lvl == 0:
            L.out = _view(out)
        elif n_dev is not None:  # whole caches: the kernel writes position n_dev - 1
            dst = order - 1 - lvl
            L.out = _view(msg_caches[dst])
            L.lse = _view(lse_caches[dst])
        else:
            dst = order - 1 - lvl
            L.out = _view(msg_caches[dst].narrow(2, n - 1, 1))
            L.lse = _view(lse_caches[dst].narrow(2, n - 1, 1))
        L.heads = heads_t
    if n_dev is not None:
        assert n_dev.dtype == torch.int32 and n_dev.is_cuda and n_dev.numel() == 1
        D.n_dev = n_dev.data_ptr()
    if noalloc:
        with _device(out):
            _lib.check(lib.pa_poly_decode_noalloc(ctypes.byref(D), _stream(out)),
                       "pa_poly_decode_noalloc")
        return out
    ws_bytes = lib.pa_poly_decode_workspace(ctypes.byref(D))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=out.device)
    D.workspace, D.workspace_bytes = ws.data_ptr(), ws_bytes
    with _device(out):
        _lib.check(lib.pa_poly_decode(ctypes.byref(D), _stream(out)), "pa_poly_decode")
    return out


def decode_prologue(items, *, eps: float, angles: Optional[Tensor], n_dev: Tensor,
                    capacity: int, overflow: Optional[Tensor] = None,
                    inv_freq: Optional[Tensor] = None, interp: float = 1.0) -> None:
    """The q norms, rotary embedding and cache appends of one decode step, one launch
    (pa_decode_prologue).  ``items``: (src [B, h, 1, d], norm weight or None, rotate,
    out [B, h, 1, d] or None, cache [B, h, capacity, d] or None) per tensor; ``angles`` is
    the [rot_dim] rotary angle row of the new position (fp32, f16 or bf16), or ``inv_freq``
    (fp32 [rot_dim / 2]) a rotary module's frequencies, whose angles the kernel forms from
    the position (with ``interp`` its interpolate_factor); the cache position, n - 1, is read
    from ``n_dev`` (device int32 [1], the step's n) on the device."""
    lib = _lib.load()
    src0 = items[0][0]
    B, _, _, d = src0.shape
    P = _lib.PaPrologue()
    P.batch, P.dim, P.count, P.capacity = B, d, len(items), int(capacity)
    P.eps = float(eps)
    keep = []
    if angles is not None:
        a = angles.detach()
        if a.dtype not in DTYPE_CODE:
            a = a.to(torch.float32)
        a = a.contiguous()
        keep.append(a)
        P.angles, P.angles_dtype, P.rot_dim = a.data_ptr(), DTYPE_CODE[a.dtype], a.numel()
    elif inv_freq is not None:
        f = inv_freq.detach().to(torch.float32).contiguous()
        keep.append(f)
        P.inv_freq, P.rot_dim, P.interp = f.data_ptr(), 2 * f.numel(), float(interp)
    assert n_dev.dtype == torch.int32 and n_dev.is_cuda and n_dev.numel() == 1
    P.n_dev = n_dev.data_ptr()
    if overflow is not None:
        assert overflow.dtype == torch.int32 and overflow.is_cuda and overflow.numel() >= 1
        P.overflow = overflow.data_ptr()
    for k, (src, w, rotate, out, cache) in enumerate(items):
        it = P.items[k]
        it.src = _view(src)
        if w is not None:
            w = w.detach().contiguous()
            keep.append(w)
            it.norm_weight, it.weight_dtype = w.data_ptr(), DTYPE_CODE[w.dtype]
        it.rotate = 1 if rotate else 0
        if out is not None:
            it.out = _view(out)
        if cache is not None:
            it.cache = _view(cache)
    with _device(src0):
        _lib.check(lib.pa_decode_prologue(ctypes.byref(P), _stream(src0)), "pa_decode_prologue")
