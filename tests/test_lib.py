"""libpolyattn.so: it loads, exports every symbol include/polyattn.h declares, its struct
layouts match the ctypes mirror, and invalid arguments are rejected before any launch (so
these run without a GPU)."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from poly_attention import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "polyattn.h").read_text()
    return sorted(set(re.findall(r"\b(pa_[a-z_0-9]+)\s*\(", text)))


def test_loads_and_version():
    lib = _lib.load()
    assert lib.pa_abi_version() == _lib.PA_ABI_VERSION


def test_exports_every_declared_symbol():
    declared = declared_functions()
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS), declared
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing


def test_struct_layouts_match():
    lib = _lib.load()
    for i, st in enumerate(_lib.STRUCTS):
        assert lib.pa_struct_size(i) == ctypes.sizeof(st), st.__name__
    assert lib.pa_struct_size(99) == 0


def test_strerror():
    lib = _lib.load()
    for code in (0, -1, -2, -3, -4, -99):
        assert isinstance(lib.pa_strerror(code), bytes)


def _valid_pass():
    p = _lib.PaPass()
    p.batch, p.heads, p.nq, p.nk, p.dim = 1, 4, 8, 8, 64
    p.scale, p.softclamp, p.causal = 0.125, 0.0, 1
    fake = 0x1000  # never dereferenced: every case below fails validation first
    for name in ("q", "k", "v", "out"):
        v = getattr(p, name)
        v.ptr, v.sb, v.sh, v.sn, v.heads, v.dtype = fake, 2048, 512, 64, 4, _lib.PA_BF16
    p.lse.ptr, p.lse.sb, p.lse.sh, p.lse.sn, p.lse.heads = fake, 32, 8, 1, 4
    p.lse.dtype = _lib.PA_F32
    return p


@pytest.mark.parametrize("breakage", [
    "null", "batch0", "dim_too_big", "heads_not_divisible", "dtype_mismatch", "lse_dtype",
    "missing_k", "out_heads",
])
def test_pass_fwd_rejects_invalid_arguments(breakage):
    lib = _lib.load()
    if breakage == "null":
        assert lib.pa_attn_pass_fwd(None, None) == _lib.PA_EINVAL
        return
    p = _valid_pass()
    want = _lib.PA_EINVAL
    if breakage == "batch0":
        p.batch = 0
    elif breakage == "dim_too_big":
        p.dim = 512
        want = _lib.PA_EUNSUPPORTED
    elif breakage == "heads_not_divisible":
        p.k.heads = 3
    elif breakage == "dtype_mismatch":
        p.v.dtype = _lib.PA_F16
    elif breakage == "lse_dtype":
        p.lse.dtype = _lib.PA_BF16
    elif breakage == "missing_k":
        p.k.ptr = None
    elif breakage == "out_heads":
        p.out.heads = 2
    assert lib.pa_attn_pass_fwd(ctypes.byref(p), None) == want


@pytest.mark.parametrize("breakage", ["null", "keys", "values", "bias", "nk"])
def test_order2_fwd_rejects_passes_that_do_not_chain(breakage):
    """pa_poly_order2_fwd takes the second pass's keys, values and key bias to be the first
    pass's queries, output and lse; anything else is refused before a launch."""
    lib = _lib.load()
    if breakage == "null":
        assert lib.pa_poly_order2_fwd(None, None, None) == _lib.PA_EINVAL
        return
    a, c = _valid_pass(), _valid_pass()
    c.k, c.v, c.bias, c.nk = a.q, a.out, a.lse, a.nq
    if breakage == "keys":
        c.k.ptr = c.k.ptr + 4096
    elif breakage == "values":
        c.v.sn = 128
    elif breakage == "bias":
        c.bias = _lib.PaView()
    elif breakage == "nk":
        c.nk = a.nq + 1
    assert lib.pa_poly_order2_fwd(ctypes.byref(a), ctypes.byref(c), None) == _lib.PA_EINVAL


def test_pass_bwd_rejects_missing_workspace():
    lib = _lib.load()
    g = _lib.PaPassGrad()
    g.fwd = _valid_pass()
    for name in ("dout", "dq", "dk", "dv"):
        setattr(g, name, getattr(g.fwd, "q"))
    assert lib.pa_attn_pass_bwd_workspace(ctypes.byref(g)) > 0
    g.workspace, g.workspace_bytes = None, 0
    assert lib.pa_attn_pass_bwd(ctypes.byref(g), None) == _lib.PA_EWORKSPACE


def test_decode_rejects_invalid_order():
    lib = _lib.load()
    d = _lib.PaDecode()
    d.order = 1
    assert lib.pa_poly_decode(ctypes.byref(d), None) == _lib.PA_EINVAL
    d.order = 2
    d.batch = d.kv_heads = d.n = d.dim = 1
    assert lib.pa_poly_decode(ctypes.byref(d), None) == _lib.PA_EINVAL  # no level tensors


def test_prologue_rejects_invalid():
    lib = _lib.load()
    p = _lib.PaPrologue()
    assert lib.pa_decode_prologue(ctypes.byref(p), None) == _lib.PA_EINVAL  # count 0
    p.batch, p.dim, p.count = 1, 64, 1
    assert lib.pa_decode_prologue(ctypes.byref(p), None) == _lib.PA_EINVAL  # no source
    it = p.items[0]
    it.src.ptr, it.src.sb, it.src.sh, it.src.sn = 0x1000, 64, 64, 64
    it.src.heads, it.src.dtype = 1, _lib.PA_BF16
    p.angles, p.rot_dim = 0x2000, 3
    assert lib.pa_decode_prologue(ctypes.byref(p), None) == _lib.PA_EINVAL  # odd rot_dim
    p.rot_dim, p.dim = 64, 512
    assert lib.pa_decode_prologue(ctypes.byref(p), None) == _lib.PA_EUNSUPPORTED
    p.dim = 64
    p.angles_dtype = 9
    assert lib.pa_decode_prologue(ctypes.byref(p), None) == _lib.PA_EINVAL  # angle dtype
    p.angles_dtype = _lib.PA_BF16
    it.cache.ptr, it.cache.heads, it.cache.dtype = 0x3000, 1, _lib.PA_BF16
    assert lib.pa_decode_prologue(ctypes.byref(p), None) == _lib.PA_EINVAL  # capacity 0


def test_rmsnorm_rejects_invalid():
    lib = _lib.load()
    r = _lib.PaRmsNorm()
    assert lib.pa_rmsnorm_fwd(ctypes.byref(r), None) == _lib.PA_EINVAL
    r.batch = r.heads = r.n = 1
    r.dim = 60  # not a multiple of 8 elements
    r.x.ptr, r.x.heads, r.x.dtype = 0x1000, 1, _lib.PA_BF16
    assert lib.pa_rmsnorm_fwd(ctypes.byref(r), None) == _lib.PA_EUNSUPPORTED
    r.dim = 64
    r.x.sb = r.x.sh = r.x.sn = 64
    assert lib.pa_rmsnorm_fwd(ctypes.byref(r), None) == _lib.PA_EINVAL  # no output view
    r.y = r.x
    r.dy = r.dx = r.x
    # rstd is optional in the forward (not written without it), required by the backward
    assert lib.pa_rmsnorm_bwd(ctypes.byref(r), None) == _lib.PA_EINVAL  # no rstd
    r.dy = r.dx = _lib.PaView()
    r.y, r.rstd = r.x, 0x2000
    r.angles, r.rot_dim, r.angles_dtype = 0x4000, 63, _lib.PA_F32
    assert lib.pa_rmsnorm_fwd(ctypes.byref(r), None) == _lib.PA_EINVAL  # odd rot_dim
    r.rot_dim, r.angles_dtype = 64, 9
    assert lib.pa_rmsnorm_fwd(ctypes.byref(r), None) == _lib.PA_EINVAL  # angle dtype
    r.angles, r.rot_dim = None, 0
    r.dy = r.dx = r.x
    r.rstd, r.dweight = 0x2000, 0x3000
    assert lib.pa_rmsnorm_bwd_workspace(ctypes.byref(r)) > 0
    assert lib.pa_rmsnorm_bwd(ctypes.byref(r), None) == _lib.PA_EWORKSPACE


def test_linear_small_rejects_invalid():
    lib = _lib.load()
    lin = _lib.PaLinear()
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EINVAL  # no rows
    lin.rows, lin.in_features, lin.dtype, lin.count = 8, 1024, _lib.PA_BF16, 1
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EINVAL  # no x
    lin.x, lin.x_stride = 0x1000, 1024
    o = lin.out[0]
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EINVAL  # no w / y
    o.w, o.w_stride, o.out_features, o.y, o.y_stride = 0x2000, 1024, 1024, 0x3000, 1024
    lin.count = 5  # more outputs than PA_LINEAR_MAX_OUT
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EINVAL
    lin.count, lin.rows = 1, 17  # more rows than a decode batch
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EUNSUPPORTED
    lin.rows, lin.in_features = 8, 1020  # not whole 16-byte chunks
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EUNSUPPORTED
    lin.in_features, lin.x = 1024, 0x1008  # misaligned x
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EUNSUPPORTED
    lin.x, lin.in_features, lin.x_stride, o.w_stride = 0x1000, 8192, 8192, 8192
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EUNSUPPORTED  # 128 KiB of x
    lin.in_features, lin.x_stride, o.w_stride = 1024, 1024, 512
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EINVAL  # w rows overlap
    o.w_stride, o.activation = 1024, 7
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EINVAL  # unknown activation
    o.activation, lin.x_sum, lin.x_sum_stride = _lib.PA_ACT_GELU, 0x5000, 1024
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EINVAL  # x_sum without x_add
    lin.x_sum, lin.norm, lin.norm_weight, lin.norm_dtype = None, 1, 0x6000, 5
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EINVAL  # norm weight dtype
    lin.norm, lin.dtype = 0, 7
    assert lib.pa_linear_small(ctypes.byref(lin), None) == _lib.PA_EINVAL
