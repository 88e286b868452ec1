"""ctypes binding of libpolyattn.so (declared in include/polyattn.h).

The structures below mirror the C structs field for field; ``pa_struct_size`` lets the
tests check the layouts against the compiled library.  Loading never touches the GPU.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libpolyattn.so"

PA_ABI_VERSION = 8
PA_MAX_ORDER = 8

PA_OK = 0
PA_EINVAL = -1
PA_EUNSUPPORTED = -2
PA_EHIP = -3
PA_EWORKSPACE = -4
PA_ESCRATCH = -5

# the static split-K scratch of pa_poly_decode_noalloc, bytes per device
PA_DECODE_SCRATCH_BYTES = 16 << 20

PA_F32, PA_F16, PA_BF16 = 0, 1, 2
PA_FLAG_MAY_DEGENERATE = 1
PA_FLAG_DISCARD_OUT = 4
PA_EPI_ROOT_SIGMOID = 1
PA_NORM_Q = 1
PA_NORM_K = 2
PA_ACC_DQ, PA_ACC_DK, PA_ACC_DV, PA_ACC_DVMUL, PA_ACC_DBIAS = 1, 2, 4, 8, 16
PA_RMS_MAX_ITEMS = 4

DTYPE_CODE = {torch.float32: PA_F32, torch.float16: PA_F16, torch.bfloat16: PA_BF16}

# every symbol include/polyattn.h declares
EXPORTED_SYMBOLS = (
    "pa_abi_version",
    "pa_strerror",
    "pa_last_hip_error",
    "pa_struct_size",
    "pa_profile_start",
    "pa_profile_stop",
    "pa_measure_clock",
    "pa_attn_pass_fwd",
    "pa_attn_pass_fwd_workspace",
    "pa_attn_pass_bwd_workspace",
    "pa_attn_pass_bwd",
    "pa_poly_order2_fwd",
    "pa_poly_decode_workspace",
    "pa_poly_decode",
    "pa_poly_decode_noalloc",
    "pa_decode_prologue",
    "pa_rmsnorm_fwd",
    "pa_rmsnorm_fwd_many",
    "pa_rmsnorm_bwd_workspace",
    "pa_rmsnorm_bwd",
    "pa_linear_small",
)


class PaView(ctypes.Structure):
    _fields_ = [
        ("ptr", c_void_p),
        ("sb", c_int64),
        ("sh", c_int64),
        ("sn", c_int64),
        ("heads", c_int32),
        ("dtype", c_int32),
    ]


class PaMask(ctypes.Structure):
    _fields_ = [("ptr", c_void_p), ("sb", c_int64), ("sn", c_int64)]


class PaEpilogue(ctypes.Structure):
    _fields_ = [("root", PaView), ("gate", PaView), ("y", PaView), ("flags", c_int32)]


class PaQkNorm(ctypes.Structure):
    _fields_ = [("q_weight", c_void_p), ("k_weight", c_void_p), ("q_eps", c_float),
                ("k_eps", c_float), ("flags", c_int32)]


class PaPass(ctypes.Structure):
    _fields_ = [
        ("batch", c_int32),
        ("heads", c_int32),
        ("nq", c_int32),
        ("nk", c_int32),
        ("dim", c_int32),
        ("scale", c_float),
        ("softclamp", c_float),
        ("causal", c_int32),
        ("flags", c_int32),
        ("q", PaView),
        ("k", PaView),
        ("v", PaView),
        ("vmul", PaView),
        ("bias", PaView),
        ("key_mask", PaMask),
        ("query_mask", PaMask),
        ("out", PaView),
        ("lse", PaView),
        ("epi", c_void_p),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("norm", c_void_p),
    ]


class PaPassGrad(ctypes.Structure):
    _fields_ = [
        ("fwd", PaPass),
        ("dout", PaView),
        ("dlse", PaView),
        ("dq", PaView),
        ("dk", PaView),
        ("dv", PaView),
        ("dvmul", PaView),
        ("dbias", PaView),
        ("accumulate", c_int32),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("droot", PaView),
        ("dgate", PaView),
    ]


class PaDecodeLevel(ctypes.Structure):
    _fields_ = [
        ("q", PaView),
        ("k", PaView),
        ("v", PaView),
        ("vmul", PaView),
        ("bias", PaView),
        ("out", PaView),
        ("lse", PaView),
        ("heads", c_int32),
    ]


class PaDecode(ctypes.Structure):
    _fields_ = [
        ("batch", c_int32),
        ("kv_heads", c_int32),
        ("n", c_int32),
        ("dim", c_int32),
        ("order", c_int32),
        ("scale", c_float),
        ("softclamp", c_float),
        ("chunk", c_int32),
        ("levels", PaDecodeLevel * PA_MAX_ORDER),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("n_dev", c_void_p),
    ]


class PaPrologueItem(ctypes.Structure):
    _fields_ = [
        ("src", PaView),
        ("norm_weight", c_void_p),
        ("weight_dtype", c_int32),
        ("rotate", c_int32),
        ("out", PaView),
        ("cache", PaView),
    ]


class PaPrologue(ctypes.Structure):
    _fields_ = [
        ("batch", c_int32),
        ("dim", c_int32),
        ("count", c_int32),
        ("capacity", c_int32),
        ("eps", c_float),
        ("angles", c_void_p),
        ("angles_dtype", c_int32),
        ("rot_dim", c_int32),
        ("pos", c_int32),
        ("n_dev", c_void_p),
        ("overflow", c_void_p),
        ("inv_freq", c_void_p),
        ("interp", c_float),
        ("items", PaPrologueItem * (2 * PA_MAX_ORDER)),
    ]


class PaRmsNorm(ctypes.Structure):
    _fields_ = [
        ("batch", c_int32),
        ("heads", c_int32),
        ("n", c_int32),
        ("dim", c_int32),
        ("eps", c_float),
        ("x", PaView),
        ("weight", c_void_p),
        ("weight_dtype", c_int32),
        ("y", PaView),
        ("rstd", c_void_p),
        ("dy", PaView),
        ("dx", PaView),
        ("dweight", c_void_p),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("angles", c_void_p),
        ("angles_dtype", c_int32),
        ("rot_dim", c_int32),
        ("angles_stride", c_int64),
    ]


PA_LINEAR_MAX_OUT = 4
PA_ACT_NONE, PA_ACT_GELU = 0, 1


class PaLinearOut(ctypes.Structure):
    _fields_ = [
        ("w", c_void_p),
        ("w_stride", c_int64),
        ("out_features", c_int32),
        ("activation", c_int32),
        ("bias", c_void_p),
        ("residual", c_void_p),
        ("residual_stride", c_int64),
        ("y", c_void_p),
        ("y_stride", c_int64),
    ]


class PaLinear(ctypes.Structure):
    _fields_ = [
        ("rows", c_int32),
        ("in_features", c_int32),
        ("dtype", c_int32),
        ("count", c_int32),
        ("x", c_void_p),
        ("x_stride", c_int64),
        ("x_add", c_void_p),
        ("x_add_stride", c_int64),
        ("x_sum", c_void_p),
        ("x_sum_stride", c_int64),
        ("norm", c_int32),
        ("norm_dtype", c_int32),
        ("norm_weight", c_void_p),
        ("norm_eps", c_float),
        ("out", PaLinearOut * PA_LINEAR_MAX_OUT),
    ]


class PaKernelTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("launches", c_int64), ("total_ms", ctypes.c_double)]


STRUCTS = (PaView, PaMask, PaPass, PaPassGrad, PaDecodeLevel, PaDecode, PaPrologueItem,
           PaPrologue, PaRmsNorm, PaLinear, PaLinearOut, PaEpilogue, PaQkNorm)


class PolyAttnError(RuntimeError):
    """A libpolyattn call returned a failure status."""

    def __init__(self, status: int, what: str, lib=None):
        msg = f"{what}: libpolyattn status {status}"
        if lib is not None:
            msg += f" ({lib.pa_strerror(status).decode()})"
            if status == PA_EHIP:
                msg += f", hipError {lib.pa_last_hip_error()}"
        super().__init__(msg)
        self.status = status


_LIB = None
_LOAD_ERROR: Exception | None = None


def _configure(lib) -> None:
    lib.pa_abi_version.restype = c_int
    lib.pa_strerror.restype = ctypes.c_char_p
    lib.pa_strerror.argtypes = [c_int]
    lib.pa_last_hip_error.restype = c_int
    lib.pa_struct_size.restype = c_size_t
    lib.pa_struct_size.argtypes = [c_int]
    lib.pa_profile_start.restype = c_int
    lib.pa_profile_stop.restype = c_int
    lib.pa_profile_stop.argtypes = [ctypes.POINTER(PaKernelTime), c_int, ctypes.POINTER(c_int)]
    lib.pa_measure_clock.restype = c_int
    lib.pa_measure_clock.argtypes = [ctypes.POINTER(ctypes.c_double), c_void_p]
    lib.pa_attn_pass_fwd.restype = c_int
    lib.pa_attn_pass_fwd.argtypes = [ctypes.POINTER(PaPass), c_void_p]
    lib.pa_attn_pass_fwd_workspace.restype = c_size_t
    lib.pa_attn_pass_fwd_workspace.argtypes = [ctypes.POINTER(PaPass)]
    lib.pa_attn_pass_bwd_workspace.restype = c_size_t
    lib.pa_attn_pass_bwd_workspace.argtypes = [ctypes.POINTER(PaPassGrad)]
    lib.pa_attn_pass_bwd.restype = c_int
    lib.pa_attn_pass_bwd.argtypes = [ctypes.POINTER(PaPassGrad), c_void_p]
    lib.pa_poly_order2_fwd.restype = c_int
    lib.pa_poly_order2_fwd.argtypes = [ctypes.POINTER(PaPass), ctypes.POINTER(PaPass), c_void_p]
    lib.pa_poly_decode_workspace.restype = c_size_t
    lib.pa_poly_decode_workspace.argtypes = [ctypes.POINTER(PaDecode)]
    lib.pa_poly_decode.restype = c_int
    lib.pa_poly_decode.argtypes = [ctypes.POINTER(PaDecode), c_void_p]
    lib.pa_poly_decode_noalloc.restype = c_int
    lib.pa_poly_decode_noalloc.argtypes = [ctypes.POINTER(PaDecode), c_void_p]
    lib.pa_decode_prologue.restype = c_int
    lib.pa_decode_prologue.argtypes = [ctypes.POINTER(PaPrologue), c_void_p]
    lib.pa_rmsnorm_fwd.restype = c_int
    lib.pa_rmsnorm_fwd.argtypes = [ctypes.POINTER(PaRmsNorm), c_void_p]
    lib.pa_rmsnorm_fwd_many.restype = c_int
    lib.pa_rmsnorm_fwd_many.argtypes = [ctypes.POINTER(PaRmsNorm), c_int, c_void_p]
    lib.pa_rmsnorm_bwd_workspace.restype = c_size_t
    lib.pa_rmsnorm_bwd_workspace.argtypes = [ctypes.POINTER(PaRmsNorm)]
    lib.pa_rmsnorm_bwd.restype = c_int
    lib.pa_rmsnorm_bwd.argtypes = [ctypes.POINTER(PaRmsNorm), c_void_p]
    lib.pa_linear_small.restype = c_int
    lib.pa_linear_small.argtypes = [ctypes.POINTER(PaLinear), c_void_p]


def load(path: str | os.PathLike | None = None):
    """Load libpolyattn.so (once); raises when it is missing or its ABI does not match."""
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "or `python poly-attention_amd/poly_attention/_build.py`"
        )
    lib = ctypes.CDLL(str(p))
    _configure(lib)
    ver = lib.pa_abi_version()
    if ver != PA_ABI_VERSION:
        raise RuntimeError(f"libpolyattn ABI {ver} != expected {PA_ABI_VERSION}")
    for i, st in enumerate(STRUCTS):
        if lib.pa_struct_size(i) != ctypes.sizeof(st):
            raise RuntimeError(
                f"libpolyattn struct {st.__name__}: C size {lib.pa_struct_size(i)} "
                f"!= ctypes size {ctypes.sizeof(st)}"
            )
    _LIB = lib
    return lib


def available() -> bool:
    """True when libpolyattn.so loads (does not initialise the GPU)."""
    global _LOAD_ERROR
    try:
        load()
        return True
    except Exception as e:  # noqa: BLE001 - reported through load_error()
        _LOAD_ERROR = e
        return False


def load_error() -> Exception | None:
    return _LOAD_ERROR


def check(status: int, what: str) -> None:
    if status != PA_OK:
        raise PolyAttnError(status, what, _LIB)


class KernelProfile:
    """Context manager timing every libpolyattn kernel launched inside it (HIP events on the
    launch stream).  After exit, ``times`` maps kernel family -> (launches, total_ms)."""

    def __init__(self):
        self.times: dict[str, tuple[int, float]] = {}

    def __enter__(self):
        check(load().pa_profile_start(), "pa_profile_start")
        return self

    def __exit__(self, *exc):
        buf = (PaKernelTime * 64)()
        n = c_int(0)
        check(load().pa_profile_stop(buf, 64, ctypes.byref(n)), "pa_profile_stop")
        self.times = {buf[i].name.decode(): (buf[i].launches, buf[i].total_ms)
                      for i in range(n.value)}
        return False


def measure_clock(device=None) -> float:
    """The GPU's shader clock in GHz under a short all-CU MFMA load on the current stream of
    ``device`` (libpolyattn pa_measure_clock): s_memtime cycles per 100 MHz s_memrealtime tick."""
    ghz = ctypes.c_double(0.0)
    stream = torch.cuda.current_stream(device).cuda_stream
    check(load().pa_measure_clock(ctypes.byref(ghz), c_void_p(stream)), "pa_measure_clock")
    return ghz.value
