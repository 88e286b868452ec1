"""GPU: pa_poly_decode_noalloc (the decode step on the library's static per-device scratch)
against pa_poly_decode (caller workspace), both through the C ABI.

Two calls in a row, the second with a smaller input (fewer batch rows, heads and cached
positions), each compared with the workspace entry point on the same inputs: the kernels
and their chunking are the same, so the outputs and the msg / lse slots the step writes are
bit-identical.  A request larger than the static scratch is refused with PA_ESCRATCH before
anything launches, and a call with a preallocated output allocates no device memory.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda")


def _case(d, B, Hq, G, n_old, dh, seed):
    gen = torch.Generator(device=d).manual_seed(seed)

    def rnd(*shape):
        return torch.randn(*shape, generator=gen, device=d).to(torch.bfloat16)

    n = n_old + 1
    q2c, q3c, v3c = rnd(B, G, n, dh), rnd(B, G, n, dh), rnd(B, G, n, dh)
    msg = rnd(B, Hq, n, dh)
    lse = torch.log(torch.arange(1, n + 1, device=d, dtype=torch.float32)) + \
        torch.randn(B, Hq, n, generator=gen, device=d)
    q1 = rnd(B, Hq, 1, dh)
    q2n = q2c[:, :, -1:].contiguous()
    return q1, q2n, q2c, q3c, v3c, msg, lse


@pytest.mark.parametrize("order_of_calls", ("large_then_small",))
def test_noalloc_decode_equals_workspace_decode(order_of_calls):
    from poly_attention import _lib, _ops

    d = dev()
    _lib.load()
    for B, Hq, G, n_old, dh, seed in ((8, 16, 4, 3000, 128, 1), (2, 8, 2, 300, 64, 2)):
        q1, q2n, q2c, q3c, v3c, msg, lse = _case(d, B, Hq, G, n_old, dh, seed)
        kw = dict(kv_heads=G, heads=Hq, softclamp=None, scale=dh ** -0.5)
        msg_a, lse_a = msg.clone(), lse.clone()
        ref = _ops.poly_decode_step([q1, q2n], [q2c, q3c], [v3c], [msg_a], [lse_a], **kw)
        msg_b, lse_b = msg.clone(), lse.clone()
        out = torch.empty_like(ref)
        torch.cuda.synchronize()
        before = torch.cuda.memory_stats(d)["allocation.all.allocated"]
        got = _ops.poly_decode_step([q1, q2n], [q2c, q3c], [v3c], [msg_b], [lse_b], noalloc=True,
                                    out=out, **kw)
        torch.cuda.synchronize()
        after = torch.cuda.memory_stats(d)["allocation.all.allocated"]
        assert after == before, f"the no-alloc call made {after - before} torch allocations"
        assert got is out
        what = f"B={B} Hq={Hq} G={G} n={n_old + 1} d={dh}"
        assert torch.equal(got, ref), f"{what}: output differs from pa_poly_decode"
        assert torch.equal(msg_b, msg_a), f"{what}: msg cache differs"
        assert torch.equal(lse_b, lse_a), f"{what}: lse cache differs"
        print(f"[no-alloc] {what}: bit-identical to pa_poly_decode", flush=True)


def test_noalloc_decode_refuses_requests_beyond_the_scratch():
    from poly_attention import _lib

    dev()
    lib = _lib.load()
    D = _lib.PaDecode()
    # no tensors at all: a request that passed the size check would still stop at the
    # missing pointers (PA_EINVAL) before any launch
    D.batch, D.kv_heads, D.n, D.dim, D.order = 256, 8, 1 << 20, 128, 2
    D.scale = 128 ** -0.5
    for t in range(2):
        D.levels[t].heads = 32
    need = lib.pa_poly_decode_workspace(ctypes.byref(D))
    assert need > _lib.PA_DECODE_SCRATCH_BYTES
    st = lib.pa_poly_decode_noalloc(ctypes.byref(D), None)
    assert st == _lib.PA_ESCRATCH, st
    assert b"static" in lib.pa_strerror(st)
