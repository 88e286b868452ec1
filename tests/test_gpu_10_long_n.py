"""GPU: long sequences, as the reference's verify_memory_efficient.py:14-43 runs them -- fp16
causal flash_poly_attention on (1, 4, N, 64) for N = 8k, 16k, 32k and 64k, forward and backward.

* Memory: the peak device memory each step adds over its inputs is printed and must stay
  linear in N (at most 16 input-sized tensors; an N x N score matrix of one head alone would be
  N / 4 of them), and peak(64k) / peak(8k) must stay near 8.
* Parity: out and dq1 of six query rows of one head (first, last, middle and near the ends)
  against the chunked oracle (oracle.order2_rows: pass 1 over every row in chunks, pass 2 for
  the chosen rows), within the fp16 bound of tests/parity.py.
* The same in bf16 at N = 16384 with a key-padding mask (left- and right-padded batch rows).
"""

import time

import pytest
import torch

import oracle.poly_oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu

B, H, D = 1, 4, 64
LENGTHS = (8192, 16384, 32768, 65536)


def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda")


def test_long_sequences_fp16_causal_memory_and_rows():
    from poly_attention.flash_poly_attention import flash_poly_attention

    d = dev()
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    peaks = {}
    for n in LENGTHS:
        gen = torch.Generator().manual_seed(n)
        ts = [torch.randn(B, H, n, D, generator=gen).to(torch.float16) for _ in range(4)]
        dout = torch.randn(B, H, n, D, generator=gen).to(torch.float16)
        g = [t.to(d).requires_grad_() for t in ts]
        dout_d = dout.to(d)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        t0 = time.perf_counter()
        out = flash_poly_attention(*g, is_causal=True)
        out.backward(dout_d)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3
        unit = B * H * n * D * 2  # one fp16 input tensor
        peak = torch.cuda.max_memory_allocated() - base
        peaks[n] = peak
        print(f"[long] N={n}: fwd+bwd {ms:.1f} ms (first call), peak over inputs "
              f"{peak / 2**20:.1f} MiB = {peak / unit:.2f} input tensors", flush=True)
        assert peak <= 16 * unit, f"N={n}: peak {peak} bytes is not linear in N"

        h = 0
        rows = torch.tensor([0, 1, 777, n // 2, n - 2, n - 1])
        sl = [t[0, h].float() for t in ts]
        ref_out, _, _, ref_dq1 = O.order2_rows(*sl, rows, dout_rows=dout[0, h, rows].float(),
                                               causal=True, chunk=2048)
        what = f"long N={n} head {h} rows {rows.tolist()}"
        assert_parity(out[0, h, rows], ref_out, torch.float16, f"{what} out")
        assert_parity(g[0].grad[0, h, rows], ref_dq1, torch.float16, f"{what} dq1", grad=True)
        del out, g, dout_d
    ratio = peaks[LENGTHS[-1]] / peaks[LENGTHS[0]]
    print(f"[long] peak(64k) / peak(8k) = {ratio:.2f}", flush=True)
    assert ratio <= 8 * 1.1


def test_long_sequence_padding_masks_bf16_causal_rows():
    """bf16 causal flash_poly_attention with a key-padding mask (the op's key mask of both
    passes, flash_poly_attention.py:109-112) at N = 16384, B = 2, 8 heads: batch 0 right-padded
    (keys from 12000 on masked), batch 1 left-padded (keys below 5000 masked).  The grid takes
    the order that gives every XCD heads of both batch rows, and the forward and dQ loops run
    over each row's live key range only.  out and dq1 of six query rows of two heads in each
    batch row (rows that keep a key) against the chunked oracle with the same mask."""
    from poly_attention.flash_poly_attention import flash_poly_attention

    d = dev()
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    Bm, Hm, n = 2, 8, 16384
    gen = torch.Generator().manual_seed(7)
    ts = [torch.randn(Bm, Hm, n, D, generator=gen).to(torch.bfloat16) for _ in range(4)]
    dout = torch.randn(Bm, Hm, n, D, generator=gen).to(torch.bfloat16)
    keep = torch.ones(Bm, n, dtype=torch.bool)
    keep[0, 12000:] = False
    keep[1, :5000] = False
    g = [t.to(d).requires_grad_() for t in ts]
    out = flash_poly_attention(*g, mask=keep.to(d), is_causal=True)
    out.backward(dout.to(d))
    torch.cuda.synchronize()
    row_sets = {0: [0, 1, 777, 11999, 12000, n - 1], 1: [5000, 5001, 8192, 12000, n - 2, n - 1]}
    for b, rows in row_sets.items():
        rows = torch.tensor(rows)
        for h in (0, 5):
            sl = [t[b, h].float() for t in ts]
            ref_out, _, _, ref_dq1 = O.order2_rows(*sl, rows, dout_rows=dout[b, h, rows].float(),
                                                   causal=True, chunk=2048, key_keep=keep[b])
            what = f"long padded N={n} batch {b} head {h} rows {rows.tolist()}"
            assert_parity(out[b, h, rows], ref_out, torch.bfloat16, f"{what} out")
            assert_parity(g[0].grad[b, h, rows], ref_dq1, torch.bfloat16, f"{what} dq1",
                          grad=True)
