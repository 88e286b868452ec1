// pa_order.h -- the workgroup -> (unit, block) order of the MFMA pass kernels: which
// (batch, head) unit and which block of it a workgroup runs.  Plain integer arithmetic with
// no HIP dependency, so that a host program can check it (tests/test_order.py).
#pragma once

#if defined(__HIPCC__)
#define PA_HD __host__ __device__ __forceinline__
#else
#define PA_HD inline
#endif

namespace pa {

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).  Map the
// hardware id to a logical id so that every XCD runs a contiguous range of logical ids --
// consecutive logical ids share a head, so its K/V stay in that XCD's L2.
constexpr int kNumXcd = 8;
PA_HD int xcd_remap(int bid, int nblocks) {
    const int per = nblocks / kNumXcd, rem = nblocks % kNumXcd;
    const int x = bid % kNumXcd, slot = bid / kNumXcd;
    return (x < rem) ? x * (per + 1) + slot : rem * (per + 1) + (x - rem) * per + slot;
}

// The unit (batch-major, head-minor) of the j-th of the nu units that XCD x runs.  Where the
// heads split evenly over the XCDs in runs of whole groups (`group` consecutive heads share
// their K / V: GQA), each XCD takes heads [x * hpx, (x + 1) * hpx) of every batch row, so that
// work that differs by batch row (padding masks) is spread over all XCDs; otherwise the XCD's
// units are consecutive.
PA_HD int xcd_unit(int x, int j, int nu, int heads, int group) {
    if (heads % (kNumXcd * group) == 0) {
        const int hpx = heads / kNumXcd;
        return (j / hpx) * heads + x * hpx + j % hpx;
    }
    return x * nu + j;
}

// (unit, rank) of workgroup bid of a grid of nblocks = units x nblk workgroups.
// heavy (causal grids, work per block falling with its rank): every XCD runs whole units and
// dispatches the heaviest blocks of all its units first, so the light blocks fill the end of
// the kernel.  Otherwise each unit's blocks are consecutive on one XCD.  When the XCD ranges
// do not hold whole units, the order is unit by unit.  heads: units per batch row; group: see
// xcd_unit.
PA_HD void block_map(int bid, int nblocks, int nblk, int heads, int group, bool heavy,
                     int& unit, int& rank) {
    const int lid = xcd_remap(bid, nblocks);
    const int per = nblocks / kNumXcd;
    if (nblocks % kNumXcd == 0 && per % nblk == 0) {
        const int x = lid / per, k = lid % per, nu = per / nblk;
        if (heavy) {
            unit = xcd_unit(x, k % nu, nu, heads, group);
            rank = k / nu;
        } else {
            unit = xcd_unit(x, k / nblk, nu, heads, group);
            rank = k % nblk;
        }
    } else {
        unit = lid / nblk;
        rank = lid % nblk;
    }
}

}  // namespace pa
