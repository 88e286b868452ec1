// pa_simt.hip -- generic attention-pass kernels: one lane per query (or key) row.
//
// These kernels implement every feature of a pass (any head dim up to 256, masks with the
// reference's finite-fill semantics, bias classes, value multiplier, GQA head mapping) in
// fp32 arithmetic.  They run whenever the MFMA kernels do not cover a request (fp32 data,
// head dims other than 64/128).  The same file holds the kernels that finish the fully-masked
// rows of the MFMA forward and backward kernels (k_fwd_fixup, the k_fix_* kernels).
#include <algorithm>

#include "pa_common.h"
#include "pa_launch.h"
#include "pa_mfma.h"

namespace pa {

constexpr int kSimtRows = 64;  // rows per workgroup: one wave, one row per lane
constexpr int kSimtKT = 32;    // keys (or queries) per LDS tile

// Stage keys [j0, j0 + kSimtKT) of K and of the effective value (v * vmul rounded to T) in
// LDS as fp32, with each key's raw bias and key-mask bit.
template <typename T, int D>
__device__ void simt_stage_keys(const PassDev& P, int b, int h, int j0, float (*sK)[D],
                                float (*sV)[D], float* sB, uint8_t* sKM) {
    for (int e = threadIdx.x; e < kSimtKT * D; e += blockDim.x) {
        const int jj = e / D, d = e % D, j = j0 + jj;
        float kv = 0.f, vv = 0.f;
        if (j < P.nk && d < P.dim) {
            kv = to_f(P.k.row<T>(b, h, j)[d]);
            vv = to_f(P.v.row<T>(b, h, j)[d]);
            if (P.vmul.ok()) vv = round_to<T>(vv * to_f(P.vmul.row<T>(b, h, j)[d]));
        }
        sK[jj][d] = kv;
        sV[jj][d] = vv;
    }
    for (int jj = threadIdx.x; jj < kSimtKT; jj += blockDim.x) {
        const int j = j0 + jj;
        sB[jj] = (j < P.nk && P.bias.ok()) ? P.bias.scalar(b, h, j) : 0.f;
        sKM[jj] = (j < P.nk && P.km.keep(b, j)) ? 1 : 0;
    }
}

// Accumulate the class-1 entries of a fully-masked row over all keys (uniform average).
// Every lane of the block must call it (it synchronises); only lanes with `degen` touch
// their accumulator (lanes holding a normal row keep theirs).
template <typename T, int D>
__device__ void simt_degenerate_rows(const PassDev& P, int b, int h, int i, bool degen, bool qok,
                                     float (*sK)[D], float (*sV)[D], float* sB, uint8_t* sKM,
                                     float* acc, float& c1) {
    c1 = 0.f;
    if (degen) {
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = 0.f;
    }
    for (int j0 = 0; j0 < P.nk; j0 += kSimtKT) {
        simt_stage_keys<T, D>(P, b, h, j0, sK, sV, sB, sKM);
        __syncthreads();
        const int cnt = min(kSimtKT, P.nk - j0);
        if (degen) {
            for (int jj = 0; jj < cnt; ++jj) {
                const int j = j0 + jj;
                const bool own_masked = !qok || (P.causal && j > i) || !sKM[jj];
                const int cls = (own_masked ? 1 : 0) + bias_class(sB[jj]);
                if (cls == 1) {
                    c1 += 1.f;
#pragma unroll
                    for (int d = 0; d < D; ++d) acc[d] += sV[jj][d];
                }
            }
        }
        __syncthreads();
    }
}

template <typename T, int D>
__device__ void simt_write_row(const PassDev& P, int b, int h, int i, const float* acc, float inv,
                               float lse) {
    T* o = P.out.wrow<T>(b, h, i);
    for (int d = 0; d < P.dim; ++d) o[d] = from_f<T>(acc[d] * inv);
    if (P.ey.ok()) {
        T* y = P.ey.wrow<T>(b, h, i);
        for (int d = 0; d < P.dim; ++d) y[d] = from_f<T>(epi_y<T>(P, b, h, i, d, round_to<T>(acc[d] * inv)));
    }
    *P.lse.wrow<float>(b, h, i) = lse;
}

template <typename T, int D>
__global__ __launch_bounds__(kSimtRows) void k_simt_fwd(PassDev P) {
    __shared__ float sK[kSimtKT][D];
    __shared__ float sV[kSimtKT][D];
    __shared__ float sB[kSimtKT];
    __shared__ uint8_t sKM[kSimtKT];
    const int b = blockIdx.z, h = blockIdx.y;
    const int i = blockIdx.x * kSimtRows + threadIdx.x;
    const bool row = i < P.nq;
    const bool qok = row && P.qm.keep(b, i);

    float q[D], acc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        q[d] = (row && d < P.dim) ? to_f(P.q.row<T>(b, h, i)[d]) : 0.f;
        acc[d] = 0.f;
    }
    float m = -INFINITY, l = 0.f;  // running max (log2 domain) and sum
    const int i_last = min(P.nq, (int)(blockIdx.x + 1) * kSimtRows) - 1;
    const int jend = P.causal ? min(P.nk, i_last + 1) : P.nk;
    for (int j0 = 0; j0 < jend; j0 += kSimtKT) {
        simt_stage_keys<T, D>(P, b, h, j0, sK, sV, sB, sKM);
        __syncthreads();
        const int cnt = min(kSimtKT, jend - j0);
        for (int jj = 0; jj < cnt; ++jj) {
            const int j = j0 + jj;
            const bool valid = qok && (!P.causal || j <= i) && sKM[jj] && bias_class(sB[jj]) == 0;
            if (!valid) continue;
            float s = 0.f;
#pragma unroll
            for (int d = 0; d < D; ++d) s += q[d] * sK[jj][d];
            const float t = (softclamp_f(s * P.scale, P.softclamp) + sB[jj]) * kLog2e;
            if (t > m) {
                const float c = exp2f(m - t);
                l *= c;
#pragma unroll
                for (int d = 0; d < D; ++d) acc[d] *= c;
                m = t;
            }
            const float p = exp2f(t - m);
            l += p;
#pragma unroll
            for (int d = 0; d < D; ++d) acc[d] += p * sV[jj][d];
        }
        __syncthreads();
    }
    const bool degen = row && !(l > 0.f);
    if (__syncthreads_or(degen)) {
        float c1;
        simt_degenerate_rows<T, D>(P, b, h, i, degen, qok, sK, sV, sB, sKM, acc, c1);
        if (degen) {
            if (c1 > 0.f) simt_write_row<T, D>(P, b, h, i, acc, 1.f / c1, -FLT_MAX);
            else simt_write_row<T, D>(P, b, h, i, acc, NAN, -INFINITY);
        }
    }
    if (row && !degen) simt_write_row<T, D>(P, b, h, i, acc, 1.f / l, (m + log2f(l)) * kLn2);
}

// 8 consecutive elements to / from fp32: 16-byte aligned rows (the MFMA kernels' loads), and
// 8-byte aligned rows (their stores) as two 8-byte accesses
template <typename T>
__device__ __forceinline__ void load8(const T* p, float* f) {
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = to_f(e[k]);
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* f) {  // 32 bytes
    const float4 a = reinterpret_cast<const float4*>(p)[0], c = reinterpret_cast<const float4*>(p)[1];
    f[0] = a.x;
    f[1] = a.y;
    f[2] = a.z;
    f[3] = a.w;
    f[4] = c.x;
    f[5] = c.y;
    f[6] = c.z;
    f[7] = c.w;
}
template <typename T>
__device__ __forceinline__ void load8_a8(const T* p, float* f) {
    const uint2 a = reinterpret_cast<const uint2*>(p)[0], c = reinterpret_cast<const uint2*>(p)[1];
    const T* ea = reinterpret_cast<const T*>(&a);
    const T* ec = reinterpret_cast<const T*>(&c);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        f[k] = to_f(ea[k]);
        f[4 + k] = to_f(ec[k]);
    }
}
template <typename T>
__device__ __forceinline__ void store8_a8(T* p, const float* f) {
    uint2 a, c;
    T* ea = reinterpret_cast<T*>(&a);
    T* ec = reinterpret_cast<T*>(&c);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        ea[k] = from_f<T>(f[k]);
        ec[k] = from_f<T>(f[4 + k]);
    }
    reinterpret_cast<uint2*>(p)[0] = a;
    reinterpret_cast<uint2*>(p)[1] = c;
}
// fp32 rows (16-byte aligned, as the fp32 MFMA kernels require): two 16-byte accesses
template <>
__device__ __forceinline__ void load8_a8<float>(const float* p, float* f) {
    load8<float>(p, f);
}
template <>
__device__ __forceinline__ void store8_a8<float>(float* p, const float* f) {
    reinterpret_cast<float4*>(p)[0] = make_float4(f[0], f[1], f[2], f[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(f[4], f[5], f[6], f[7]);
}

constexpr int kFixThreads = 1024;  // per-head reductions: many rows in flight on one CU

// p[0] + p[S] + p[2 S] + ... (n terms, stride S) in that order, eight loads in flight at a
// time (partial sums are few; a loop of one load per step waits a round trip per term)
template <int S>
__device__ __forceinline__ float ordered_sum(const float* p, int n) {
    constexpr int U = 8;
    float a = 0.f;
    for (int c0 = 0; c0 < n; c0 += U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = c0 + u < n ? p[(int64_t)(c0 + u) * S] : 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u) a += x[u];
    }
    return a;
}

// S0 of k_fwd_fixup, one slot's share (key rows slot, slot + R, ...): U key rows per round,
// every load of a round (key term, mask byte, value row) issued before the first is used, rows
// past the end reading the last row and counting for nothing.  One memory round trip per
// round: with the key terms loaded first and the value rows behind them (two round trips a
// round, four rows) the left-padded config-2 pass took 35 us here.  VM: the values are
// v * vmul, rounded to T.
template <typename T, int D, bool VM, bool HB, bool HK>
__device__ __forceinline__ void fixup_s0(const PassDev& P, int b, int h, int slot, int c0,
                                         float (&acc)[8], int& n0, int& n1) {
    constexpr int R = kFixThreads / (D / 8), U = VM ? 4 : 8;  // 16 spills at 1024 threads
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
    for (int j0 = slot; j0 < P.nk; j0 += R * U) {
        float x[U], v8[U][8], m8[VM ? U : 1][8];
        bool kp[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int jc = min(j0 + u * R, P.nk - 1);
            x[u] = HB ? P.bias.scalar(b, h, jc) : 0.f;
            kp[u] = HK ? P.km.p[(int64_t)b * P.km.sb + (int64_t)jc * P.km.sn] != 0 : true;
            load8<T>(P.v.row<T>(b, h, jc) + c0, v8[u]);
            if constexpr (VM) load8<T>(P.vmul.row<T>(b, h, jc) + c0, m8[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (j0 + u * R >= P.nk) break;
            const int cls = bias_class(x[u]);
            if (cls == 1 && kp[u]) ++n1;
            if (cls != 0) continue;
            ++n0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if constexpr (VM) acc[e] += round_to<T>(v8[u][e] * m8[u][e]);
                else acc[e] += v8[u][e];
            }
        }
    }
}

template <typename T, int D, bool VM>
__device__ __forceinline__ void fixup_s0_any(const PassDev& P, int b, int h, int slot, int c0,
                                             float (&acc)[8], int& n0, int& n1) {
    const bool hb = P.bias.ok(), hk = P.km.p != nullptr;
    if (hb) hk ? fixup_s0<T, D, VM, true, true>(P, b, h, slot, c0, acc, n0, n1)
               : fixup_s0<T, D, VM, true, false>(P, b, h, slot, c0, acc, n0, n1);
    else hk ? fixup_s0<T, D, VM, false, true>(P, b, h, slot, c0, acc, n0, n1)
            : fixup_s0<T, D, VM, false, false>(P, b, h, slot, c0, acc, n0, n1);
}

// Finish the rows an MFMA forward left fully masked (their lse holds NaN), one workgroup per
// (b, query head).  Every key of bias class 0 is masked for such a row (else the row would
// hold a normal entry), so its class-1 entries are all bias-class-0 keys plus its own
// unmasked bias-class-1 keys, and its output is (S0 + the latter's values) / c1, with S0 the
// sum of the bias-class-0 keys' effective values -- one sum for every such row of the head.
template <typename T, int D>
__global__ __launch_bounds__(kFixThreads) void k_fwd_fixup(PassDev P) {
    constexpr int LPR = D / 8, R = kFixThreads / LPR;  // lanes per key row, key slots
    constexpr int E = D / 64;  // columns per lane when finishing a row
    const int h = blockIdx.x, b = blockIdx.y;
    const int tid = threadIdx.x;
    bool any = false;
    {
        constexpr int RU = 4;  // rows per thread per round, all loads in flight together
        for (int i0 = tid; i0 < P.nq; i0 += kFixThreads * RU) {
            float l[RU];
#pragma unroll
            for (int u = 0; u < RU; ++u) l[u] = *P.lse.row<float>(b, h, min(i0 + u * kFixThreads, P.nq - 1));
#pragma unroll
            for (int u = 0; u < RU; ++u) any |= i0 + u * kFixThreads < P.nq && isnan(l[u]);
        }
    }
    if (!__syncthreads_or(any)) return;

    // S0 and the counts of bias-class-0 and unmasked bias-class-1 keys
    const int slot = tid / LPR, c0 = (tid % LPR) * 8;
    float acc[8];
    int n0 = 0, n1 = 0;
    if (P.vmul.ok()) fixup_s0_any<T, D, true>(P, b, h, slot, c0, acc, n0, n1);
    else fixup_s0_any<T, D, false>(P, b, h, slot, c0, acc, n0, n1);
    __shared__ float sS[R][D];
    __shared__ int sN[R][2];
    __shared__ float sT[D];
    __shared__ int sCnt[2];
#pragma unroll
    for (int e = 0; e < 8; ++e) sS[slot][c0 + e] = acc[e];
    if (c0 == 0) {
        sN[slot][0] = n0;
        sN[slot][1] = n1;
    }
    __syncthreads();
    if (tid < D) {
        float a = 0.f;
#pragma unroll 16  // the LDS reads issued ahead of the (ordered) sums
        for (int r = 0; r < R; ++r) a += sS[r][tid];
        sT[tid] = a;
    } else if (tid < D + 2) {
        int a = 0;
#pragma unroll 16  // the LDS reads issued ahead of the (ordered) sums
        for (int r = 0; r < R; ++r) a += sN[r][tid - D];
        sCnt[tid - D] = a;
    }
    __syncthreads();
    const int N0 = sCnt[0], N1 = sCnt[1];

    if constexpr (sizeof(T) == 2) {
        if (N1 == 0 && !P.ey.ok()) {
            // no unmasked bias-class-1 key: every fully-masked row is S0 / N0.  Round it once,
            // then each thread finds its rows (their lse loaded before any store) and copies it
            constexpr int RB = 8;
            __shared__ __attribute__((aligned(16))) uint32_t sRow[D / 2];
            if (tid < D / 2) {
                const float inv = N0 > 0 ? 1.f / (float)N0 : NAN;
                float y0 = sT[2 * tid] * inv, y1 = sT[2 * tid + 1] * inv;
                asm volatile("" : "+v"(y0), "+v"(y1));  // round the fp32 products, then convert
                sRow[tid] = pack2<T>(y0, y1);
            }
            __syncthreads();
            const float fill = N0 > 0 ? -FLT_MAX : -INFINITY;
            for (int i0 = tid; i0 < P.nq; i0 += kFixThreads * RB) {
                bool dg[RB];
#pragma unroll
                for (int u = 0; u < RB; ++u) {
                    const int i = i0 + u * kFixThreads;
                    dg[u] = i < P.nq && isnan(*P.lse.row<float>(b, h, i));
                }
#pragma unroll
                for (int u = 0; u < RB; ++u) {
                    if (!dg[u]) continue;
                    const int i = i0 + u * kFixThreads;
                    T* o = P.out.wrow<T>(b, h, i);
#pragma unroll
                    for (int c = 0; c < D / 4; ++c)
                        *reinterpret_cast<u32x2_t*>(o + 4 * c) = *reinterpret_cast<const u32x2_t*>(&sRow[2 * c]);
                    *P.lse.wrow<float>(b, h, i) = fill;
                }
            }
            return;
        }
    }

    // each wave finds its fully-masked rows 64 at a time and writes them, lanes as columns
    const int w = tid / 64, lane = tid % 64;
    for (int i0 = w * 64; i0 < P.nq; i0 += blockDim.x) {
        const int i = i0 + lane;
        uint64_t m = __ballot(i < P.nq && isnan(*P.lse.row<float>(b, h, i)));
        while (m) {
            const int r = i0 + __ffsll((unsigned long long)m) - 1;
            m &= m - 1;
            float sum[E];
#pragma unroll
            for (int e = 0; e < E; ++e) sum[e] = sT[lane + 64 * e];
            int c1 = N0;
            if (N1 > 0 && P.qm.keep(b, r)) {  // the row's unmasked bias-class-1 keys
                const int jend = P.causal ? min(P.nk, r + 1) : P.nk;
                for (int j0 = 0; j0 < jend; j0 += 64) {
                    const int j = j0 + lane;
                    const bool f = j < jend && P.km.keep(b, j) &&
                                   bias_class(P.bias.scalar(b, h, j)) == 1;
                    uint64_t fm = __ballot(f);
                    c1 += __popcll(fm);
                    while (fm) {
                        const int jk = j0 + __ffsll((unsigned long long)fm) - 1;
                        fm &= fm - 1;
#pragma unroll
                        for (int e = 0; e < E; ++e) {
                            const int d = lane + 64 * e;
                            float vv = to_f(P.v.row<T>(b, h, jk)[d]);
                            if (P.vmul.ok()) vv = round_to<T>(vv * to_f(P.vmul.row<T>(b, h, jk)[d]));
                            sum[e] += vv;
                        }
                    }
                }
            }
            const float inv = c1 > 0 ? 1.f / (float)c1 : NAN;
            T* o = P.out.wrow<T>(b, h, r);
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const int d = lane + 64 * e;
                o[d] = from_f<T>(sum[e] * inv);
                if (P.ey.ok()) P.ey.wrow<T>(b, h, r)[d] = from_f<T>(epi_y<T>(P, b, h, r, d, round_to<T>(sum[e] * inv)));
            }
            if (lane == 0) *P.lse.wrow<float>(b, h, r) = c1 > 0 ? -FLT_MAX : -INFINITY;
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward

// Number of class-1 entries (score -finfo.max) of the fully-masked row i.  Every key of bias
// class 0 is masked for such a row (else the row would hold a normal entry), so the count is
// the (b, key head)'s bias-class-0 keys plus the row's unmasked bias-class-1 keys; the latter
// exist only where the bias holds -finfo.max on kept keys and the row's query is kept.  With
// the per-key-head counts of a masked MFMA backward (G.ws_kcnt) the row loop runs only then.
__device__ __forceinline__ float degenerate_count(const GradDev& G, int b, int h, int i) {
    const PassDev& P = G.f;
    const bool qok = P.qm.keep(b, i);
    if (G.ws_kcnt) {
        const int32_t* kc = G.ws_kcnt + 2 * ((int64_t)b * G.hk + h / (P.heads / G.hk));
        if (!qok || kc[1] == 0) return (float)kc[0];
    }
    float c1 = 0.f;
    for (int j = 0; j < P.nk; ++j) {
        const bool own_masked = !qok || (P.causal && j > i) || !P.km.keep(b, j);
        const float bj = P.bias.ok() ? P.bias.scalar(b, h, j) : 0.f;
        if ((own_masked ? 1 : 0) + bias_class(bj) == 1) c1 += 1.f;
    }
    return c1;
}

// Per row: D = rowsum(dO * O) - dlse, so that dS = P (dP - D) carries the softmax and the
// logsumexp gradients.  A fully-masked row has P = 1/c1 on its c1 class-1 entries, and its
// lse is absorbed to -finfo.max, so logsumexp's backward exp(s - lse) weighs each class-1
// entry by 1 (not 1/c1): there D = rowsum(dO * O) - c1 * dlse.
template <typename T, int D>
__global__ __launch_bounds__(kSimtRows) void k_bwd_pre(GradDev G) {
    const PassDev& P = G.f;
    const int b = blockIdx.z, h = blockIdx.y;
    const int i = blockIdx.x * kSimtRows + threadIdx.x;
    if (i >= P.nq) return;
    const T* o = P.out.row<T>(b, h, i);
    const T* go = G.dout.row<T>(b, h, i);
    float dsum = 0.f;
    for (int d = 0; d < P.dim; ++d) dsum += to_f(o[d]) * to_f(go[d]);
    const float dl = G.dlse.ok() ? *G.dlse.row<float>(b, h, i) : 0.f;
    const float l = *P.lse.row<float>(b, h, i);
    float lseb = l, invc = 0.f;
    if (l > kMaskedThreshold) {
        dsum -= dl;
    } else {
        const float c1 = degenerate_count(G, b, h, i);
        lseb = INFINITY;
        invc = c1 > 0.f ? 1.f / c1 : 0.f;
        // an all -inf row (c1 == 0): its NaN output has no gradient here
        dsum = c1 > 0.f ? dsum - c1 * dl : 0.f;
    }
    const int64_t r = ((int64_t)b * P.heads + h) * P.nq + i;
    G.ws_D[r] = dsum;
    G.ws_lse[r] = lseb;
    G.ws_invc[r] = invc;
}

// The same preprocess for 16-bit types with head dims that are multiples of 8: LPR lanes
// per row read 16 bytes each (a wave covers 64/LPR whole rows per load), then reduce.
constexpr int kPreRows = 4;  // rows per lane group of k_bwd_pre_vec, all loads issued first
template <typename T, int LPR>
__global__ __launch_bounds__(256) void k_bwd_pre_vec(GradDev G) {
    const PassDev& P = G.f;
    constexpr int kRows = 256 / LPR;  // lane groups per workgroup
    const int h = blockIdx.y, b = blockIdx.z;
    const int sub = threadIdx.x % LPR, d0 = sub * 8;
    const int i0 = (int)blockIdx.x * kRows * kPreRows + (int)threadIdx.x / LPR;
    const int64_t row0 = ((int64_t)b * P.heads + h) * P.nq;
    // a lane group takes rows i0, i0 + kRows, ... of (b, h): every load of its rows goes out
    // before the first is used (one memory round trip per workgroup)
    uint4 ov[kPreRows], gv[kPreRows];
    float dl[kPreRows], l[kPreRows];
#pragma unroll
    for (int u = 0; u < kPreRows; ++u) {
        const int i = min(i0 + u * kRows, P.nq - 1);
        ov[u] = gv[u] = make_uint4(0u, 0u, 0u, 0u);
        if (d0 < P.dim) {
            ov[u] = *reinterpret_cast<const uint4*>(P.out.row<T>(b, h, i) + d0);
            gv[u] = *reinterpret_cast<const uint4*>(G.dout.row<T>(b, h, i) + d0);
        }
        dl[u] = G.dlse.ok() ? *G.dlse.row<float>(b, h, i) : 0.f;
        l[u] = *P.lse.row<float>(b, h, i);
    }
#pragma unroll
    for (int u = 0; u < kPreRows; ++u) {
        const int i = i0 + u * kRows;
        const T* oe = reinterpret_cast<const T*>(&ov[u]);
        const T* ge = reinterpret_cast<const T*>(&gv[u]);
        float dsum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dsum += to_f(oe[e]) * to_f(ge[e]);
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) dsum += __shfl_xor(dsum, off);
        if (sub != 0 || i >= P.nq) continue;
        float lseb = l[u], invc = 0.f;
        if (l[u] > kMaskedThreshold) {
            dsum -= dl[u];
        } else {  // fully-masked row (rare): count its class-1 entries
            const float c1 = degenerate_count(G, b, h, i);
            lseb = INFINITY;
            invc = c1 > 0.f ? 1.f / c1 : 0.f;
            dsum = c1 > 0.f ? dsum - c1 * dl[u] : 0.f;
        }
        G.ws_D[row0 + i] = dsum;
        G.ws_lse[row0 + i] = lseb;
        G.ws_invc[row0 + i] = invc;
    }
}

// probability of entry (i, j) given the row's (lse, 1/c1) and the entry's mask state
__device__ __forceinline__ float entry_prob(bool normal, bool own_ok, int bcls, float y_plus_bias,
                                            float lseb, float invc) {
    if (normal) return (own_ok && bcls == 0) ? exp2f((y_plus_bias - lseb) * kLog2e) : 0.f;
    return ((own_ok ? 0 : 1) + bcls == 1) ? invc : 0.f;
}

template <typename T, int D>
__global__ __launch_bounds__(kSimtRows) void k_simt_bwd_dq(GradDev G) {
    const PassDev& P = G.f;
    __shared__ float sK[kSimtKT][D];
    __shared__ float sV[kSimtKT][D];
    __shared__ float sB[kSimtKT];
    __shared__ uint8_t sKM[kSimtKT];
    const int b = blockIdx.z, h = blockIdx.y;
    const int i = blockIdx.x * kSimtRows + threadIdx.x;
    const bool row = i < P.nq;
    const bool qok = row && P.qm.keep(b, i);
    const int64_t r = ((int64_t)b * P.heads + h) * P.nq + (row ? i : 0);
    const float Dp = row ? G.ws_D[r] : 0.f;
    const float lseb = row ? G.ws_lse[r] : 0.f;
    const float invc = row ? G.ws_invc[r] : 0.f;
    const bool normal = lseb != INFINITY;

    float q[D], go[D], dq[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        q[d] = (row && d < P.dim) ? to_f(P.q.row<T>(b, h, i)[d]) : 0.f;
        go[d] = (row && d < P.dim) ? to_f(G.dout.row<T>(b, h, i)[d]) : 0.f;
        dq[d] = 0.f;
    }
    const int i_last = min(P.nq, (int)(blockIdx.x + 1) * kSimtRows) - 1;
    const bool any_degen = __syncthreads_or(row && !normal);
    const int jend = (P.causal && !any_degen) ? min(P.nk, i_last + 1) : P.nk;
    for (int j0 = 0; j0 < jend; j0 += kSimtKT) {
        simt_stage_keys<T, D>(P, b, h, j0, sK, sV, sB, sKM);
        __syncthreads();
        const int cnt = min(kSimtKT, jend - j0);
        if (row) {
            for (int jj = 0; jj < cnt; ++jj) {
                const int j = j0 + jj;
                const bool own_ok = qok && (!P.causal || j <= i) && sKM[jj];
                const int bcls = bias_class(sB[jj]);
                float s = 0.f;
#pragma unroll
                for (int d = 0; d < D; ++d) s += q[d] * sK[jj][d];
                const float y = softclamp_f(s * P.scale, P.softclamp);
                const float p = entry_prob(normal, own_ok, bcls, y + sB[jj], lseb, invc);
                if (p == 0.f || !own_ok) continue;  // no score gradient reaches q
                float dp = 0.f;
#pragma unroll
                for (int d = 0; d < D; ++d) dp += go[d] * sV[jj][d];
                const float g = p * (dp - Dp) * softclamp_grad(y, P.softclamp) * P.scale;
#pragma unroll
                for (int d = 0; d < D; ++d) dq[d] += g * sK[jj][d];
            }
        }
        __syncthreads();
    }
    if (!row) return;
    T* o = G.dq.wrow<T>(b, h, i);
    const bool acc = (G.accumulate & PA_ACC_DQ) != 0;
    for (int d = 0; d < P.dim; ++d) o[d] = from_f<T>(dq[d] + (acc ? to_f(o[d]) : 0.f));
}

// One lane per key row of key head kh; loops over the query heads of its group.
template <typename T, int D>
__global__ __launch_bounds__(kSimtRows) void k_simt_bwd_dkv(GradDev G) {
    const PassDev& P = G.f;
    __shared__ float sQ[kSimtKT][D];
    __shared__ float sO[kSimtKT][D];  // dO rows
    __shared__ float sL[kSimtKT], sI[kSimtKT], sD[kSimtKT];
    __shared__ uint8_t sQM[kSimtKT];
    const int b = blockIdx.z, kh = blockIdx.y;
    const int j = blockIdx.x * kSimtRows + threadIdx.x;
    const bool col = j < P.nk;
    const int rep = P.heads / G.hk;
    const int h0 = kh * rep;  // first pass head of this group (k.row(b, h0, j) maps to kh)

    float kk[D], vv[D], dk[D], dv[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        float kv = 0.f, v = 0.f;
        if (col && d < P.dim) {
            kv = to_f(P.k.row<T>(b, h0, j)[d]);
            v = to_f(P.v.row<T>(b, h0, j)[d]);
            if (P.vmul.ok()) v = round_to<T>(v * to_f(P.vmul.row<T>(b, h0, j)[d]));
        }
        kk[d] = kv;
        vv[d] = v;
        dk[d] = 0.f;
        dv[d] = 0.f;
    }
    const bool kmok = col && P.km.keep(b, j);
    const float bj = (col && P.bias.ok()) ? P.bias.scalar(b, h0, j) : 0.f;
    const int bcls = bias_class(bj);
    float dbias = 0.f;
    const int j_first = blockIdx.x * kSimtRows;

    for (int h = h0; h < h0 + rep; ++h) {
        for (int i0 = 0; i0 < P.nq; i0 += kSimtKT) {
            // per-row scalars first: a causal tile entirely above this block's keys can be
            // skipped unless one of its rows is fully masked
            for (int ii = threadIdx.x; ii < kSimtKT; ii += blockDim.x) {
                const int i = i0 + ii;
                const int64_t r = ((int64_t)b * P.heads + h) * P.nq + i;
                const bool ok = i < P.nq;
                sL[ii] = ok ? G.ws_lse[r] : 0.f;
                sI[ii] = ok ? G.ws_invc[r] : 0.f;
                sD[ii] = ok ? G.ws_D[r] : 0.f;
                sQM[ii] = (ok && P.qm.keep(b, i)) ? 1 : 0;
            }
            __syncthreads();
            bool tile_degen = false;
            const int cnt = min(kSimtKT, P.nq - i0);
            for (int ii = 0; ii < cnt; ++ii) tile_degen |= (sL[ii] == INFINITY);
            const bool skip = P.causal && !tile_degen && (i0 + cnt - 1 < j_first);
            if (!skip) {
                for (int e = threadIdx.x; e < kSimtKT * D; e += blockDim.x) {
                    const int ii = e / D, d = e % D, i = i0 + ii;
                    const bool ok = i < P.nq && d < P.dim;
                    sQ[ii][d] = ok ? to_f(P.q.row<T>(b, h, i)[d]) : 0.f;
                    sO[ii][d] = ok ? to_f(G.dout.row<T>(b, h, i)[d]) : 0.f;
                }
            }
            __syncthreads();
            if (!skip && col) {
                for (int ii = 0; ii < cnt; ++ii) {
                    const int i = i0 + ii;
                    const bool normal = sL[ii] != INFINITY;
                    const bool own_ok = sQM[ii] && (!P.causal || j <= i) && kmok;
                    float s = 0.f;
#pragma unroll
                    for (int d = 0; d < D; ++d) s += sQ[ii][d] * kk[d];
                    const float y = softclamp_f(s * P.scale, P.softclamp);
                    const float p = entry_prob(normal, own_ok, bcls, y + bj, sL[ii], sI[ii]);
                    if (p == 0.f) continue;
                    float dp = 0.f;
#pragma unroll
                    for (int d = 0; d < D; ++d) dp += sO[ii][d] * vv[d];
                    const float ds = p * (dp - sD[ii]);
                    dbias += ds;
#pragma unroll
                    for (int d = 0; d < D; ++d) dv[d] += p * sO[ii][d];
                    if (own_ok) {
                        const float g = ds * softclamp_grad(y, P.softclamp) * P.scale;
#pragma unroll
                        for (int d = 0; d < D; ++d) dk[d] += g * sQ[ii][d];
                    }
                }
            }
            __syncthreads();
        }
    }
    if (!col) return;
    {
        T* o = G.dk.wrow<T>(b, h0, j);
        const bool acc = (G.accumulate & PA_ACC_DK) != 0;
        for (int d = 0; d < P.dim; ++d) o[d] = from_f<T>(dk[d] + (acc ? to_f(o[d]) : 0.f));
    }
    {
        T* o = G.dv.wrow<T>(b, h0, j);
        const bool acc = (G.accumulate & PA_ACC_DV) != 0;
        const T* mul = P.vmul.ok() ? P.vmul.row<T>(b, h0, j) : nullptr;
        for (int d = 0; d < P.dim; ++d) {
            const float g = mul ? dv[d] * to_f(mul[d]) : dv[d];
            o[d] = from_f<T>(g + (acc ? to_f(o[d]) : 0.f));
        }
    }
    if (P.vmul.ok()) {
        T* o = G.dvmul.wrow<T>(b, h0, j);
        const bool acc = (G.accumulate & PA_ACC_DVMUL) != 0;
        const T* v = P.v.row<T>(b, h0, j);
        for (int d = 0; d < P.dim; ++d)
            o[d] = from_f<T>(dv[d] * to_f(v[d]) + (acc ? to_f(o[d]) : 0.f));
    }
    if (G.dbias.ok()) {
        float* o = G.dbias.wrow<float>(b, h0, j);
        *o = dbias + ((G.accumulate & PA_ACC_DBIAS) ? *o : 0.f);
    }
}

// ---------------------------------------------------------------------------------------
// masked passes on the MFMA backward kernels
//
// The MFMA kernels compute the normal rows of a masked pass exactly once the key mask is
// folded into a per-key additive term (the raw bias on kept keys, -inf on masked ones: the
// kernels turn any non-class-0 term into probability 0), and the preprocess gives every
// fully-masked row lse = +inf, which makes its probabilities 0 there.  The kernels below add
// the fully-masked rows' part.  Such a row i has probability 1/c1_i on its class-1 entries:
//   (A) every key of bias class 0 (all masked for the row, so no score gradient), and
//   (B) its unmasked keys of bias class 1 (only where the bias holds -finfo.max).
// Part A is the same key set for every fully-masked row of a head, so over those rows it is a
// rank-one update: dV[j] += u = sum_i dO_i / c1_i and dbias[j] += u . V[j] - sum_i D_i / c1_i
// on each bias-class-0 key j.  Part B is a plain loop over the rare (row, key) pairs.

// Per (b, key head): the count of bias-class-0 keys and of unmasked bias-class-1 keys (part
// B exists only where the latter is nonzero; with kcnt), (with kterm) the per-key term the
// MFMA kernels read as their bias, rows of stride nkp, and (with live) the range [first, last
// + 1) of the keys that are kept and of bias class 0 -- the only keys that enter a normal row;
// [nk, 0) when there is none.  The MFMA forward and dQ kernels start and end their key loops
// at the range (padding masks: the masked prefix or suffix is not even loaded).  A workgroup walks a key row in rounds
// of kKeyTermThreads x kKeyTermPer keys, every load of a round issued before its first use (the
// key-mask bytes may alias the key-term stores, so a loop mixing them would load one key at
// a time); at 4096 keys that is one round instead of 16 dependent steps.
constexpr int kKeyTermThreads = 1024, kKeyTermPer = 4;
__global__ __launch_bounds__(kKeyTermThreads) void k_key_terms(GradDev G, float* kterm, int nkp,
                                                               int32_t* kcnt, int32_t* live) {
    const PassDev& P = G.f;
    const int kh = blockIdx.x, b = blockIdx.y;
    const int h0 = kh * (P.heads / G.hk);
    int c0 = 0, c1 = 0, lo = P.nk, hi = 0;
    for (int j0 = 0; j0 < P.nk; j0 += kKeyTermThreads * kKeyTermPer) {
        float x[kKeyTermPer];
        bool kept[kKeyTermPer];
#pragma unroll
        for (int u = 0; u < kKeyTermPer; ++u) {
            const int j = j0 + u * kKeyTermThreads + (int)threadIdx.x;
            x[u] = (j < P.nk && P.bias.ok()) ? P.bias.scalar(b, h0, j) : 0.f;
            kept[u] = j < P.nk && P.km.keep(b, j);
        }
#pragma unroll
        for (int u = 0; u < kKeyTermPer; ++u) {
            const int j = j0 + u * kKeyTermThreads + (int)threadIdx.x;
            if (j >= P.nk) break;
            const int cls = bias_class(x[u]);
            c0 += cls == 0;
            c1 += cls == 1 && kept[u];
            if (cls == 0 && kept[u]) {
                lo = min(lo, j);
                hi = j + 1;
            }
            if (kterm) kterm[((int64_t)b * G.hk + kh) * nkp + j] = kept[u] ? x[u] : -INFINITY;
        }
    }
    if (!kcnt && !live) return;  // whole workgroup: nothing to reduce
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        c0 += __shfl_xor(c0, off);
        c1 += __shfl_xor(c1, off);
        lo = min(lo, __shfl_xor(lo, off));
        hi = max(hi, __shfl_xor(hi, off));
    }
    __shared__ int s0[kKeyTermThreads / 64], s1[kKeyTermThreads / 64];
    __shared__ int slo[kKeyTermThreads / 64], shi[kKeyTermThreads / 64];
    const int w = threadIdx.x / 64;
    if (threadIdx.x % 64 == 0) {
        s0[w] = c0;
        s1[w] = c1;
        slo[w] = lo;
        shi[w] = hi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int t0 = 0, t1 = 0, tlo = P.nk, thi = 0;
        for (int k = 0; k < (int)blockDim.x / 64; ++k) {
            t0 += s0[k];
            t1 += s1[k];
            tlo = min(tlo, slo[k]);
            thi = max(thi, shi[k]);
        }
        const int64_t u = (int64_t)b * G.hk + kh;
        if (kcnt) {
            kcnt[2 * u] = t0;
            kcnt[2 * u + 1] = t1;
        }
        if (live) {
            live[2 * u] = tlo;
            live[2 * u + 1] = thi;
        }
    }
}

__device__ __forceinline__ bool degenerate_row(const GradDev& G, int64_t r) {
    return G.ws_lse[r] == INFINITY && G.ws_invc[r] > 0.f;
}

// Part A sums over the fully-masked rows, one workgroup per (b, query head, chunk of
// kFixRowChunk rows): D/8 lanes per row, 16 bytes of dO and of O each; each lane group's rows
// go eight at a time with every load issued first (rows that are not fully masked weigh 0).
// A fully-masked row is known by its lse entry, which is not finite (+inf from the preprocess
// kernel, or the dQ kernel's seed of +inf); its preprocess is done here, from the original
// masks: c1 (its class-1 entries), 1/c1 and D = rowsum(dO * O) - c1 * dlse, written back as
// lse = +inf, 1/c1, D for the part B kernels.  The row slots are then summed through LDS into
// the chunk's partial row (fixed order: the sums are deterministic).  A chunk without such a
// row writes zeros after one scan of its lse.
template <typename T, int D>
__global__ __launch_bounds__(256) void k_fix_rows(GradDev G) {
    const PassDev& P = G.f;
    constexpr int LPR = D / 8, R = 256 / LPR, U = 8;  // lanes per row, row slots, rows per round
    static_assert(kFixRowChunk % (R * U) == 0, "whole rounds per chunk");
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int slot = threadIdx.x / LPR, c0 = (threadIdx.x % LPR) * 8;
    const int64_t row0 = ((int64_t)b * P.heads + h) * P.nq;
    const int i0 = c * kFixRowChunk, i1 = min(P.nq, i0 + kFixRowChunk);
    float* part = G.ws_part + (((int64_t)b * P.heads + h) * fix_row_chunks(P.nq) + c) * (D + 2);
    bool any = false;
    {
        static_assert(kFixRowChunk % 256 == 0, "whole rounds per chunk");
        float l[kFixRowChunk / 256];  // the chunk's rows, all loads in flight together
#pragma unroll
        for (int k = 0; k < kFixRowChunk / 256; ++k) l[k] = G.ws_lse[row0 + min(i0 + (int)threadIdx.x + 256 * k, i1 - 1)];
#pragma unroll
        for (int k = 0; k < kFixRowChunk / 256; ++k) any |= !isfinite(l[k]);
    }
    if (!__syncthreads_or(any)) {
        for (int e = threadIdx.x; e < D + 2; e += 256) part[e] = 0.f;  // D + 2 may exceed 256
        return;
    }
    float u[8], wsum = 0.f, cnt = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) u[e] = 0.f;
    // the key head's class counts (see degenerate_count): c1 of a fully-masked row is the
    // class-0 count unless the row's query is kept and unmasked class-1 keys exist
    int kc0 = 0, kc1 = 1;
    if (G.ws_kcnt) {
        const int32_t* kc = G.ws_kcnt + 2 * ((int64_t)b * G.hk + h / (P.heads / G.hk));
        kc0 = kc[0];
        kc1 = kc[1];
    }
    for (int ib = i0 + slot; ib < i1; ib += R * U) {
        float li[U], dl[U], g8[U][8], o8[U][8];
        bool qk[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            // every load of the round before the first use (a load behind a lane-dependent
            // condition would make the branch's join wait for it)
            const int i = min(ib + k * R, i1 - 1);
            li[k] = G.ws_lse[row0 + i];
            dl[k] = G.dlse.ok() ? *G.dlse.row<float>(b, h, i) : 0.f;
            qk[k] = P.qm.keep(b, i);
            load8<T>(G.dout.row<T>(b, h, i) + c0, g8[k]);
            load8<T>(P.out.row<T>(b, h, i) + c0, o8[k]);
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
            // the row's preprocess, for fully-masked rows: whether the preprocess kernel or
            // the dQ kernel (seed form) ran, such a row's lse entry is not finite
            float ds = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ds += o8[k][e] * g8[k][e];
#pragma unroll
            for (int off = LPR / 2; off > 0; off >>= 1) ds += __shfl_xor(ds, off);
            const int i = ib + k * R;
            float ic = 0.f, dd = 0.f;
            if (i < i1 && !isfinite(li[k])) {
                const float c1 = G.ws_kcnt && (!qk[k] || kc1 == 0) ? (float)kc0
                                                                 : degenerate_count(G, b, h, i);
                ic = c1 > 0.f ? 1.f / c1 : 0.f;
                dd = c1 > 0.f ? ds - c1 * dl[k] : 0.f;
                if (c0 == 0) {  // the canonical entries the part B kernels read
                    G.ws_lse[row0 + i] = INFINITY;
                    G.ws_invc[row0 + i] = ic;
                    G.ws_D[row0 + i] = dd;
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) u[e] += ic * g8[k][e];
            wsum += ic * dd;
            cnt += ic > 0.f ? 1.f : 0.f;
        }
    }
    __shared__ float sU[R][D];
    __shared__ float sW[R], sC[R];
#pragma unroll
    for (int e = 0; e < 8; ++e) sU[slot][c0 + e] = u[e];
    if (c0 == 0) {
        sW[slot] = wsum;
        sC[slot] = cnt;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < D + 2; e += 256) {  // D + 2 may exceed 256
        float a = 0.f;
        if (e < D) {
#pragma unroll 16  // the LDS reads issued ahead of the (ordered) sums
            for (int r = 0; r < R; ++r) a += sU[r][e];
        } else {
            const float* src = e == D ? sW : sC;
#pragma unroll 16  // the LDS reads issued ahead of the (ordered) sums
            for (int r = 0; r < R; ++r) a += src[r];
        }
        part[e] = a;
    }
}

// The part A sums of query head h over its row chunks (entry e of [sum dO / c1 | sum D / c1 |
// count]), in chunk order.
template <int D>
__device__ __forceinline__ float part_sum(const GradDev& G, int b, int h, int e) {
    const int C = fix_row_chunks(G.f.nq);
    return ordered_sum<D + 2>(G.ws_part + ((int64_t)b * G.f.heads + h) * C * (D + 2) + e, C);
}

constexpr int kFixKeys = 256;  // keys per k_fix_keys workgroup

// Part A updates of key head kh: dV (and dvmul) and dbias of the bias-class-0 keys,
// read-modify-write on what the MFMA dK/dV kernel stored; D/8 lanes per key row, each lane
// group's keys four at a time with their loads issued first.
template <typename T, int D>
__global__ __launch_bounds__(256) void k_fix_keys(GradDev G) {
    const PassDev& P = G.f;
    constexpr int LPR = D / 8, R = 256 / LPR, U = 4;
    static_assert(kFixKeys % (R * U) == 0, "whole rounds per workgroup");
    const int kh = blockIdx.y, b = blockIdx.z;
    const int rep = P.heads / G.hk, h0 = kh * rep;
    __shared__ float sU[D];
    __shared__ float sWC[2];
    const int tid = threadIdx.x;
    for (int e = tid; e < D + 2; e += 256) {  // D + 2 may exceed 256
        float a = 0.f;
        for (int hh = 0; hh < rep; ++hh) a += part_sum<D>(G, b, h0 + hh, e);
        if (e < D) sU[e] = a;
        else sWC[e - D] = a;
    }
    __syncthreads();
    if (sWC[1] == 0.f) return;  // no fully-masked row in the group
    const int slot = tid / LPR, c0 = (tid % LPR) * 8;
    const bool vm = P.vmul.ok();
    float u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) u[e] = sU[c0 + e];
    for (int jb = blockIdx.x * kFixKeys + slot; jb < (int)(blockIdx.x + 1) * kFixKeys; jb += R * U) {
        bool ok[U];
        float v[U][8], m[U][8], g[U][8];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int j = min(jb + k * R, P.nk - 1);
            ok[k] = jb + k * R < P.nk && (!P.bias.ok() || bias_class(P.bias.scalar(b, h0, j)) == 0);
            load8(P.v.row<T>(b, h0, j) + c0, v[k]);
            if (vm) load8(P.vmul.row<T>(b, h0, j) + c0, m[k]);
            load8_a8(G.dv.wrow<T>(b, h0, j) + c0, g[k]);
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int j = jb + k * R;
            float dot = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                dot += u[e] * (vm ? round_to<T>(v[k][e] * m[k][e]) : v[k][e]);
                g[k][e] += vm ? u[e] * m[k][e] : u[e];
            }
            if (ok[k]) {
                store8_a8(G.dv.wrow<T>(b, h0, j) + c0, g[k]);
                if (vm) {
                    T* dm = G.dvmul.wrow<T>(b, h0, j) + c0;
                    float gm[8];
                    load8_a8(dm, gm);
#pragma unroll
                    for (int e = 0; e < 8; ++e) gm[e] += u[e] * v[k][e];
                    store8_a8(dm, gm);
                }
            }
#pragma unroll
            for (int off = LPR / 2; off > 0; off >>= 1) dot += __shfl_xor(dot, off);
            if (ok[k] && c0 == 0 && G.dbias.ok()) *G.dbias.wrow<float>(b, h0, j) += dot - sWC[0];
        }
    }
}

// Part B, query side: dQ of the fully-masked kept rows through their unmasked bias-class-1
// keys (one lane per row).
template <typename T, int D>
__global__ __launch_bounds__(kSimtRows) void k_fix_rows_b(GradDev G) {
    const PassDev& P = G.f;
    __shared__ float sK[kSimtKT][D];
    __shared__ float sV[kSimtKT][D];
    __shared__ float sB[kSimtKT];
    __shared__ uint8_t sKM[kSimtKT];
    const int b = blockIdx.z, h = blockIdx.y;
    const int kh = h / (P.heads / G.hk);
    if (G.ws_kcnt[2 * ((int64_t)b * G.hk + kh) + 1] == 0) return;
    const int i = blockIdx.x * kSimtRows + threadIdx.x;
    const int64_t r = ((int64_t)b * P.heads + h) * P.nq + i;
    const bool dg = i < P.nq && degenerate_row(G, r) && P.qm.keep(b, i);
    if (!__syncthreads_or(dg)) return;
    const float Dp = dg ? G.ws_D[r] : 0.f;
    const float ic = dg ? G.ws_invc[r] : 0.f;
    float q[D], go[D], dq[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        q[d] = dg ? to_f(P.q.row<T>(b, h, i)[d]) : 0.f;
        go[d] = dg ? to_f(G.dout.row<T>(b, h, i)[d]) : 0.f;
        dq[d] = 0.f;
    }
    const int i_last = min(P.nq, (int)(blockIdx.x + 1) * kSimtRows) - 1;
    const int jend = P.causal ? min(P.nk, i_last + 1) : P.nk;
    for (int j0 = 0; j0 < jend; j0 += kSimtKT) {
        simt_stage_keys<T, D>(P, b, h, j0, sK, sV, sB, sKM);
        __syncthreads();
        const int cnt = min(kSimtKT, jend - j0);
        bool any = false;
        for (int jj = 0; jj < cnt; ++jj) any |= bias_class(sB[jj]) == 1 && sKM[jj];
        if (any && dg) {
            for (int jj = 0; jj < cnt; ++jj) {
                const int j = j0 + jj;
                if (bias_class(sB[jj]) != 1 || !sKM[jj] || (P.causal && j > i)) continue;
                float s = 0.f, dp = 0.f;
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    s += q[d] * sK[jj][d];
                    dp += go[d] * sV[jj][d];
                }
                const float y = softclamp_f(s * P.scale, P.softclamp);
                const float g = ic * (dp - Dp) * softclamp_grad(y, P.softclamp) * P.scale;
#pragma unroll
                for (int d = 0; d < D; ++d) dq[d] += g * sK[jj][d];
            }
        }
        __syncthreads();
    }
    if (!dg) return;
    T* o = G.dq.wrow<T>(b, h, i);
    for (int d = 0; d < D; ++d) o[d] = from_f<T>(to_f(o[d]) + dq[d]);
}

// Part B, key side: dK, dV (dvmul) and dbias of the unmasked bias-class-1 keys from the
// fully-masked kept rows of every query head of the group (one lane per key).
template <typename T, int D>
__global__ __launch_bounds__(kSimtRows) void k_fix_keys_b(GradDev G) {
    const PassDev& P = G.f;
    __shared__ float sQ[kSimtKT][D];
    __shared__ float sO[kSimtKT][D];
    __shared__ float sL[kSimtKT], sI[kSimtKT], sD[kSimtKT];
    const int b = blockIdx.z, kh = blockIdx.y;
    if (G.ws_kcnt[2 * ((int64_t)b * G.hk + kh) + 1] == 0) return;
    const int rep = P.heads / G.hk, h0 = kh * rep;
    const int j = blockIdx.x * kSimtRows + threadIdx.x;
    const bool mine = j < P.nk && P.km.keep(b, j) && bias_class(P.bias.scalar(b, h0, j)) == 1;
    if (!__syncthreads_or(mine)) return;
    float kk[D], vv[D], dk[D], dv[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        float kv = 0.f, v = 0.f;
        if (mine) {
            kv = to_f(P.k.row<T>(b, h0, j)[d]);
            v = to_f(P.v.row<T>(b, h0, j)[d]);
            if (P.vmul.ok()) v = round_to<T>(v * to_f(P.vmul.row<T>(b, h0, j)[d]));
        }
        kk[d] = kv;
        vv[d] = v;
        dk[d] = 0.f;
        dv[d] = 0.f;
    }
    float dbias = 0.f;
    const int j_first = blockIdx.x * kSimtRows;
    for (int h = h0; h < h0 + rep; ++h) {
        if (part_sum<D>(G, b, h, D + 1) == 0.f) continue;
        for (int i0 = 0; i0 < P.nq; i0 += kSimtKT) {
            const int cnt = min(kSimtKT, P.nq - i0);
            if (P.causal && i0 + cnt - 1 < j_first) continue;  // every row precedes these keys
            for (int ii = threadIdx.x; ii < kSimtKT; ii += blockDim.x) {
                const int i = i0 + ii;
                const int64_t r = ((int64_t)b * P.heads + h) * P.nq + i;
                const bool dg = i < P.nq && degenerate_row(G, r) && P.qm.keep(b, i);
                sL[ii] = dg ? 1.f : 0.f;
                sI[ii] = dg ? G.ws_invc[r] : 0.f;
                sD[ii] = dg ? G.ws_D[r] : 0.f;
            }
            __syncthreads();
            bool any = false;
            for (int ii = 0; ii < cnt; ++ii) any |= sL[ii] != 0.f;
            if (any) {
                for (int e = threadIdx.x; e < kSimtKT * D; e += blockDim.x) {
                    const int ii = e / D, d = e % D, i = i0 + ii;
                    const bool ok = i < P.nq;
                    sQ[ii][d] = ok ? to_f(P.q.row<T>(b, h, i)[d]) : 0.f;
                    sO[ii][d] = ok ? to_f(G.dout.row<T>(b, h, i)[d]) : 0.f;
                }
            }
            __syncthreads();
            if (any && mine) {
                for (int ii = 0; ii < cnt; ++ii) {
                    if (sL[ii] == 0.f || (P.causal && j > i0 + ii)) continue;
                    float s = 0.f, dp = 0.f;
#pragma unroll
                    for (int d = 0; d < D; ++d) {
                        s += sQ[ii][d] * kk[d];
                        dp += sO[ii][d] * vv[d];
                    }
                    const float y = softclamp_f(s * P.scale, P.softclamp);
                    const float ds = sI[ii] * (dp - sD[ii]);
                    const float g = ds * softclamp_grad(y, P.softclamp) * P.scale;
                    dbias += ds;
#pragma unroll
                    for (int d = 0; d < D; ++d) {
                        dv[d] += sI[ii] * sO[ii][d];
                        dk[d] += g * sQ[ii][d];
                    }
                }
            }
            __syncthreads();
        }
    }
    if (!mine) return;
    {
        T* o = G.dk.wrow<T>(b, h0, j);
        for (int d = 0; d < D; ++d) o[d] = from_f<T>(to_f(o[d]) + dk[d]);
    }
    {
        T* o = G.dv.wrow<T>(b, h0, j);
        const T* mul = P.vmul.ok() ? P.vmul.row<T>(b, h0, j) : nullptr;
        for (int d = 0; d < D; ++d) o[d] = from_f<T>(to_f(o[d]) + (mul ? dv[d] * to_f(mul[d]) : dv[d]));
    }
    if (P.vmul.ok()) {
        T* o = G.dvmul.wrow<T>(b, h0, j);
        const T* v = P.v.row<T>(b, h0, j);
        for (int d = 0; d < D; ++d) o[d] = from_f<T>(to_f(o[d]) + dv[d] * to_f(v[d]));
    }
    if (G.dbias.ok()) *G.dbias.wrow<float>(b, h0, j) += dbias;
}

// ---------------------------------------------------------------------------------------
// the module epilogue's backward (torch's autograd of y = round(round(r * o) * g'),
// g' = round(sigmoid(gate)), r = root or round(sigmoid(root)), each step rounded as torch
// rounds its intermediate tensors):
//   gt = round(dy * g'), dgate = round(round(dy * t) * (1 - g') * g')        (t = round(r * o))
//   dO = round(gt * r),  droot = sum over the heads sharing the root of round(gt * o)
//                                (times (1 - r) * r for a sigmoid root)
// Grid (row chunks, root head, batch); a thread takes W consecutive elements of one row of
// the root's [B, hr, nq, dim] (the pass's without a root) and the rep query heads sharing it.

template <typename T, int W>
struct alignas(sizeof(T) * W) EpiVec {
    T v[W];
};

template <typename T, int W>
__global__ __launch_bounds__(256) void k_epi_bwd(GradDev G, T* dO, int hr) {
    using V = EpiVec<T, W>;
    const PassDev& P = G.f;
    const int rep = P.heads / hr;
    const int rh = blockIdx.y, b = blockIdx.z;
    const int cpr = P.dim / W;  // chunks per row
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= P.nq * cpr) return;
    const int i = c / cpr, d = (c % cpr) * W;
    const bool has_r = P.er.ok(), has_g = P.eg.ok(), sig = (P.eflags & PA_EPI_ROOT_SIGMOID) != 0;
    float rp[W], dr[W];
    V rv;
    if (has_r) rv = *reinterpret_cast<const V*>(P.er.row<T>(b, rh * rep, i) + d);
#pragma unroll
    for (int e = 0; e < W; ++e) {
        rp[e] = has_r ? to_f(rv.v[e]) : 1.f;
        if (has_r && sig) rp[e] = round_to<T>(sigmoid_f(rp[e]));
        dr[e] = 0.f;
    }
    for (int k = 0; k < rep; ++k) {
        const int h = rh * rep + k;
        const V ov = *reinterpret_cast<const V*>(P.out.row<T>(b, h, i) + d);
        const V yv = *reinterpret_cast<const V*>(G.dout.row<T>(b, h, i) + d);
        V gv;
        if (has_g) gv = *reinterpret_cast<const V*>(P.eg.row<T>(b, h, i) + d);
        V go, dg;
#pragma unroll
        for (int e = 0; e < W; ++e) {
            const float o = to_f(ov.v[e]), dy = to_f(yv.v[e]);
            float gt = dy;
            if (has_g) {
                const float gp = round_to<T>(sigmoid_f(to_f(gv.v[e])));
                const float t = has_r ? round_to<T>(rp[e] * o) : o;
                gt = round_to<T>(dy * gp);
                dg.v[e] = from_f<T>(round_to<T>(dy * t) * (1.f - gp) * gp);
            }
            float g_o = gt;
            if (has_r) {
                g_o = round_to<T>(gt * rp[e]);
                dr[e] += round_to<T>(gt * o);
            }
            go.v[e] = from_f<T>(g_o);
        }
        *reinterpret_cast<V*>(dO + (((int64_t)b * P.heads + h) * P.nq + i) * P.dim + d) = go;
        if (has_g) *reinterpret_cast<V*>(G.dgate.wrow<T>(b, h, i) + d) = dg;
    }
    if (has_r) {
        V out;
#pragma unroll
        for (int e = 0; e < W; ++e) out.v[e] = from_f<T>(sig ? dr[e] * (1.f - rp[e]) * rp[e] : dr[e]);
        *reinterpret_cast<V*>(G.droot.wrow<T>(b, rh * rep, i) + d) = out;
    }
}

// ---------------------------------------------------------------------------------------
// launchers

template <typename T, int D>
static void launch_simt_fwd_t(const PassDev& P, hipStream_t s) {
    dim3 grid((P.nq + kSimtRows - 1) / kSimtRows, P.heads, P.batch);
    ProfScope ps("simt_fwd", s);
    hipLaunchKernelGGL((k_simt_fwd<T, D>), grid, dim3(kSimtRows), 0, s, P);
}
template <typename T, int D>
static void launch_fwd_fixup_t(const PassDev& P, hipStream_t s) {
    ProfScope ps("fwd_fixup", s);
    hipLaunchKernelGGL((k_fwd_fixup<T, D>), dim3(P.heads, P.batch), dim3(kFixThreads), 0, s, P);
}
template <typename T, int D>
static void launch_simt_bwd_t(const GradDev& G, hipStream_t s, bool pre, bool dq, bool dkv) {
    const PassDev& P = G.f;
    dim3 qgrid((P.nq + kSimtRows - 1) / kSimtRows, P.heads, P.batch);
    if (pre) {
        ProfScope ps("bwd_pre", s);
        auto al16 = [](const DView& v) {
            return (uintptr_t)v.p % 16 == 0 && v.sb % 8 == 0 && v.sh % 8 == 0 && v.sn % 8 == 0;
        };
        const bool vec = sizeof(T) == 2 && P.dim % 8 == 0 && al16(P.out) && al16(G.dout);
        if (vec) {
            int lpr = 1;
            while (lpr * 8 < P.dim) lpr <<= 1;
            const dim3 blocks((unsigned)(((int64_t)P.nq * lpr + 256 * kPreRows - 1) / (256 * kPreRows)),
                              P.heads, P.batch);
            switch (lpr) {
                case 1: hipLaunchKernelGGL((k_bwd_pre_vec<T, 1>), dim3(blocks), dim3(256), 0, s, G); break;
                case 2: hipLaunchKernelGGL((k_bwd_pre_vec<T, 2>), dim3(blocks), dim3(256), 0, s, G); break;
                case 4: hipLaunchKernelGGL((k_bwd_pre_vec<T, 4>), dim3(blocks), dim3(256), 0, s, G); break;
                case 8: hipLaunchKernelGGL((k_bwd_pre_vec<T, 8>), dim3(blocks), dim3(256), 0, s, G); break;
                case 16: hipLaunchKernelGGL((k_bwd_pre_vec<T, 16>), dim3(blocks), dim3(256), 0, s, G); break;
                default: hipLaunchKernelGGL((k_bwd_pre_vec<T, 32>), dim3(blocks), dim3(256), 0, s, G); break;
            }
        } else {
            hipLaunchKernelGGL((k_bwd_pre<T, D>), qgrid, dim3(kSimtRows), 0, s, G);
        }
    }
    if (dq) {
        ProfScope ps("simt_bwd_dq", s);
        hipLaunchKernelGGL((k_simt_bwd_dq<T, D>), qgrid, dim3(kSimtRows), 0, s, G);
    }
    if (dkv) {
        dim3 kgrid((P.nk + kSimtRows - 1) / kSimtRows, G.hk, P.batch);
        ProfScope ps("simt_bwd_dkv", s);
        hipLaunchKernelGGL((k_simt_bwd_dkv<T, D>), kgrid, dim3(kSimtRows), 0, s, G);
    }
}

template <typename T>
static void simt_fwd_d(const PassDev& P, hipStream_t s) {
    const int d = P.dim;
    if (d <= 16) launch_simt_fwd_t<T, 16>(P, s);
    else if (d <= 32) launch_simt_fwd_t<T, 32>(P, s);
    else if (d <= 64) launch_simt_fwd_t<T, 64>(P, s);
    else if (d <= 128) launch_simt_fwd_t<T, 128>(P, s);
    else launch_simt_fwd_t<T, 256>(P, s);
}

template <typename T>
static void simt_bwd_d(const GradDev& G, hipStream_t s, bool pre, bool dq, bool dkv) {
    const int d = G.f.dim;
    if (d <= 16) launch_simt_bwd_t<T, 16>(G, s, pre, dq, dkv);
    else if (d <= 32) launch_simt_bwd_t<T, 32>(G, s, pre, dq, dkv);
    else if (d <= 64) launch_simt_bwd_t<T, 64>(G, s, pre, dq, dkv);
    else if (d <= 128) launch_simt_bwd_t<T, 128>(G, s, pre, dq, dkv);
    else launch_simt_bwd_t<T, 256>(G, s, pre, dq, dkv);
}

template <typename T, int D>
static void launch_mask_fixups_t(const GradDev& G, hipStream_t s) {
    const PassDev& P = G.f;
    {
        ProfScope ps("fix_rows", s);
        hipLaunchKernelGGL((k_fix_rows<T, D>), dim3(fix_row_chunks(P.nq), P.heads, P.batch), dim3(256), 0, s, G);
    }
    {
        ProfScope ps("fix_keys", s);
        const dim3 grid((P.nk + kFixKeys - 1) / kFixKeys, G.hk, P.batch);
        hipLaunchKernelGGL((k_fix_keys<T, D>), grid, dim3(256), 0, s, G);
    }
    if (P.bias.ok()) {  // part B needs keys of bias class 1
        ProfScope ps("fix_part_b", s);
        const dim3 qgrid((P.nq + kSimtRows - 1) / kSimtRows, P.heads, P.batch);
        const dim3 kgrid((P.nk + kSimtRows - 1) / kSimtRows, G.hk, P.batch);
        hipLaunchKernelGGL((k_fix_rows_b<T, D>), qgrid, dim3(kSimtRows), 0, s, G);
        hipLaunchKernelGGL((k_fix_keys_b<T, D>), kgrid, dim3(kSimtRows), 0, s, G);
    }
}

template <typename T>
static void launch_epi_bwd_t(const GradDev& G, T* dO, int hr, hipStream_t s) {
    const PassDev& P = G.f;
    auto rows4 = [](const DView& v) {
        return !v.ok() || ((uintptr_t)v.p % 16 == 0 && v.sb % 4 == 0 && v.sh % 4 == 0 && v.sn % 4 == 0);
    };
    const bool vec = P.dim % 4 == 0 && rows4(P.out) && rows4(G.dout) && rows4(P.er) &&
                     rows4(P.eg) && rows4(G.droot) && rows4(G.dgate);
    const int w = vec ? 4 : 1;
    const dim3 grid((unsigned)(((int64_t)P.nq * (P.dim / w) + 255) / 256), hr, P.batch);
    if (vec) hipLaunchKernelGGL((k_epi_bwd<T, 4>), grid, dim3(256), 0, s, G, dO, hr);
    else hipLaunchKernelGGL((k_epi_bwd<T, 1>), grid, dim3(256), 0, s, G, dO, hr);
}

void launch_epi_bwd(const GradDev& G, void* dO, int hr, int dtype, hipStream_t s) {
    ProfScope ps("epi_bwd", s);
    if (dtype == PA_F32) launch_epi_bwd_t<float>(G, (float*)dO, hr, s);
    else if (dtype == PA_F16) launch_epi_bwd_t<f16>(G, (f16*)dO, hr, s);
    else launch_epi_bwd_t<bf16>(G, (bf16*)dO, hr, s);
}

void launch_key_terms(const GradDev& G, float* kterm, int nkp, int32_t* kcnt, int32_t* live,
                      hipStream_t s) {
    ProfScope ps("key_terms", s);
    hipLaunchKernelGGL(k_key_terms, dim3(G.hk, G.f.batch), dim3(kKeyTermThreads), 0, s, G, kterm,
                       nkp, kcnt, live);
}

template <typename T>
static void mask_fixups_d(const GradDev& G, hipStream_t s) {
    if (G.f.dim == 64) launch_mask_fixups_t<T, 64>(G, s);
    else if (G.f.dim == 128) launch_mask_fixups_t<T, 128>(G, s);
    else launch_mask_fixups_t<T, 256>(G, s);
}

// head dims 64 and 128 (every MFMA dtype) and 256 (16-bit)
void launch_mask_fixups(const GradDev& G, int dtype, hipStream_t s) {
    if (dtype == PA_F32) G.f.dim == 64 ? launch_mask_fixups_t<float, 64>(G, s) : launch_mask_fixups_t<float, 128>(G, s);
    else if (dtype == PA_F16) mask_fixups_d<f16>(G, s);
    else mask_fixups_d<bf16>(G, s);
}

void launch_simt_fwd(const PassDev& P, int dtype, hipStream_t s) {
    if (dtype == PA_F32) simt_fwd_d<float>(P, s);
    else if (dtype == PA_F16) simt_fwd_d<f16>(P, s);
    else simt_fwd_d<bf16>(P, s);
}
template <typename T>
static void fwd_fixup_d(const PassDev& P, hipStream_t s) {
    if (P.dim == 64) launch_fwd_fixup_t<T, 64>(P, s);
    else if (P.dim == 128) launch_fwd_fixup_t<T, 128>(P, s);
    else launch_fwd_fixup_t<T, 256>(P, s);
}

// head dims 64 and 128 (every MFMA dtype) and 256 (16-bit)
void launch_fwd_fixup(const PassDev& P, int dtype, hipStream_t s) {
    if (dtype == PA_F32) P.dim == 64 ? launch_fwd_fixup_t<float, 64>(P, s) : launch_fwd_fixup_t<float, 128>(P, s);
    else if (dtype == PA_F16) fwd_fixup_d<f16>(P, s);
    else fwd_fixup_d<bf16>(P, s);
}
void launch_simt_bwd(const GradDev& G, int dtype, hipStream_t s, bool pre, bool dq, bool dkv) {
    if (dtype == PA_F32) simt_bwd_d<float>(G, s, pre, dq, dkv);
    else if (dtype == PA_F16) simt_bwd_d<f16>(G, s, pre, dq, dkv);
    else simt_bwd_d<bf16>(G, s, pre, dq, dkv);
}

}  // namespace pa
