// pa_mfma_f32.hip -- fp32 attention passes on the matrix cores (v_mfma_f32_32x32x2_f32),
// head dim 64 or 128: the forward (every pass feature), and the backward of unmasked passes
// (k_mfma_bwd_f32_dq / k_mfma_bwd_f32_dkv, described at the kernels).
//
// Forward:
// A workgroup of nw waves (1, 2 or 4, chosen by the grid size) owns 32 * nw queries of one
// (batch, head); each wave owns 32.  Per 32-key tile staged in LDS (K, the effective value
// v * vmul, the key term):
//   S^T = K Q^T: D/2 MFMAs with K[key = l%32][2s + l/32] from LDS as A and the wave's
//     Q[q = l%32][2s + l/32] held in registers as B, so lane l holds query l % 32 and the keys
//     8*(r/4) + 4*(l/32) + (r%4) of its 16 accumulator registers r -- the softmax state is per
//     lane, combined with the lane 32 apart;
//   O^T += V^T P^T: MFMA step r pairs the two keys lanes l < 32 and l >= 32 hold in register r,
//     so the probabilities enter as B straight from the score registers and V[key][d] is read
//     from LDS as A (consecutive d across lanes).
// Everything stays fp32 (no operand rounding), exp2 on the hardware unit, an online softmax
// with the running max shared by the lane pair.  Masks, key bias classes, value multiplier,
// softclamp, causal limits and the module epilogue follow the pass semantics of polyattn.h;
// rows left fully masked get lse = NaN for k_fwd_fixup, as in the 16-bit kernels.
#include <algorithm>

#include "pa_common.h"
#include "pa_launch.h"
#include "pa_mfma.h"

namespace pa {

constexpr int kF32BN = 32;  // keys per tile
#ifndef PA_F32_SPLIT
#define PA_F32_SPLIT 1  // small grids: the forward split over the keys (k_mfma_fwd_f32_split)
#endif

__device__ __forceinline__ f32x16_t mfma_32x32x2(float a, float b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// One wave's online-softmax state for its 32 queries: O^T accumulators, the running max (log2
// units, shared by the lane pair) and the lane's partial sum.
template <int D>
struct F32Acc {
    f32x16_t o[D / 32];
    float m, l;
};

// One 32-key tile (rows j0 .. j0 + 31 staged at sK / sV with row stride D + 1, key term sB):
// S^T = K Q^T, the softmax update, O^T += V^T P^T.
template <int D>
__device__ __forceinline__ void f32_tile(F32Acc<D>& a, const float (&qf)[D / 2], const float* sK,
                                         const float* sV, const float* sB, int j0, int qi, int col,
                                         int hh, const PassDev& P, bool sc, bool causal) {
    constexpr int RS = D + 1;
    f32x16_t s = zero16();
#pragma unroll
    for (int st = 0; st < D / 2; ++st) s = mfma_32x32x2(sK[col * RS + 2 * st + hh], qf[st], s);
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int jj = 8 * (r / 4) + 4 * hh + (r % 4);
        float y = s[r] * P.scale;
        if (sc) y = softclamp_f(y, P.softclamp);
        float t = y * kLog2e + sB[jj];
        if (causal && j0 + jj > qi) t = -INFINITY;
        s[r] = t;
        tmax = fmaxf(tmax, t);
    }
    const float mnew = fmaxf(a.m, xhalf_max(tmax));
    if (mnew > a.m) {
        const float c = a.m == -INFINITY ? 0.f : fast_exp2(a.m - mnew);
        a.l *= c;
#pragma unroll
        for (int x = 0; x < D / 32; ++x)
#pragma unroll
            for (int r = 0; r < 16; ++r) a.o[x][r] *= c;
        a.m = mnew;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float p = a.m == -INFINITY ? 0.f : fast_exp2(s[r] - a.m);
        s[r] = p;
        a.l += p;
    }
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int jj = 8 * (r / 4) + 4 * hh + (r % 4);
            a.o[x] = mfma_32x32x2(sV[jj * RS + 32 * x + col], s[r], a.o[x]);
        }
}

// The 32 queries' outputs, lse (NaN for a row left fully masked, for k_fwd_fixup) and the
// module epilogue.
template <int D>
__device__ __forceinline__ void f32_store(const F32Acc<D>& a, const PassDev& P, int b, int h,
                                          int qi, int hh) {
    const float lt = xhalf_sum(a.l);
    if (qi >= P.nq) return;
    const bool degenerate = !(lt > 0.f) || !P.qm.keep(b, qi);
    const float inv = degenerate ? 0.f : 1.f / lt;
    float* orow = P.out.wrow<float>(b, h, qi);
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * x + 8 * g + 4 * hh;
            const float4 v = make_float4(a.o[x][4 * g] * inv, a.o[x][4 * g + 1] * inv,
                                         a.o[x][4 * g + 2] * inv, a.o[x][4 * g + 3] * inv);
            *reinterpret_cast<float4*>(orow + d) = v;
            if (P.ey.ok()) {
                float* yrow = P.ey.wrow<float>(b, h, qi);
                yrow[d] = epi_y<float>(P, b, h, qi, d, v.x);
                yrow[d + 1] = epi_y<float>(P, b, h, qi, d + 1, v.y);
                yrow[d + 2] = epi_y<float>(P, b, h, qi, d + 2, v.z);
                yrow[d + 3] = epi_y<float>(P, b, h, qi, d + 3, v.w);
            }
        }
    if (hh == 0) *P.lse.wrow<float>(b, h, qi) = degenerate ? NAN : (a.m + log2f(lt)) * kLn2;
}

// Q[qi][2s + hh] of the lane's query (zeros past the last query)
template <int D>
__device__ __forceinline__ void f32_load_q(const PassDev& P, int b, int h, int qi, int hh,
                                           float (&qf)[D / 2]) {
    const bool qrow = qi < P.nq;
    const float* qr = P.q.row<float>(b, h, qrow ? qi : 0);
#pragma unroll
    for (int s = 0; s < D / 2; ++s) qf[s] = qrow ? qr[2 * s + hh] : 0.f;
}

template <int D>
__global__ __launch_bounds__(256) void k_mfma_fwd_f32(PassDev P) {
    constexpr int RS = D + 1;  // LDS row stride (odd: the K reads of 32 rows hit 32 banks)
    __shared__ float sK[kF32BN * RS];
    __shared__ float sV[kF32BN * RS];
    __shared__ float sB[kF32BN];  // key term in log2 units: bias * log2e, -inf when masked

    const int nw = blockDim.x >> 6;
    const int BM = 32 * nw;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const bool causal = P.causal != 0;
    const int nqb = (P.nq + BM - 1) / BM;
    int bh, rank;
    if (causal) block_order<true>(nqb, P.heads, P.k.hdiv, bh, rank);
    else block_order<false>(nqb, P.heads, P.k.hdiv, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;
    const int h = bh % P.heads, b = bh / P.heads;
    const int col = lane & 31, hh = lane >> 5;
    const int q0 = qb * BM + w * 32;
    const int qi = q0 + col;

    float qf[D / 2];  // Q[qi][2s + hh]
    f32_load_q<D>(P, b, h, qi, hh, qf);
    F32Acc<D> a;
#pragma unroll
    for (int x = 0; x < D / 32; ++x) a.o[x] = zero16();
    a.m = -INFINITY;
    a.l = 0.f;

    const bool sc = P.softclamp > 0.f, has_vmul = P.vmul.ok(), has_bias = P.bias.ok();
    const int kend = causal ? min(P.nk, qb * BM + BM) : P.nk;
    const int wave_kend = causal ? min(kend, q0 + 32) : kend;

    // a key tile's K rows, effective value rows and key term travel through registers: the
    // next tile's loads are in flight while the current tile is computed
    constexpr int NL = kF32BN * (D / 4) / 64;  // 16-byte loads per thread and tensor (one wave)
    const int nload = kF32BN * (D / 4);
    float4 rk[NL], rv[NL];
    float rb = 0.f;
    auto load_tile = [&](int j0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int e = tid + i * (int)blockDim.x;
            const int jj = e / (D / 4), c4 = (e % (D / 4)) * 4, j = j0 + jj;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (e < nload && j < P.nk) {
                kv = *reinterpret_cast<const float4*>(P.k.row<float>(b, h, j) + c4);
                vv = *reinterpret_cast<const float4*>(P.v.row<float>(b, h, j) + c4);
                if (has_vmul) {
                    const float4 mm = *reinterpret_cast<const float4*>(P.vmul.row<float>(b, h, j) + c4);
                    vv.x *= mm.x;
                    vv.y *= mm.y;
                    vv.z *= mm.z;
                    vv.w *= mm.w;
                }
            }
            rk[i] = kv;
            rv[i] = vv;
        }
        if (tid < kF32BN) {
            const int j = j0 + tid;
            rb = -INFINITY;
            if (j < P.nk && P.km.keep(b, j)) {
                const float x = has_bias ? P.bias.scalar(b, h, j) : 0.f;
                rb = bias_class(x) == 0 ? x * kLog2e : -INFINITY;
            }
        }
    };
    auto store_tile = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int e = tid + i * (int)blockDim.x;
            if (e < nload) {
                const int jj = e / (D / 4), c4 = (e % (D / 4)) * 4;
                float* dk = sK + jj * RS + c4;
                float* dv = sV + jj * RS + c4;
                dk[0] = rk[i].x;
                dk[1] = rk[i].y;
                dk[2] = rk[i].z;
                dk[3] = rk[i].w;
                dv[0] = rv[i].x;
                dv[1] = rv[i].y;
                dv[2] = rv[i].z;
                dv[3] = rv[i].w;
            }
        }
        if (tid < kF32BN) sB[tid] = rb;
    };

    if (kend > 0) load_tile(0);
    for (int j0 = 0; j0 < kend; j0 += kF32BN) {
        store_tile();
        __syncthreads();
        if (j0 + kF32BN < kend) load_tile(j0 + kF32BN);
        if (j0 < wave_kend)  // wave-uniform: the causal limit of this wave's queries
            f32_tile<D>(a, qf, sK, sV, sB, j0, qi, col, hh, P, sc, causal);
        __syncthreads();
    }
    f32_store<D>(a, P, b, h, qi, hh);  // no barriers below
}

// Split over the keys, for grids too small to occupy the chip (config 1: 8 heads x 1024
// queries is 256 blocks of 32 queries): NS waves share one 32-query block, wave w taking key
// tiles w, w + NS, ...  Each wave stages its own tiles in its own LDS region (wave-level order
// only: a wave's LDS operations complete in order), keeps its own softmax state, and after a
// workgroup barrier leaves (m, l, O) in its region; wave 0 merges the NS states (scaled by
// 2^(m_w - max m)) and stores.
template <int D, int NS>
__global__ __launch_bounds__(64 * NS) void k_mfma_fwd_f32_split(PassDev P) {
    constexpr int RS = D + 1;
    constexpr int TILE = 2 * kF32BN * RS + kF32BN;  // K, V rows and the key term
    static_assert(TILE >= (D / 32) * 16 * 64 + 2 * 64, "a wave's region holds its state");
    __shared__ float sT[NS][TILE];
    const int lane = threadIdx.x & 63, w = wave_id();
    float* sK = sT[w];
    float* sV = sK + kF32BN * RS;
    float* sB = sV + kF32BN * RS;
    const bool causal = P.causal != 0;
    const int nqb = (P.nq + 31) / 32;
    int bh, rank;
    if (causal) block_order<true>(nqb, P.heads, P.k.hdiv, bh, rank);
    else block_order<false>(nqb, P.heads, P.k.hdiv, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;
    const int h = bh % P.heads, b = bh / P.heads;
    const int col = lane & 31, hh = lane >> 5;
    const int q0 = qb * 32, qi = q0 + col;

    float qf[D / 2];
    f32_load_q<D>(P, b, h, qi, hh, qf);
    F32Acc<D> a;
#pragma unroll
    for (int x = 0; x < D / 32; ++x) a.o[x] = zero16();
    a.m = -INFINITY;
    a.l = 0.f;
    const bool sc = P.softclamp > 0.f, has_vmul = P.vmul.ok(), has_bias = P.bias.ok();
    const int kend = causal ? min(P.nk, q0 + 32) : P.nk;

    constexpr int NL = kF32BN * (D / 4) / 64;  // 16-byte loads per lane and tensor
    float4 rk[NL], rv[NL];
    float rb = 0.f;
    auto load_tile = [&](int j0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int e = lane + 64 * i, jj = e / (D / 4), c4 = (e % (D / 4)) * 4, j = j0 + jj;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (j < P.nk) {
                kv = *reinterpret_cast<const float4*>(P.k.row<float>(b, h, j) + c4);
                vv = *reinterpret_cast<const float4*>(P.v.row<float>(b, h, j) + c4);
                if (has_vmul) {
                    const float4 mm = *reinterpret_cast<const float4*>(P.vmul.row<float>(b, h, j) + c4);
                    vv.x *= mm.x;
                    vv.y *= mm.y;
                    vv.z *= mm.z;
                    vv.w *= mm.w;
                }
            }
            rk[i] = kv;
            rv[i] = vv;
        }
        if (lane < kF32BN) {
            const int j = j0 + lane;
            rb = -INFINITY;
            if (j < P.nk && P.km.keep(b, j)) {
                const float x = has_bias ? P.bias.scalar(b, h, j) : 0.f;
                rb = bias_class(x) == 0 ? x * kLog2e : -INFINITY;
            }
        }
    };
    auto store_tile = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int e = lane + 64 * i, jj = e / (D / 4), c4 = (e % (D / 4)) * 4;
            float* dk = sK + jj * RS + c4;
            float* dv = sV + jj * RS + c4;
            dk[0] = rk[i].x;
            dk[1] = rk[i].y;
            dk[2] = rk[i].z;
            dk[3] = rk[i].w;
            dv[0] = rv[i].x;
            dv[1] = rv[i].y;
            dv[2] = rv[i].z;
            dv[3] = rv[i].w;
        }
        if (lane < kF32BN) sB[lane] = rb;
    };
    // a wave's own LDS writes before its reads (and its reads before the next tile's writes)
    auto wave_sync = []() __attribute__((always_inline)) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        asm volatile("" ::: "memory");
    };

    const int ntiles = (kend + kF32BN - 1) / kF32BN;
    if (w < ntiles) load_tile(w * kF32BN);
    for (int t = w; t < ntiles; t += NS) {  // wave-uniform
        wave_sync();
        store_tile();
        wave_sync();
        if (t + NS < ntiles) load_tile((t + NS) * kF32BN);
        f32_tile<D>(a, qf, sK, sV, sB, t * kF32BN, qi, col, hh, P, sc, causal);
    }

    // every wave's state into its region, then wave 0 merges
    __syncthreads();
    {
        float* so = sT[w];
#pragma unroll
        for (int x = 0; x < D / 32; ++x)
#pragma unroll
            for (int r = 0; r < 16; ++r) so[(x * 16 + r) * 64 + lane] = a.o[x][r];
        so[(D / 32) * 16 * 64 + lane] = a.m;
        so[(D / 32) * 16 * 64 + 64 + lane] = a.l;
    }
    __syncthreads();
    if (w != 0) return;  // no barriers below
    float mt = -INFINITY;
#pragma unroll
    for (int v = 0; v < NS; ++v) mt = fmaxf(mt, sT[v][(D / 32) * 16 * 64 + lane]);
    F32Acc<D> r;
#pragma unroll
    for (int x = 0; x < D / 32; ++x) r.o[x] = zero16();
    r.m = mt;
    r.l = 0.f;
#pragma unroll
    for (int v = 0; v < NS; ++v) {
        const float* so = sT[v];
        const float mv = so[(D / 32) * 16 * 64 + lane];
        const float c = mv == -INFINITY ? 0.f : fast_exp2(mv - mt);
        r.l += so[(D / 32) * 16 * 64 + 64 + lane] * c;
#pragma unroll
        for (int x = 0; x < D / 32; ++x)
#pragma unroll
            for (int q = 0; q < 16; ++q) r.o[x][q] += so[(x * 16 + q) * 64 + lane] * c;
    }
    f32_store<D>(r, P, b, h, qi, hh);
}

// ---------------------------------------------------------------------------------------
// backward (unmasked passes; after the row preprocess: ws_lse, ws_D)

// Stage 32 rows [r0, r0 + 32) of two [n, D] fp32 views of (b, h) in LDS (row stride RS)
// through registers; rows past n read as zero.
template <int D>
struct F32Rows {
    static constexpr int NL = kF32BN * (D / 4) / 64;  // 16-byte loads per thread (one wave)
    float4 a[NL], c[NL];
    __device__ __forceinline__ void load(const DView& va, const DView& vc, const DView& vm, int b,
                                         int h, int r0, int n, int t0 = -1, int ts = 0) {
        const int nload = kF32BN * (D / 4);
        if (t0 < 0) {  // spread over the workgroup
            t0 = threadIdx.x;
            ts = blockDim.x;
        }
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int e = t0 + i * ts;
            const int rr = e / (D / 4), c4 = (e % (D / 4)) * 4, r = r0 + rr;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
            if (e < nload && r < n) {
                x = *reinterpret_cast<const float4*>(va.row<float>(b, h, r) + c4);
                y = *reinterpret_cast<const float4*>(vc.row<float>(b, h, r) + c4);
                if (vm.ok()) {  // effective value v * vmul
                    const float4 mm = *reinterpret_cast<const float4*>(vm.row<float>(b, h, r) + c4);
                    y.x *= mm.x;
                    y.y *= mm.y;
                    y.z *= mm.z;
                    y.w *= mm.w;
                }
            }
            a[i] = x;
            c[i] = y;
        }
    }
    __device__ __forceinline__ void store(float* sa, float* sc, int t0 = -1, int ts = 0) const {
        constexpr int RS = D + 1;
        const int nload = kF32BN * (D / 4);
        if (t0 < 0) {
            t0 = threadIdx.x;
            ts = blockDim.x;
        }
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int e = t0 + i * ts;
            if (e < nload) {
                const int rr = e / (D / 4), c4 = (e % (D / 4)) * 4;
                float* da = sa + rr * RS + c4;
                float* dc = sc + rr * RS + c4;
                da[0] = a[i].x;
                da[1] = a[i].y;
                da[2] = a[i].z;
                da[3] = a[i].w;
                dc[0] = c[i].x;
                dc[1] = c[i].y;
                dc[2] = c[i].z;
                dc[3] = c[i].w;
            }
        }
    }
};

__device__ __forceinline__ float key_term_l2(const PassDev& P, int b, int h, int j) {
    if (j >= P.nk) return -INFINITY;
    const float x = P.bias.ok() ? P.bias.scalar(b, h, j) : 0.f;
    return bias_class(x) == 0 ? x * kLog2e : -INFINITY;
}

// one 4-element group of an output row: value (+ the old value with accumulate)
__device__ __forceinline__ void store4(float* p, float4 v, bool acc) {
    if (acc) {
        const float4 o = *reinterpret_cast<const float4*>(p);
        v.x += o.x;
        v.y += o.y;
        v.z += o.z;
        v.w += o.w;
    }
    *reinterpret_cast<float4*>(p) = v;
}

// dQ, query-major: per key tile S^T = K Q^T and dP^T = V dO^T (lane = query), dS, then
// dQ^T += K^T dS^T with dS entering as B from the score registers.
// dQ of one 32-key tile (rows j0 .. j0 + 31 staged at sK / sV, key term sB): S = Q K^T and
// dP = dO V^T (lane = query), dS = P (dP - D), dQ^T += K^T dS^T with dS entering as B.
template <int D>
__device__ __forceinline__ void f32_dq_tile(f32x16_t (&dq)[D / 32], const float (&qf)[D / 2],
                                            const float (&of)[D / 2], const float* sK,
                                            const float* sV, const float* sB, int j0, int qi,
                                            int col, int hh, const PassDev& P, bool sc,
                                            bool causal, float lse_l2, float dsum) {
    constexpr int RS = D + 1;
    f32x16_t s = zero16(), dp = zero16();
#pragma unroll
    for (int t = 0; t < D / 2; ++t) {
        s = mfma_32x32x2(sK[col * RS + 2 * t + hh], qf[t], s);
        dp = mfma_32x32x2(sV[col * RS + 2 * t + hh], of[t], dp);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int jj = 8 * (i / 4) + 4 * hh + (i % 4);
        float y = s[i] * P.scale;
        if (sc) y = softclamp_f(y, P.softclamp);
        float t = y * kLog2e + sB[jj];
        if (causal && j0 + jj > qi) t = -INFINITY;
        const float p = fast_exp2(t - lse_l2);
        s[i] = p * (dp[i] - dsum) * softclamp_grad(y, P.softclamp) * P.scale;
    }
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int jj = 8 * (i / 4) + 4 * hh + (i % 4);
            dq[x] = mfma_32x32x2(sK[jj * RS + 32 * x + col], s[i], dq[x]);
        }
}

// dK / dV / dbias of one 32-query tile (rows i0 .. i0 + 31 of Q and dO at sQ / sO, their lse
// (log2) and D at sL / sD) against the wave's 32 keys (lane = key).
template <int D>
__device__ __forceinline__ void f32_dkv_tile(f32x16_t (&dk)[D / 32], f32x16_t (&dv)[D / 32],
                                             float& dbias, const float (&kf)[D / 2],
                                             const float (&vf)[D / 2], const float* sQ,
                                             const float* sO, const float* sL, const float* sD,
                                             int i0, int kj, int col, int hh, const PassDev& P,
                                             bool sc, bool causal, float bk) {
    constexpr int RS = D + 1;
    f32x16_t s = zero16(), dp = zero16();
#pragma unroll
    for (int t = 0; t < D / 2; ++t) {
        s = mfma_32x32x2(sQ[col * RS + 2 * t + hh], kf[t], s);
        dp = mfma_32x32x2(sO[col * RS + 2 * t + hh], vf[t], dp);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int ii = 8 * (i / 4) + 4 * hh + (i % 4);
        float y = s[i] * P.scale;
        if (sc) y = softclamp_f(y, P.softclamp);
        float t = y * kLog2e + bk;
        if (causal && i0 + ii < kj) t = -INFINITY;
        const float p = fast_exp2(t - sL[ii]);
        const float ds = p * (dp[i] - sD[ii]);
        dbias += ds;
        s[i] = p;
        dp[i] = ds * softclamp_grad(y, P.softclamp) * P.scale;
    }
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int ii = 8 * (i / 4) + 4 * hh + (i % 4);
            dv[x] = mfma_32x32x2(sO[ii * RS + 32 * x + col], s[i], dv[x]);
            dk[x] = mfma_32x32x2(sQ[ii * RS + 32 * x + col], dp[i], dk[x]);
        }
}

template <int D>
__global__ __launch_bounds__(256) void k_mfma_bwd_f32_dq(GradDev G) {
    constexpr int RS = D + 1;
    const PassDev& P = G.f;
    __shared__ float sK[kF32BN * RS];
    __shared__ float sV[kF32BN * RS];
    __shared__ float sB[kF32BN];
    const int nw = blockDim.x >> 6;
    const int BM = 32 * nw;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const bool causal = P.causal != 0;
    const int nqb = (P.nq + BM - 1) / BM;
    int bh, rank;
    if (causal) block_order<true>(nqb, P.heads, P.k.hdiv, bh, rank);
    else block_order<false>(nqb, P.heads, P.k.hdiv, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;
    const int h = bh % P.heads, b = bh / P.heads;
    const int col = lane & 31, hh = lane >> 5;
    const int q0 = qb * BM + w * 32, qi = q0 + col;
    const bool qrow = qi < P.nq;
    float qf[D / 2], of[D / 2];
    {
        const float* qr = P.q.row<float>(b, h, qrow ? qi : 0);
        const float* orr = G.dout.row<float>(b, h, qrow ? qi : 0);
#pragma unroll
        for (int s = 0; s < D / 2; ++s) {
            qf[s] = qrow ? qr[2 * s + hh] : 0.f;
            of[s] = qrow ? orr[2 * s + hh] : 0.f;
        }
    }
    const int64_t r = ((int64_t)b * P.heads + h) * P.nq + (qrow ? qi : 0);
    const float lse_l2 = qrow ? G.ws_lse[r] * kLog2e : INFINITY;
    const float dsum = qrow ? G.ws_D[r] : 0.f;
    f32x16_t dq[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) dq[x] = zero16();
    const bool sc = P.softclamp > 0.f;
    const int kend = causal ? min(P.nk, qb * BM + BM) : P.nk;
    const int wave_kend = causal ? min(kend, q0 + 32) : kend;
    F32Rows<D> st;
    float rb = 0.f;
    if (kend > 0) {
        st.load(P.k, P.v, P.vmul, b, h, 0, P.nk);
        if (tid < kF32BN) rb = key_term_l2(P, b, h, tid);
    }
    for (int j0 = 0; j0 < kend; j0 += kF32BN) {
        st.store(sK, sV);
        if (tid < kF32BN) sB[tid] = rb;
        __syncthreads();
        if (j0 + kF32BN < kend) {
            st.load(P.k, P.v, P.vmul, b, h, j0 + kF32BN, P.nk);
            if (tid < kF32BN) rb = key_term_l2(P, b, h, j0 + kF32BN + tid);
        }
        if (j0 < wave_kend)
            f32_dq_tile<D>(dq, qf, of, sK, sV, sB, j0, qi, col, hh, P, sc, causal, lse_l2, dsum);
        __syncthreads();
    }
    if (!qrow) return;
    float* row = G.dq.wrow<float>(b, h, qi);
    const bool acc = (G.accumulate & PA_ACC_DQ) != 0;
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            store4(row + 32 * x + 8 * g + 4 * hh,
                   make_float4(dq[x][4 * g], dq[x][4 * g + 1], dq[x][4 * g + 2], dq[x][4 * g + 3]), acc);
}

// dK / dV / dbias, key-major: the wave's 32 keys (K and the effective value in registers as B
// operands) against the query tiles of every query head of the group: C = Q K^T and
// dP = dO V^T (lane = key), dV^T += dO^T P and dK^T += Q^T dS with P / dS entering as B.
template <int D>
__global__ __launch_bounds__(256) void k_mfma_bwd_f32_dkv(GradDev G) {
    constexpr int RS = D + 1;
    const PassDev& P = G.f;
    __shared__ float sQ[kF32BN * RS];
    __shared__ float sO[kF32BN * RS];
    __shared__ float sL[kF32BN], sD[kF32BN];
    const int nw = blockDim.x >> 6;
    const int BK = 32 * nw;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const bool causal = P.causal != 0;
    const int nkb = (P.nk + BK - 1) / BK;
    int unit, kblk;  // causal: the first key blocks carry the most work
    if (causal) block_order<true>(nkb, G.hk, 1, unit, kblk);
    else block_order<false>(nkb, G.hk, 1, unit, kblk);
    const int kh = unit % G.hk, b = unit / G.hk;
    const int rep = P.heads / G.hk, h0 = kh * rep;
    const int col = lane & 31, hh = lane >> 5;
    const int k0 = kblk * BK + w * 32, kj = k0 + col;
    const bool krow = kj < P.nk;
    float kf[D / 2], vf[D / 2];
    {
        const float* kr = P.k.row<float>(b, h0, krow ? kj : 0);
        const float* vr = P.v.row<float>(b, h0, krow ? kj : 0);
        const float* mr = P.vmul.ok() ? P.vmul.row<float>(b, h0, krow ? kj : 0) : nullptr;
#pragma unroll
        for (int s = 0; s < D / 2; ++s) {
            kf[s] = krow ? kr[2 * s + hh] : 0.f;
            vf[s] = krow ? vr[2 * s + hh] * (mr ? mr[2 * s + hh] : 1.f) : 0.f;
        }
    }
    const float bk = key_term_l2(P, b, h0, kj);  // -inf past nk
    f32x16_t dk[D / 32], dv[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
        dk[x] = zero16();
        dv[x] = zero16();
    }
    float dbias = 0.f;
    const bool sc = P.softclamp > 0.f;
    const int i_start = causal ? (kblk * BK / kF32BN) * kF32BN : 0;
    const DView none = {nullptr, 0, 0, 0, 1, PA_F32};
    for (int hr = 0; hr < rep; ++hr) {
        const int h = h0 + hr;
        const int64_t row0 = ((int64_t)b * P.heads + h) * P.nq;
        F32Rows<D> st;
        float rl = 0.f, rd = 0.f;
        auto load_rows = [&](int i0) __attribute__((always_inline)) {
            st.load(P.q, G.dout, none, b, h, i0, P.nq);
            if (tid < kF32BN) {
                const int i = i0 + tid;
                rl = i < P.nq ? G.ws_lse[row0 + i] * kLog2e : INFINITY;
                rd = i < P.nq ? G.ws_D[row0 + i] : 0.f;
            }
        };
        if (i_start < P.nq) load_rows(i_start);
        for (int i0 = i_start; i0 < P.nq; i0 += kF32BN) {
            st.store(sQ, sO);
            if (tid < kF32BN) {
                sL[tid] = rl;
                sD[tid] = rd;
            }
            __syncthreads();
            if (i0 + kF32BN < P.nq) load_rows(i0 + kF32BN);
            if (!causal || i0 + kF32BN - 1 >= k0)  // wave-uniform: some query reaches a key
                f32_dkv_tile<D>(dk, dv, dbias, kf, vf, sQ, sO, sL, sD, i0, kj, col, hh, P, sc,
                                causal, bk);
            __syncthreads();
        }
    }
    dbias = xhalf_sum(dbias);
    if (!krow) return;
    const float* mr = P.vmul.ok() ? P.vmul.row<float>(b, h0, kj) : nullptr;
    const float* vr = P.v.row<float>(b, h0, kj);
    float* dkr = G.dk.wrow<float>(b, h0, kj);
    float* dvr = G.dv.wrow<float>(b, h0, kj);
    float* dmr = mr ? G.dvmul.wrow<float>(b, h0, kj) : nullptr;
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * x + 8 * g + 4 * hh;
            store4(dkr + d, make_float4(dk[x][4 * g], dk[x][4 * g + 1], dk[x][4 * g + 2], dk[x][4 * g + 3]),
                   (G.accumulate & PA_ACC_DK) != 0);
            float4 e = make_float4(dv[x][4 * g], dv[x][4 * g + 1], dv[x][4 * g + 2], dv[x][4 * g + 3]);
            if (mr) {
                const float4 m4 = *reinterpret_cast<const float4*>(mr + d);
                const float4 v4 = *reinterpret_cast<const float4*>(vr + d);
                store4(dmr + d, make_float4(e.x * v4.x, e.y * v4.y, e.z * v4.z, e.w * v4.w),
                       (G.accumulate & PA_ACC_DVMUL) != 0);
                e = make_float4(e.x * m4.x, e.y * m4.y, e.z * m4.z, e.w * m4.w);
            }
            store4(dvr + d, e, (G.accumulate & PA_ACC_DV) != 0);
        }
    if (hh == 0 && G.dbias.ok()) {
        float* o = G.dbias.wrow<float>(b, h0, kj);
        *o = dbias + ((G.accumulate & PA_ACC_DBIAS) ? *o : 0.f);
    }
}

// The backward split like k_mfma_fwd_f32_split, for grids too small to occupy the chip: NS
// waves share one 32-row block, each taking every NS-th tile into its own LDS region (wave-level
// order only); after a workgroup barrier every wave leaves its partial sums in its region and
// wave 0 adds them in wave order (deterministic) and stores.
__device__ __forceinline__ void f32_wave_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
}

template <int D, int NS>
__global__ __launch_bounds__(64 * NS) void k_mfma_bwd_f32_dq_split(GradDev G) {
    constexpr int RS = D + 1;
    constexpr int TILE = 2 * kF32BN * RS + kF32BN;
    static_assert(TILE >= (D / 32) * 16 * 64, "a wave's region holds its partial dQ");
    const PassDev& P = G.f;
    __shared__ float sT[NS][TILE];
    const int lane = threadIdx.x & 63, w = wave_id();
    float* sK = sT[w];
    float* sV = sK + kF32BN * RS;
    float* sB = sV + kF32BN * RS;
    const bool causal = P.causal != 0;
    const int nqb = (P.nq + 31) / 32;
    int bh, rank;
    if (causal) block_order<true>(nqb, P.heads, P.k.hdiv, bh, rank);
    else block_order<false>(nqb, P.heads, P.k.hdiv, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;
    const int h = bh % P.heads, b = bh / P.heads;
    const int col = lane & 31, hh = lane >> 5;
    const int q0 = qb * 32, qi = q0 + col;
    const bool qrow = qi < P.nq;
    float qf[D / 2], of[D / 2];
    {
        const float* qr = P.q.row<float>(b, h, qrow ? qi : 0);
        const float* orr = G.dout.row<float>(b, h, qrow ? qi : 0);
#pragma unroll
        for (int t = 0; t < D / 2; ++t) {
            qf[t] = qrow ? qr[2 * t + hh] : 0.f;
            of[t] = qrow ? orr[2 * t + hh] : 0.f;
        }
    }
    const int64_t r = ((int64_t)b * P.heads + h) * P.nq + (qrow ? qi : 0);
    const float lse_l2 = qrow ? G.ws_lse[r] * kLog2e : INFINITY;
    const float dsum = qrow ? G.ws_D[r] : 0.f;
    f32x16_t dq[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) dq[x] = zero16();
    const bool sc = P.softclamp > 0.f;
    const int kend = causal ? min(P.nk, q0 + 32) : P.nk;
    const int ntiles = (kend + kF32BN - 1) / kF32BN;
    F32Rows<D> st;
    float rb = 0.f;
    if (w < ntiles) {
        st.load(P.k, P.v, P.vmul, b, h, w * kF32BN, P.nk, lane, 64);
        if (lane < kF32BN) rb = key_term_l2(P, b, h, w * kF32BN + lane);
    }
    for (int t = w; t < ntiles; t += NS) {  // wave-uniform
        f32_wave_sync();
        st.store(sK, sV, lane, 64);
        if (lane < kF32BN) sB[lane] = rb;
        f32_wave_sync();
        if (t + NS < ntiles) {
            st.load(P.k, P.v, P.vmul, b, h, (t + NS) * kF32BN, P.nk, lane, 64);
            if (lane < kF32BN) rb = key_term_l2(P, b, h, (t + NS) * kF32BN + lane);
        }
        f32_dq_tile<D>(dq, qf, of, sK, sV, sB, t * kF32BN, qi, col, hh, P, sc, causal, lse_l2,
                       dsum);
    }
    __syncthreads();
    {
        float* so = sT[w];
#pragma unroll
        for (int x = 0; x < D / 32; ++x)
#pragma unroll
            for (int i = 0; i < 16; ++i) so[(x * 16 + i) * 64 + lane] = dq[x][i];
    }
    __syncthreads();
    if (w != 0 || !qrow) return;  // no barriers below
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float a = 0.f;
#pragma unroll
            for (int v = 0; v < NS; ++v) a += sT[v][(x * 16 + i) * 64 + lane];
            dq[x][i] = a;
        }
    float* row = G.dq.wrow<float>(b, h, qi);
    const bool acc = (G.accumulate & PA_ACC_DQ) != 0;
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            store4(row + 32 * x + 8 * g + 4 * hh,
                   make_float4(dq[x][4 * g], dq[x][4 * g + 1], dq[x][4 * g + 2], dq[x][4 * g + 3]), acc);
}

template <int D, int NS>
__global__ __launch_bounds__(64 * NS) void k_mfma_bwd_f32_dkv_split(GradDev G) {
    constexpr int RS = D + 1;
    constexpr int TILE = 2 * kF32BN * RS + 2 * kF32BN;
    static_assert(TILE >= 2 * (D / 32) * 16 * 64 + 64, "a wave's region holds its partial sums");
    const PassDev& P = G.f;
    __shared__ float sT[NS][TILE];
    const int lane = threadIdx.x & 63, w = wave_id();
    float* sQ = sT[w];
    float* sO = sQ + kF32BN * RS;
    float* sL = sO + kF32BN * RS;
    float* sD = sL + kF32BN;
    const bool causal = P.causal != 0;
    const int nkb = (P.nk + 31) / 32;
    int unit, kblk;
    if (causal) block_order<true>(nkb, G.hk, 1, unit, kblk);
    else block_order<false>(nkb, G.hk, 1, unit, kblk);
    const int kh = unit % G.hk, b = unit / G.hk;
    const int rep = P.heads / G.hk, h0 = kh * rep;
    const int col = lane & 31, hh = lane >> 5;
    const int k0 = kblk * 32, kj = k0 + col;
    const bool krow = kj < P.nk;
    float kf[D / 2], vf[D / 2];
    {
        const float* kr = P.k.row<float>(b, h0, krow ? kj : 0);
        const float* vr = P.v.row<float>(b, h0, krow ? kj : 0);
        const float* mr = P.vmul.ok() ? P.vmul.row<float>(b, h0, krow ? kj : 0) : nullptr;
#pragma unroll
        for (int t = 0; t < D / 2; ++t) {
            kf[t] = krow ? kr[2 * t + hh] : 0.f;
            vf[t] = krow ? vr[2 * t + hh] * (mr ? mr[2 * t + hh] : 1.f) : 0.f;
        }
    }
    const float bk = key_term_l2(P, b, h0, kj);  // -inf past nk
    f32x16_t dk[D / 32], dv[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
        dk[x] = zero16();
        dv[x] = zero16();
    }
    float dbias = 0.f;
    const bool sc = P.softclamp > 0.f;
    // the query tiles of every query head of the group, from the block's first reachable tile
    const int i_start = causal ? k0 : 0;
    const int ntq = P.nq > i_start ? (P.nq - i_start + kF32BN - 1) / kF32BN : 0;
    const int ntiles = ntq * rep;
    const DView none = {nullptr, 0, 0, 0, 1, PA_F32};
    F32Rows<D> st;
    float rl = 0.f, rd = 0.f;
    auto load_rows = [&](int t) __attribute__((always_inline)) {
        const int h = h0 + t / ntq, i0 = i_start + (t % ntq) * kF32BN;
        const int64_t row0 = ((int64_t)b * P.heads + h) * P.nq;
        st.load(P.q, G.dout, none, b, h, i0, P.nq, lane, 64);
        if (lane < kF32BN) {
            const int i = i0 + lane;
            rl = i < P.nq ? G.ws_lse[row0 + i] * kLog2e : INFINITY;
            rd = i < P.nq ? G.ws_D[row0 + i] : 0.f;
        }
    };
    if (w < ntiles) load_rows(w);
    for (int t = w; t < ntiles; t += NS) {  // wave-uniform
        f32_wave_sync();
        st.store(sQ, sO, lane, 64);
        if (lane < kF32BN) {
            sL[lane] = rl;
            sD[lane] = rd;
        }
        f32_wave_sync();
        const int i0 = i_start + (t % ntq) * kF32BN;
        if (t + NS < ntiles) load_rows(t + NS);
        f32_dkv_tile<D>(dk, dv, dbias, kf, vf, sQ, sO, sL, sD, i0, kj, col, hh, P, sc, causal, bk);
    }
    __syncthreads();
    {
        float* so = sT[w];
#pragma unroll
        for (int x = 0; x < D / 32; ++x)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                so[(x * 16 + i) * 64 + lane] = dk[x][i];
                so[((D / 32 + x) * 16 + i) * 64 + lane] = dv[x][i];
            }
        so[2 * (D / 32) * 16 * 64 + lane] = dbias;
    }
    __syncthreads();
    if (w != 0) return;  // no barriers below
    float db = 0.f;
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float a = 0.f, c = 0.f;
#pragma unroll
            for (int v = 0; v < NS; ++v) {
                a += sT[v][(x * 16 + i) * 64 + lane];
                c += sT[v][((D / 32 + x) * 16 + i) * 64 + lane];
            }
            dk[x][i] = a;
            dv[x][i] = c;
        }
#pragma unroll
    for (int v = 0; v < NS; ++v) db += sT[v][2 * (D / 32) * 16 * 64 + lane];
    dbias = xhalf_sum(db);
    if (!krow) return;
    const float* mr = P.vmul.ok() ? P.vmul.row<float>(b, h0, kj) : nullptr;
    const float* vr = P.v.row<float>(b, h0, kj);
    float* dkr = G.dk.wrow<float>(b, h0, kj);
    float* dvr = G.dv.wrow<float>(b, h0, kj);
    float* dmr = mr ? G.dvmul.wrow<float>(b, h0, kj) : nullptr;
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * x + 8 * g + 4 * hh;
            store4(dkr + d, make_float4(dk[x][4 * g], dk[x][4 * g + 1], dk[x][4 * g + 2], dk[x][4 * g + 3]),
                   (G.accumulate & PA_ACC_DK) != 0);
            float4 e = make_float4(dv[x][4 * g], dv[x][4 * g + 1], dv[x][4 * g + 2], dv[x][4 * g + 3]);
            if (mr) {
                const float4 m4 = *reinterpret_cast<const float4*>(mr + d);
                const float4 v4 = *reinterpret_cast<const float4*>(vr + d);
                store4(dmr + d, make_float4(e.x * v4.x, e.y * v4.y, e.z * v4.z, e.w * v4.w),
                       (G.accumulate & PA_ACC_DVMUL) != 0);
                e = make_float4(e.x * m4.x, e.y * m4.y, e.z * m4.z, e.w * m4.w);
            }
            store4(dvr + d, e, (G.accumulate & PA_ACC_DV) != 0);
        }
    if (hh == 0 && G.dbias.ok()) {
        float* o = G.dbias.wrow<float>(b, h0, kj);
        *o = dbias + ((G.accumulate & PA_ACC_DBIAS) ? *o : 0.f);
    }
}

bool mfma_bwd_f32_supported(const GradDev& G) {
    const PassDev& P = G.f;
    if (P.dim != 64 && P.dim != 128) return false;
    if (P.km.p || P.qm.p || (P.flags & PA_FLAG_MAY_DEGENERATE)) return false;
    for (const DView* v : {&P.q, &P.k, &P.v, &G.dout, &G.dq, &G.dk, &G.dv})
        if (!aligned_rows_host(*v, 4)) return false;
    if (P.vmul.ok() && (!aligned_rows_host(P.vmul, 4) || !aligned_rows_host(G.dvmul, 4))) return false;
    return true;
}

void launch_mfma_bwd_f32(const GradDev& G, hipStream_t s) {
    const PassDev& P = G.f;
    auto waves = [](int64_t units, int n) {
        int nw = 4;
        while (nw > 1 && units * ((n + 32 * nw - 1) / (32 * nw)) < 512) nw >>= 1;
        return nw;
    };
    // grids of fewer than 512 blocks of 32 rows: the tiles of a block split over four waves
    // (block counts in 64 bits: a product past 2^31 must not wrap into the small-grid test)
    const int64_t qblocks = (int64_t)P.batch * P.heads * ((P.nq + 31) / 32);
    const int64_t kblocks = (int64_t)P.batch * G.hk * ((P.nk + 31) / 32);
    if (PA_F32_SPLIT && qblocks < 512 && (P.nk + kF32BN - 1) / kF32BN >= 4) {
        ProfScope ps("mfma_bwd_f32_dq_split", s);
        if (P.dim == 64) hipLaunchKernelGGL((k_mfma_bwd_f32_dq_split<64, 4>), dim3((uint32_t)qblocks), dim3(256), 0, s, G);
        else hipLaunchKernelGGL((k_mfma_bwd_f32_dq_split<128, 4>), dim3((uint32_t)qblocks), dim3(256), 0, s, G);
    } else {
        const int nw = waves((int64_t)P.batch * P.heads, P.nq);
        const dim3 grid(P.batch * P.heads * ((P.nq + 32 * nw - 1) / (32 * nw)));
        ProfScope ps("mfma_bwd_f32_dq", s);
        if (P.dim == 64) hipLaunchKernelGGL((k_mfma_bwd_f32_dq<64>), grid, dim3(64 * nw), 0, s, G);
        else hipLaunchKernelGGL((k_mfma_bwd_f32_dq<128>), grid, dim3(64 * nw), 0, s, G);
    }
    if (PA_F32_SPLIT && kblocks < 512 && (P.heads / G.hk) * ((P.nq + kF32BN - 1) / kF32BN) >= 4) {
        ProfScope ps("mfma_bwd_f32_dkv_split", s);
        if (P.dim == 64) hipLaunchKernelGGL((k_mfma_bwd_f32_dkv_split<64, 4>), dim3((uint32_t)kblocks), dim3(256), 0, s, G);
        else hipLaunchKernelGGL((k_mfma_bwd_f32_dkv_split<128, 4>), dim3((uint32_t)kblocks), dim3(256), 0, s, G);
    } else {
        const int nw = waves((int64_t)P.batch * G.hk, P.nk);
        const dim3 grid(P.batch * G.hk * ((P.nk + 32 * nw - 1) / (32 * nw)));
        ProfScope ps("mfma_bwd_f32_dkv", s);
        if (P.dim == 64) hipLaunchKernelGGL((k_mfma_bwd_f32_dkv<64>), grid, dim3(64 * nw), 0, s, G);
        else hipLaunchKernelGGL((k_mfma_bwd_f32_dkv<128>), grid, dim3(64 * nw), 0, s, G);
    }
}

bool mfma_fwd_f32_supported(const PassDev& P) {
    if (P.dim != 64 && P.dim != 128) return false;
    for (const DView* v : {&P.q, &P.k, &P.v, &P.out})
        if (!aligned_rows_host(*v, 4)) return false;
    if (P.vmul.ok() && !aligned_rows_host(P.vmul, 4)) return false;
    return true;
}

void launch_mfma_fwd_f32(const PassDev& P, hipStream_t s) {
    const int units = P.batch * P.heads;
    // grids of fewer than 512 blocks of 32 queries leave most of the chip idle: split the keys
    // of a block over 4 waves (the kernel's 332-512 registers allow one wave per SIMD), when
    // there are that many key tiles
    const int64_t blocks32 = (int64_t)units * ((P.nq + 31) / 32);
    const int tiles = (P.nk + kF32BN - 1) / kF32BN;
    if (PA_F32_SPLIT && blocks32 < 512 && tiles >= 4) {
        ProfScope ps("mfma_fwd_f32_split", s);
        if (P.dim == 64) hipLaunchKernelGGL((k_mfma_fwd_f32_split<64, 4>), dim3((uint32_t)blocks32), dim3(64 * 4), 0, s, P);
        else hipLaunchKernelGGL((k_mfma_fwd_f32_split<128, 4>), dim3((uint32_t)blocks32), dim3(64 * 4), 0, s, P);
        return;
    }
    // waves per workgroup: the most that still give the grid two workgroups per CU
    int nw = 4;
    while (nw > 1 && (int64_t)units * ((P.nq + 32 * nw - 1) / (32 * nw)) < 512) nw >>= 1;
    const dim3 grid(units * ((P.nq + 32 * nw - 1) / (32 * nw)));
    ProfScope ps("mfma_fwd_f32", s);
    if (P.dim == 64) hipLaunchKernelGGL((k_mfma_fwd_f32<64>), grid, dim3(64 * nw), 0, s, P);
    else hipLaunchKernelGGL((k_mfma_fwd_f32<128>), grid, dim3(64 * nw), 0, s, P);
}

}  // namespace pa
