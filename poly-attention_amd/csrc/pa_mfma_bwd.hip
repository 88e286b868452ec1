// pa_mfma_bwd.hip -- MFMA backward of one attention pass (bf16 / f16, head dim 64 or 128).
//
// After k_bwd_pre has written per row lse and D = rowsum(dO * O) - dlse:
//   k_mfma_bwd_dkv (key-major, no atomics): a workgroup owns 128 keys of one key head
//     (4 waves x 32 keys, K and V kept in registers as B operands) and sweeps the query
//     tiles of every query head of its group: S = Q K^T and dP = dO V^T give, per lane,
//     16 queries of the lane's key; P = exp2(S*scale*log2e + bias - lse*log2e) and
//     dS = P (dP - D) feed dV^T += dO^T P and dK^T += Q^T dS through transposed LDS copies of
//     Q and dO, and the key bias gradient is the column sum of dS.
//   k_mfma_bwd_dq (query-major, no atomics): a workgroup owns 128 queries (4 waves x 32) and
//     sweeps the key tiles: S^T = K Q^T, dP^T = V dO^T, dS^T, then dQ^T += K^T dS^T.
// The dQ kernel pipelines its two 32-key blocks by hand: every MFMA of one block is followed
// by the VALU work of a few of the other block's gradient entries, scheduling barriers keeping
// the chunks in order (the same done for the dK/dV kernel's two query blocks measured 5% slower,
// so that kernel leaves the interleaving to the compiler).
// Both recompute P from the saved lse.  They read no masks: for a masked pass the host folds
// the key mask into the key bias and gives fully-masked rows lse = +inf (probability 0 here),
// and the generic kernels add those rows' part afterwards.
#include <algorithm>

#include "pa_common.h"
#include "pa_launch.h"
#include "pa_mfma.h"

namespace pa {

constexpr int kBwdThreads = 256;

#ifndef PA_DQ_CHUNKS
#define PA_DQ_CHUNKS 1  // dQ kernel (no softclamp): the two key blocks in an explicit chunk pipeline
#endif
#ifndef PA_BWD_DMA
#define PA_BWD_DMA 1  // direct-to-LDS backward kernels where they apply
#endif

// ---------------------------------------------------------------------------------------
// dK / dV / dbias

constexpr int kKvBK = 128;  // keys per workgroup
constexpr int kKvBQ = 64;   // queries per tile

template <int D>
struct KvTile {
    static constexpr int RS = D + 8;        // row-major stride (elements)
    static constexpr int TS = kKvBQ + 4;    // transposed stride (elements)
    static constexpr int BLOCKS = (kKvBQ / 4) * (D / 8);  // 4-row x 8-column blocks per tensor
    static constexpr int NB = (2 * BLOCKS + kBwdThreads - 1) / kBwdThreads;
};

template <int D>
struct KvStage {
    u32x4_t w[KvTile<D>::NB][4];
    float lse, dsum;
};

// Per (batch, query head) pointers of the query-side tiles.
template <typename T>
struct QuerySide {
    const T* q;
    const T* dout;
    int64_t qsn, osn;
    const float* lse;
    const float* dsum;
    int32_t nq;
};

template <typename T>
__device__ __forceinline__ QuerySide<T> query_side(const GradDev& G, int b, int h) {
    const PassDev& P = G.f;
    QuerySide<T> s;
    s.q = P.q.row<T>(b, h, 0);
    s.dout = G.dout.row<T>(b, h, 0);
    s.qsn = P.q.sn;
    s.osn = G.dout.sn;
    const int64_t row0 = ((int64_t)b * P.heads + h) * P.nq;
    s.lse = G.ws_lse + row0;
    s.dsum = G.ws_D + row0;
    s.nq = P.nq;
    return s;
}

template <typename T, int D>
__device__ __forceinline__ void kv_load(const QuerySide<T>& qs, int q0, KvStage<D>& st) {
    using TL = KvTile<D>;
    const int tid = threadIdx.x;
    const u32x4_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int c = 0; c < TL::NB; ++c) {
        const int task = tid + c * kBwdThreads;
        if (task < 2 * TL::BLOCKS) {
            const int tensor = task / TL::BLOCKS, blk = task % TL::BLOCKS;
            const int rg = blk / (D / 8), cc = blk % (D / 8);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = q0 + rg * 4 + r;
                u32x4_t x = zero;
                if (q < qs.nq) {
                    const T* src = tensor == 0 ? qs.q + q * qs.qsn : qs.dout + q * qs.osn;
                    x = *reinterpret_cast<const u32x4_t*>(src + cc * 8);
                }
                st.w[c][r] = x;
            }
        }
    }
    if (tid < kKvBQ) {
        const int q = q0 + tid;
        st.lse = q < qs.nq ? qs.lse[q] * kLog2e : INFINITY;
        st.dsum = q < qs.nq ? qs.dsum[q] : 0.f;
    }
}

template <typename T, int D>
__device__ __forceinline__ void kv_store(const KvStage<D>& st, T* sQ, T* sO, T* sQt, T* sOt,
                                         float* sL, float* sD) {
    using TL = KvTile<D>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int c = 0; c < TL::NB; ++c) {
        const int task = tid + c * kBwdThreads;
        if (task < 2 * TL::BLOCKS) {
            const int tensor = task / TL::BLOCKS, blk = task % TL::BLOCKS;
            const int rg = blk / (D / 8), cc = blk % (D / 8);
            T* rows = tensor == 0 ? sQ : sO;
            T* trans = tensor == 0 ? sQt : sOt;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                *reinterpret_cast<u32x4_t*>(rows + (rg * 4 + r) * TL::RS + cc * 8) = st.w[c][r];
            store_block_transposed(st.w[c], reinterpret_cast<uint16_t*>(trans + (cc * 8) * TL::TS + rg * 4),
                                   TL::TS);
        }
    }
    if (tid < kKvBQ) {
        sL[tid] = st.lse;
        sD[tid] = st.dsum;
    }
}

template <typename T, int D, bool CAUSAL, bool SOFTCLAMP, bool HAS_VMUL, bool HAS_BIAS>
__global__ __launch_bounds__(kBwdThreads, D == 64 ? 2 : 1) void k_mfma_bwd_dkv(GradDev G) {
    using TL = KvTile<D>;
    using M = Mma<T>;
    typedef typename M::frag frag;
    const PassDev& P = G.f;
    __shared__ __attribute__((aligned(16))) T sQ[kKvBQ * TL::RS];
    __shared__ __attribute__((aligned(16))) T sO[kKvBQ * TL::RS];
    __shared__ __attribute__((aligned(16))) T sQt[D * TL::TS];
    __shared__ __attribute__((aligned(16))) T sOt[D * TL::TS];
    __shared__ __attribute__((aligned(16))) float sL[kKvBQ];
    __shared__ __attribute__((aligned(16))) float sD[kKvBQ];

    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int hh = lane >> 5, kcol = lane & 31;
    const int nkb = (P.nk + kKvBK - 1) / kKvBK;
    int unit, kblk;  // causal: the first key blocks carry the most work
    block_order<CAUSAL>(nkb, G.hk, 1, unit, kblk);
    const int kh = unit % G.hk, b = unit / G.hk;
    const int rep = P.heads / G.hk;
    const int h0 = kh * rep;
    const int kw0 = kblk * kKvBK + w * 32;  // first key of this wave
    const int key = kw0 + kcol;
    const bool key_ok = key < P.nk;

    // K and effective V of the lane's key as B operands (elements c*16 + 8*hh .. +7)
    frag kf[D / 16], vf[D / 16];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        u32x4_t kr = {0u, 0u, 0u, 0u}, vr = {0u, 0u, 0u, 0u};
        if (key_ok) {
            kr = *reinterpret_cast<const u32x4_t*>(P.k.row<T>(b, h0, key) + c * 16 + 8 * hh);
            vr = *reinterpret_cast<const u32x4_t*>(P.v.row<T>(b, h0, key) + c * 16 + 8 * hh);
            if (HAS_VMUL)
                vr = mul_round8<T>(vr, *reinterpret_cast<const u32x4_t*>(P.vmul.row<T>(b, h0, key) + c * 16 + 8 * hh));
        }
        kf[c] = __builtin_bit_cast(frag, kr);
        vf[c] = __builtin_bit_cast(frag, vr);
    }
    float bias_l2 = key_ok ? 0.f : -INFINITY;
    if (HAS_BIAS && key_ok) {
        const float x = P.bias.scalar(b, h0, key);
        bias_l2 = bias_class(x) == 0 ? x * kLog2e : -INFINITY;
    }
    const float sl2 = P.scale * kLog2e;
    const float cinv = SOFTCLAMP ? P.scale / P.softclamp : 0.f;
    const float crec = SOFTCLAMP ? 1.f / P.softclamp : 0.f;

    f32x16_t dk[D / 32], dv[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
        dk[x] = zero16();
        dv[x] = zero16();
    }
    float dbias = 0.f;

    const int q_start = CAUSAL ? (kblk * kKvBK / kKvBQ) * kKvBQ : 0;
    const int ntiles = P.nq > q_start ? (P.nq - q_start + kKvBQ - 1) / kKvBQ : 0;
    // head dim 256: the next tile is loaded just before it is stored, not held in registers
    // across the compute (the register file is full: fewer spills, 2.95 against 3.90 ms per
    // launch at N = 4096)
    constexpr bool PREFETCH = D < 256;
    KvStage<D> st;
    for (int h = h0; h < h0 + rep; ++h) {
        const QuerySide<T> qs = query_side<T>(G, b, h);
        if (PREFETCH && ntiles > 0) kv_load<T, D>(qs, q_start, st);
        for (int t = 0; t < ntiles; ++t) {
            const int q0 = q_start + t * kKvBQ;
            if (!PREFETCH) kv_load<T, D>(qs, q0, st);
            kv_store<T, D>(st, sQ, sO, sQt, sOt, sL, sD);
            __syncthreads();
            if (PREFETCH && t + 1 < ntiles) kv_load<T, D>(qs, q0 + kKvBQ, st);
            // head dim 256, not causal: the two query halves one after the other (unrolled, the
            // scheduler kept both halves' temporaries live: 479 against 106 spilled registers,
            // 3.75 against 1.80 ms per launch at N = 2048); causal, unrolled was faster
#pragma unroll(D == 256 && !CAUSAL ? 1 : 2)
            for (int qb = 0; qb < 2; ++qb) {
                const int qbase = q0 + qb * 32;
                if (CAUSAL && qbase + 31 < kw0) continue;  // every query precedes every key
                f32x16_t s = zero16(), dp = zero16();
#pragma unroll
                for (int c = 0; c < D / 16; ++c) {
                    const int off = (qb * 32 + kcol) * TL::RS + c * 16 + 8 * hh;
                    s = M::run(ld_frag<T>(sQ + off), kf[c], s);
                    dp = M::run(ld_frag<T>(sO + off), vf[c], dp);
                }
                // P: register i holds query qbase + 8*(i/4) + 4*hh + (i%4) of the lane's key
                float yv[16];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 Lv = *reinterpret_cast<const float4*>(sL + qb * 32 + 8 * g + 4 * hh);
                    const float L[4] = {Lv.x, Lv.y, Lv.z, Lv.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * g + r;
                        float x;
                        if (SOFTCLAMP) {
                            yv[i] = tanhf(s[i] * cinv);  // softclamp(s*scale) / c
                            x = yv[i] * (P.softclamp * kLog2e) + bias_l2 - L[r];
                        } else {
                            x = fmaf(s[i], sl2, bias_l2 - L[r]);
                        }
                        s[i] = fast_exp2(x);
                    }
                }
                if (CAUSAL && qbase < kw0 + 31) {  // queries before the lane's key: P = 0
                    const int lim = key - qbase - 4 * hh;
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (8 * (i / 4) + (i % 4) < lim) s[i] = 0.f;
                }
                // dS = P (dP - D); the key bias gradient is its column sum
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 Dv = *reinterpret_cast<const float4*>(sD + qb * 32 + 8 * g + 4 * hh);
                    const float Dd[4] = {Dv.x, Dv.y, Dv.z, Dv.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * g + r;
                        float dsv = s[i] * (dp[i] - Dd[r]);
                        dbias += dsv;
                        if (SOFTCLAMP) dsv *= (1.f - yv[i] * yv[i]);
                        dp[i] = dsv;
                    }
                }
#pragma unroll
                for (int t2 = 0; t2 < 2; ++t2) {
                    const frag pf = acc_to_frag<T>(s, t2);
                    const frag df = acc_to_frag<T>(dp, t2);
#pragma unroll
                    for (int x = 0; x < D / 32; ++x) {
                        const int toff = (x * 32 + kcol) * TL::TS + qb * 32 + 16 * t2 + 4 * hh;
                        dv[x] = M::run(lds_runs<T>(sOt + toff), pf, dv[x]);
                        dk[x] = M::run(lds_runs<T>(sQt + toff), df, dk[x]);
                    }
                }
            }
            __syncthreads();
        }
    }

    dbias += __shfl_xor(dbias, 32);
    if (!key_ok) return;
    (void)crec;
    // dK = scale * dK^T^T ; registers: d = x*32 + 8g + 4hh + r
    T* dkrow = G.dk.wrow<T>(b, h0, key);
    T* dvrow = G.dv.wrow<T>(b, h0, key);
    const bool acc_k = (G.accumulate & PA_ACC_DK) != 0;
    const bool acc_v = (G.accumulate & PA_ACC_DV) != 0;
    const bool acc_m = (G.accumulate & PA_ACC_DVMUL) != 0;
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = x * 32 + 8 * g + 4 * hh;
            float kv[4], vv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                kv[r] = dk[x][4 * g + r] * P.scale;
                vv[r] = dv[x][4 * g + r];
            }
            if (acc_k)
#pragma unroll
                for (int r = 0; r < 4; ++r) kv[r] += to_f(dkrow[d + r]);
            u32x2_t pk;
            pk[0] = pack2<T>(kv[0], kv[1]);
            pk[1] = pack2<T>(kv[2], kv[3]);
            *reinterpret_cast<u32x2_t*>(dkrow + d) = pk;
            if (HAS_VMUL) {
                const T* mrow = P.vmul.row<T>(b, h0, key);
                const T* vrow = P.v.row<T>(b, h0, key);
                T* dmrow = G.dvmul.wrow<T>(b, h0, key);
                float gv[4], gm[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    gv[r] = vv[r] * to_f(mrow[d + r]) + (acc_v ? to_f(dvrow[d + r]) : 0.f);
                    gm[r] = vv[r] * to_f(vrow[d + r]) + (acc_m ? to_f(dmrow[d + r]) : 0.f);
                }
                pk[0] = pack2<T>(gv[0], gv[1]);
                pk[1] = pack2<T>(gv[2], gv[3]);
                *reinterpret_cast<u32x2_t*>(dvrow + d) = pk;
                pk[0] = pack2<T>(gm[0], gm[1]);
                pk[1] = pack2<T>(gm[2], gm[3]);
                *reinterpret_cast<u32x2_t*>(dmrow + d) = pk;
            } else {
                if (acc_v)
#pragma unroll
                    for (int r = 0; r < 4; ++r) vv[r] += to_f(dvrow[d + r]);
                pk[0] = pack2<T>(vv[0], vv[1]);
                pk[1] = pack2<T>(vv[2], vv[3]);
                *reinterpret_cast<u32x2_t*>(dvrow + d) = pk;
            }
        }
    }
    if (hh == 0 && G.dbias.ok()) {
        float* o = G.dbias.wrow<float>(b, h0, key);
        *o = dbias + ((G.accumulate & PA_ACC_DBIAS) ? *o : 0.f);
    }
}

// ---------------------------------------------------------------------------------------
// Direct-to-LDS dK / dV / dbias (no value multiplier): the Q and dO tiles of every query
// tile, with their lse and D rows, travel HBM -> LDS by buffer_load ... lds, four stages
// filled and waited for in pairs (tiles i+2 and i+3 in flight while tiles i and i+1 are
// computed, one barrier per pair; the query heads of a KV group form one flat tile sequence).  Q and dO stay row-major in LDS and are read both by rows (S = Q K^T,
// dP = dO V^T) and transposed (dV^T += dO^T P, dK^T += Q^T dS, ds_read_b64_tr_b16), under a
// chunk swizzle that serves both patterns.  The tile's lse and D rows enter as accumulator
// seeds: S starts at -lse/scale (so P = exp2(scale*log2e*S + bias)) and dP at -D (so
// dS = P dP); with softclamp the lse is kept in the log2 domain instead.  When the dQ kernel
// ran first (GradDev::seeds) it wrote the rows in this form and the waves read the loaded
// rows directly; otherwise each wave converts them into a copy of its own.

// chunk swizzle for tiles read by rows (16 rows x one chunk per quarter-wave) and transposed
// (4 rows x 4 chunks per half-wave): rows of one parity in a 16-row group get distinct
// chunks, and rows r, r+2 of an aligned group of four differ in the chunk's bit 2 (D = 64);
// a 4-bit reversal of the row for D = 128
template <int D>
__device__ __forceinline__ int swz_qt(int r) {
    if (D == 64) {
        const int v = (r >> 1) & 7;
        return ((v & 1) << 2) | (v & 2) | ((v >> 2) & 1);
    }
    const int v = r & 15;
    return ((v & 1) << 3) | ((v & 2) << 1) | ((v >> 1) & 2) | ((v >> 3) & 1);
}

constexpr int kKvStages = 3;

template <typename T, int D, bool CAUSAL, bool SOFTCLAMP, bool HAS_BIAS>
__global__ __launch_bounds__(kBwdThreads, D == 64 ? 2 : 1) void k_mfma_bwd_dkv_dma(GradDev G) {
    using M = Mma<T>;
    typedef typename M::frag frag;
    constexpr int BQ = kKvBQ, CPR = D / 8, ELEMS = BQ * D;
    constexpr int NL = BQ * CPR / kBwdThreads;  // chunks per thread and tensor
    static_assert(BQ * CPR % kBwdThreads == 0, "tile must split evenly over the threads");
    const PassDev& P = G.f;
    constexpr int NSTG = 4;  // query tiles filled and waited for in pairs
    __shared__ __attribute__((aligned(16))) T sQ[NSTG * ELEMS];
    __shared__ __attribute__((aligned(16))) T sO[NSTG * ELEMS];
    __shared__ __attribute__((aligned(16))) float sLraw[NSTG][BQ];
    __shared__ __attribute__((aligned(16))) float sDraw[NSTG][BQ];
    __shared__ __attribute__((aligned(16))) float sLw[4][BQ];  // per-wave converted seeds
    __shared__ __attribute__((aligned(16))) float sDw[4][BQ];

    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int hh = lane >> 5, kcol = lane & 31;
    const int nkb = (P.nk + kKvBK - 1) / kKvBK;
    int unit, kblk;  // causal: the first key blocks carry the most work
    block_order<CAUSAL>(nkb, G.hk, 1, unit, kblk);
    const int kh = unit % G.hk, b = unit / G.hk;
    const int rep = P.heads / G.hk;
    const int h0 = kh * rep;
    const int kw0 = kblk * kKvBK + w * 32;  // first key of this wave
    const int key = kw0 + kcol;
    const bool key_ok = key < P.nk;

    frag kf[D / 16], vf[D / 16];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        u32x4_t kr = {0u, 0u, 0u, 0u}, vr = {0u, 0u, 0u, 0u};
        if (key_ok) {
            kr = *reinterpret_cast<const u32x4_t*>(P.k.row<T>(b, h0, key) + c * 16 + 8 * hh);
            vr = *reinterpret_cast<const u32x4_t*>(P.v.row<T>(b, h0, key) + c * 16 + 8 * hh);
        }
        kf[c] = __builtin_bit_cast(frag, kr);
        vf[c] = __builtin_bit_cast(frag, vr);
    }
    float bias_l2 = key_ok ? 0.f : -INFINITY;
    if (HAS_BIAS && key_ok) {
        const float x = P.bias.scalar(b, h0, key);
        bias_l2 = bias_class(x) == 0 ? x * kLog2e : -INFINITY;
    }
    // retire the compiler-visible loads before the first direct load
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        kf[c] = opaque(kf[c]);
        vf[c] = opaque(vf[c]);
    }
    bias_l2 = opaque(bias_l2);
    const float sl2 = P.scale * kLog2e;
    const float cinv = SOFTCLAMP ? P.scale / P.softclamp : 0.f;
    const float cl2 = SOFTCLAMP ? P.softclamp * kLog2e : 0.f;
    const float lmul = SOFTCLAMP ? kLog2e : -1.f / P.scale;  // lse -> seed / log2 value
    const bool need_dbias = G.dbias.ok();

    f32x16_t dk[D / 32], dv[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
        dk[x] = zero16();
        dv[x] = zero16();
    }
    float dbias = 0.f;

    // a key block none of whose keys has a bias-class-0 term (masked keys: padding) receives
    // nothing from any query: the sweep is skipped and the block's gradients are written as
    // zero.  Every wave reads the whole block's terms, so all reach the same decision.
    static_assert(kKvBK == 128, "two keys per lane");
    bool block_dead = false;
    if (HAS_BIAS) {
        const int k0 = kblk * kKvBK;
        const float y0 = k0 + lane < P.nk ? P.bias.scalar(b, h0, k0 + lane) : -INFINITY;
        const float y1 = k0 + 64 + lane < P.nk ? P.bias.scalar(b, h0, k0 + 64 + lane) : -INFINITY;
        block_dead = !__any(bias_class(y0) == 0 || bias_class(y1) == 0);
    }

    const int q_start = CAUSAL ? (kblk * kKvBK / BQ) * BQ : 0;
    const int nt = P.nq > q_start ? (P.nq - q_start + BQ - 1) / BQ : 0;  // tiles per query head
    const int total = block_dead ? 0 : nt * rep;

    // direct loads: thread tid carries chunk n*256 + tid of a tile: row p / CPR, chunk p % CPR
    const int qsn = (int)P.q.sn, osn = (int)G.dout.sn;
    uint32_t offq[NL], offo[NL];
#pragma unroll
    for (int n = 0; n < NL; ++n) {
        const int p = n * kBwdThreads + tid, r = p / CPR, ph = p % CPR;
        offq[n] = (uint32_t)((r * qsn + (ph ^ swz_qt<D>(r)) * 8) * 2);
        offo[n] = (uint32_t)((r * osn + (ph ^ swz_qt<D>(r)) * 8) * 2);
    }
    const uint32_t lds_q = lds_addr(sQ), lds_o = lds_addr(sO);
    const uint32_t lds_l = lds_addr(&sLraw[0][0]), lds_d = lds_addr(&sDraw[0][0]);
    const uint32_t qbytes = (uint32_t)(((int64_t)(P.nq - 1) * qsn + D) * 2);
    const uint32_t obytes = (uint32_t)(((int64_t)(P.nq - 1) * osn + D) * 2);
    // load cursor: the tiles go head by head (the query heads of this KV group), query tiles
    // in order; the buffer descriptors change only with the head
    int cur_h = h0, cur_q0 = q_start;
    const int q_end = q_start + nt * BQ;
    srd_t rq, ro, rl, rd;
    auto set_head = [&](int h) __attribute__((always_inline)) {
        rq = make_srd(P.q.row<T>(b, h, 0), qbytes);
        ro = make_srd(G.dout.row<T>(b, h, 0), obytes);
        const int64_t row0 = ((int64_t)b * P.heads + h) * P.nq;
        rl = make_srd(G.ws_lse + row0, (uint32_t)(P.nq * 4));
        rd = make_srd(G.ws_D + row0, (uint32_t)(P.nq * 4));
    };
    set_head(h0);
    auto issue = [&](int stage) __attribute__((always_inline)) {
        const int q0 = cur_q0;
        const uint32_t sq = lds_q + (uint32_t)(stage * ELEMS * 2), so = lds_o + (uint32_t)(stage * ELEMS * 2);
#pragma unroll
        for (int n = 0; n < NL; ++n) {
            dma16(rq, sq + (uint32_t)((n * kBwdThreads + w * 64) * 16), offq[n] + (uint32_t)(q0 * qsn * 2));
            dma16(ro, so + (uint32_t)((n * kBwdThreads + w * 64) * 16), offo[n] + (uint32_t)(q0 * osn * 2));
        }
        // lse and D rows: 256 bytes each, four lanes of every wave
        if (lane < 4) {
            const uint32_t o = (uint32_t)(w * 64 + 16 * lane);
            dma16(rl, lds_l + (uint32_t)(stage * BQ * 4 + w * 64), o + (uint32_t)(q0 * 4));
            dma16(rd, lds_d + (uint32_t)(stage * BQ * 4 + w * 64), o + (uint32_t)(q0 * 4));
        }
        cur_q0 += BQ;
        if (cur_q0 == q_end) {
            cur_q0 = q_start;
            if (++cur_h < h0 + rep) set_head(cur_h);
        }
    };

    // per-lane LDS element offsets: rows qb*32 + kcol, chunk 2c + hh (row reads) and rows
    // 4*hh + j/4 (+16*t2 + 8*u + 32*qb), columns 32x + (lane & 31) (transposed reads)
    int roff[D / 16];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) roff[c] = kcol * D + (((2 * c + hh) ^ swz_qt<D>(kcol)) * 8);
    // (the swizzle depends on row bit 3, so the two 4-row runs u = 0, 1 get their own offsets)
    int toff[2][D / 32];
    {
        const int g = lane >> 4, j = lane & 15;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int r = 8 * u + 4 * (g >> 1) + (j >> 2);
#pragma unroll
            for (int x = 0; x < D / 32; ++x) {
                const int ch = 4 * x + 2 * (g & 1) + ((j & 3) >> 1);
                toff[u][x] = r * D + ((ch ^ swz_qt<D>(r)) * 8) + 4 * (j & 1);
            }
        }
    }
    auto tr_frag = [&](const T* base, int row0, int x) __attribute__((always_inline)) -> frag {
        const u32x2_t lo = lds_read_tr(base + row0 * D + toff[0][x]);
        const u32x2_t hi = lds_read_tr(base + row0 * D + toff[1][x]);
        const u32x4_t v4 = {lo[0], lo[1], hi[0], hi[1]};
        return __builtin_bit_cast(frag, v4);
    };

    if (total > 0) issue(0);
    if (total > 1) issue(1);
    int st = 0;
    int q0 = q_start;  // first query of the tile being computed
    for (int idx = 0; idx < total; ++idx, q0 = (q0 + BQ == q_end) ? q_start : q0 + BQ) {
        // query tiles in pairs, one workgroup barrier per pair: at an even tile both tiles of
        // the pair have landed and every wave is done with the previous pair, whose stages
        // receive the next pair (half the barriers of one per tile: -1.5% on this kernel)
        if (!(idx & 1)) {
            wait_vmcnt<0>();
            lds_barrier();
            if (idx + 2 < total) issue((st + 2) & 3);
            if (idx + 3 < total) issue((st + 3) & 3);
        }
        const T* Qt = sQ + st * ELEMS;
        const T* Ot = sO + st * ELEMS;
        // the tile's seeds: -lse/scale (log2-domain lse with softclamp), -D; read from the
        // loaded rows when the dQ kernel wrote them in that form, else converted into this
        // wave's copy
        const float* seed_l = &sLraw[st][0];
        const float* seed_d = &sDraw[st][0];
        if (!G.seeds) {
            sLw[w][lane] = sLraw[st][lane] * lmul;
            sDw[w][lane] = -sDraw[st][lane];
            seed_l = &sLw[w][0];
            seed_d = &sDw[w][0];
        }
        // the two 32-query blocks in a software pipeline: the MFMAs of one block are issued in
        // the same basic block as the VALU work of the other
        auto scores = [&](int qb, f32x16_t& s, f32x16_t& dp) __attribute__((always_inline)) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 lv = *reinterpret_cast<const float4*>(seed_l + qb * 32 + 8 * g + 4 * hh);
                const float4 dv4 = *reinterpret_cast<const float4*>(seed_d + qb * 32 + 8 * g + 4 * hh);
                if (SOFTCLAMP) {
                    s[4 * g] = s[4 * g + 1] = s[4 * g + 2] = s[4 * g + 3] = 0.f;
                } else {
                    s[4 * g] = lv.x;
                    s[4 * g + 1] = lv.y;
                    s[4 * g + 2] = lv.z;
                    s[4 * g + 3] = lv.w;
                }
                dp[4 * g] = dv4.x;
                dp[4 * g + 1] = dv4.y;
                dp[4 * g + 2] = dv4.z;
                dp[4 * g + 3] = dv4.w;
            }
#pragma unroll
            for (int c = 0; c < D / 16; ++c) {
                const int off = qb * 32 * D + roff[c];
                s = M::run(ld_frag<T>(Qt + off), kf[c], s);
                dp = M::run(ld_frag<T>(Ot + off), vf[c], dp);
            }
        };
        // queries before the lane's key or past the last query: scores -> -inf (P = 0).
        // Register i holds query qbase + 8*(i/4) + 4*hh + (i%4) of the lane's key.
        auto mask = [&](int qb, f32x16_t& s) __attribute__((always_inline)) {
            const int qbase = q0 + qb * 32;
            if ((CAUSAL && qbase < kw0 + 32) || qbase + 32 > P.nq) {
                keep_branch();
                const int lo = CAUSAL ? key - qbase - 4 * hh : -(1 << 30);
                const int hi = P.nq - qbase - 4 * hh;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int o = 8 * (i / 4) + (i % 4);
                    if (o < lo || o >= hi) s[i] = -INFINITY;
                }
            }
        };
        // P, dS = P (dP - D) (the key bias gradient is its column sum), packed as B operands
        auto grads = [&](int qb, f32x16_t& s, f32x16_t& dp, frag (&pf)[2], frag (&df)[2])
                         __attribute__((always_inline)) {
            float yv[16];
            if (SOFTCLAMP) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 lv = *reinterpret_cast<const float4*>(seed_l + qb * 32 + 8 * g + 4 * hh);
                    const float L[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * g + r;
                        yv[i] = s[i] == -INFINITY ? 1.f : tanhf(s[i] * cinv);
                        s[i] = s[i] == -INFINITY ? 0.f : fast_exp2(yv[i] * cl2 + bias_l2 - L[r]);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) s[i] = fast_exp2(fmaf(s[i], sl2, bias_l2));
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) dp[i] *= s[i];
            if (need_dbias) {
                float a0 = 0.f, a1 = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i += 2) {
                    a0 += dp[i];
                    a1 += dp[i + 1];
                }
                dbias += a0 + a1;
            }
            if (SOFTCLAMP)
#pragma unroll
                for (int i = 0; i < 16; ++i) dp[i] *= (1.f - yv[i] * yv[i]);
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
                pf[t2] = acc_to_frag<T>(s, t2);
                df[t2] = acc_to_frag<T>(dp, t2);
            }
        };
        auto accumulate = [&](int qb, const frag (&pf)[2], const frag (&df)[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
                for (int x = 0; x < D / 32; ++x) {
                    dv[x] = M::run(tr_frag(Ot, qb * 32 + 16 * t2, x), pf[t2], dv[x]);
                    dk[x] = M::run(tr_frag(Qt, qb * 32 + 16 * t2, x), df[t2], dk[x]);
                }
        };
        f32x16_t s0, dp0, s1, dp1;
        frag pf0[2], df0[2], pf1[2], df1[2];
        scores(0, s0, dp0);
        mask(0, s0);
        scores(1, s1, dp1);
        grads(0, s0, dp0, pf0, df0);
        mask(1, s1);
        accumulate(0, pf0, df0);
        grads(1, s1, dp1, pf1, df1);
        accumulate(1, pf1, df1);
        st = (st + 1) & 3;
    }

    dbias += __shfl_xor(dbias, 32);
    if (!key_ok) return;
    T* dkrow = G.dk.wrow<T>(b, h0, key);
    T* dvrow = G.dv.wrow<T>(b, h0, key);
    const bool acc_k = (G.accumulate & PA_ACC_DK) != 0;
    const bool acc_v = (G.accumulate & PA_ACC_DV) != 0;
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = x * 32 + 8 * g + 4 * hh;
            float kv[4], vv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                kv[r] = dk[x][4 * g + r] * P.scale + (acc_k ? to_f(dkrow[d + r]) : 0.f);
                vv[r] = dv[x][4 * g + r] + (acc_v ? to_f(dvrow[d + r]) : 0.f);
            }
            u32x2_t pk;
            pk[0] = pack2<T>(kv[0], kv[1]);
            pk[1] = pack2<T>(kv[2], kv[3]);
            *reinterpret_cast<u32x2_t*>(dkrow + d) = pk;
            pk[0] = pack2<T>(vv[0], vv[1]);
            pk[1] = pack2<T>(vv[2], vv[3]);
            *reinterpret_cast<u32x2_t*>(dvrow + d) = pk;
        }
    }
    if (hh == 0 && need_dbias) {
        float* o = G.dbias.wrow<float>(b, h0, key);
        *o = dbias + ((G.accumulate & PA_ACC_DBIAS) ? *o : 0.f);
    }
}

// ---------------------------------------------------------------------------------------
// dQ

constexpr int kDqBM = 128;  // queries per workgroup
constexpr int kDqBN = 64;   // keys per tile

template <int D>
struct DqTile {
    static constexpr int RS = D + 8;
    static constexpr int TS = kDqBN + 4;
    static constexpr int BLOCKS = (kDqBN / 4) * (D / 8);
    static constexpr int NB = (2 * BLOCKS + kBwdThreads - 1) / kBwdThreads;
};

// Per (batch, key head) pointers of the key-side tiles.
template <typename T>
struct KeyRows {
    const T* k;
    const T* v;
    const T* vm;
    int64_t ksn, vsn, msn;
    const char* bias;
    int64_t bsn;
    int32_t bdt;
    int32_t nk;
};

template <typename T>
__device__ __forceinline__ KeyRows<T> key_rows(const PassDev& P, int b, int h) {
    KeyRows<T> s;
    s.k = P.k.row<T>(b, h, 0);
    s.v = P.v.row<T>(b, h, 0);
    s.vm = P.vmul.ok() ? P.vmul.row<T>(b, h, 0) : nullptr;
    s.ksn = P.k.sn;
    s.vsn = P.v.sn;
    s.msn = P.vmul.sn;
    s.bias = P.bias.ok() ? P.bias.p + P.bias.idx(b, h, 0) * (P.bias.dtype == PA_F32 ? 4 : 2) : nullptr;
    s.bsn = P.bias.sn;
    s.bdt = P.bias.dtype;
    s.nk = P.nk;
    return s;
}

template <int D>
struct DqStage {
    u32x4_t w[DqTile<D>::NB][4];
    float bias;
};

template <typename T, int D, bool HAS_VMUL, bool HAS_BIAS>
__device__ __forceinline__ void dq_load(const KeyRows<T>& ks, int j0, DqStage<D>& st) {
    using TL = DqTile<D>;
    const int tid = threadIdx.x;
    const u32x4_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int c = 0; c < TL::NB; ++c) {
        const int task = tid + c * kBwdThreads;
        if (task < 2 * TL::BLOCKS) {
            const int tensor = task / TL::BLOCKS, blk = task % TL::BLOCKS;
            const int rg = blk / (D / 8), cc = blk % (D / 8);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = j0 + rg * 4 + r;
                u32x4_t x = zero;
                if (j < ks.nk) {
                    if (tensor == 0) {
                        x = *reinterpret_cast<const u32x4_t*>(ks.k + j * ks.ksn + cc * 8);
                    } else {
                        x = *reinterpret_cast<const u32x4_t*>(ks.v + j * ks.vsn + cc * 8);
                        if (HAS_VMUL)
                            x = mul_round8<T>(x, *reinterpret_cast<const u32x4_t*>(ks.vm + j * ks.msn + cc * 8));
                    }
                }
                st.w[c][r] = x;
            }
        }
    }
    if (tid < kDqBN) {
        const int j = j0 + tid;
        float bv = -INFINITY;
        if (j < ks.nk) {
            bv = 0.f;
            if (HAS_BIAS) {
                const float x = load_any(ks.bias, ks.bdt, j * ks.bsn);
                bv = bias_class(x) == 0 ? x * kLog2e : -INFINITY;
            }
        }
        st.bias = bv;
    }
}

template <typename T, int D>
__device__ __forceinline__ void dq_store(const DqStage<D>& st, T* sK, T* sV, T* sKt, float* sB) {
    using TL = DqTile<D>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int c = 0; c < TL::NB; ++c) {
        const int task = tid + c * kBwdThreads;
        if (task < 2 * TL::BLOCKS) {
            const int tensor = task / TL::BLOCKS, blk = task % TL::BLOCKS;
            const int rg = blk / (D / 8), cc = blk % (D / 8);
            T* rows = tensor == 0 ? sK : sV;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                *reinterpret_cast<u32x4_t*>(rows + (rg * 4 + r) * TL::RS + cc * 8) = st.w[c][r];
            if (tensor == 0)
                store_block_transposed(st.w[c], reinterpret_cast<uint16_t*>(sKt + (cc * 8) * TL::TS + rg * 4),
                                       TL::TS);
        }
    }
    if (tid < kDqBN) sB[tid] = st.bias;
}

template <typename T, int D, bool CAUSAL, bool SOFTCLAMP, bool HAS_VMUL, bool HAS_BIAS>
__global__ __launch_bounds__(kBwdThreads, D == 64 ? 2 : 1) void k_mfma_bwd_dq(GradDev G) {
    using TL = DqTile<D>;
    using M = Mma<T>;
    typedef typename M::frag frag;
    const PassDev& P = G.f;
    __shared__ __attribute__((aligned(16))) T sK[kDqBN * TL::RS];
    __shared__ __attribute__((aligned(16))) T sV[kDqBN * TL::RS];
    __shared__ __attribute__((aligned(16))) T sKt[D * TL::TS];
    __shared__ __attribute__((aligned(16))) float sB[kDqBN];

    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int hh = lane >> 5, kcol = lane & 31;
    const int nqb = (P.nq + kDqBM - 1) / kDqBM;
    int unit, rank;
    block_order<CAUSAL>(nqb, P.heads, P.k.hdiv, unit, rank);
    const int qblk = CAUSAL ? nqb - 1 - rank : rank;  // heaviest first
    const int h = unit % P.heads, b = unit / P.heads;
    const int qw0 = qblk * kDqBM + w * 32;
    const int qi = qw0 + kcol;
    const bool q_ok = qi < P.nq;

    frag qf[D / 16], of[D / 16];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        u32x4_t qr = {0u, 0u, 0u, 0u}, orr = {0u, 0u, 0u, 0u};
        if (q_ok) {
            qr = *reinterpret_cast<const u32x4_t*>(P.q.row<T>(b, h, qi) + c * 16 + 8 * hh);
            orr = *reinterpret_cast<const u32x4_t*>(G.dout.row<T>(b, h, qi) + c * 16 + 8 * hh);
        }
        qf[c] = __builtin_bit_cast(frag, qr);
        of[c] = __builtin_bit_cast(frag, orr);
    }
    const int64_t row = ((int64_t)b * P.heads + h) * P.nq + (q_ok ? qi : 0);
    const float lse_l2 = q_ok ? G.ws_lse[row] * kLog2e : INFINITY;
    const float dpi = q_ok ? G.ws_D[row] : 0.f;
    const float sl2 = P.scale * kLog2e;
    const float cinv = SOFTCLAMP ? P.scale / P.softclamp : 0.f;

    f32x16_t dq[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) dq[x] = zero16();

    const int kend = CAUSAL ? min(P.nk, qblk * kDqBM + kDqBM) : P.nk;
    const int ntiles = (kend + kDqBN - 1) / kDqBN;
    const KeyRows<T> ks = key_rows<T>(P, b, h);
    DqStage<D> st;
    dq_load<T, D, HAS_VMUL, HAS_BIAS>(ks, 0, st);
    for (int t = 0; t < ntiles; ++t) {
        const int j0 = t * kDqBN;
        dq_store<T, D>(st, sK, sV, sKt, sB);
        __syncthreads();
        if (t + 1 < ntiles) dq_load<T, D, HAS_VMUL, HAS_BIAS>(ks, j0 + kDqBN, st);
        if (!(CAUSAL && j0 > qw0 + 31)) {
            const bool diag = CAUSAL && (j0 + kDqBN - 1 > qw0);
            // head dim 256: the two key blocks one after the other (unrolled, the register file
            // spilled up to 200 registers; rolled, none: 1.39 against 2.02 ms per launch at
            // N = 4096, causal)
#pragma unroll(D == 256 ? 1 : 2)
            for (int kb = 0; kb < 2; ++kb) {
                f32x16_t s = zero16(), dp = zero16();
#pragma unroll
                for (int c = 0; c < D / 16; ++c) {
                    const int off = (kb * 32 + kcol) * TL::RS + c * 16 + 8 * hh;
                    s = M::run(ld_frag<T>(sK + off), qf[c], s);
                    dp = M::run(ld_frag<T>(sV + off), of[c], dp);
                }
                // P^T: register i holds key j0 + kb*32 + 8*(i/4) + 4*hh + (i%4) of the lane's query
                float yv[16];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 bb = *reinterpret_cast<const float4*>(sB + kb * 32 + 8 * g + 4 * hh);
                    const float bv[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * g + r;
                        float x;
                        if (SOFTCLAMP) {
                            yv[i] = tanhf(s[i] * cinv);
                            x = yv[i] * (P.softclamp * kLog2e) + bv[r] - lse_l2;
                        } else {
                            x = fmaf(s[i], sl2, bv[r] - lse_l2);
                        }
                        s[i] = fast_exp2(x);
                    }
                }
                if (diag) {  // keys after the lane's query: P = 0
                    const int lim = qi - j0 - kb * 32 - 4 * hh;
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (8 * (i / 4) + (i % 4) > lim) s[i] = 0.f;
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    float dsv = s[i] * (dp[i] - dpi);
                    if (SOFTCLAMP) dsv *= (1.f - yv[i] * yv[i]);
                    s[i] = dsv;
                }
#pragma unroll
                for (int t2 = 0; t2 < 2; ++t2) {
                    const frag df = acc_to_frag<T>(s, t2);
#pragma unroll
                    for (int x = 0; x < D / 32; ++x) {
                        const int toff = (x * 32 + kcol) * TL::TS + kb * 32 + 16 * t2 + 4 * hh;
                        dq[x] = M::run(lds_runs<T>(sKt + toff), df, dq[x]);
                    }
                }
            }
        }
        __syncthreads();
    }
    if (!q_ok) return;
    T* dqrow = G.dq.wrow<T>(b, h, qi);
    const bool acc = (G.accumulate & PA_ACC_DQ) != 0;
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = x * 32 + 8 * g + 4 * hh;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = dq[x][4 * g + r] * P.scale + (acc ? to_f(dqrow[d + r]) : 0.f);
            u32x2_t pk;
            pk[0] = pack2<T>(v[0], v[1]);
            pk[1] = pack2<T>(v[2], v[3]);
            *reinterpret_cast<u32x2_t*>(dqrow + d) = pk;
        }
    }
}

// ---------------------------------------------------------------------------------------
// Direct-to-LDS dQ (no value multiplier): K, V and the raw key bias of every key tile travel
// HBM -> LDS by buffer_load ... lds, three stages deep.  K is read by rows (S^T = K Q^T) and
// transposed (dQ^T += K^T dS^T) under the dual-pattern swizzle, V by rows only.  Each wave
// converts the tile's key bias into accumulator seeds (bias / scale; log2 domain with
// softclamp), so that P^T = exp2(scale*log2e*S^T - lse*log2e).  Three workgroups per CU at
// head dim 64 (the register budget fits without spills).
template <typename T, int D, bool CAUSAL, bool SOFTCLAMP, bool HAS_BIAS>
__global__ __launch_bounds__(kBwdThreads, D == 64 ? 3 : 1) void k_mfma_bwd_dq_dma(GradDev G) {
    using M = Mma<T>;
    typedef typename M::frag frag;
    constexpr int BN = kDqBN, CPR = D / 8, ELEMS = BN * D;
    constexpr int NL = BN * CPR / kBwdThreads;
    constexpr int NOPS = 2 * NL + (HAS_BIAS ? 1 : 0);
    constexpr bool FOLD = HAS_BIAS && !SOFTCLAMP;
    static_assert(BN * CPR % kBwdThreads == 0, "tile must split evenly over the threads");
    const PassDev& P = G.f;
    __shared__ __attribute__((aligned(16))) T sK[kKvStages * ELEMS];
    __shared__ __attribute__((aligned(16))) T sV[kKvStages * ELEMS];
    __shared__ __attribute__((aligned(16))) float sBraw[kKvStages][BN];
    __shared__ __attribute__((aligned(16))) float sBw[4][BN];

    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int hh = lane >> 5, kcol = lane & 31;
    const int nqb = (P.nq + kDqBM - 1) / kDqBM;
    int unit, rank;
    block_order<CAUSAL>(nqb, P.heads, P.k.hdiv, unit, rank);
    const int qblk = CAUSAL ? nqb - 1 - rank : rank;  // heaviest first
    const int h = unit % P.heads, b = unit / P.heads;
    const int qw0 = qblk * kDqBM + w * 32;
    const int qi = qw0 + kcol;
    const bool q_ok = qi < P.nq;

    // rows past the end read row 0 and are zeroed: every prologue load goes out before the
    // first is used (a branch around a load makes its join wait for the loads before it)
    const int qc = q_ok ? qi : 0;
    frag qf[D / 16], of[D / 16];
    u32x4_t orows[D / 16];
    float l = 0.f, dl = 0.f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        u32x4_t qr = *reinterpret_cast<const u32x4_t*>(P.q.row<T>(b, h, qc) + c * 16 + 8 * hh);
        u32x4_t orr = *reinterpret_cast<const u32x4_t*>(G.dout.row<T>(b, h, qc) + c * 16 + 8 * hh);
        if (!q_ok) qr = orr = u32x4_t{0u, 0u, 0u, 0u};
        qf[c] = __builtin_bit_cast(frag, qr);
        of[c] = __builtin_bit_cast(frag, orr);
    }
    if (G.fused_pre) {
#pragma unroll
        for (int c = 0; c < D / 16; ++c)
            orows[c] = *reinterpret_cast<const u32x4_t*>(P.out.row<T>(b, h, qc) + c * 16 + 8 * hh);
        l = *P.lse.row<float>(b, h, qc);
        if (G.dlse.ok()) dl = *G.dlse.row<float>(b, h, qc);
    }
    const int64_t row = ((int64_t)b * P.heads + h) * P.nq + qc;
    float lse_l2, dpi;
    if (G.fused_pre) {
        // the preprocess of this wave's rows: D = rowsum(dO * O) - dlse, lse (+inf for a
        // fully-masked row), also written for the dK/dV kernel that runs next
        float part = 0.f;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            const u32x4_t grow = __builtin_bit_cast(u32x4_t, of[c]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float o0, o1, g0, g1;
                unpack2<T>(orows[c][e], o0, o1);
                unpack2<T>(grow[e], g0, g1);
                part += o0 * g0;
                part += o1 * g1;
            }
        }
        const float dsum = xhalf_sum(part);
        if (!q_ok) l = dl = 0.f;
        const bool normal = l > kMaskedThreshold;
        const float lseb = normal ? l : INFINITY;
        dpi = normal ? dsum - dl : 0.f;
        lse_l2 = q_ok ? lseb * kLog2e : INFINITY;
        if (q_ok && hh == 0) {
            if (G.seeds) {
                G.ws_D[row] = -dpi;
                G.ws_lse[row] = lseb * (SOFTCLAMP ? kLog2e : -1.f / P.scale);
            } else {
                G.ws_D[row] = dpi;
                G.ws_lse[row] = lseb;
            }
        }
    } else {
        lse_l2 = q_ok ? G.ws_lse[row] * kLog2e : INFINITY;
        dpi = q_ok ? G.ws_D[row] : 0.f;
    }
    // retire the compiler-visible loads before the first direct load
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        qf[c] = opaque(qf[c]);
        of[c] = opaque(of[c]);
    }
    lse_l2 = opaque(lse_l2);
    dpi = opaque(dpi);
    const float sl2 = P.scale * kLog2e;
    const float cinv = SOFTCLAMP ? P.scale / P.softclamp : 0.f;
    const float cl2 = SOFTCLAMP ? P.softclamp * kLog2e : 0.f;

    f32x16_t dq[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) dq[x] = zero16();

    const int ksn = (int)P.k.sn, vsn = (int)P.v.sn;
    const srd_t rk = make_srd(P.k.row<T>(b, h, 0), (uint32_t)(((int64_t)(P.nk - 1) * ksn + D) * 2));
    const srd_t rv = make_srd(P.v.row<T>(b, h, 0), (uint32_t)(((int64_t)(P.nk - 1) * vsn + D) * 2));
    const int bes = P.bias.dtype == PA_F32 ? 4 : 2;
    const float bmul = FOLD ? 1.f / P.scale : kLog2e;
    srd_t rb = {0, 0, 0, 0};
    if (HAS_BIAS) rb = make_srd(P.bias.p + P.bias.idx(b, h, 0) * bes, (uint32_t)(P.nk * bes));
    uint32_t offk[NL], offv[NL];
#pragma unroll
    for (int n = 0; n < NL; ++n) {
        const int p = n * kBwdThreads + tid, r = p / CPR, ph = p % CPR;
        offk[n] = (uint32_t)((r * ksn + (ph ^ swz_qt<D>(r)) * 8) * 2);
        offv[n] = (uint32_t)((r * vsn + (ph ^ swz_qt<D>(r)) * 8) * 2);
    }
    const int bq = BN * bes / 4;  // bias bytes per wave
    const uint32_t lds_k = lds_addr(sK), lds_v = lds_addr(sV), lds_b = lds_addr(&sBraw[0][0]);
    auto issue = [&](int j0, int stage) __attribute__((always_inline)) {
        const uint32_t tk = (uint32_t)(j0 * ksn * 2), tv = (uint32_t)(j0 * vsn * 2);
        const uint32_t kd = lds_k + (uint32_t)(stage * ELEMS * 2), vd = lds_v + (uint32_t)(stage * ELEMS * 2);
#pragma unroll
        for (int n = 0; n < NL; ++n) {
            dma16(rk, kd + (uint32_t)((n * kBwdThreads + w * 64) * 16), offk[n] + tk);
            dma16(rv, vd + (uint32_t)((n * kBwdThreads + w * 64) * 16), offv[n] + tv);
        }
        if (HAS_BIAS && 16 * lane < bq)
            dma16(rb, lds_b + (uint32_t)(stage * BN * 4 + w * bq), (uint32_t)(w * bq + 16 * lane + j0 * bes));
    };

    int roff[D / 16];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) roff[c] = kcol * D + (((2 * c + hh) ^ swz_qt<D>(kcol)) * 8);
    int toff[2][D / 32];
    {
        const int g = lane >> 4, j = lane & 15;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int r = 8 * u + 4 * (g >> 1) + (j >> 2);
#pragma unroll
            for (int x = 0; x < D / 32; ++x) {
                const int ch = 4 * x + 2 * (g & 1) + ((j & 3) >> 1);
                toff[u][x] = r * D + ((ch ^ swz_qt<D>(r)) * 8) + 4 * (j & 1);
            }
        }
    }

    const int kend = CAUSAL ? min(P.nk, qblk * kDqBM + kDqBM) : P.nk;
    // tiles [tb, te): with the range of keys that can enter a normal row (masked passes), the
    // tiles outside it are neither loaded nor visited; t counts from tb
    int tb = 0, te = (kend + BN - 1) / BN;
    if (HAS_BIAS && P.live) {
        const int hd = P.bias.hdiv;
        const int32_t* r = P.live + 2 * ((int64_t)b * (P.heads / hd) + h / hd);
        const int lo = r[0], hi = r[1];
        te = min(te, (hi + BN - 1) / BN);
        tb = min(lo / BN, te);
    }
    const int ntiles = te - tb;
    const int nact = max(0, (CAUSAL ? min(te, (qw0 + 31) / BN + 1) : te) - tb);
    if (ntiles > 0) issue(tb * BN, 0);
    if (ntiles > 1) issue((tb + 1) * BN, 1);
    int st = 0;
    auto enter = [&](int t) __attribute__((always_inline)) {
        if (t + 1 < ntiles) wait_vmcnt<NOPS>();
        else wait_vmcnt<0>();
        lds_barrier();
        if (t + 2 < ntiles) issue((tb + t + 2) * BN, st == 0 ? 2 : st - 1);
    };
    // this wave's converted copy of a tile's key terms; true when every one is -inf (masked
    // keys: every probability of the tile is 0)
    auto conv_bias = [&](int stg) __attribute__((always_inline)) -> bool {
        float x;
        if (bes == 4) x = sBraw[stg][lane];
        else x = (float)reinterpret_cast<const T*>(&sBraw[stg][0])[lane];
        const float xw = bias_class(x) == 0 ? x * bmul : -INFINITY;
        sBw[w][lane] = xw;
        return !__any(xw != -INFINITY);
    };
    for (int t = 0; t < nact; ++t) {
        enter(t);
        if (HAS_BIAS) {
            // tiles of masked keys are passed through (loads and barriers only); the last
            // active tile is computed even then (its probabilities are 0)
            bool dead = conv_bias(st);
            while (dead && t + 1 < nact) {
                st = st == 2 ? 0 : st + 1;
                enter(++t);
                dead = conv_bias(st);
            }
        }
        const int j0 = (tb + t) * BN;
        const T* Kt = sK + st * ELEMS;
        const T* Vt = sV + st * ELEMS;
        // the two 32-key blocks in a software pipeline (MFMAs of one beside the VALU of the other)
        auto scores = [&](int kb, f32x16_t& s, f32x16_t& dp) __attribute__((always_inline)) {
            s = zero16();
            dp = zero16();
            if (FOLD) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 bb = *reinterpret_cast<const float4*>(&sBw[w][kb * 32 + 8 * g + 4 * hh]);
                    s[4 * g] = bb.x;
                    s[4 * g + 1] = bb.y;
                    s[4 * g + 2] = bb.z;
                    s[4 * g + 3] = bb.w;
                }
            }
#pragma unroll
            for (int c = 0; c < D / 16; ++c) {
                const int off = kb * 32 * D + roff[c];
                s = M::run(ld_frag<T>(Kt + off), qf[c], s);
                dp = M::run(ld_frag<T>(Vt + off), of[c], dp);
            }
        };
        // keys after the lane's query or past the last key: scores -> -inf (P = 0).  Register i
        // holds key j0 + kb*32 + 8*(i/4) + 4*hh + (i%4) of the lane's query.
        auto mask = [&](int kb, f32x16_t& s) __attribute__((always_inline)) {
            const int kb0 = j0 + kb * 32;
            if ((CAUSAL && kb0 + 31 > qw0) || kb0 + 32 > P.nk) {
                keep_branch();
                int lim = P.nk - 1 - kb0;
                if (CAUSAL) lim = min(lim, qi - kb0);
                lim -= 4 * hh;
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (8 * (i / 4) + (i % 4) > lim) s[i] = -INFINITY;
            }
        };
        // dS^T = P^T (dP^T - D), packed as B operands
        auto grads = [&](int kb, f32x16_t& s, const f32x16_t& dp, frag (&df)[2]) __attribute__((always_inline)) {
            float yv[16];
            if (SOFTCLAMP) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    float bv[4] = {0.f, 0.f, 0.f, 0.f};
                    if (HAS_BIAS) {
                        const float4 bb = *reinterpret_cast<const float4*>(&sBw[w][kb * 32 + 8 * g + 4 * hh]);
                        bv[0] = bb.x;
                        bv[1] = bb.y;
                        bv[2] = bb.z;
                        bv[3] = bb.w;
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * g + r;
                        yv[i] = s[i] == -INFINITY ? 1.f : tanhf(s[i] * cinv);
                        s[i] = s[i] == -INFINITY ? 0.f : fast_exp2(yv[i] * cl2 + bv[r] - lse_l2);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) s[i] = fast_exp2(fmaf(s[i], sl2, -lse_l2));
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float dsv = s[i] * (dp[i] - dpi);
                if (SOFTCLAMP) dsv *= (1.f - yv[i] * yv[i]);
                s[i] = dsv;
            }
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) df[t2] = acc_to_frag<T>(s, t2);
        };
        auto accumulate = [&](int kb, const frag (&df)[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
                for (int x = 0; x < D / 32; ++x) {
                    const int row0 = kb * 32 + 16 * t2;
                    const u32x2_t lo = lds_read_tr(Kt + row0 * D + toff[0][x]);
                    const u32x2_t hi = lds_read_tr(Kt + row0 * D + toff[1][x]);
                    const u32x4_t v4 = {lo[0], lo[1], hi[0], hi[1]};
                    dq[x] = M::run(__builtin_bit_cast(frag, v4), df[t2], dq[x]);
                }
        };
        f32x16_t s0, dp0, s1, dp1;
        frag df0[2], df1[2];
#if PA_DQ_CHUNKS
        if constexpr (!SOFTCLAMP) {
            // Explicit pipeline of the two key blocks: (A) scores of block 0; (B) scores of
            // block 1, each MFMA followed by the VALU work of two of block 0's gradient
            // entries; (C) dQ of block 0, each MFMA followed by four of block 1's entries;
            // (D) dQ of block 1.  Scheduling barriers keep the chunks in this order.
            auto grads2 = [&](f32x16_t& sv, const f32x16_t& dpv, int j, u32x4_t (&dfr)[2])
                              __attribute__((always_inline)) {
                // entries 2j, 2j+1: P = exp2(S*scale*log2e - lse), dS = P (dP - D), packed
                const float p0 = fast_exp2(fmaf(sv[2 * j], sl2, -lse_l2));
                const float p1 = fast_exp2(fmaf(sv[2 * j + 1], sl2, -lse_l2));
                dfr[j / 4][j % 4] = pack2<T>(p0 * (dpv[2 * j] - dpi), p1 * (dpv[2 * j + 1] - dpi));
            };
            scores(0, s0, dp0);
            mask(0, s0);
            __builtin_amdgcn_sched_barrier(0);
            u32x4_t dfr0[2], dfr1[2];
            {
                // (B): each chunk reads the next chunk's K or V fragment, issues its MFMA and
                // forms two of block 0's entries
                s1 = zero16();
                dp1 = zero16();
                if (FOLD) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const float4 bb = *reinterpret_cast<const float4*>(&sBw[w][32 + 8 * g + 4 * hh]);
                        s1[4 * g] = bb.x;
                        s1[4 * g + 1] = bb.y;
                        s1[4 * g + 2] = bb.z;
                        s1[4 * g + 3] = bb.w;
                    }
                }
                auto frag_b = [&](int i) __attribute__((always_inline)) -> frag {
                    return ld_frag<T>((i % 2 == 0 ? Kt : Vt) + 32 * D + roff[i / 2]);
                };
                frag cur = frag_b(0);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < 2 * (D / 16); ++i) {
                    const int c = i / 2;
                    frag nxt = cur;
                    if (i + 1 < 2 * (D / 16)) nxt = frag_b(i + 1);
                    if (i % 2 == 0) s1 = M::run(cur, qf[c], s1);
                    else dp1 = M::run(cur, of[c], dp1);
                    constexpr int per = 2 * (D / 16) / 8;  // MFMAs per pair of entries
                    if (i % per == 0) grads2(s0, dp0, i / per, dfr0);
                    cur = nxt;
                    __builtin_amdgcn_sched_barrier(0);
                }
                // block 0's packed entries are consumed here, before the mask branch below,
                // so that their VALU work is not sunk out of the region
                dfr0[0] = opaque(dfr0[0]);
                dfr0[1] = opaque(dfr0[1]);
            }
            df0[0] = __builtin_bit_cast(frag, dfr0[0]);
            df0[1] = __builtin_bit_cast(frag, dfr0[1]);
            mask(1, s1);
            __builtin_amdgcn_sched_barrier(0);
            {
                // (C): each chunk reads the next chunk's transposed K fragment, issues its dQ
                // MFMA and forms four of block 1's entries
                auto frag_c = [&](int i) __attribute__((always_inline)) -> frag {
                    const int t2 = i / (D / 32), x = i % (D / 32);
                    const u32x2_t lo = lds_read_tr(Kt + 16 * t2 * D + toff[0][x]);
                    const u32x2_t hi = lds_read_tr(Kt + 16 * t2 * D + toff[1][x]);
                    const u32x4_t v4 = {lo[0], lo[1], hi[0], hi[1]};
                    return __builtin_bit_cast(frag, v4);
                };
                frag cur = frag_c(0);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < 2 * (D / 32); ++i) {
                    const int t2 = i / (D / 32), x = i % (D / 32);
                    frag nxt = cur;
                    if (i + 1 < 2 * (D / 32)) nxt = frag_c(i + 1);
                    dq[x] = M::run(cur, df0[t2], dq[x]);
#pragma unroll
                    for (int jj = 0; jj < 8 / (2 * (D / 32)); ++jj)
                        grads2(s1, dp1, i * (8 / (2 * (D / 32))) + jj, dfr1);
                    cur = nxt;
                    __builtin_amdgcn_sched_barrier(0);
                }
                dfr1[0] = opaque(dfr1[0]);
                dfr1[1] = opaque(dfr1[1]);
            }
            df1[0] = __builtin_bit_cast(frag, dfr1[0]);
            df1[1] = __builtin_bit_cast(frag, dfr1[1]);
            accumulate(1, df1);
            st = st == 2 ? 0 : st + 1;
            continue;
        }
#endif
        scores(0, s0, dp0);
        mask(0, s0);
        scores(1, s1, dp1);
        grads(0, s0, dp0, df0);
        mask(1, s1);
        accumulate(0, df0);
        grads(1, s1, dp1, df1);
        accumulate(1, df1);
        st = st == 2 ? 0 : st + 1;
    }
    for (int t = nact; t < ntiles; ++t) {
        enter(t);
        st = st == 2 ? 0 : st + 1;
    }

    if (!q_ok) return;
    T* dqrow = G.dq.wrow<T>(b, h, qi);
    const bool acc = (G.accumulate & PA_ACC_DQ) != 0;
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = x * 32 + 8 * g + 4 * hh;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = dq[x][4 * g + r] * P.scale + (acc ? to_f(dqrow[d + r]) : 0.f);
            u32x2_t pk;
            pk[0] = pack2<T>(v[0], v[1]);
            pk[1] = pack2<T>(v[2], v[3]);
            *reinterpret_cast<u32x2_t*>(dqrow + d) = pk;
        }
    }
}

// ---------------------------------------------------------------------------------------

bool mfma_bwd_supported(const GradDev& G, int dtype) {
    const PassDev& P = G.f;
    if (dtype == PA_F32) return mfma_bwd_f32_supported(G);
    if (dtype != PA_BF16 && dtype != PA_F16) return false;
    if (P.dim != 64 && P.dim != 128 && P.dim != 256) return false;
    const DView* loads[] = {&P.q, &P.k, &P.v, &G.dout};
    for (const DView* v : loads)
        if (!aligned_rows_host(*v, 8)) return false;
    if (P.vmul.ok() && !aligned_rows_host(P.vmul, 8)) return false;
    const DView* stores[] = {&G.dq, &G.dk, &G.dv};
    for (const DView* v : stores)
        if (!aligned_rows_host(*v, 4)) return false;
    if (P.vmul.ok() && !aligned_rows_host(G.dvmul, 4)) return false;
    return true;
}

// the direct-to-LDS kernels address the query-side (or key-side) tensors of one head with
// 32-bit byte offsets up to the end of the last tile
static bool bwd_dma_ok(const GradDev& G) {
    const PassDev& P = G.f;
    const int64_t qspan = std::max(P.q.sn, G.dout.sn) * ((int64_t)P.nq + 2 * kKvBQ) * 2;
    const int64_t kspan = std::max(P.k.sn, P.v.sn) * ((int64_t)P.nk + 2 * 64) * 2;
    if (!(qspan < ((int64_t)1 << 31) && kspan < ((int64_t)1 << 31))) return false;
    // lse / D rows travel in whole 16-byte chunks
    return P.nq % 4 == 0;
}

// the direct-to-LDS dQ kernel also reads the key bias as one contiguous row of whole chunks
static bool bwd_dq_dma_ok(const GradDev& G) {
    const PassDev& P = G.f;
    const int64_t kspan = std::max(P.k.sn, P.v.sn) * ((int64_t)P.nk + 2 * kDqBN) * 2;
    if (!(kspan < ((int64_t)1 << 31))) return false;
    if (P.bias.ok()) {
        const int64_t es = P.bias.dtype == PA_F32 ? 4 : 2;
        if (P.bias.sn != 1) return false;
        if ((uintptr_t)P.bias.p % 16 != 0 || (P.bias.sh * es) % 16 != 0 || (P.bias.sb * es) % 16 != 0) return false;
        if ((P.nk * es) % 16 != 0) return false;
    }
    return true;
}

// The preprocess folded into the direct-to-LDS dQ kernel (which then runs first): it loads
// the O rows of its queries beside dO with 16-byte loads.
bool mfma_bwd_fuses_pre(const GradDev& G) {
    const PassDev& P = G.f;
    if (!PA_BWD_DMA || P.vmul.ok() || P.q.dtype == PA_F32) return false;
    if (P.dim != 64 && P.dim != 128) return false;
    return bwd_dq_dma_ok(G) && aligned_rows_host(P.out, 8);
}

template <typename T, int D, bool C, bool S, bool V, bool B>
static void launch_dq(const GradDev& G, hipStream_t s) {
    const PassDev& P = G.f;
    dim3 grid(((P.nq + kDqBM - 1) / kDqBM) * P.heads * P.batch);
    ProfScope ps("mfma_bwd_dq", s);
    // head dim 256: the register-staged kernels only (their direct-to-LDS stages would not
    // fit in LDS)
    if constexpr (D != 256) {
        if (!V && PA_BWD_DMA && bwd_dq_dma_ok(G)) {
            hipLaunchKernelGGL((k_mfma_bwd_dq_dma<T, D, C, S, B>), grid, dim3(kBwdThreads), 0, s, G);
            return;
        }
    }
    hipLaunchKernelGGL((k_mfma_bwd_dq<T, D, C, S, V, B>), grid, dim3(kBwdThreads), 0, s, G);
}

template <typename T, int D, bool C, bool S, bool V, bool B>
static void launch_bwd_t(const GradDev& G0, hipStream_t s) {
    const PassDev& P = G0.f;
    const bool kv_dma = D != 256 && !V && PA_BWD_DMA && bwd_dma_ok(G0);
    GradDev G = G0;
    // the dQ kernel writes the preprocess in the direct-to-LDS dK/dV kernel's seed form
    G.seeds = (G.fused_pre && kv_dma) ? 1 : 0;
    if (G.fused_pre) launch_dq<T, D, C, S, V, B>(G, s);  // writes the preprocess for dK/dV
    {
        dim3 grid(((P.nk + kKvBK - 1) / kKvBK) * G.hk * P.batch);
        ProfScope ps("mfma_bwd_dkv", s);
        bool done = false;
        if constexpr (D != 256) {  // head dim 256: the register-staged kernel only
            if (kv_dma) {
                hipLaunchKernelGGL((k_mfma_bwd_dkv_dma<T, D, C, S, B>), grid, dim3(kBwdThreads), 0, s, G);
                done = true;
            }
        }
        if (!done)
            hipLaunchKernelGGL((k_mfma_bwd_dkv<T, D, C, S, V, B>), grid, dim3(kBwdThreads), 0, s, G);
    }
    if (!G.fused_pre) launch_dq<T, D, C, S, V, B>(G, s);
}

template <typename T, int D, bool C, bool S>
static void launch_bwd_vb(const GradDev& G, hipStream_t s) {
    const bool v = G.f.vmul.ok(), b = G.f.bias.ok();
    if (v) b ? launch_bwd_t<T, D, C, S, true, true>(G, s) : launch_bwd_t<T, D, C, S, true, false>(G, s);
    else b ? launch_bwd_t<T, D, C, S, false, true>(G, s) : launch_bwd_t<T, D, C, S, false, false>(G, s);
}

template <typename T, int D>
static void launch_bwd_d(const GradDev& G, hipStream_t s) {
    const bool c = G.f.causal != 0, sc = G.f.softclamp > 0.f;
    if (c) sc ? launch_bwd_vb<T, D, true, true>(G, s) : launch_bwd_vb<T, D, true, false>(G, s);
    else sc ? launch_bwd_vb<T, D, false, true>(G, s) : launch_bwd_vb<T, D, false, false>(G, s);
}

void launch_mfma_bwd(const GradDev& G, int dtype, hipStream_t s) {
    if (dtype == PA_F32) {
        launch_mfma_bwd_f32(G, s);
        return;
    }
    if (dtype == PA_BF16) {
        if (G.f.dim == 64) launch_bwd_d<bf16, 64>(G, s);
        else if (G.f.dim == 128) launch_bwd_d<bf16, 128>(G, s);
        else launch_bwd_d<bf16, 256>(G, s);
    } else {
        if (G.f.dim == 64) launch_bwd_d<f16, 64>(G, s);
        else if (G.f.dim == 128) launch_bwd_d<f16, 128>(G, s);
        else launch_bwd_d<f16, 256>(G, s);
    }
}

}  // namespace pa
