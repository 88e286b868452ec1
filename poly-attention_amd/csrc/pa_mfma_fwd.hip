// pa_mfma_fwd.hip -- MFMA forward attention pass for bf16 / f16, head dim 64 or 128 (gfx950).
//
// Common scheme: 32 queries per wave.  Per key tile a wave computes the transposed scores
// S^T = K . Q^T with v_mfma_f32_32x32x16_{bf16,f16}: the 32x32 accumulator layout gives lane
// l the column q = l % 32 and 16 key rows per block, so the online-softmax state (running max
// m, sum l, the output rescale) is a per-lane scalar.  The probabilities, rounded to the input
// type, stay in registers as the B operand of O^T += V^T . P^T (keys permuted consistently
// between the two operands, see pa_mfma.h).
//
// Softmax: log2 domain (bare v_exp_f32, scale*log2(e) folded into one FMA; without softclamp
// the running max is taken on the raw scores).  The running max is updated lazily: it moves
// (and the output is rescaled) only when a tile's max exceeds it by more than kFwdTau, so
// probabilities stay <= 2^kFwdTau (exact in fp32 and within the input type's exponent range);
// after the first tiles this almost never happens.  Row sums accumulate the rounded
// probabilities with v_dot2 (the same values the MFMA consumes).  Without softclamp (and
// without a bias added to the logits) the direct-to-LDS kernel takes no per-tile max at all:
// it forms the probabilities against the running max and checks their sum instead
// (FwdWave::probs_checked), so no reduction sits between the score MFMAs and the
// exponentials, and it pipelines a wave's two query blocks so that each one's probabilities
// are formed while the matrix core runs the other's products.
//
// Kernels:
//  * k_mfma_fwd_dma (default): K, V and the key bias travel HBM -> LDS by direct loads,
//    four stages of 64-key tiles filled and waited for in pairs (one barrier per two tiles);
//    V^T operands come from transposing LDS reads; without softclamp the key bias is folded
//    into the score accumulators.
//  * k_mfma_fwd: register-staged loads with a transposing LDS store; the general kernel
//    (value multiplier, key masks, strided biases, very long rows).
//
// Rows whose every key is masked are left with lse = NaN for k_fwd_fixup, which applies the
// reference's finite-fill semantics to them.  Workgroups are mapped XCD-aware (pa_mfma.h); in
// causal grids each XCD dispatches the heaviest query blocks of all its heads first.
//
#include <algorithm>
#include <type_traits>

#include "pa_common.h"
#include "pa_launch.h"
#include "pa_mfma.h"

namespace pa {

#ifndef PA_FWD_KB64
#define PA_FWD_KB64 2
#endif
#ifndef PA_FWD_USPLIT
#define PA_FWD_USPLIT 1  // QB = 2 with sum-checked probabilities: the two query blocks pipelined
#endif
#ifndef PA_FWD_QB64
#define PA_FWD_QB64 2  // 32-query blocks per wave in the direct-to-LDS kernel at head dim 64
#endif

constexpr int kFwdBM = 128;  // query rows per workgroup
constexpr int kFwdThreads = 256;
constexpr float kFwdTau = 8.f;  // lazy-rescale threshold (log2 units)
// sum-checked probabilities (PLAIN scores): largest tile sum per lane accepted without a max
constexpr float kFwdSumCap = 8192.f;
#ifndef PA_FWD_SUMCHECK
#define PA_FWD_SUMCHECK 1
#endif


// Key tile of BN = 32 * KB keys: KB accumulator blocks per wave and tile.
template <int D, int KB>
struct FwdTile {
    static constexpr int BN = 32 * KB;
    static constexpr int KS = D + 8;   // K row stride in LDS (elements)
    static constexpr int VS = BN + 4;  // V^T row stride in LDS (elements)
    static constexpr int BLOCKS = (BN / 4) * (D / 8);  // 4-key x 8-dim blocks per tensor
    static constexpr int NB = (2 * BLOCKS + kFwdThreads - 1) / kFwdThreads;
};

// Per-workgroup key-side pointers (batch and head resolved once).
template <typename T>
struct KeySide {
    const T* k;
    const T* v;
    const T* vm;
    int64_t ksn, vsn, msn;
    const char* bias;
    int64_t bsn;
    int32_t bdt;
    const uint8_t* km;
    int64_t kmsn;
    int32_t nk;
};

template <typename T>
__device__ __forceinline__ KeySide<T> key_side(const PassDev& P, int b, int h) {
    KeySide<T> s;
    s.k = P.k.row<T>(b, h, 0);
    s.v = P.v.row<T>(b, h, 0);
    s.vm = P.vmul.ok() ? P.vmul.row<T>(b, h, 0) : nullptr;
    s.ksn = P.k.sn;
    s.vsn = P.v.sn;
    s.msn = P.vmul.sn;
    s.bias = P.bias.ok() ? P.bias.p + P.bias.idx(b, h, 0) * (P.bias.dtype == PA_F32 ? 4 : 2) : nullptr;
    s.bsn = P.bias.sn;
    s.bdt = P.bias.dtype;
    s.km = P.km.p ? P.km.p + (int64_t)b * P.km.sb : nullptr;
    s.kmsn = P.km.sn;
    s.nk = P.nk;
    return s;
}

// The module epilogue (pa_pass.epi) at one lane's output store: the lane holds 4 * NG outputs
// of row qi, 4 consecutive columns from d = (k / 4) * 32 + (k % 4) * 8 + 4 * hh for k < NG,
// rounded and packed in o[k].  Every root and gate word is loaded before any is used: the
// store is the kernel's tail, where a load per element would serialise on memory latency.
// The root and gate presence are template arguments: with a run-time choice between a loaded
// row and the lane's own output the compiler loads through a selected pointer, which puts the
// output array in scratch memory in every kernel that calls this.
template <typename T, int NG, bool HR, bool HG>
__device__ __forceinline__ void epi_store_rows(const PassDev& P, int b, int h, int qi, int hh,
                                               const u32x2_t (&o)[NG], bool sig) {
    u32x2_t r[NG], g[NG];
#pragma unroll
    for (int k = 0; k < NG; ++k) {
        const int d = (k / 4) * 32 + (k % 4) * 8 + 4 * hh;
        if constexpr (HR) r[k] = *reinterpret_cast<const u32x2_t*>(P.er.row<T>(b, h, qi) + d);
        else r[k] = o[k];
        if constexpr (HG) g[k] = *reinterpret_cast<const u32x2_t*>(P.eg.row<T>(b, h, qi) + d);
        else g[k] = o[k];
    }
    T* yrow = P.ey.wrow<T>(b, h, qi);
#pragma unroll
    for (int k = 0; k < NG; ++k) {
        const int d = (k / 4) * 32 + (k % 4) * 8 + 4 * hh;
        u32x2_t y4;
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            float o0, o1, r0, r1, g0, g1;
            unpack2<T>(o[k][w], o0, o1);
            unpack2<T>(r[k][w], r0, r1);
            unpack2<T>(g[k][w], g0, g1);
            y4[w] = pack2<T>(epi_combine<T>(o0, r0, g0, HR, HG, sig),
                             epi_combine<T>(o1, r1, g1, HR, HG, sig));
        }
        *reinterpret_cast<u32x2_t*>(yrow + d) = y4;
    }
}

template <typename T, int NG>
__device__ __forceinline__ void epi_store_lane(const PassDev& P, int b, int h, int qi, int hh,
                                               const u32x2_t (&o)[NG]) {
    const bool sig = (P.eflags & PA_EPI_ROOT_SIGMOID) != 0;
    if (P.er.ok()) {
        if (P.eg.ok()) epi_store_rows<T, NG, true, true>(P, b, h, qi, hh, o, sig);
        else epi_store_rows<T, NG, true, false>(P, b, h, qi, hh, o, sig);
    } else {
        if (P.eg.ok()) epi_store_rows<T, NG, false, true>(P, b, h, qi, hh, o, sig);
        else epi_store_rows<T, NG, false, false>(P, b, h, qi, hh, o, sig);
    }
}

// Registers holding one K tile and one V tile (+ key bias) between global load and LDS store.
template <int D, int KB>
struct FwdStage {
    u32x4_t w[FwdTile<D, KB>::NB][4];
    float bias;
};

// Issue the global loads of K rows [jk, jk + BN) (when lk) and V rows / key bias [jv, jv + BN)
// (when lv); rows past the end read as zero, their bias as -inf.
template <typename T, int D, int KB, bool HAS_VMUL, bool HAS_BIAS>
__device__ __forceinline__ void fwd_load(const KeySide<T>& ks, int jk, bool lk, int jv, bool lv,
                                         FwdStage<D, KB>& st) {
    using TL = FwdTile<D, KB>;
    const int tid = threadIdx.x;
    const u32x4_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int c = 0; c < TL::NB; ++c) {
        const int task = tid + c * kFwdThreads;
        if (task < 2 * TL::BLOCKS) {
            const int tensor = task / TL::BLOCKS, blk = task % TL::BLOCKS;
            const int rg = blk / (D / 8), cc = blk % (D / 8);
            if (tensor == 0 ? lk : lv) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int j = (tensor == 0 ? jk : jv) + rg * 4 + r;
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
    }
    if (HAS_BIAS && lv && tid < TL::BN) {
        const int j = jv + tid;
        float bv = -INFINITY;
        if (j < ks.nk && (!ks.km || ks.km[j * ks.kmsn])) {
            bv = 0.f;
            if (ks.bias) {
                const float x = load_any(ks.bias, ks.bdt, j * ks.bsn);
                bv = bias_class(x) == 0 ? x * kLog2e : -INFINITY;
            }
        }
        st.bias = bv;
    }
}

template <typename T, int D, int KB, bool HAS_BIAS>
__device__ __forceinline__ void fwd_store(const FwdStage<D, KB>& st, T* sK, bool sk, T* sVt, float* sB,
                                          bool sv) {
    using TL = FwdTile<D, KB>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int c = 0; c < TL::NB; ++c) {
        const int task = tid + c * kFwdThreads;
        if (task < 2 * TL::BLOCKS) {
            const int tensor = task / TL::BLOCKS, blk = task % TL::BLOCKS;
            const int rg = blk / (D / 8), cc = blk % (D / 8);
            if (tensor == 0) {
                if (sk) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        *reinterpret_cast<u32x4_t*>(sK + (rg * 4 + r) * TL::KS + cc * 8) = st.w[c][r];
                }
            } else if (sv) {
                store_block_transposed(st.w[c], reinterpret_cast<uint16_t*>(sVt + (cc * 8) * TL::VS + rg * 4),
                                       TL::VS);
            }
        }
    }
    if (HAS_BIAS && sv && tid < TL::BN) sB[tid] = st.bias;
}

// Per-wave state and the pieces of one pipeline step.  BIAS_IN_LOGITS: the key bias is added
// to the scores in logits() (otherwise it is absent or already inside the scores).
template <typename T, int D, int KB, bool CAUSAL, bool SOFTCLAMP, bool HAS_BIAS,
          bool BIAS_IN_LOGITS = HAS_BIAS>
struct FwdWave {
    using TL = FwdTile<D, KB>;
    using M = Mma<T>;
    typedef typename M::frag frag;
    static constexpr int BN = TL::BN;
    static constexpr bool PLAIN = !BIAS_IN_LOGITS && !SOFTCLAMP;  // max taken on raw scores

    frag qf[D / 16];
    f32x16_t o[D / 32];
    float m, l;
    int kcol, hh, q0, qi, nk;
    float sl2, cinv, cl2;

    // S^T block kb of a key tile: s[kb] = K[kb*32 + row, :] . Q^T
    __device__ __forceinline__ void scores(const T* K, f32x16_t (&s)[KB]) const {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            s[kb] = zero16();
#pragma unroll
            for (int c = 0; c < D / 16; ++c)
                s[kb] = M::run(ld_frag<T>(K + (kb * 32 + kcol) * TL::KS + c * 16 + 8 * hh), qf[c], s[kb]);
        }
    }

    // causal diagonal / past-the-end keys of the tile at j0 -> -inf (raw scores).  Register i
    // of block kb holds key j0 + kb*32 + 8*(i/4) + 4*hh + (i%4).
    __device__ __forceinline__ void mask_edges(f32x16_t (&s)[KB], int j0) const {
        if ((CAUSAL && j0 + BN - 1 > q0) || (!HAS_BIAS && j0 + BN > nk)) {
            keep_branch();
            int lim = HAS_BIAS ? (1 << 30) : nk - 1 - j0;
            if (CAUSAL) lim = min(lim, qi - j0);
            lim -= 4 * hh;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (kb * 32 + 8 * (i / 4) + (i % 4) > lim) s[kb][i] = -INFINITY;
        }
    }

    // as mask_edges, but past-the-end keys are masked by position also with a key bias
    __device__ __forceinline__ void mask_edges_nk(f32x16_t (&s)[KB], int j0) const {
        if ((CAUSAL && j0 + BN - 1 > q0) || (j0 + BN > nk)) {
            keep_branch();
            int lim = nk - 1 - j0;
            if (CAUSAL) lim = min(lim, qi - j0);
            lim -= 4 * hh;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (kb * 32 + 8 * (i / 4) + (i % 4) > lim) s[kb][i] = -INFINITY;
        }
    }

    // scores -> log2-domain logits in place (bias / softclamp paths); returns the max over the
    // query's logits of this tile (PLAIN: of the raw scores, times scale*log2e)
    __device__ __forceinline__ float logits(f32x16_t (&s)[KB], const float* sB) const {
        // four independent max chains (short dependency chains), combined at the end
        float mq[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float bv[4] = {0.f, 0.f, 0.f, 0.f};
                if (BIAS_IN_LOGITS) {
                    const float4 bb = *reinterpret_cast<const float4*>(sB + kb * 32 + 8 * g + 4 * hh);
                    bv[0] = bb.x;
                    bv[1] = bb.y;
                    bv[2] = bb.z;
                    bv[3] = bb.w;
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float x = s[kb][4 * g + r];
                    if (!PLAIN) {
                        if (SOFTCLAMP) x = (x == -INFINITY) ? -INFINITY : cl2 * tanhf(x * cinv) + bv[r];
                        else x = fmaf(x, sl2, bv[r]);
                        s[kb][4 * g + r] = x;
                    }
                    mq[r] = fmaxf(mq[r], x);
                }
            }
        }
        const float mx = xhalf_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3])));
        return PLAIN ? mx * sl2 : mx;
    }

    // probabilities against the max msub, rounded to T and packed as the PV B operands; returns
    // the lane's sum of the rounded probabilities
    __device__ __forceinline__ float probs(const f32x16_t (&s)[KB], float msub, u32x4_t (&pk)[KB][2]) const {
        float lt[4] = {0.f, 0.f, 0.f, 0.f};  // independent accumulation chains
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float x0 = s[kb][8 * t2 + 2 * k], x1 = s[kb][8 * t2 + 2 * k + 1];
                    const float p0 = PLAIN ? fast_exp2(fmaf(x0, sl2, -msub)) : fast_exp2(x0 - msub);
                    const float p1 = PLAIN ? fast_exp2(fmaf(x1, sl2, -msub)) : fast_exp2(x1 - msub);
                    const uint32_t w = pack2<T>(p0, p1);
                    pk[kb][t2][k] = w;
                    lt[k] = sum_pair<T>(w, lt[k]);
                }
        return (lt[0] + lt[1]) + (lt[2] + lt[3]);
    }

    // Probabilities of a tile without a per-tile max (PLAIN scores): they are formed against the
    // running max m first; a lane whose tile sum is not in [0, kFwdSumCap] -- some probability
    // above kFwdSumCap, a non-finite value, or m still -inf before the first tile -- makes the
    // wave take the tile's max, move m (settle) and form them again.  Every probability that
    // reaches the MFMA is therefore <= kFwdSumCap, and m only ever holds a maximum the lane's
    // scores reached.  Saves the max reduction (two VALU instructions per four scores) on all
    // but the rare tiles where the scores rise.
    __device__ __forceinline__ float probs_checked(f32x16_t (&s)[KB], const float* sB, u32x4_t (&pk)[KB][2]) {
        float lt = probs(s, m, pk);
        if (__any(!(lt <= kFwdSumCap))) {
            keep_branch();
            settle(logits(s, sB), true);
            lt = probs(s, m == -INFINITY ? 0.f : m, pk);
        }
        return lt;
    }

    // lazy rescale: only when some lane's tile max exceeds its running max by more than
    // kFwdTau (by anything, with `always`) does the running max move (rescaling O and l)
    __device__ __forceinline__ void settle(float mx, bool always = false) {
        if (always) {
            const float m_new = fmaxf(m, mx);
            const float alpha = (m_new > m) ? fast_exp2(m - m_new) : 1.f;
            l *= alpha;
#pragma unroll
            for (int x = 0; x < D / 32; ++x)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[x][i] *= alpha;
            m = m_new;
            return;
        }
        if (__any(mx > m + kFwdTau)) {
            keep_branch();
            const float m_new = fmaxf(m, mx);
            const float alpha = (m_new > m) ? fast_exp2(m - m_new) : 1.f;
            l *= alpha;
#pragma unroll
            for (int x = 0; x < D / 32; ++x)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[x][i] *= alpha;
            m = m_new;
        }
    }

    // V^T operand fragments of one tile (read early so the LDS latency hides behind the softmax)
    __device__ __forceinline__ void load_v(const T* Vt, frag (&vf)[KB][2][D / 32]) const {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
                for (int x = 0; x < D / 32; ++x)
                    vf[kb][t2][x] = lds_runs<T>(Vt + (x * 32 + kcol) * TL::VS + kb * 32 + 16 * t2 + 4 * hh);
    }

    // O^T += V^T . P^T for one tile
    __device__ __forceinline__ void pv(const frag (&vf)[KB][2][D / 32], const u32x4_t (&pk)[KB][2]) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
                const frag pb = __builtin_bit_cast(frag, pk[kb][t2]);
#pragma unroll
                for (int x = 0; x < D / 32; ++x) o[x] = M::run(vf[kb][t2][x], pb, o[x]);
            }
    }
};

template <typename T, int D, int KB, bool CAUSAL, bool SOFTCLAMP, bool HAS_VMUL, bool HAS_BIAS>
__global__ __launch_bounds__(kFwdThreads, D == 64 ? 2 : 1) void k_mfma_fwd(PassDev P) {
    using TL = FwdTile<D, KB>;
    constexpr int BN = TL::BN;
    using W = FwdWave<T, D, KB, CAUSAL, SOFTCLAMP, HAS_BIAS>;
    typedef typename W::frag frag;
    __shared__ __attribute__((aligned(16))) T sK[2][BN * TL::KS];
    __shared__ __attribute__((aligned(16))) T sVt[2][D * TL::VS];
    __shared__ __attribute__((aligned(16))) float sB[2][BN];

    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int nqb = (P.nq + kFwdBM - 1) / kFwdBM;
    int bh, rank;
    block_order<CAUSAL>(nqb, P.heads, P.k.hdiv, bh, rank);
    const int qb = CAUSAL ? nqb - 1 - rank : rank;
    const int h = bh % P.heads, b = bh / P.heads;

    W wv;
    wv.hh = lane >> 5;
    wv.kcol = lane & 31;
    wv.q0 = qb * kFwdBM + w * 32;
    wv.qi = wv.q0 + wv.kcol;
    wv.nk = P.nk;
    wv.sl2 = P.scale * kLog2e;
    wv.cinv = SOFTCLAMP ? P.scale / P.softclamp : 0.f;
    wv.cl2 = SOFTCLAMP ? P.softclamp * kLog2e : 0.f;
    wv.m = -INFINITY;
    wv.l = 0.f;
    // Q^T operand fragments: lane (q, hh) holds Q[q][c*16 + 8*hh .. +7]
    {
        const int qi = wv.qi;
        const T* qrow = P.q.row<T>(b, h, qi < P.nq ? qi : 0);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            u32x4_t raw = {0u, 0u, 0u, 0u};
            if (qi < P.nq) raw = *reinterpret_cast<const u32x4_t*>(qrow + c * 16 + 8 * wv.hh);
            wv.qf[c] = __builtin_bit_cast(frag, raw);
        }
    }
#pragma unroll
    for (int x = 0; x < D / 32; ++x) wv.o[x] = zero16();

    const KeySide<T> ks = key_side<T>(P, b, h);
    const int kend = CAUSAL ? min(P.nk, qb * kFwdBM + kFwdBM) : P.nk;
    const int ntiles = (kend + BN - 1) / BN;
    // a wave skips the tiles that lie wholly above its causal diagonal
    const int wave_last = CAUSAL ? (wv.q0 + 31) : (1 << 30);

    // prologue: K_0, V_0 (+ bias_0), K_1 in LDS; S_0 in registers
    FwdStage<D, KB> st;
    fwd_load<T, D, KB, HAS_VMUL, HAS_BIAS>(ks, 0, true, 0, true, st);
    fwd_store<T, D, KB, HAS_BIAS>(st, sK[0], true, sVt[0], sB[0], true);
    if (ntiles > 1) {
        fwd_load<T, D, KB, HAS_VMUL, HAS_BIAS>(ks, BN, true, 0, false, st);
        fwd_store<T, D, KB, HAS_BIAS>(st, sK[1], true, sVt[0], sB[0], false);
    }
    __syncthreads();

    f32x16_t sa[KB], sb[KB];
    wv.scores(sK[0], sa);
    wv.mask_edges(sa, 0);

    // one pipeline step: softmax + PV of tile t (scores in `cur`), scores of tile t+1 into `nxt`
    auto step = [&](f32x16_t (&cur)[KB], f32x16_t (&nxt)[KB], int t) __attribute__((always_inline)) {
        const int j0 = t * BN;
        const bool more_k = t + 2 < ntiles, more_v = t + 1 < ntiles;
        fwd_load<T, D, KB, HAS_VMUL, HAS_BIAS>(ks, j0 + 2 * BN, more_k, j0 + BN, more_v, st);
        const bool act = j0 <= wave_last, act_next = more_v && j0 + BN <= wave_last;
        const float* bt = sB[t & 1];
        u32x4_t pk[KB][2];
        frag vf[KB][2][D / 32];
        if (act) {
            wv.settle(wv.logits(cur, bt));
            // one basic block of independent work: the score MFMAs of tile t+1 (computed even
            // when that tile is skipped or absent; the result is then unused) beside the
            // exponentials of tile t
            wv.scores(sK[(t + 1) & 1], nxt);
            wv.load_v(sVt[t & 1], vf);
            wv.l += wv.probs(cur, wv.m == -INFINITY ? 0.f : wv.m, pk);
            wv.pv(vf, pk);
            if (act_next) wv.mask_edges(nxt, j0 + BN);
        }
        fwd_store<T, D, KB, HAS_BIAS>(st, sK[t & 1], more_k, sVt[(t + 1) & 1], sB[(t + 1) & 1], more_v);
        __syncthreads();
    };
    for (int t = 0; t < ntiles; t += 2) {
        step(sa, sb, t);
        if (t + 1 < ntiles) step(sb, sa, t + 1);
    }

    const float l = xhalf_sum(wv.l);
    const int qi = wv.qi;
    if (qi >= P.nq) return;
    const bool degenerate = !(l > 0.f) || !P.qm.keep(b, qi);
    const float inv = degenerate ? 0.f : 1.f / l;
    T* orow = P.out.wrow<T>(b, h, qi);
    u32x2_t pk[D / 8];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = x * 32 + 8 * g + 4 * wv.hh;
            u32x2_t& p = pk[4 * x + g];
            p[0] = pack2<T>(wv.o[x][4 * g] * inv, wv.o[x][4 * g + 1] * inv);
            p[1] = pack2<T>(wv.o[x][4 * g + 2] * inv, wv.o[x][4 * g + 3] * inv);
            *reinterpret_cast<u32x2_t*>(orow + d) = p;
        }
    }
    if (P.ey.ok()) epi_store_lane<T, D / 8>(P, b, h, qi, wv.hh, pk);
    if (wv.hh == 0) *P.lse.wrow<float>(b, h, qi) = degenerate ? NAN : (wv.m + log2f(l)) * kLn2;
}

// ---------------------------------------------------------------------------------------
// Direct-to-LDS variant (no value multiplier, no key mask, unit-stride key bias): K, V and the
// raw key bias travel HBM -> LDS with buffer_load ... lds (no registers, no VALU), three LDS
// stages deep so that the loads of tile t+2 are in flight while tile t is computed.  K and V
// stay row-major in LDS with the 16-byte chunks of each row XOR-swizzled, so that the K
// fragment reads (ds_read_b128) and the transposing V^T reads (ds_read_b64_tr_b16) spread
// over the LDS banks.  Rows past the last key lie outside the buffer range and read as zeros
// (their scores are masked).  Every vector-memory operation inside the tile loop is one of
// these loads, so the waits are explicit: before the barrier of step t each wave waits until
// only tile t+1's loads are outstanding.  Each wave converts the raw bias of its tile
// (class filter, log2 domain) into a wave-private LDS row.

constexpr int kFwdStages = 4;  // LDS stages of 64-key tiles, filled and waited for in pairs

// chunk swizzles (16-byte chunk index within a row, as a function of the row)
// K (read as 16-byte fragments, 32 rows per block): for d = 64 the chunk is XORed with a
// permutation of row bits 1-3, which the counters measure as free of LDS bank conflicts (a
// row + row/8 rotation cost about one conflict cycle per LDS read)
template <int D>
__device__ __forceinline__ int swz_k(int r) {
    r &= 31;
    if (D == 64) {
        const int v = (r >> 1) & 7;
        return ((v & 1) << 2) | (v & 2) | ((v >> 2) & 1);
    }
    return r & 15;
}
template <int D>
__device__ __forceinline__ int swz_v(int r) {
    return D == 64 ? 2 * (r & 3) : 4 * (r & 3);
}

template <int D, int KB>
struct DmaTile {
    static constexpr int BN = 32 * KB;
    static constexpr int CPR = D / 8;                  // 16-byte chunks per row
    static constexpr int NL = BN * CPR / kFwdThreads;  // loads per thread and tensor
    static constexpr int ELEMS = BN * D;               // elements per tensor tile
    static_assert(BN * CPR % kFwdThreads == 0, "tile must split evenly over the threads");
};

// QB query blocks of 32 per wave (workgroup = 128 * QB queries): with QB = 2 every K and V
// fragment read from LDS feeds two MFMAs, and each wave carries two independent softmax chains.
template <typename T, int D, int KB, int QB, bool CAUSAL, bool SOFTCLAMP, bool HAS_BIAS>
__global__ __launch_bounds__(kFwdThreads, D == 64 ? 2 : 1) void k_mfma_fwd_dma(PassDev P) {
    using TL = DmaTile<D, KB>;
    constexpr int BN = TL::BN, NL = TL::NL, BM = kFwdBM * QB;
    // without softclamp the key bias enters the scores as the MFMA accumulator's initial value
    // (bias / scale, so that scale*log2e*(s + bias/scale) is the log2-domain logit)
    constexpr bool FOLD = HAS_BIAS && !SOFTCLAMP;
    using W = FwdWave<T, D, KB, CAUSAL, SOFTCLAMP, HAS_BIAS, HAS_BIAS && SOFTCLAMP>;
    using M = Mma<T>;
    typedef typename W::frag frag;
    constexpr int NSTG = kFwdStages;
    __shared__ __attribute__((aligned(16))) T sK[NSTG * TL::ELEMS];
    __shared__ __attribute__((aligned(16))) T sV[NSTG * TL::ELEMS];
    __shared__ __attribute__((aligned(16))) float sBraw[NSTG][BN];  // raw bias bytes
    __shared__ __attribute__((aligned(16))) float sBw[4][BN];             // per-wave converted

    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int nqb = (P.nq + BM - 1) / BM;
    int bh, rank;
    block_order<CAUSAL>(nqb, P.heads, P.k.hdiv, bh, rank);
    const int qb = CAUSAL ? nqb - 1 - rank : rank;
    const int h = bh % P.heads, b = bh / P.heads;
    const int hh = lane >> 5, kcol = lane & 31;
    const int wq0 = qb * BM + w * 32 * QB;  // this wave's first query

    W wv[QB];
#pragma unroll
    for (int u = 0; u < QB; ++u) {
        W& v = wv[u];
        v.hh = hh;
        v.kcol = kcol;
        v.q0 = wq0 + 32 * u;
        v.qi = v.q0 + kcol;
        v.nk = P.nk;
        v.sl2 = P.scale * kLog2e;
        v.cinv = SOFTCLAMP ? P.scale / P.softclamp : 0.f;
        v.cl2 = SOFTCLAMP ? P.softclamp * kLog2e : 0.f;
        v.m = -INFINITY;
        v.l = 0.f;
        const int qi = v.qi;
        // rows past the end read row 0 and are zeroed: no branch around a load (a branch's join
        // waits for the loads issued before it)
        const T* qrow = P.q.row<T>(b, h, qi < P.nq ? qi : 0);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            u32x4_t raw = *reinterpret_cast<const u32x4_t*>(qrow + c * 16 + 8 * hh);
            if (qi >= P.nq) raw = u32x4_t{0u, 0u, 0u, 0u};
            v.qf[c] = __builtin_bit_cast(frag, raw);
        }
#pragma unroll
        for (int x = 0; x < D / 32; ++x) v.o[x] = zero16();
    }
    // the Q loads are the only compiler-visible vector-memory operations: retire them before
    // the first direct load, so that no compiler-inserted wait can stall on the latter
#pragma unroll
    for (int u = 0; u < QB; ++u)
#pragma unroll
        for (int c = 0; c < D / 16; ++c) wv[u].qf[c] = opaque(wv[u].qf[c]);

    // buffers over this (batch, head)'s rows [0, nk) of K and V, and its key bias
    const int ksn = (int)P.k.sn, vsn = (int)P.v.sn;
    const srd_t rk = make_srd(P.k.row<T>(b, h, 0), (uint32_t)(((int64_t)(P.nk - 1) * ksn + D) * 2));
    const srd_t rv = make_srd(P.v.row<T>(b, h, 0), (uint32_t)(((int64_t)(P.nk - 1) * vsn + D) * 2));
    const int bes = P.bias.dtype == PA_F32 ? 4 : 2;  // bias element size
    const float bmul = FOLD ? 1.f / P.scale : kLog2e;
    srd_t rb = {0, 0, 0, 0};
    if (HAS_BIAS) rb = make_srd(P.bias.p + P.bias.idx(b, h, 0) * bes, (uint32_t)(P.nk * bes));
    // per-thread byte offsets (tile-relative) of the chunks this thread loads: chunk
    // p = n*256 + tid of the tile sits at row p / CPR, physical chunk p % CPR
    uint32_t offk[NL], offv[NL];
#pragma unroll
    for (int n = 0; n < NL; ++n) {
        const int p = n * kFwdThreads + tid, r = p / TL::CPR, ph = p % TL::CPR;
        offk[n] = (uint32_t)((r * ksn + (ph ^ swz_k<D>(r)) * 8) * 2);
        offv[n] = (uint32_t)((r * vsn + (ph ^ swz_v<D>(r)) * 8) * 2);
    }
    // bias: each wave loads a quarter of the tile's BN * bes bytes with its first lanes
    const int bq = BN * bes / 4;  // bytes per wave
    const uint32_t offb = (uint32_t)(w * bq + 16 * lane);
    const uint32_t lds_k = lds_addr(sK), lds_v = lds_addr(sV), lds_b = lds_addr(&sBraw[0][0]);
    auto issue = [&](int j0, int stage) __attribute__((always_inline)) {
        const uint32_t tk = (uint32_t)(j0 * ksn * 2), tv = (uint32_t)(j0 * vsn * 2);
        const uint32_t kd = lds_k + (uint32_t)(stage * TL::ELEMS * 2), vd = lds_v + (uint32_t)(stage * TL::ELEMS * 2);
#pragma unroll
        for (int n = 0; n < NL; ++n) {
            dma16(rk, kd + (uint32_t)((n * kFwdThreads + w * 64) * 16), offk[n] + tk);
            dma16(rv, vd + (uint32_t)((n * kFwdThreads + w * 64) * 16), offv[n] + tv);
        }
        // one (partially active) bias load per wave: lanes past the wave's quarter stay idle
        if (HAS_BIAS && 16 * lane < bq)
            dma16(rb, lds_b + (uint32_t)(stage * BN * 4 + w * bq), offb + (uint32_t)(j0 * bes));
    };

    // per-lane LDS element offsets of the MFMA operands (tile-relative)
    int koff[D / 16];  // K rows kcol (+32*kb), chunk 2c + hh
#pragma unroll
    for (int c = 0; c < D / 16; ++c) koff[c] = kcol * D + (((2 * c + hh) ^ swz_k<D>(kcol)) * 8);
    int voff[D / 32];  // V rows 4*hh + j/4 (+16*t2 + 8*u + 32*kb), columns 32x + (lane & 31)
    {
        const int g = lane >> 4, j = lane & 15;
        const int r = 4 * (g >> 1) + (j >> 2);
#pragma unroll
        for (int x = 0; x < D / 32; ++x) {
            const int ch = 4 * x + 2 * (g & 1) + ((j & 3) >> 1);
            voff[x] = r * D + ((ch ^ swz_v<D>(r)) * 8) + 4 * (j & 1);
        }
    }

    const int kend = CAUSAL ? min(P.nk, qb * BM + BM) : P.nk;
    // tiles [tb, te): with the range of keys that can enter a normal row (masked passes), the
    // tiles outside it are neither loaded nor visited
    int tb = 0, te = (kend + BN - 1) / BN;
    if (HAS_BIAS && P.live) {
        const int hd = P.bias.hdiv;
        const int32_t* r = P.live + 2 * ((int64_t)b * (P.heads / hd) + h / hd);
        const int lo = r[0], hi = r[1];
        te = min(te, (hi + BN - 1) / BN);
        tb = min(lo / BN, te);
    }
    const int ntl = te - tb;  // tiles loaded
    const int wave_last = CAUSAL ? (wq0 + 32 * QB - 1) : (1 << 30);

    if (ntl > 0) issue(tb * BN, 0);
    if (ntl > 1) issue((tb + 1) * BN, 1);

    // tiles [tb, tb + nact) hold keys at or below this wave's last query; the remaining tiles
    // of the workgroup only pass through (loads and barriers), in a loop of their own so that
    // the compute loop has a single path
    const int nact = max(0, (CAUSAL ? min(te, wave_last / BN + 1) : te) - tb);
    int st = 0;
    auto next_st = [](int s) __attribute__((always_inline)) { return (s + 1) & 3; };
    // tiles in pairs, one workgroup barrier per pair: at an even tile both tiles of the pair
    // have landed and every wave is done with the previous pair, whose stages receive the
    // next pair (half the barriers of one per tile: -1% on this kernel).  u: the tile's index
    // from tb
    auto enter = [&](int u) __attribute__((always_inline)) {
        if (u & 1) return;
        wait_vmcnt<0>();
        lds_barrier();
        if (u + 2 < ntl) issue((tb + u + 2) * BN, (st + 2) & 3);
        if (u + 3 < ntl) issue((tb + u + 3) * BN, (st + 3) & 3);
    };
    for (int u = 0; u < nact; ++u) {
        const int j0 = (tb + u) * BN;
        enter(u);
        const T* K = sK + st * TL::ELEMS;
        const T* V = sV + st * TL::ELEMS;
        if (HAS_BIAS) {
            // this wave's converted copy of the tile's bias: class filtered; log2 domain
            // (softclamp) or divided by the scale (folded into the scores)
            float x;
            if (bes == 4) x = sBraw[st][lane];
            else x = (float)reinterpret_cast<const T*>(&sBraw[st][0])[lane];
            const float xw = bias_class(x) == 0 ? x * bmul : -INFINITY;
            sBw[w][lane] = xw;
            // a tile whose every key term is -inf (masked keys: padding) adds nothing to any
            // row; a row that has seen only such keys keeps m = -inf and l = 0 either way
            if (!__any(xw != -INFINITY)) {
                st = next_st(st);
                continue;
            }
        }
#if PA_FWD_USPLIT
        if constexpr (QB == 2 && W::PLAIN && PA_FWD_SUMCHECK) {
            // The wave's two query blocks in a pipeline: (A) scores of block 0; (B) scores of
            // block 1 among block 0's probabilities; (C) O += V^T P^T of block 0 among block 1's
            // probabilities; (D) O += V^T P^T of block 1.  In B and C each MFMA is followed by
            // the VALU work of four probabilities (scheduling barriers keep the chunks in
            // order), so the matrix core runs while the wave forms probabilities.
            frag kf[KB][D / 16];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int c = 0; c < D / 16; ++c) kf[kb][c] = ld_frag<T>(K + kb * 32 * D + koff[c]);
            f32x16_t s[QB][KB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                f32x16_t init = zero16();
                if (FOLD) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const float4 bb = *reinterpret_cast<const float4*>(&sBw[w][kb * 32 + 8 * g + 4 * hh]);
                        init[4 * g] = bb.x;
                        init[4 * g + 1] = bb.y;
                        init[4 * g + 2] = bb.z;
                        init[4 * g + 3] = bb.w;
                    }
                }
                s[0][kb] = init;
                s[1][kb] = init;
            }
            // four probabilities of block u (registers 4 (i % 4) .. +3 of key block i / 4) into
            // the packed operands and the four sum chains
            auto chunk = [&](int u, int i, float msub, u32x4_t (&pk)[KB][2], float (&lts)[4])
                             __attribute__((always_inline)) {
                const int kb = i / 4, r0 = 4 * (i % 4);
                const float sl2 = wv[u].sl2;
                const float p0 = fast_exp2(fmaf(s[u][kb][r0], sl2, -msub));
                const float p1 = fast_exp2(fmaf(s[u][kb][r0 + 1], sl2, -msub));
                const float p2 = fast_exp2(fmaf(s[u][kb][r0 + 2], sl2, -msub));
                const float p3 = fast_exp2(fmaf(s[u][kb][r0 + 3], sl2, -msub));
                const uint32_t w0 = pack2<T>(p0, p1), w1 = pack2<T>(p2, p3);
                pk[kb][r0 / 8][(r0 % 8) / 2] = w0;
                pk[kb][r0 / 8][(r0 % 8) / 2 + 1] = w1;
                lts[(2 * i) % 4] = sum_pair<T>(w0, lts[(2 * i) % 4]);
                lts[(2 * i + 1) % 4] = sum_pair<T>(w1, lts[(2 * i + 1) % 4]);
            };
            // the rare path of a block whose probabilities failed the sum check
            auto recheck = [&](int u, float lt, u32x4_t (&pk)[KB][2]) __attribute__((always_inline)) {
                if (__any(!(lt <= kFwdSumCap))) {
                    keep_branch();
                    wv[u].settle(wv[u].logits(s[u], sBw[w]), true);
                    lt = wv[u].probs(s[u], wv[u].m == -INFINITY ? 0.f : wv[u].m, pk);
                }
                wv[u].l += lt;
            };
            // (A)
#pragma unroll
            for (int c = 0; c < D / 16; ++c)
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) s[0][kb] = M::run(kf[kb][c], wv[0].qf[c], s[0][kb]);
            wv[0].mask_edges_nk(s[0], j0);
            // the first tile: O and l are still 0, so the running max is just the tile's (no
            // attempt against m = -inf that the sum check would send back)
            if (u == 0) wv[0].m = wv[0].logits(s[0], sBw[w]);
            __builtin_amdgcn_sched_barrier(0);
            // (B)
            u32x4_t pk0[KB][2];
            float lt0;
            {
                const float msub = wv[0].m;
                float lts[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < KB * (D / 16); ++i) {
                    const int c = i / KB, kb = i % KB;
                    s[1][kb] = M::run(kf[kb][c], wv[1].qf[c], s[1][kb]);
                    chunk(0, i, msub, pk0, lts);
                    __builtin_amdgcn_sched_barrier(0);
                }
                lt0 = (lts[0] + lts[1]) + (lts[2] + lts[3]);
            }
            frag vf[KB][2][D / 32];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
                    for (int x = 0; x < D / 32; ++x) {
                        const T* base = V + (kb * 32 + 16 * t2) * D + voff[x];
                        const u32x2_t lo = lds_read_tr(base);
                        const u32x2_t hi = lds_read_tr(base + 8 * D);
                        const u32x4_t v4 = {lo[0], lo[1], hi[0], hi[1]};
                        vf[kb][t2][x] = __builtin_bit_cast(frag, v4);
                    }
            recheck(0, lt0, pk0);
            wv[1].mask_edges_nk(s[1], j0);
            if (u == 0) wv[1].m = wv[1].logits(s[1], sBw[w]);
            __builtin_amdgcn_sched_barrier(0);
            // (C)
            u32x4_t pk1[KB][2];
            float lt1;
            {
                const float msub = wv[1].m;
                float lts[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < KB * 2 * (D / 32); ++i) {
                    const int kb = i / (2 * (D / 32)), t2 = (i / (D / 32)) % 2, x = i % (D / 32);
                    wv[0].o[x] = M::run(vf[kb][t2][x], __builtin_bit_cast(frag, pk0[kb][t2]), wv[0].o[x]);
                    chunk(1, i, msub, pk1, lts);
                    __builtin_amdgcn_sched_barrier(0);
                }
                lt1 = (lts[0] + lts[1]) + (lts[2] + lts[3]);
            }
            recheck(1, lt1, pk1);
            // (D)
            wv[1].pv(vf, pk1);
            st = next_st(st);
            continue;
        }
#endif
        f32x16_t s[QB][KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            f32x16_t init = zero16();
            if (FOLD) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 bb = *reinterpret_cast<const float4*>(&sBw[w][kb * 32 + 8 * g + 4 * hh]);
                    init[4 * g] = bb.x;
                    init[4 * g + 1] = bb.y;
                    init[4 * g + 2] = bb.z;
                    init[4 * g + 3] = bb.w;
                }
            }
#pragma unroll
            for (int u = 0; u < QB; ++u) s[u][kb] = init;
#pragma unroll
            for (int c = 0; c < D / 16; ++c) {
                const frag a = ld_frag<T>(K + kb * 32 * D + koff[c]);
#pragma unroll
                for (int u = 0; u < QB; ++u) s[u][kb] = M::run(a, wv[u].qf[c], s[u][kb]);
            }
        }
        constexpr bool SUMCHK = PA_FWD_SUMCHECK && W::PLAIN;
#pragma unroll
        for (int u = 0; u < QB; ++u) {
            wv[u].mask_edges_nk(s[u], j0);
            if (!SUMCHK) wv[u].settle(wv[u].logits(s[u], sBw[w]));
        }
        frag vf[KB][2][D / 32];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
                for (int x = 0; x < D / 32; ++x) {
                    const T* base = V + (kb * 32 + 16 * t2) * D + voff[x];
                    const u32x2_t lo = lds_read_tr(base);
                    const u32x2_t hi = lds_read_tr(base + 8 * D);
                    const u32x4_t v4 = {lo[0], lo[1], hi[0], hi[1]};
                    vf[kb][t2][x] = __builtin_bit_cast(frag, v4);
                }
#pragma unroll
        for (int u = 0; u < QB; ++u) {
            u32x4_t pk[KB][2];
            if (SUMCHK) wv[u].l += wv[u].probs_checked(s[u], sBw[w], pk);
            else wv[u].l += wv[u].probs(s[u], wv[u].m == -INFINITY ? 0.f : wv[u].m, pk);
            wv[u].pv(vf, pk);
        }
        st = next_st(st);
    }
    for (int u = nact; u < ntl; ++u) {
        enter(u);
        st = next_st(st);
    }

#pragma unroll
    for (int u = 0; u < QB; ++u) {
        const W& v = wv[u];
        const float l = xhalf_sum(v.l);
        const int qi = v.qi;
        if (qi < P.nq) {
            const bool degenerate = !(l > 0.f) || !P.qm.keep(b, qi);
            const float inv = degenerate ? 0.f : 1.f / l;
            T* orow = P.out.wrow<T>(b, h, qi);
            u32x2_t pk[D / 8];
#pragma unroll
            for (int x = 0; x < D / 32; ++x) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = x * 32 + 8 * g + 4 * hh;
                    u32x2_t& p = pk[4 * x + g];
                    p[0] = pack2<T>(v.o[x][4 * g] * inv, v.o[x][4 * g + 1] * inv);
                    p[1] = pack2<T>(v.o[x][4 * g + 2] * inv, v.o[x][4 * g + 3] * inv);
                    *reinterpret_cast<u32x2_t*>(orow + d) = p;
                }
            }
            if (P.ey.ok()) epi_store_lane<T, D / 8>(P, b, h, qi, hh, pk);
            if (hh == 0) *P.lse.wrow<float>(b, h, qi) = degenerate ? NAN : (v.m + log2f(l)) * kLn2;
        }
    }
}

// The direct-to-LDS kernel addresses K / V with 32-bit byte offsets up to the end of the last
// tile and reads the key bias as one contiguous row; other cases take the register-staged
// kernel.
// ---------------------------------------------------------------------------------------
// Short passes (nq, nk <= 64, head dim 64, not causal, no value multiplier or key mask: the
// PolyViT shape): one (batch, head) unit per wave, kShortUnits units per workgroup.  Such a
// pass is one key tile per unit and a few microseconds of dependent latency (loads, 16 MFMAs,
// softmax, 16 MFMAs, store); what sets the time is how many units run at once.  The general
// kernels' 256-query workgroups (three LDS stages, up to 256 VGPRs per lane) fit two or three
// per CU, so 1024 units took two rounds; here each wave stages only its own K and V^T tile
// (18 KB) and works on it alone -- no workgroup barrier, a wave may finish independently.

constexpr int kShortUnits = 4;  // waves per workgroup
#ifndef PA_FWD_SHORT_SPLIT
#define PA_FWD_SHORT_SPLIT 2
#endif
// waves per unit: each takes 2 / kShortSplit of the unit's two 32-query blocks and stages the
// unit's K / V^T tile itself.  With 2 (two waves per SIMD at PolyViT's 1024 units, the second
// K / V read of a unit served by L2) the pass took 16.5 against 17.5 us event-timed, PolyViT
// 1.130 against 1.144 ms.
constexpr int kShortSplit = PA_FWD_SHORT_SPLIT;
static_assert(kShortSplit == 1 || kShortSplit == 2, "short-pass split");

template <typename T>
__device__ __forceinline__ void unpack8(const u32x4_t& r, float (&out)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) unpack2<T>(r[i], out[2 * i], out[2 * i + 1]);
}
// y = (x * rs) * w in fp32, each product rounded to fp32 before the caller's conversion to T,
// as pa_rmsnorm_fwd computes it.  The empty asm operand makes the fp32 product a value of its
// own: otherwise the second product and the conversion to f16 become one mixed-precision FMA
// (v_fma_mixlo_f16, a single rounding), which differs from the norm kernel in rare cases.
__device__ __forceinline__ void norm_scale(const float (&x)[8], float rs, const float (&w)[8],
                                           float (&y)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        y[e] = (x[e] * rs) * w[e];
        asm volatile("" : "+v"(y[e]));
    }
}
template <typename T>
__device__ __forceinline__ u32x4_t pack8(const float (&v)[8]) {
    u32x4_t r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack2<T>(v[2 * i], v[2 * i + 1]);
    return r;
}

// RMSNorm of one 32-row block held as Q^T fragments, bit-identical to pa_rmsnorm_fwd: lane
// (q, hh) holds row q's feature chunks 2c + hh (8 features each), the partner half lane ^ 32
// the others; the chunk sums combine as that kernel's butterfly over its 8 lanes does: chunk
// pairs first, then (t0 + t1) + (t2 + t3)
template <typename T>
__device__ __forceinline__ void norm_q_frags(u32x4_t (&q)[4], const u32x4_t (&wf)[4], float eps) {
    constexpr int D = 64;
    float x[D / 16][8], t[D / 16];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        unpack8<T>(q[c], x[c]);
        float sc = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sc += x[c][e] * x[c][e];
        t[c] = sc + __shfl_xor(sc, 32);
    }
    const float rs = rsqrtf(((t[0] + t[1]) + (t[2] + t[3])) * (1.f / D) + eps);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        float wq[8], y[8];
        unpack8<T>(wf[c], wq);
        norm_scale(x[c], rs, wq, y);
        q[c] = pack8<T>(y);
    }
}

// The lane's norm weight fragments of a Q^T operand row (as norm_q_frags takes them), loaded
// beside the row data; without a norm (w null) a valid row is read instead and not used, so
// that no load sits behind a branch (a branch's join waits for the loads issued before it)
template <typename T>
__device__ __forceinline__ void load_wq_frags(u32x4_t (&wf)[4], const void* w, const T* fallback,
                                              int hh) {
    const T* p = w ? static_cast<const T*>(w) : fallback;
#pragma unroll
    for (int c = 0; c < 4; ++c) wf[c] = *reinterpret_cast<const u32x4_t*>(p + c * 16 + 8 * hh);
}

// RMSNorm of a row chunk (8 features) whose row's 8 chunks sit in 8 consecutive lanes, summed
// by pa_rmsnorm_fwd's butterfly; w = this lane's 8 weights
template <typename T>
__device__ __forceinline__ void norm_row_chunk(u32x4_t& k, const float (&w)[8], float eps) {
    constexpr int D = 64;
    float x[8];
    unpack8<T>(k, x);
    float sc = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sc += x[e] * x[e];
#pragma unroll
    for (int off = 1; off < D / 8; off <<= 1) sc += __shfl_xor(sc, off);
    const float rs = rsqrtf(sc * (1.f / D) + eps);
    float y[8];
    norm_scale(x, rs, w, y);
    k = pack8<T>(y);
}

// One 32-query block (queries q0 .. q0 + 31 as Q^T fragments q) of a short pass against the
// unit's staged 64-key tile (K row-major, V^T, key term Bk when the pass has one); leaves O,
// m and l in wv.
template <typename T, class W>
__device__ __forceinline__ void short_block(W& wv, const PassDev& P, int q0, int lane,
                                            const u32x4_t (&q)[4], const T* Ks, const T* Vt,
                                            const float* Bk, bool softclamp) {
    constexpr int D = 64, KB = 2;
    typedef typename W::frag frag;
    wv.hh = lane >> 5;
    wv.kcol = lane & 31;
    wv.q0 = q0;
    wv.qi = q0 + wv.kcol;
    wv.nk = P.nk;
    wv.sl2 = P.scale * kLog2e;
    wv.cinv = softclamp ? P.scale / P.softclamp : 0.f;
    wv.cl2 = softclamp ? P.softclamp * kLog2e : 0.f;
    wv.m = -INFINITY;
    wv.l = 0.f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) wv.qf[c] = __builtin_bit_cast(frag, q[c]);
#pragma unroll
    for (int x = 0; x < D / 32; ++x) wv.o[x] = zero16();
    f32x16_t s[KB];
    wv.scores(Ks, s);
    wv.mask_edges(s, 0);
    wv.settle(wv.logits(s, Bk));
    u32x4_t pk[KB][2];
    frag vf[KB][2][D / 32];
    wv.load_v(Vt, vf);
    wv.l += wv.probs(s, wv.m == -INFINITY ? 0.f : wv.m, pk);
    wv.pv(vf, pk);
}

// The finished block's rows normalised and rounded to T (lane (q, hh): features
// x*32 + 8g + 4hh .. +3 in ow[4x + g]) and its lse (NaN for a degenerate row); with `store`
// written to out, lse and the epilogue's y for the rows below nq.  Returns the lse.
template <typename T, class W>
__device__ __forceinline__ float short_finish(const W& wv, const PassDev& P, int b, int h,
                                              bool store, u32x2_t (&ow)[8]) {
    constexpr int D = 64;
    const float l = xhalf_sum(wv.l);
    const int qi = wv.qi;
    const bool degenerate = !(l > 0.f) || (qi < P.nq && !P.qm.keep(b, qi));
    const float inv = degenerate ? 0.f : 1.f / l;
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            ow[4 * x + g][0] = pack2<T>(wv.o[x][4 * g] * inv, wv.o[x][4 * g + 1] * inv);
            ow[4 * x + g][1] = pack2<T>(wv.o[x][4 * g + 2] * inv, wv.o[x][4 * g + 3] * inv);
        }
    const float lse = degenerate ? NAN : (wv.m + log2f(l)) * kLn2;
    if (store && qi < P.nq) {
        T* orow = P.out.wrow<T>(b, h, qi);
#pragma unroll
        for (int x = 0; x < D / 32; ++x)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<u32x2_t*>(orow + x * 32 + 8 * g + 4 * wv.hh) = ow[4 * x + g];
        if (P.ey.ok()) epi_store_lane<T, D / 8>(P, b, h, qi, wv.hh, ow);
        if (wv.hh == 0) *P.lse.wrow<float>(b, h, qi) = lse;
    }
    return lse;
}

template <typename T, bool SOFTCLAMP, bool HAS_BIAS>
__global__ __launch_bounds__(kFwdThreads, 2) void k_mfma_fwd_short(PassDev P) {
    constexpr int D = 64, KB = 2;
    using TL = FwdTile<D, KB>;
    constexpr int BN = TL::BN;
    using W = FwdWave<T, D, KB, false, SOFTCLAMP, HAS_BIAS>;
    __shared__ __attribute__((aligned(16))) T sK[kShortUnits][BN * TL::KS];
    __shared__ __attribute__((aligned(16))) T sVt[kShortUnits][D * TL::VS];
    __shared__ __attribute__((aligned(16))) float sB[kShortUnits][BN];
    const int lane = threadIdx.x & 63, w = wave_id();
    constexpr int QPW = 2 / kShortSplit;  // 32-query blocks per wave
    const int task = blockIdx.x * kShortUnits + w;
    const int unit = task / kShortSplit, qb0 = (task % kShortSplit) * QPW;
    // whole waves; nothing below synchronises waves
    if (unit >= P.batch * P.heads || 32 * qb0 >= P.nq) return;
    const int h = unit % P.heads, b = unit / P.heads;
    T* Ks = sK[w];
    T* Vt = sVt[w];
    float* Bk = sB[w];
    const u32x4_t zero = {0u, 0u, 0u, 0u};
    const int hh = lane >> 5, kcol = lane & 31;

    // Every global load of the unit is issued before the first wait (one memory round trip):
    // the Q^T fragments of the wave's 32-query blocks, the K and V rows of both 4-key x 8-dim
    // block rounds, the key bias.  Rows past nq / nk are read from the last row (no branch
    // around a load) and replaced by zeros afterwards.
    static_assert(TL::BLOCKS % 64 == 0 && BN == 64, "short-pass tile");
    constexpr int NR = TL::BLOCKS / 64;  // block rounds per lane
    u32x4_t qraw[QPW][D / 16];
#pragma unroll
    for (int u = 0; u < QPW; ++u) {
        const T* qrow = P.q.row<T>(b, h, min(32 * (qb0 + u) + kcol, P.nq - 1));
#pragma unroll
        for (int c = 0; c < D / 16; ++c) qraw[u][c] = *reinterpret_cast<const u32x4_t*>(qrow + c * 16 + 8 * hh);
    }
    u32x4_t kw[NR][4], vw[NR][4];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int blk = lane + 64 * i, rg = blk / (D / 8), cc = blk % (D / 8);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = min(rg * 4 + r, P.nk - 1);
            kw[i][r] = *reinterpret_cast<const u32x4_t*>(P.k.row<T>(b, h, j) + cc * 8);
            vw[i][r] = *reinterpret_cast<const u32x4_t*>(P.v.row<T>(b, h, j) + cc * 8);
        }
    }
    float braw = 0.f;  // lane j's key bias (BN = 64 keys, one per lane)
    if (HAS_BIAS) braw = P.bias.scalar(b, h, min(lane, P.nk - 1));
    // the norm weights, loaded with the rows (see load_wq_frags)
    u32x4_t wqf[4], wkr;
    load_wq_frags<T>(wqf, (P.nflags & PA_NORM_Q) ? P.qnw : nullptr, P.q.row<T>(b, h, 0), hh);
    wkr = *reinterpret_cast<const u32x4_t*>(
        ((P.nflags & PA_NORM_K) ? static_cast<const T*>(P.knw) : P.k.row<T>(b, h, 0)) + (lane % (D / 8)) * 8);
#pragma unroll
    for (int u = 0; u < QPW; ++u)
        if (32 * (qb0 + u) + kcol >= P.nq)
#pragma unroll
            for (int c = 0; c < D / 16; ++c) qraw[u][c] = zero;
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if ((lane + 64 * i) / (D / 8) * 4 + r >= P.nk) kw[i][r] = vw[i][r] = zero;

    // optional RMSNorms of the queries and keys
    if (P.nflags & PA_NORM_Q)
#pragma unroll
        for (int u = 0; u < QPW; ++u) norm_q_frags<T>(qraw[u], wqf, P.qeps);
    if (P.nflags & PA_NORM_K) {
        float wk[8];
        unpack8<T>(wkr, wk);
#pragma unroll
        for (int i = 0; i < NR; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) norm_row_chunk<T>(kw[i][r], wk, P.keps);
    }

    // this unit's keys into LDS: K row-major, V transposed (4-key x 8-dim blocks), the key term
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int blk = lane + 64 * i, rg = blk / (D / 8), cc = blk % (D / 8);
#pragma unroll
        for (int r = 0; r < 4; ++r) *reinterpret_cast<u32x4_t*>(Ks + (rg * 4 + r) * TL::KS + cc * 8) = kw[i][r];
        store_block_transposed(vw[i], reinterpret_cast<uint16_t*>(Vt + (cc * 8) * TL::VS + rg * 4), TL::VS);
    }
    if (HAS_BIAS) Bk[lane] = lane < P.nk && bias_class(braw) == 0 ? braw * kLog2e : -INFINITY;
    // one wave's LDS operations complete in order: wait for the writes, fence the compiler
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");

#pragma unroll
    for (int u = 0; u < QPW; ++u) {  // this wave's 32-query blocks
        if (32 * (qb0 + u) >= P.nq) break;  // wave-uniform
        W wv;
        short_block<T>(wv, P, 32 * (qb0 + u), lane, qraw[u], Ks, Vt, Bk, SOFTCLAMP);
        u32x2_t ow[D / 8];
        short_finish<T>(wv, P, b, h, true, ow);
    }
}

// ---------------------------------------------------------------------------------------
// Both passes of an order-2 chain in one launch, where each is a short pass of the same heads
// and the second pass's keys, values and key bias are the first pass's queries, output and
// lse (the chain's q2, msg and lse23; poly_attention.py:48-116):
//   pass 1: msg = attn(q2, q3, v3), lse23;   pass 2: out = attn(q1, q2, msg; key bias lse23).
// Two waves per (batch, head) unit, one per 32-row block p: each loads its rows of q2 and q1
// and its half of pass 1's K / V rows in one memory round trip, normalises q2 once for both
// passes (its pass-1 query norm is the pass-2 key norm), stages its half of pass 1's K / V^T
// tile and of pass 2's K tile, runs pass 1 for its q2 block, hands the rounded msg rows and
// their lse (as the key term) to pass 2's V^T tile in LDS -- also storing them as pass 1's
// outputs -- and runs pass 2 for its q1 block.  A unit's two waves meet at two workgroup
// barriers, which every wave reaches: a padding unit recomputes the last unit and stores
// nothing.  Per unit it reads q1, q2, q3, v3 once (32 KB at the PolyViT shape) and writes
// msg, lse23 and out, where the two launches read 48 KB; the results are the two passes'
// bits.

constexpr int kO2Units = kShortUnits / 2;  // units per workgroup

template <typename T, bool SOFTCLAMP>
__global__ __launch_bounds__(kFwdThreads, 2) void k_mfma_order2_short(PassDev P1, PassDev P2) {
    constexpr int D = 64, KB = 2;
    using TL = FwdTile<D, KB>;
    constexpr int BN = TL::BN;
    static_assert(BN == 64 && kShortUnits == 4, "order-2 short tile");
    using W1 = FwdWave<T, D, KB, false, SOFTCLAMP, false>;
    using W2 = FwdWave<T, D, KB, false, SOFTCLAMP, true>;
    __shared__ __attribute__((aligned(16))) T sK1[kO2Units][BN * TL::KS];
    __shared__ __attribute__((aligned(16))) T sVt1[kO2Units][D * TL::VS];
    __shared__ __attribute__((aligned(16))) T sK2[kO2Units][BN * TL::KS];
    __shared__ __attribute__((aligned(16))) T sVt2[kO2Units][D * TL::VS];
    __shared__ __attribute__((aligned(16))) float sB2[kO2Units][BN];
    const int lane = threadIdx.x & 63, w = wave_id();
    const int units = P1.batch * P1.heads;
    const int slot = w >> 1, p = w & 1;  // unit slot in the workgroup, 32-row block
    const int task = blockIdx.x * kO2Units + slot;
    const bool live = task < units;
    const int unit = live ? task : units - 1;
    const int h = unit % P1.heads, b = unit / P1.heads;
    const int hh = lane >> 5, kcol = lane & 31, row = 32 * p + kcol;
    const u32x4_t zero = {0u, 0u, 0u, 0u};
    const int n2 = P1.nq;  // q2 rows: pass 1's queries, pass 2's keys

    // loads: q2 and q1 rows of block p as Q^T fragments, pass 1's K / V rows 32p .. 32p + 31
    // as 4-key x 8-dim blocks (one per lane); rows past the end read from the last row, zeroed
    const int rg = lane / (D / 8) + 8 * p, cc = lane % (D / 8);
    u32x4_t q2r[D / 16], q1r[D / 16], kw[4], vw[4];
    {
        const T* r2 = P1.q.row<T>(b, h, min(row, n2 - 1));
        const T* r1 = P2.q.row<T>(b, h, min(row, P2.nq - 1));
#pragma unroll
        for (int c = 0; c < D / 16; ++c) q2r[c] = *reinterpret_cast<const u32x4_t*>(r2 + c * 16 + 8 * hh);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) q1r[c] = *reinterpret_cast<const u32x4_t*>(r1 + c * 16 + 8 * hh);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = min(rg * 4 + r, P1.nk - 1);
            kw[r] = *reinterpret_cast<const u32x4_t*>(P1.k.row<T>(b, h, j) + cc * 8);
            vw[r] = *reinterpret_cast<const u32x4_t*>(P1.v.row<T>(b, h, j) + cc * 8);
        }
    }
    // the norm weights, loaded with the rows (see load_wq_frags)
    u32x4_t w2f[4], w1f[4], wkr;
    load_wq_frags<T>(w2f, (P1.nflags & PA_NORM_Q) ? P1.qnw : nullptr, P1.q.row<T>(b, h, 0), hh);
    load_wq_frags<T>(w1f, (P2.nflags & PA_NORM_Q) ? P2.qnw : nullptr, P2.q.row<T>(b, h, 0), hh);
    wkr = *reinterpret_cast<const u32x4_t*>(
        ((P1.nflags & PA_NORM_K) ? static_cast<const T*>(P1.knw) : P1.k.row<T>(b, h, 0)) + cc * 8);
    if (row >= n2)
#pragma unroll
        for (int c = 0; c < D / 16; ++c) q2r[c] = zero;
    if (row >= P2.nq)
#pragma unroll
        for (int c = 0; c < D / 16; ++c) q1r[c] = zero;
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (rg * 4 + r >= P1.nk) kw[r] = vw[r] = zero;

    if (P1.nflags & PA_NORM_Q) norm_q_frags<T>(q2r, w2f, P1.qeps);
    if (P2.nflags & PA_NORM_Q) norm_q_frags<T>(q1r, w1f, P2.qeps);
    if (P1.nflags & PA_NORM_K) {
        float wk[8];
        unpack8<T>(wkr, wk);
#pragma unroll
        for (int r = 0; r < 4; ++r) norm_row_chunk<T>(kw[r], wk, P1.keps);
    }

    // stage: pass 1's K rows / V^T columns of this block, pass 2's K rows (normalised q2)
#pragma unroll
    for (int r = 0; r < 4; ++r) *reinterpret_cast<u32x4_t*>(sK1[slot] + (rg * 4 + r) * TL::KS + cc * 8) = kw[r];
    store_block_transposed(vw, reinterpret_cast<uint16_t*>(sVt1[slot] + (cc * 8) * TL::VS + rg * 4), TL::VS);
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
        *reinterpret_cast<u32x4_t*>(sK2[slot] + row * TL::KS + c * 16 + 8 * hh) = q2r[c];
    __syncthreads();

    // pass 1 for q2 block p; its rounded msg rows and lse become pass 2's values and key term
    u32x2_t ow[D / 8];
    float lse = 0.f;
    const bool run1 = 32 * p < n2;  // wave-uniform
    if (run1) {
        W1 wv;
        short_block<T>(wv, P1, 32 * p, lane, q2r, sK1[slot], sVt1[slot], nullptr, SOFTCLAMP);
        lse = short_finish<T>(wv, P1, b, h, live && !(P1.flags & PA_FLAG_DISCARD_OUT), ow);
    }
    {
        const bool keep = run1 && row < n2;
        uint16_t* vt = reinterpret_cast<uint16_t*>(sVt2[slot]);
#pragma unroll
        for (int x = 0; x < D / 32; ++x)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int e2 = 0; e2 < 2; ++e2) {
                    const uint32_t wd = keep ? ow[4 * x + g][e2] : 0u;
                    const int d = x * 32 + 8 * g + 4 * hh + 2 * e2;
                    vt[d * TL::VS + row] = (uint16_t)(wd & 0xffffu);
                    vt[(d + 1) * TL::VS + row] = (uint16_t)(wd >> 16);
                }
        if (hh == 0) sB2[slot][row] = keep && bias_class(lse) == 0 ? lse * kLog2e : -INFINITY;
    }
    __syncthreads();

    // pass 2 for q1 block p
    if (32 * p < P2.nq) {
        W2 wv;
        short_block<T>(wv, P2, 32 * p, lane, q1r, sK2[slot], sVt2[slot], sB2[slot], SOFTCLAMP);
        u32x2_t ow2[D / 8];
        short_finish<T>(wv, P2, b, h, live, ow2);
    }
}

#ifndef PA_FWD_SHORT
#define PA_FWD_SHORT 1  // the short-pass kernel where it applies
#endif

static bool dma_ok(const PassDev& P, int bn) {
    const int64_t rows = (int64_t)P.nk + 2 * bn;
    const int64_t span = std::max(P.k.sn, P.v.sn) * rows * 2;
    if (!(span < ((int64_t)1 << 31))) return false;
    if (P.km.p) return false;
    if (P.bias.ok() && P.bias.sn != 1) return false;
    if (P.bias.ok()) {
        const int64_t es = P.bias.dtype == PA_F32 ? 4 : 2;
        if ((uintptr_t)P.bias.p % 16 != 0 || (P.bias.sh * es) % 16 != 0 || (P.bias.sb * es) % 16 != 0) return false;
        if ((P.nk * es) % 16 != 0) return false;  // whole 16-byte chunks in range
    }
    return true;
}


// ---------------------------------------------------------------------------------------

// 32-key blocks per key tile (64-key tiles)
template <int D, bool SOFTCLAMP>
constexpr int kFwdKB = (D == 64 && !SOFTCLAMP) ? PA_FWD_KB64 : (D == 256 ? 1 : 2);

bool mfma_fwd_supported(const PassDev& P, int dtype) {
    if (dtype == PA_F32) return mfma_fwd_f32_supported(P);
    if (dtype != PA_BF16 && dtype != PA_F16) return false;
    if (P.dim != 64 && P.dim != 128 && P.dim != 256) return false;
    if (!(P.scale > 0.f)) return false;  // the raw-score running max assumes a positive scale
    if (!aligned_rows_host(P.q, 8) || !aligned_rows_host(P.k, 8) || !aligned_rows_host(P.v, 8)) return false;
    if (P.vmul.ok() && !aligned_rows_host(P.vmul, 8)) return false;
    if (!aligned_rows_host(P.out, 4)) return false;
    // the epilogue's root / gate / y rows travel in 8-byte words
    for (const DView* e : {&P.er, &P.eg, &P.ey})
        if (e->ok() && !aligned_rows_host(*e, 4)) return false;
    return true;
}

bool mfma_fwd_short_applies(const PassDev& P, int dtype) {
    return PA_FWD_SHORT && (dtype == PA_BF16 || dtype == PA_F16) && P.dim == 64 && !P.causal &&
           !P.vmul.ok() && P.nq <= 64 && P.nk <= 64 && !P.km.p;
}

template <typename T, int D, bool C, bool S, bool V, bool B>
static void launch_t(const PassDev& P, hipStream_t s) {
    if constexpr (D == 64 && !C && !V) {
        if (mfma_fwd_short_applies(P, sizeof(T) == 2 ? PA_BF16 : PA_F32)) {
            const int units = P.batch * P.heads;
            ProfScope ps("mfma_fwd_short", s);
            hipLaunchKernelGGL((k_mfma_fwd_short<T, S, B>),
                               dim3((units * kShortSplit + kShortUnits - 1) / kShortUnits),
                               dim3(kFwdThreads), 0, s, P);
            return;
        }
    }
    constexpr int KB = kFwdKB<D, S>;
    const int nqb = (P.nq + kFwdBM - 1) / kFwdBM;
    dim3 grid(nqb * P.heads * P.batch);
    ProfScope ps("mfma_fwd", s);
    // head dim 256: the register-staged kernel only (four direct-to-LDS stages of its tiles
    // would need 256 KB of LDS)
    if constexpr (D != 256) {
        if (!V && dma_ok(P, 32 * KB)) {
            constexpr int QB = (D == 64) ? PA_FWD_QB64 : 1;
            const int nqb2 = (P.nq + kFwdBM * QB - 1) / (kFwdBM * QB);
            hipLaunchKernelGGL((k_mfma_fwd_dma<T, D, KB, QB, C, S, B>), dim3(nqb2 * P.heads * P.batch),
                               dim3(kFwdThreads), 0, s, P);
            return;
        }
    }
    hipLaunchKernelGGL((k_mfma_fwd<T, D, KB, C, S, V, B>), grid, dim3(kFwdThreads), 0, s, P);
}

template <typename T, int D, bool C, bool S>
static void launch_vb(const PassDev& P, hipStream_t s) {
    const bool v = P.vmul.ok(), b = P.bias.ok() || P.km.p;
    if (v) b ? launch_t<T, D, C, S, true, true>(P, s) : launch_t<T, D, C, S, true, false>(P, s);
    else b ? launch_t<T, D, C, S, false, true>(P, s) : launch_t<T, D, C, S, false, false>(P, s);
}

template <typename T, int D>
static void launch_d(const PassDev& P, hipStream_t s) {
    const bool c = P.causal != 0, sc = P.softclamp > 0.f;
    if (c) sc ? launch_vb<T, D, true, true>(P, s) : launch_vb<T, D, true, false>(P, s);
    else sc ? launch_vb<T, D, false, true>(P, s) : launch_vb<T, D, false, false>(P, s);
}

void launch_mfma_fwd(const PassDev& P, int dtype, hipStream_t s) {
    if (dtype == PA_F32) {
        launch_mfma_fwd_f32(P, s);
        return;
    }
    if (dtype == PA_BF16) {
        if (P.dim == 64) launch_d<bf16, 64>(P, s);
        else if (P.dim == 128) launch_d<bf16, 128>(P, s);
        else launch_d<bf16, 256>(P, s);
    } else {
        if (P.dim == 64) launch_d<f16, 64>(P, s);
        else if (P.dim == 128) launch_d<f16, 128>(P, s);
        else launch_d<f16, 256>(P, s);
    }
}

bool mfma_order2_short_applies(const PassDev& P1, const PassDev& P2, int dtype) {
    if (!(dtype == PA_BF16 || dtype == PA_F16)) return false;
    if (!mfma_fwd_supported(P1, dtype) || !mfma_fwd_supported(P2, dtype)) return false;
    if (!mfma_fwd_short_applies(P1, dtype) || !mfma_fwd_short_applies(P2, dtype)) return false;
    if (P1.batch != P2.batch || P1.heads != P2.heads || P2.nk != P1.nq) return false;
    if ((P1.softclamp > 0.f) != (P2.softclamp > 0.f)) return false;
    // pass 1 has no key term and no epilogue; no query masks
    if (P1.bias.ok() || P1.ey.ok() || P1.qm.p || P2.qm.p) return false;
    // q2 is normalised once: pass 2's key norm must be pass 1's query norm
    const bool nq1 = (P1.nflags & PA_NORM_Q) != 0, nk2 = (P2.nflags & PA_NORM_K) != 0;
    if (nq1 != nk2) return false;
    if (nq1 && (P1.qnw != P2.knw || P1.qeps != P2.keps)) return false;
    return true;
}

template <typename T>
static void launch_o2(const PassDev& P1, const PassDev& P2, hipStream_t s) {
    const int units = P1.batch * P1.heads;
    const dim3 grid((units + kO2Units - 1) / kO2Units);
    ProfScope ps("mfma_order2_short", s);
    if (P1.softclamp > 0.f) hipLaunchKernelGGL((k_mfma_order2_short<T, true>), grid, dim3(kFwdThreads), 0, s, P1, P2);
    else hipLaunchKernelGGL((k_mfma_order2_short<T, false>), grid, dim3(kFwdThreads), 0, s, P1, P2);
}

void launch_order2_short(const PassDev& P1, const PassDev& P2, int dtype, hipStream_t s) {
    if (dtype == PA_BF16) launch_o2<bf16>(P1, P2, s);
    else launch_o2<f16>(P1, P2, s);
}

}  // namespace pa
