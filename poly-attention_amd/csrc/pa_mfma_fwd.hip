// pa_mfma_fwd.hip -- MFMA forward attention pass for bf16 / f16, head dim 64 or 128 (gfx950).
//
// Workgroup = 4 waves = 128 query rows of one (batch, pass head); each wave owns 32 queries.
// Per key tile (64 keys) a wave computes the transposed scores S^T = K . Q^T with
// v_mfma_f32_32x32x16_{bf16,f16}: the 32x32 accumulator layout gives lane l the column
// q = l % 32 and 16 key rows, so the online-softmax state (running max m, sum l and the
// rescale of the output) is a per-lane scalar.  The probabilities, rounded to the input
// type, stay in registers as the B operand of O^T += V^T . P^T (keys permuted consistently
// between the two operands, see pa_mfma.h), V being staged transposed in LDS.  K / V tiles
// are double buffered: the global loads of tile t+1 are in flight while tile t is computed.
// Exponentials run in the log2 domain (bare v_exp_f32) with scale*log2(e) folded into one
// FMA; without a key bias the running max is taken on the raw scores.  The output rescale
// is skipped when no lane's running max moved.  Workgroups are mapped XCD-aware (pa_mfma.h)
// and causal query blocks run heaviest first.
//
// Rows whose every key is masked are left with lse = NaN for k_simt_fixup, which applies the
// reference's finite-fill semantics to them.
#include "pa_common.h"
#include "pa_launch.h"
#include "pa_mfma.h"

namespace pa {

#ifndef PA_FWD_KB64
#define PA_FWD_KB64 2
#endif

constexpr int kFwdBM = 128;  // query rows per workgroup
constexpr int kFwdThreads = 256;

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

// Registers holding one tile's global loads between issue and LDS store.
template <int D, int KB>
struct FwdStage {
    u32x4_t w[FwdTile<D, KB>::NB][4];
    float bias;
};

template <typename T, int D, int KB, bool HAS_VMUL, bool HAS_BIAS>
__device__ __forceinline__ void fwd_load_tile(const KeySide<T>& ks, int j0, FwdStage<D, KB>& st) {
    using TL = FwdTile<D, KB>;
    const int tid = threadIdx.x;
    const u32x4_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int c = 0; c < TL::NB; ++c) {
        const int task = tid + c * kFwdThreads;
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
    if (HAS_BIAS && tid < TL::BN) {
        const int j = j0 + tid;
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
__device__ __forceinline__ void fwd_store_tile(const FwdStage<D, KB>& st, T* sK, T* sVt, float* sB) {
    using TL = FwdTile<D, KB>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int c = 0; c < TL::NB; ++c) {
        const int task = tid + c * kFwdThreads;
        if (task < 2 * TL::BLOCKS) {
            const int tensor = task / TL::BLOCKS, blk = task % TL::BLOCKS;
            const int rg = blk / (D / 8), cc = blk % (D / 8);
            if (tensor == 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    *reinterpret_cast<u32x4_t*>(sK + (rg * 4 + r) * TL::KS + cc * 8) = st.w[c][r];
            } else {
                store_block_transposed(st.w[c], reinterpret_cast<uint16_t*>(sVt + (cc * 8) * TL::VS + rg * 4),
                                       TL::VS);
            }
        }
    }
    if (HAS_BIAS && tid < TL::BN) sB[tid] = st.bias;
}

template <typename T, int D, int KB, bool CAUSAL, bool SOFTCLAMP, bool HAS_VMUL, bool HAS_BIAS>
__global__ __launch_bounds__(kFwdThreads, D == 64 ? 2 : 1) void k_mfma_fwd(PassDev P) {
    using TL = FwdTile<D, KB>;
    constexpr int BN = TL::BN;
    using M = Mma<T>;
    typedef typename M::frag frag;
    constexpr bool PLAIN = !HAS_BIAS && !SOFTCLAMP;  // max taken on raw scores
    __shared__ __attribute__((aligned(16))) T sK[2][BN * TL::KS];
    __shared__ __attribute__((aligned(16))) T sVt[2][D * TL::VS];
    __shared__ __attribute__((aligned(16))) float sB[2][BN];

    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int hh = lane >> 5, kcol = lane & 31;
    const int nqb = (P.nq + kFwdBM - 1) / kFwdBM;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int qb = CAUSAL ? nqb - 1 - lid % nqb : lid % nqb;
    const int bh = lid / nqb;
    const int h = bh % P.heads, b = bh / P.heads;
    const int q0 = qb * kFwdBM + w * 32;
    const int qi = q0 + kcol;

    // Q^T operand fragments: lane (q, hh) holds Q[q][c*16 + 8*hh .. +7]
    frag qf[D / 16];
    {
        const T* qrow = P.q.row<T>(b, h, qi < P.nq ? qi : 0);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            u32x4_t raw = {0u, 0u, 0u, 0u};
            if (qi < P.nq) raw = *reinterpret_cast<const u32x4_t*>(qrow + c * 16 + 8 * hh);
            qf[c] = __builtin_bit_cast(frag, raw);
        }
    }
    f32x16_t o[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) o[x] = zero16();
    float m = -INFINITY, l = 0.f;
    const float sl2 = P.scale * kLog2e;
    const float cinv = SOFTCLAMP ? P.scale / P.softclamp : 0.f;
    const float cl2 = SOFTCLAMP ? P.softclamp * kLog2e : 0.f;

    const KeySide<T> ks = key_side<T>(P, b, h);
    const int kend = CAUSAL ? min(P.nk, qb * kFwdBM + kFwdBM) : P.nk;
    const int ntiles = (kend + BN - 1) / BN;

    FwdStage<D, KB> st;
    fwd_load_tile<T, D, KB, HAS_VMUL, HAS_BIAS>(ks, 0, st);
    fwd_store_tile<T, D, KB, HAS_BIAS>(st, sK[0], sVt[0], sB[0]);
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const int j0 = t * BN;
        if (t + 1 < ntiles) fwd_load_tile<T, D, KB, HAS_VMUL, HAS_BIAS>(ks, j0 + BN, st);
        if (!(CAUSAL && j0 > q0 + 31)) {
            const T* K = sK[buf];
            const T* Vt = sVt[buf];
            f32x16_t s[KB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                s[kb] = zero16();
#pragma unroll
                for (int c = 0; c < D / 16; ++c)
                    s[kb] = M::run(ld_frag<T>(K + (kb * 32 + kcol) * TL::KS + c * 16 + 8 * hh), qf[c], s[kb]);
            }
            // scores in the log2 domain (raw when PLAIN) plus the key bias
            if (!PLAIN) {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        float bv[4] = {0.f, 0.f, 0.f, 0.f};
                        if (HAS_BIAS) {
                            const float4 bb = *reinterpret_cast<const float4*>(sB[buf] + kb * 32 + 8 * g + 4 * hh);
                            bv[0] = bb.x;
                            bv[1] = bb.y;
                            bv[2] = bb.z;
                            bv[3] = bb.w;
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float x = s[kb][4 * g + r];
                            s[kb][4 * g + r] = (SOFTCLAMP ? cl2 * tanhf(x * cinv) : x * sl2) + bv[r];
                        }
                    }
                }
            }
            // causal diagonal / past-the-end tiles: register i of block kb holds key
            // j0 + kb*32 + 8*(i/4) + 4*hh + (i%4), valid while that offset stays <= lim
            if ((CAUSAL && j0 + BN - 1 > q0) || (!HAS_BIAS && j0 + BN > P.nk)) {
                int lim = HAS_BIAS ? (1 << 30) : P.nk - 1 - j0;
                if (CAUSAL) lim = min(lim, qi - j0);
                lim -= 4 * hh;
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (kb * 32 + 8 * (i / 4) + (i % 4) > lim) s[kb][i] = -INFINITY;
            }
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
            mx = xhalf_max(mx);
            if (PLAIN) mx *= sl2;
            const float m_new = fmaxf(m, mx);
            if (__any(m_new > m)) {
                const float alpha = (m_new > m) ? fast_exp2(m - m_new) : 1.f;
                l *= alpha;
#pragma unroll
                for (int x = 0; x < D / 32; ++x)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[x][i] *= alpha;
                m = m_new;
            }
            const float m_sub = (m == -INFINITY) ? 0.f : m;
            // P^T operands and O^T += V^T . P^T
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float p = PLAIN ? fast_exp2(fmaf(s[kb][i], sl2, -m_sub)) : fast_exp2(s[kb][i] - m_sub);
                    s[kb][i] = p;
                    l += p;
                }
#pragma unroll
                for (int t2 = 0; t2 < 2; ++t2) {
                    const frag pb = acc_to_frag<T>(s[kb], t2);
                    const int kbase = kb * 32 + 16 * t2 + 4 * hh;
#pragma unroll
                    for (int x = 0; x < D / 32; ++x)
                        o[x] = M::run(lds_runs<T>(Vt + (x * 32 + kcol) * TL::VS + kbase), pb, o[x]);
                }
            }
        }
        if (t + 1 < ntiles) fwd_store_tile<T, D, KB, HAS_BIAS>(st, sK[buf ^ 1], sVt[buf ^ 1], sB[buf ^ 1]);
        __syncthreads();
    }

    l = xhalf_sum(l);
    if (qi >= P.nq) return;
    const bool degenerate = !(l > 0.f) || !P.qm.keep(b, qi);
    const float inv = degenerate ? 0.f : 1.f / l;
    T* orow = P.out.wrow<T>(b, h, qi);
#pragma unroll
    for (int x = 0; x < D / 32; ++x) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = x * 32 + 8 * g + 4 * hh;
            u32x2_t pk;
            pk[0] = pack2<T>(o[x][4 * g] * inv, o[x][4 * g + 1] * inv);
            pk[1] = pack2<T>(o[x][4 * g + 2] * inv, o[x][4 * g + 3] * inv);
            *reinterpret_cast<u32x2_t*>(orow + d) = pk;
        }
    }
    if (hh == 0) *P.lse.wrow<float>(b, h, qi) = degenerate ? NAN : (m + log2f(l)) * kLn2;
}

// ---------------------------------------------------------------------------------------

// 32-key blocks per key tile: 128-key tiles at head dim 64 (without softclamp, whose tanh
// temporaries would spill), 64-key tiles otherwise
template <int D, bool SOFTCLAMP>
constexpr int kFwdKB = (D == 64 && !SOFTCLAMP) ? PA_FWD_KB64 : 2;

bool mfma_fwd_supported(const PassDev& P, int dtype) {
    if (dtype != PA_BF16 && dtype != PA_F16) return false;
    if (P.dim != 64 && P.dim != 128) return false;
    if (!aligned_rows_host(P.q, 8) || !aligned_rows_host(P.k, 8) || !aligned_rows_host(P.v, 8)) return false;
    if (P.vmul.ok() && !aligned_rows_host(P.vmul, 8)) return false;
    if (!aligned_rows_host(P.out, 4)) return false;
    return true;
}

template <typename T, int D, bool C, bool S, bool V, bool B>
static void launch_t(const PassDev& P, hipStream_t s) {
    constexpr int KB = kFwdKB<D, S>;
    const int nqb = (P.nq + kFwdBM - 1) / kFwdBM;
    dim3 grid(nqb * P.heads * P.batch);
    ProfScope ps("mfma_fwd", s);
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
    if (dtype == PA_BF16) {
        if (P.dim == 64) launch_d<bf16, 64>(P, s);
        else launch_d<bf16, 128>(P, s);
    } else {
        if (P.dim == 64) launch_d<f16, 64>(P, s);
        else launch_d<f16, 128>(P, s);
    }
}

}  // namespace pa
