// pa_mfma_fwd.hip -- MFMA forward attention pass for bf16 / f16, head dim 64 or 128 (gfx950).
//
// Workgroup = 4 waves = 128 query rows of one (batch, pass head); each wave owns 32 queries.
// Per key tile (64 keys) a wave computes the transposed scores S^T = K . Q^T with
// v_mfma_f32_32x32x16_{bf16,f16}: the 32x32 accumulator layout gives lane l the column
// q = l % 32 and 16 key rows, so the online-softmax state (running max m, sum l and the
// rescale of the output) is a per-lane scalar.  The probabilities, rounded to the input
// type, stay in registers as the B operand of O^T += V^T . P^T (keys permuted consistently
// between the two operands), V being staged transposed in LDS.  K / V tiles are double
// buffered: the global loads of tile t+1 are in flight while tile t is computed.
// The exponentials run in the log2 domain with scale*log2(e) folded into one multiply.
//
// Rows whose every key is masked are left with lse = NaN for k_simt_fixup, which applies the
// reference's finite-fill semantics to them.
#include "pa_common.h"
#include "pa_launch.h"
#include "pa_mfma.h"

namespace pa {

constexpr int kFwdBM = 128;  // query rows per workgroup
constexpr int kFwdBN = 64;   // keys per tile
constexpr int kFwdThreads = 256;

template <typename T, int D>
struct FwdTile {
    static constexpr int KS = D + 8;          // K row stride in LDS (elements)
    static constexpr int VS = kFwdBN + 4;     // V^T row stride in LDS (elements)
    static constexpr int KCH = kFwdBN * D / 8 / kFwdThreads;  // 16-B K chunks per thread
    static constexpr int VTASKS = (kFwdBN / 4) * (D / 8);    // 4-key x 8-dim V blocks
    static constexpr int VT = (VTASKS + kFwdThreads - 1) / kFwdThreads;
};

// Registers holding one tile's global loads between issue and LDS store.
template <typename T, int D>
struct FwdStage {
    u32x4_t k[FwdTile<T, D>::KCH];
    u32x4_t v[FwdTile<T, D>::VT][4];
    float bias;
};

template <typename T, int D, bool HAS_VMUL>
__device__ __forceinline__ void fwd_load_tile(const PassDev& P, int b, int h, int j0,
                                              FwdStage<T, D>& st) {
    using TL = FwdTile<T, D>;
    const int tid = threadIdx.x;
    const u32x4_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int c = 0; c < TL::KCH; ++c) {
        const int e = tid + c * kFwdThreads;
        const int row = e / (D / 8), ch = e % (D / 8);
        const int j = j0 + row;
        st.k[c] = (j < P.nk) ? *reinterpret_cast<const u32x4_t*>(P.k.row<T>(b, h, j) + ch * 8) : zero;
    }
#pragma unroll
    for (int c = 0; c < TL::VT; ++c) {
        const int task = tid + c * kFwdThreads;
        const int dc = task % (D / 8), kg = task / (D / 8);
        if (task < TL::VTASKS) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = j0 + kg * 4 + r;
                if (j < P.nk) {
                    u32x4_t v = *reinterpret_cast<const u32x4_t*>(P.v.row<T>(b, h, j) + dc * 8);
                    if (HAS_VMUL)
                        v = mul_round8<T>(v, *reinterpret_cast<const u32x4_t*>(P.vmul.row<T>(b, h, j) + dc * 8));
                    st.v[c][r] = v;
                } else {
                    st.v[c][r] = zero;
                }
            }
        }
    }
    if (tid < kFwdBN) {
        const int j = j0 + tid;
        float bv = -INFINITY;
        if (j < P.nk && P.km.keep(b, j)) {
            bv = 0.f;
            if (P.bias.ok()) {
                const float x = P.bias.scalar(b, h, j);
                bv = bias_class(x) == 0 ? x * kLog2e : -INFINITY;
            }
        }
        st.bias = bv;
    }
}

template <typename T, int D>
__device__ __forceinline__ void fwd_store_tile(const FwdStage<T, D>& st, T* sK, T* sVt, float* sB) {
    using TL = FwdTile<T, D>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int c = 0; c < TL::KCH; ++c) {
        const int e = tid + c * kFwdThreads;
        const int row = e / (D / 8), ch = e % (D / 8);
        *reinterpret_cast<u32x4_t*>(sK + row * TL::KS + ch * 8) = st.k[c];
    }
#pragma unroll
    for (int c = 0; c < TL::VT; ++c) {
        const int task = tid + c * kFwdThreads;
        const int dc = task % (D / 8), kg = task / (D / 8);
        if (task < TL::VTASKS) {
            // transpose a 4-key x 8-dim block: V^T[d][k0..k0+3] for the 8 dims
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint32_t w0 = st.v[c][0][m], w1 = st.v[c][1][m];
                const uint32_t w2 = st.v[c][2][m], w3 = st.v[c][3][m];
                u32x2_t even, odd;
                even[0] = (w0 & 0xffffu) | (w1 << 16);
                even[1] = (w2 & 0xffffu) | (w3 << 16);
                odd[0] = (w0 >> 16) | (w1 & 0xffff0000u);
                odd[1] = (w2 >> 16) | (w3 & 0xffff0000u);
                const int d = dc * 8 + 2 * m;
                *reinterpret_cast<u32x2_t*>(sVt + d * TL::VS + kg * 4) = even;
                *reinterpret_cast<u32x2_t*>(sVt + (d + 1) * TL::VS + kg * 4) = odd;
            }
        }
    }
    if (tid < kFwdBN) sB[tid] = st.bias;
}

template <typename T, int D, bool CAUSAL, bool SOFTCLAMP, bool HAS_VMUL>
__global__ __launch_bounds__(kFwdThreads, D == 64 ? 2 : 1) void k_mfma_fwd(PassDev P) {
    using TL = FwdTile<T, D>;
    using M = Mma<T>;
    typedef typename M::frag frag;
    __shared__ __attribute__((aligned(16))) T sK[2][kFwdBN * TL::KS];
    __shared__ __attribute__((aligned(16))) T sVt[2][D * TL::VS];
    __shared__ __attribute__((aligned(16))) float sB[2][kFwdBN];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int q0 = qb * kFwdBM + w * 32;
    const int qi = q0 + (lane & 31);
    const int hh = lane >> 5;
    const int kcol = lane & 31;

    // Q^T operand fragments: lane (q, hh) holds Q[q][c*16 + 8*hh .. +7]
    frag qf[D / 16];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        u32x4_t raw = {0u, 0u, 0u, 0u};
        if (qi < P.nq) raw = *reinterpret_cast<const u32x4_t*>(P.q.row<T>(b, h, qi) + c * 16 + 8 * hh);
        qf[c] = __builtin_bit_cast(frag, raw);
    }
    f32x16_t o[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[x][i] = 0.f;
    float m = -INFINITY, l = 0.f;
    const float sl2 = P.scale * kLog2e;
    const float cinv = SOFTCLAMP ? P.scale / P.softclamp : 0.f;
    const float cl2 = SOFTCLAMP ? P.softclamp * kLog2e : 0.f;

    const int kend = CAUSAL ? min(P.nk, qb * kFwdBM + kFwdBM) : P.nk;
    const int ntiles = (kend + kFwdBN - 1) / kFwdBN;

    FwdStage<T, D> st;
    fwd_load_tile<T, D, HAS_VMUL>(P, b, h, 0, st);
    fwd_store_tile<T, D>(st, sK[0], sVt[0], sB[0]);
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const int j0 = t * kFwdBN;
        if (t + 1 < ntiles) fwd_load_tile<T, D, HAS_VMUL>(P, b, h, j0 + kFwdBN, st);
        if (!(CAUSAL && j0 > q0 + 31)) {
            const T* K = sK[buf];
            const T* Vt = sVt[buf];
            const float* Bs = sB[buf];
            f32x16_t s[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) s[kb][i] = 0.f;
#pragma unroll
                for (int c = 0; c < D / 16; ++c) {
                    const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(
                        K + (kb * 32 + kcol) * TL::KS + c * 16 + 8 * hh);
                    s[kb] = M::run(__builtin_bit_cast(frag, raw), qf[c], s[kb]);
                }
            }
            // scores in the log2 domain, bias / masks, running max
            const bool diag = CAUSAL && (j0 + kFwdBN - 1 > q0);
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int kr = kb * 32 + 8 * g + 4 * hh;  // first of 4 consecutive keys
                    const float4 bb = *reinterpret_cast<const float4*>(Bs + kr);
                    const float bv[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * g + r;
                        float x;
                        if (SOFTCLAMP) x = cl2 * tanhf(s[kb][i] * cinv) + bv[r];
                        else x = s[kb][i] * sl2 + bv[r];
                        if (diag && (j0 + kr + r > qi)) x = -INFINITY;
                        s[kb][i] = x;
                        mx = fmaxf(mx, x);
                    }
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m, mx);
            const float alpha = (m == m_new) ? 1.f : exp2f(m - m_new);
            const float m_sub = (m_new == -INFINITY) ? 0.f : m_new;
            m = m_new;
            l *= alpha;
#pragma unroll
            for (int x = 0; x < D / 32; ++x)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[x][i] *= alpha;
            // P^T operands and O^T += V^T . P^T
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int t2 = 0; t2 < 2; ++t2) {
                    float p[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        p[e] = exp2f(s[kb][8 * t2 + e] - m_sub);
                        l += p[e];
                    }
                    u32x4_t praw;
#pragma unroll
                    for (int k = 0; k < 4; ++k) praw[k] = pack2<T>(p[2 * k], p[2 * k + 1]);
                    const frag pb = __builtin_bit_cast(frag, praw);
                    const int kbase = kb * 32 + 16 * t2 + 4 * hh;
#pragma unroll
                    for (int x = 0; x < D / 32; ++x) {
                        const T* vrow = Vt + (x * 32 + kcol) * TL::VS + kbase;
                        const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vrow);
                        const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vrow + 8);
                        const u32x4_t vraw = {lo[0], lo[1], hi[0], hi[1]};
                        o[x] = M::run(__builtin_bit_cast(frag, vraw), pb, o[x]);
                    }
                }
            }
        }
        if (t + 1 < ntiles) fwd_store_tile<T, D>(st, sK[buf ^ 1], sVt[buf ^ 1], sB[buf ^ 1]);
        __syncthreads();
    }

    l += __shfl_xor(l, 32);
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

bool mfma_fwd_supported(const PassDev& P, int dtype) {
    if (dtype != PA_BF16 && dtype != PA_F16) return false;
    if (P.dim != 64 && P.dim != 128) return false;
    if (!aligned_rows_host(P.q, 8) || !aligned_rows_host(P.k, 8) || !aligned_rows_host(P.v, 8)) return false;
    if (P.vmul.ok() && !aligned_rows_host(P.vmul, 8)) return false;
    if (!aligned_rows_host(P.out, 4)) return false;
    return true;
}

template <typename T, int D, bool C, bool S, bool V>
static void launch_t(const PassDev& P, hipStream_t s) {
    dim3 grid((P.nq + kFwdBM - 1) / kFwdBM, P.heads, P.batch);
    ProfScope ps("mfma_fwd", s);
    hipLaunchKernelGGL((k_mfma_fwd<T, D, C, S, V>), grid, dim3(kFwdThreads), 0, s, P);
}

template <typename T, int D>
static void launch_d(const PassDev& P, hipStream_t s) {
    const bool c = P.causal != 0, sc = P.softclamp > 0.f, v = P.vmul.ok();
    if (c) {
        if (sc) v ? launch_t<T, D, true, true, true>(P, s) : launch_t<T, D, true, true, false>(P, s);
        else v ? launch_t<T, D, true, false, true>(P, s) : launch_t<T, D, true, false, false>(P, s);
    } else {
        if (sc) v ? launch_t<T, D, false, true, true>(P, s) : launch_t<T, D, false, true, false>(P, s);
        else v ? launch_t<T, D, false, false, true>(P, s) : launch_t<T, D, false, false, false>(P, s);
    }
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
