// pa_mfma_f32.hip -- fp32 attention-pass forward on the matrix cores (v_mfma_f32_32x32x2_f32),
// head dim 64 or 128.
//
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

__device__ __forceinline__ f32x16_t mfma_32x32x2(float a, float b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
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
    if (causal) block_order<true>(nqb, bh, rank);
    else block_order<false>(nqb, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;
    const int h = bh % P.heads, b = bh / P.heads;
    const int col = lane & 31, hh = lane >> 5;
    const int q0 = qb * BM + w * 32;
    const int qi = q0 + col;
    const bool qrow = qi < P.nq;

    float qf[D / 2];  // Q[qi][2s + hh]
    {
        const float* qr = P.q.row<float>(b, h, qrow ? qi : 0);
#pragma unroll
        for (int s = 0; s < D / 2; ++s) qf[s] = qrow ? qr[2 * s + hh] : 0.f;
    }
    f32x16_t o[D / 32];
#pragma unroll
    for (int x = 0; x < D / 32; ++x) o[x] = zero16();
    float m = -INFINITY, l = 0.f;  // running max (log2 units, shared by the lane pair), partial sum

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
        if (j0 < wave_kend) {  // wave-uniform: the causal limit of this wave's queries
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
            const float mnew = fmaxf(m, xhalf_max(tmax));
            if (mnew > m) {
                const float c = m == -INFINITY ? 0.f : fast_exp2(m - mnew);
                l *= c;
#pragma unroll
                for (int x = 0; x < D / 32; ++x)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[x][r] *= c;
                m = mnew;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = m == -INFINITY ? 0.f : fast_exp2(s[r] - m);
                s[r] = p;
                l += p;
            }
#pragma unroll
            for (int x = 0; x < D / 32; ++x)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int jj = 8 * (r / 4) + 4 * hh + (r % 4);
                    o[x] = mfma_32x32x2(sV[jj * RS + 32 * x + col], s[r], o[x]);
                }
        }
        __syncthreads();
    }

    const float lt = xhalf_sum(l);
    if (!qrow) return;  // no barriers below
    const bool degenerate = !(lt > 0.f) || !P.qm.keep(b, qi);
    const float inv = degenerate ? 0.f : 1.f / lt;
    float* orow = P.out.wrow<float>(b, h, qi);
#pragma unroll
    for (int x = 0; x < D / 32; ++x)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * x + 8 * g + 4 * hh;
            const float4 v = make_float4(o[x][4 * g] * inv, o[x][4 * g + 1] * inv,
                                         o[x][4 * g + 2] * inv, o[x][4 * g + 3] * inv);
            *reinterpret_cast<float4*>(orow + d) = v;
            if (P.ey.ok()) {
                float* yrow = P.ey.wrow<float>(b, h, qi);
                yrow[d] = epi_y<float>(P, b, h, qi, d, v.x);
                yrow[d + 1] = epi_y<float>(P, b, h, qi, d + 1, v.y);
                yrow[d + 2] = epi_y<float>(P, b, h, qi, d + 2, v.z);
                yrow[d + 3] = epi_y<float>(P, b, h, qi, d + 3, v.w);
            }
        }
    if (hh == 0) *P.lse.wrow<float>(b, h, qi) = degenerate ? NAN : (m + log2f(lt)) * kLn2;
}

bool mfma_fwd_f32_supported(const PassDev& P) {
    if (P.dim != 64 && P.dim != 128) return false;
    for (const DView* v : {&P.q, &P.k, &P.v, &P.out})
        if (!aligned_rows_host(*v, 4)) return false;
    if (P.vmul.ok() && !aligned_rows_host(P.vmul, 4)) return false;
    return true;
}

void launch_mfma_fwd_f32(const PassDev& P, hipStream_t s) {
    // waves per workgroup: the most that still give the grid two workgroups per CU
    const int units = P.batch * P.heads;
    int nw = 4;
    while (nw > 1 && (int64_t)units * ((P.nq + 32 * nw - 1) / (32 * nw)) < 512) nw >>= 1;
    const dim3 grid(units * ((P.nq + 32 * nw - 1) / (32 * nw)));
    ProfScope ps("mfma_fwd_f32", s);
    if (P.dim == 64) hipLaunchKernelGGL((k_mfma_fwd_f32<64>), grid, dim3(64 * nw), 0, s, P);
    else hipLaunchKernelGGL((k_mfma_fwd_f32<128>), grid, dim3(64 * nw), 0, s, P);
}

}  // namespace pa
