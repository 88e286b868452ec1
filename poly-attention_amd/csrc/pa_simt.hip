// pa_simt.hip -- generic attention-pass kernels: one lane per query (or key) row.
//
// These kernels implement every feature of a pass (any head dim up to 256, masks with the
// reference's finite-fill semantics, bias classes, value multiplier, GQA head mapping) in
// fp32 arithmetic.  They run whenever the MFMA kernels do not cover a request (fp32 data,
// head dims other than 64/128, masked rows) and they finish the rare fully-masked rows of
// an MFMA forward (k_simt_fixup).
#include "pa_common.h"
#include "pa_launch.h"

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

// Finish the rows an MFMA forward left fully masked (their lse holds NaN).
template <typename T, int D>
__global__ __launch_bounds__(kSimtRows) void k_simt_fixup(PassDev P) {
    __shared__ float sK[kSimtKT][D];
    __shared__ float sV[kSimtKT][D];
    __shared__ float sB[kSimtKT];
    __shared__ uint8_t sKM[kSimtKT];
    const int b = blockIdx.z, h = blockIdx.y;
    const int i = blockIdx.x * kSimtRows + threadIdx.x;
    const bool row = i < P.nq;
    const bool degen = row && isnan(*P.lse.row<float>(b, h, i));
    if (!__syncthreads_or(degen)) return;
    const bool qok = row && P.qm.keep(b, i);
    float acc[D], c1;
    simt_degenerate_rows<T, D>(P, b, h, i, degen, qok, sK, sV, sB, sKM, acc, c1);
    if (degen) {
        if (c1 > 0.f) simt_write_row<T, D>(P, b, h, i, acc, 1.f / c1, -FLT_MAX);
        else simt_write_row<T, D>(P, b, h, i, acc, NAN, -INFINITY);
    }
}

// ---------------------------------------------------------------------------------------
// backward

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
        const bool qok = P.qm.keep(b, i);
        float c1 = 0.f;
        for (int j = 0; j < P.nk; ++j) {
            const bool own_masked = !qok || (P.causal && j > i) || !P.km.keep(b, j);
            const float bj = P.bias.ok() ? P.bias.scalar(b, h, j) : 0.f;
            if ((own_masked ? 1 : 0) + bias_class(bj) == 1) c1 += 1.f;
        }
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
template <typename T, int LPR>
__global__ __launch_bounds__(256) void k_bwd_pre_vec(GradDev G) {
    const PassDev& P = G.f;
    constexpr int kRows = 256 / LPR;
    const int64_t total = (int64_t)P.batch * P.heads * P.nq;
    const int64_t r = (int64_t)blockIdx.x * kRows + threadIdx.x / LPR;
    const int sub = threadIdx.x % LPR;
    if (r >= total) return;  // whole LPR-lane groups leave together
    const int i = (int)(r % P.nq);
    const int h = (int)((r / P.nq) % P.heads), b = (int)(r / ((int64_t)P.nq * P.heads));
    const int d0 = sub * 8;
    float dsum = 0.f;
    if (d0 < P.dim) {
        const uint4 ov = *reinterpret_cast<const uint4*>(P.out.row<T>(b, h, i) + d0);
        const uint4 gv = *reinterpret_cast<const uint4*>(G.dout.row<T>(b, h, i) + d0);
        const T* oe = reinterpret_cast<const T*>(&ov);
        const T* ge = reinterpret_cast<const T*>(&gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) dsum += to_f(oe[e]) * to_f(ge[e]);
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) dsum += __shfl_xor(dsum, off);
    if (sub != 0) return;
    const float dl = G.dlse.ok() ? *G.dlse.row<float>(b, h, i) : 0.f;
    const float l = *P.lse.row<float>(b, h, i);
    float lseb = l, invc = 0.f;
    if (l > kMaskedThreshold) {
        dsum -= dl;
    } else {  // fully-masked row (rare): count its class-1 entries
        const bool qok = P.qm.keep(b, i);
        float c1 = 0.f;
        for (int j = 0; j < P.nk; ++j) {
            const bool own_masked = !qok || (P.causal && j > i) || !P.km.keep(b, j);
            const float bj = P.bias.ok() ? P.bias.scalar(b, h, j) : 0.f;
            if ((own_masked ? 1 : 0) + bias_class(bj) == 1) c1 += 1.f;
        }
        lseb = INFINITY;
        invc = c1 > 0.f ? 1.f / c1 : 0.f;
        dsum = c1 > 0.f ? dsum - c1 * dl : 0.f;
    }
    G.ws_D[r] = dsum;
    G.ws_lse[r] = lseb;
    G.ws_invc[r] = invc;
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
// launchers

template <typename T, int D>
static void launch_simt_fwd_t(const PassDev& P, hipStream_t s) {
    dim3 grid((P.nq + kSimtRows - 1) / kSimtRows, P.heads, P.batch);
    ProfScope ps("simt_fwd", s);
    hipLaunchKernelGGL((k_simt_fwd<T, D>), grid, dim3(kSimtRows), 0, s, P);
}
template <typename T, int D>
static void launch_simt_fixup_t(const PassDev& P, hipStream_t s) {
    dim3 grid((P.nq + kSimtRows - 1) / kSimtRows, P.heads, P.batch);
    ProfScope ps("simt_fixup", s);
    hipLaunchKernelGGL((k_simt_fixup<T, D>), grid, dim3(kSimtRows), 0, s, P);
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
            const int64_t total = (int64_t)P.batch * P.heads * P.nq;
            const unsigned blocks = (unsigned)((total * lpr + 255) / 256);
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
static void simt_fwd_d(const PassDev& P, hipStream_t s, bool fixup) {
    const int d = P.dim;
    if (fixup) {
        if (d <= 16) launch_simt_fixup_t<T, 16>(P, s);
        else if (d <= 32) launch_simt_fixup_t<T, 32>(P, s);
        else if (d <= 64) launch_simt_fixup_t<T, 64>(P, s);
        else if (d <= 128) launch_simt_fixup_t<T, 128>(P, s);
        else launch_simt_fixup_t<T, 256>(P, s);
        return;
    }
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

void launch_simt_fwd(const PassDev& P, int dtype, hipStream_t s) {
    if (dtype == PA_F32) simt_fwd_d<float>(P, s, false);
    else if (dtype == PA_F16) simt_fwd_d<f16>(P, s, false);
    else simt_fwd_d<bf16>(P, s, false);
}
void launch_simt_fixup(const PassDev& P, int dtype, hipStream_t s) {
    if (dtype == PA_F32) simt_fwd_d<float>(P, s, true);
    else if (dtype == PA_F16) simt_fwd_d<f16>(P, s, true);
    else simt_fwd_d<bf16>(P, s, true);
}
void launch_simt_bwd(const GradDev& G, int dtype, hipStream_t s, bool pre, bool dq, bool dkv) {
    if (dtype == PA_F32) simt_bwd_d<float>(G, s, pre, dq, dkv);
    else if (dtype == PA_F16) simt_bwd_d<f16>(G, s, pre, dq, dkv);
    else simt_bwd_d<bf16>(G, s, pre, dq, dkv);
}

}  // namespace pa
