// pa_decode.hip -- single-token decode over the poly KV cache.
//
// A decode step of an order-n poly attention reads every cached tensor once; it is HBM
// bound.  Phase 1 splits the cached positions 0..n-2 of every level into chunks and computes,
// per (level, batch, head, chunk), the softmax partial (m, l, sum p v) with coalesced,
// non-temporal 16-byte loads; the K row of a position is read once and shared by the query
// heads of its KV group.  With one or two level heads per KV group k_dec_partial streams K,
// values and biases in one pass with an online softmax; with more, k_dec_partial_grp scores
// the K rows for all heads first and then streams the values head by head.  Phase 2
// (k_dec_combine) runs one workgroup
// per (batch, KV group): level by level (deepest first) it merges the chunk partials,
// adds the new position n-1 -- whose value and bias are the step results of the deeper
// level -- and writes the level's msg / lse cache slot (or the final output).
#include <algorithm>
#include <mutex>

#include "pa_common.h"
#include "pa_launch.h"

namespace pa {

struct DecLevelDev {
    DView q, k, v, vmul, bias, out, lse;  // hdiv relative to the level head count
    int32_t heads;                        // level head count
    int32_t rep;                          // level heads per KV group
    int32_t out_rep, lse_rep;             // view heads per level head (replicated writes)
    float* ws;                            // partial records [B][heads][nchunks][rec]
};

struct DecodeDev {
    int32_t batch, kv_heads, n, dim, order, chunk, nchunks, rec, lpr;
    float scale, softclamp;
    // when set, the step's position count is read here (n above is then its upper bound) and
    // the msg / lse caches of the non-final levels are written at position n-1
    const int32_t* n_dev;
    DecLevelDev L[PA_MAX_ORDER];
};

__device__ __forceinline__ int step_n(const DecodeDev& D) {
    if (!D.n_dev) return D.n;
    const int n = *D.n_dev;
    return n < 1 ? 1 : (n > D.n ? D.n : n);  // clamped: a bad count cannot read out of bounds
}

constexpr int kDecThreads = 256;
constexpr int kDecHB = 4;      // grouped kernel: level heads scored per pass over a chunk's K rows
constexpr int kDecVH = 4;      // grouped kernel: level heads per sweep over a chunk's value rows
constexpr int kDecRows = 8;    // rows in flight per row group (streaming kernel: heads x rows)
constexpr float kDecTau = 8.f;  // lazy-rescale headroom of the partial's running max (log2 units)
constexpr int kDecChunkWork = 4096;  // level heads per KV group x positions of one chunk, at most
constexpr int kDecMaxHeadsPerGroup = 64;
constexpr int kDecMaxGroupElems = 8192;  // level heads per KV group * head dim

template <typename T> struct Vec16;
template <> struct Vec16<bf16> { typedef uint4 type; static constexpr int n = 8; };
template <> struct Vec16<f16> { typedef uint4 type; static constexpr int n = 8; };
template <> struct Vec16<float> { typedef uint4 type; static constexpr int n = 4; };

// 16-byte streaming load: the cache is read once per step, so it bypasses cache retention
template <typename T>
__device__ __forceinline__ void load16(const T* p, float* out) {
    constexpr int E = Vec16<T>::n;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int i = 0; i < E; ++i) out[i] = to_f(e[i]);
}

// merge (m2, l2, a2) into (m, l, a); m in the log2 domain, -inf when empty
template <int E>
__device__ __forceinline__ void merge_state(float& m, float& l, float* a, float m2, float l2,
                                            const float* a2) {
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) return;
    const float c1 = exp2f(m - mn), c2 = exp2f(m2 - mn);
    l = l * c1 + l2 * c2;
#pragma unroll
    for (int i = 0; i < E; ++i) a[i] = a[i] * c1 + a2[i] * c2;
    m = mn;
}

// Sum over the LPR lanes of a row group (LPR <= 16 stays inside a 16-lane DPP row).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                                 0xF, 0xF, false));
}
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
    if (LPR >= 2) x += dpp_f<0xB1>(x);   // quad_perm [1,0,3,2]
    if (LPR >= 4) x += dpp_f<0x4E>(x);   // quad_perm [2,3,0,1]
    if (LPR >= 8) x += dpp_f<0x141>(x);  // row_half_mirror
    if (LPR >= 16) x += dpp_f<0x140>(x); // row_mirror
    if (LPR >= 32) x += __shfl_xor(x, 16);
    if (LPR >= 64) x += __shfl_xor(x, 32);
    return x;
}

// Streaming variant (one or two level heads per KV group), one workgroup per (chunk of cached
// positions, batch, KV group, level), one pass:
// each row group of LPR lanes walks its positions (row groups interleaved, so a wave's loads
// cover consecutive rows) with U = kDecRows / HB rows in flight, reads the K row once for
// HB level heads of the group together with those heads' value rows (times vmul for middle
// levels) and key biases, and keeps a per-head online softmax state (running max m in the
// log2 domain, sum l, sum p v over its E elements) with a lazy rescale.  At the end the row
// groups of a wave merge through lane exchanges, the four waves through LDS, and the chunk
// record (m, l, sum p v) is written.  More than HB heads per group re-read the K rows per
// batch of heads.
template <typename T, int LPR, int HB>
__global__ __launch_bounds__(kDecThreads) void k_dec_partial(DecodeDev D) {
    constexpr int E = Vec16<T>::n;
    constexpr int KG = kDecThreads / LPR;  // row groups per workgroup
    constexpr int NW = kDecThreads / 64;
    constexpr int U = kDecRows / HB;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    __shared__ float s_ml[NW][HB][2];
    __shared__ float s_acc[NW][HB][256];

    const int c = blockIdx.x, bg = blockIdx.y, t = blockIdx.z;
    const int b = bg / D.kv_heads, g = bg % D.kv_heads;
    const DecLevelDev& L = D.L[t];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = tid % LPR, kg = tid / LPR;
    const int d0 = sub * E;
    const bool dok = d0 < D.dim;
    const int C = D.chunk;
    const int j_begin = c * C;
    const int cnt = min(C, step_n(D) - 1 - j_begin);
    const int rep = L.rep, h0 = g * rep;
    if (cnt <= 0) {
        // a chunk past the step's positions (grid sized for the capacity): empty records
        for (int hh = tid; hh < rep; hh += kDecThreads) {
            float* rec = L.ws + (((int64_t)b * L.heads + h0 + hh) * D.nchunks + c) * D.rec;
            rec[0] = -INFINITY;
            rec[1] = 0.f;
        }
        return;
    }
    const float cinv = D.softclamp > 0.f ? D.scale / D.softclamp : 0.f;
    const float cl2 = D.softclamp * kLog2e;
    const float sl2 = D.scale * kLog2e;
    const bool has_vmul = L.vmul.ok(), has_bias = L.bias.ok();
    const T* kbase = L.k.row<T>(b, h0, 0) + d0;
    const int64_t ksn = L.k.sn, vsn = L.v.sn, msn = L.vmul.sn;
    auto raw16 = [&](const T* p) __attribute__((always_inline)) -> u32x4 {
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    };
    auto unpack = [&](const u32x4& r, float* out) __attribute__((always_inline)) {
        const T* e = reinterpret_cast<const T*>(&r);
#pragma unroll
        for (int i = 0; i < E; ++i) out[i] = to_f(e[i]);
    };

    for (int hb0 = 0; hb0 < rep; hb0 += HB) {
        const int nh = min(HB, rep - hb0);
        float qv[HB][E], acc[HB][E], m[HB], l[HB];
        const T* vbase[HB];
        const T* mbase[HB];
#pragma unroll
        for (int hh = 0; hh < HB; ++hh) {
            const int h = h0 + hb0 + (hh < nh ? hh : 0);
            if (hh < nh && dok) load16<T>(L.q.row<T>(b, h, 0) + d0, qv[hh]);
            else
#pragma unroll
                for (int e = 0; e < E; ++e) qv[hh][e] = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) acc[hh][e] = 0.f;
            m[hh] = -INFINITY;
            l[hh] = 0.f;
            vbase[hh] = L.v.row<T>(b, h, 0) + d0;
            mbase[hh] = has_vmul ? L.vmul.row<T>(b, h, 0) + d0 : nullptr;
        }
        for (int jl0 = kg; jl0 < cnt; jl0 += KG * U) {
            // loads of U rows: K (shared by the heads), then per head value, multiplier, bias
            u32x4 kr[U], vr[HB][U], mr[HB][U];
            float bz[HB][U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int jl = jl0 + u * KG;
                const bool ok = jl < cnt && dok;
                const int64_t j = j_begin + (jl < cnt ? jl : 0);
                kr[u] = ok ? raw16(kbase + j * ksn) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
                for (int hh = 0; hh < HB; ++hh) {
                    const bool hok = ok && hh < nh;
                    vr[hh][u] = hok ? raw16(vbase[hh] + j * vsn) : u32x4{0u, 0u, 0u, 0u};
                    mr[hh][u] = (hok && has_vmul) ? raw16(mbase[hh] + j * msn) : u32x4{0u, 0u, 0u, 0u};
                    bz[hh][u] = (jl < cnt && hh < nh && has_bias) ? L.bias.scalar(b, h0 + hb0 + hh, (int)j) : 0.f;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int jl = jl0 + u * KG;
                float kf[E];
                unpack(kr[u], kf);
#pragma unroll
                for (int hh = 0; hh < HB; ++hh) {
                    if (hh >= nh) break;
                    float part = 0.f;
#pragma unroll
                    for (int e = 0; e < E; ++e) part += qv[hh][e] * kf[e];
                    const float dot = group_sum<LPR>(part);
                    float x = D.softclamp > 0.f ? cl2 * tanhf(dot * cinv) : dot * sl2;
                    const float bj = bz[hh][u];
                    x = (jl < cnt && bias_class(bj) == 0) ? x + bj * kLog2e : -INFINITY;
                    // lazy rescale: the running max moves only past kDecTau of headroom
                    if (x > m[hh] + kDecTau) {
                        const float alpha = __builtin_amdgcn_exp2f(m[hh] - x);  // 0 when m = -inf
                        l[hh] *= alpha;
#pragma unroll
                        for (int e = 0; e < E; ++e) acc[hh][e] *= alpha;
                        m[hh] = x;
                    }
                    const float pj = __builtin_amdgcn_exp2f(x - (m[hh] == -INFINITY ? 0.f : m[hh]));
                    l[hh] += pj;
                    float vf[E];
                    unpack(vr[hh][u], vf);
                    if (has_vmul) {
                        float mf[E];
                        unpack(mr[hh][u], mf);
#pragma unroll
                        for (int e = 0; e < E; ++e) vf[e] = round_to<T>(vf[e] * mf[e]);
                    }
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[hh][e] += pj * vf[e];
                }
            }
        }
        // merge the row groups of each wave (lanes LPR, 2 LPR, ... apart), then the waves
#pragma unroll
        for (int hh = 0; hh < HB; ++hh) {
            if (hh >= nh) break;
            float mw = m[hh];
            for (int off = LPR; off < 64; off <<= 1) mw = fmaxf(mw, __shfl_xor(mw, off));
            const float cs = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[hh] - mw);
            float lw = l[hh] * cs;
            float aw[E];
#pragma unroll
            for (int e = 0; e < E; ++e) aw[e] = acc[hh][e] * cs;
            for (int off = LPR; off < 64; off <<= 1) {
                lw += __shfl_xor(lw, off);
#pragma unroll
                for (int e = 0; e < E; ++e) aw[e] += __shfl_xor(aw[e], off);
            }
            if (lane < LPR && dok)
#pragma unroll
                for (int e = 0; e < E; ++e) s_acc[wave][hh][d0 + e] = aw[e];
            if (lane == 0) {
                s_ml[wave][hh][0] = mw;
                s_ml[wave][hh][1] = lw;
            }
        }
        __syncthreads();
        for (int hh = 0; hh < nh; ++hh) {
            float mt = -INFINITY;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) mt = fmaxf(mt, s_ml[w2][hh][0]);
            float cw[NW], lt = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) {
                cw[w2] = mt == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_ml[w2][hh][0] - mt);
                lt += s_ml[w2][hh][1] * cw[w2];
            }
            float* rec = L.ws + (((int64_t)b * L.heads + h0 + hb0 + hh) * D.nchunks + c) * D.rec;
            for (int x = tid; x < D.dim; x += kDecThreads) {
                float a = 0.f;
#pragma unroll
                for (int w2 = 0; w2 < NW; ++w2) a += s_acc[w2][hh][x] * cw[w2];
                rec[2 + x] = a;
            }
            if (tid == 0) {
                rec[0] = mt;
                rec[1] = lt;
            }
        }
        __syncthreads();
    }
}

// Grouped variant (more than two level heads per KV group), one workgroup per (chunk of
// cached positions, batch, KV group, level), in three phases:
//   1. the chunk's key biases (the deeper level's lse, log2 domain) are staged in LDS, then
//      each row group of LPR lanes reads whole K rows (16 bytes per lane, kDecU rows in
//      flight) and adds the score of every level head of the group;
//   2. per head: max, p = 2^(s - max) in place, and the sum, over the chunk;
//   3. the values (times vmul for middle levels) of kDecVH heads at a time are streamed
//      together, one FMA per element, reduced over the row groups and written as the
//      chunk records (m, l, sum p v).
template <typename T, int LPR, bool VM>
__global__ __launch_bounds__(kDecThreads) void k_dec_partial_grp(DecodeDev D) {
    constexpr int E = Vec16<T>::n;
    constexpr int KG = kDecThreads / LPR;
    constexpr int kDecU = kDecRows;
    __shared__ float s_sc[kDecChunkWork];
    __shared__ float s_ml[kDecMaxHeadsPerGroup][2];
    __shared__ float s_acc[kDecThreads / 64][kDecVH][256];

    const int c = blockIdx.x, bg = blockIdx.y, t = blockIdx.z;
    const int b = bg / D.kv_heads, g = bg % D.kv_heads;
    const DecLevelDev& L = D.L[t];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = tid % LPR, kg = tid / LPR;
    const int d0 = sub * E;
    const bool dok = d0 < D.dim;
    const int C = D.chunk;
    const int j_begin = c * C;
    const int cnt = min(C, step_n(D) - 1 - j_begin);
    const int rep = L.rep, h0 = g * rep;
    if (cnt <= 0) {
        // a chunk past the step's positions (grid sized for the capacity): empty records
        for (int hh = tid; hh < rep; hh += kDecThreads) {
            float* rec = L.ws + (((int64_t)b * L.heads + h0 + hh) * D.nchunks + c) * D.rec;
            rec[0] = -INFINITY;
            rec[1] = 0.f;
        }
        return;
    }
    const float cinv = D.softclamp > 0.f ? D.scale / D.softclamp : 0.f;
    const float cl2 = D.softclamp * kLog2e;
    const float sl2 = D.scale * kLog2e;

    // 1a. biases
    for (int x = tid; x < rep * cnt; x += kDecThreads) {
        const int hh = x / cnt, jl = x % cnt;
        float bv = 0.f;
        if (L.bias.ok()) {
            const float bj = L.bias.scalar(b, h0 + hh, j_begin + jl);
            bv = bias_class(bj) == 0 ? bj * kLog2e : -INFINITY;
        }
        s_sc[hh * C + jl] = bv;
    }
    __syncthreads();

    // 1b. scores, heads in batches of kDecHB (K re-read per batch when rep > kDecHB)
    const T* kbase = L.k.row<T>(b, h0, 0) + d0;
    const int64_t ksn = L.k.sn;
    for (int hb0 = 0; hb0 < rep; hb0 += kDecHB) {
        float qv[kDecHB][E];
#pragma unroll
        for (int hh = 0; hh < kDecHB; ++hh) {
            if (hb0 + hh < rep && dok) load16<T>(L.q.row<T>(b, h0 + hb0 + hh, 0) + d0, qv[hh]);
            else
#pragma unroll
                for (int e = 0; e < E; ++e) qv[hh][e] = 0.f;
        }
        for (int jl0 = kg; jl0 < cnt; jl0 += KG * kDecU) {
            float kf[kDecU][E];
#pragma unroll
            for (int u = 0; u < kDecU; ++u) {
                const int jl = jl0 + u * KG;
                if (jl < cnt && dok) load16<T>(kbase + (j_begin + jl) * ksn, kf[u]);
                else
#pragma unroll
                    for (int e = 0; e < E; ++e) kf[u][e] = 0.f;
            }
#pragma unroll
            for (int hh = 0; hh < kDecHB; ++hh) {
                if (hb0 + hh >= rep) break;
#pragma unroll
                for (int u = 0; u < kDecU; ++u) {
                    float part = 0.f;
#pragma unroll
                    for (int e = 0; e < E; ++e) part += qv[hh][e] * kf[u][e];
                    const float dot = group_sum<LPR>(part);
                    const int jl = jl0 + u * KG;
                    if (sub == 0 && jl < cnt) {
                        const float x = D.softclamp > 0.f ? cl2 * tanhf(dot * cinv) : dot * sl2;
                        s_sc[(hb0 + hh) * C + jl] += x;
                    }
                }
            }
        }
    }
    __syncthreads();

    // 2. per-head max, exponentials and sum
    for (int hh = wave; hh < rep; hh += kDecThreads / 64) {
        float* sc = s_sc + hh * C;
        float mx = -INFINITY;
        for (int jl = lane; jl < cnt; jl += 64) mx = fmaxf(mx, sc[jl]);
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        const float msub = mx == -INFINITY ? 0.f : mx;
        float sum = 0.f;
        for (int jl = lane; jl < cnt; jl += 64) {
            const float p = __builtin_amdgcn_exp2f(sc[jl] - msub);
            sc[jl] = p;
            sum += p;
        }
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
        if (lane == 0) {
            s_ml[hh][0] = mx;
            s_ml[hh][1] = sum;
        }
    }
    __syncthreads();

    // 3. values: the heads of the group in sweeps of kDecVH over the chunk's rows, VU rows per
    // row group and head in flight (one pipeline drain and one record write-out per sweep).
    // VM: some level of the launch has a value multiplier, whose rows then share the budget
    // of loads in flight (four rows without one, one with: the kernel stays within 128 VGPRs,
    // four waves per SIMD)
    constexpr int VU = VM ? 1 : 4;
    const bool has_vmul = VM && L.vmul.ok();
    const int64_t vsn = L.v.sn, msn = L.vmul.sn;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    auto raw16 = [&](const T* q) __attribute__((always_inline)) -> u32x4 {
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q));
    };
    for (int hb0 = 0; hb0 < rep; hb0 += kDecVH) {
        const int nh = min(kDecVH, rep - hb0);
        const T* vbase[kDecVH];
        const T* mbase[kDecVH];
        float acc[kDecVH][E];
#pragma unroll
        for (int hh = 0; hh < kDecVH; ++hh) {
            const int h = h0 + hb0 + (hh < nh ? hh : 0);
            vbase[hh] = L.v.row<T>(b, h, 0) + d0;
            mbase[hh] = has_vmul ? L.vmul.row<T>(b, h, 0) + d0 : nullptr;
#pragma unroll
            for (int e = 0; e < E; ++e) acc[hh][e] = 0.f;
        }
        for (int jl0 = kg; jl0 < cnt; jl0 += KG * VU) {
            u32x4 vr[kDecVH][VU], mr[kDecVH][VU];
#pragma unroll
            for (int u = 0; u < VU; ++u) {
                const int jl = jl0 + u * KG;
                const int64_t j = j_begin + (jl < cnt ? jl : 0);
#pragma unroll
                for (int hh = 0; hh < kDecVH; ++hh) {
                    const bool ok = jl < cnt && dok && hh < nh;
                    vr[hh][u] = ok ? raw16(vbase[hh] + j * vsn) : u32x4{0u, 0u, 0u, 0u};
                    mr[hh][u] = (ok && has_vmul) ? raw16(mbase[hh] + j * msn) : u32x4{0u, 0u, 0u, 0u};
                }
            }
#pragma unroll
            for (int u = 0; u < VU; ++u) {
                const int jl = jl0 + u * KG;
#pragma unroll
                for (int hh = 0; hh < kDecVH; ++hh) {
                    if (hh >= nh) break;
                    const float pj = jl < cnt ? s_sc[(hb0 + hh) * C + jl] : 0.f;
                    const T* ve = reinterpret_cast<const T*>(&vr[hh][u]);
                    const T* me = reinterpret_cast<const T*>(&mr[hh][u]);
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        float v = to_f(ve[e]);
                        if (has_vmul) v = round_to<T>(v * to_f(me[e]));
                        acc[hh][e] += pj * v;
                    }
                }
            }
        }
#pragma unroll
        for (int hh = 0; hh < kDecVH; ++hh) {
            if (hh >= nh) break;
            for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
                for (int e = 0; e < E; ++e) acc[hh][e] += __shfl_xor(acc[hh][e], off);
            if (lane < LPR && dok)
#pragma unroll
                for (int e = 0; e < E; ++e) s_acc[wave][hh][d0 + e] = acc[hh][e];
        }
        __syncthreads();
        for (int hh = 0; hh < nh; ++hh) {
            float* rec = L.ws + (((int64_t)b * L.heads + h0 + hb0 + hh) * D.nchunks + c) * D.rec;
            for (int x = tid; x < D.dim; x += kDecThreads) {
                float a = 0.f;
#pragma unroll
                for (int w2 = 0; w2 < kDecThreads / 64; ++w2) a += s_acc[w2][hh][x];
                rec[2 + x] = a;
            }
            if (tid == 0) {
                rec[0] = s_ml[hb0 + hh][0];
                rec[1] = s_ml[hb0 + hh][1];
            }
        }
        __syncthreads();
    }
}

// The new position of one (level, head) and the write of its step result: (mm, ll, acc) is
// the merged state of the cached positions, part the raw q.k of the new position, vnew its
// value and bnew its bias (the deeper level's step results).
template <typename T>
__device__ __forceinline__ float dec_finish(const DecodeDev& D, const DecLevelDev& L, int b, int h,
                                           int hh, int lane, bool final_level, int n, float mm,
                                           float ll, float (&acc)[4], float part,
                                           const float (&vnew)[4], float bnew, float* s_msg2,
                                           float* s_lse2) {
    const int dim = D.dim, nold = n - 1;
    const bool new_ok = bias_class(bnew) == 0;
    if (new_ok) {
        const float tt = (softclamp_f(part * D.scale, D.softclamp) + bnew) * kLog2e;
        const float mn = fmaxf(mm, tt);
        const float c1 = exp2f(mm - mn), c2 = exp2f(tt - mn);
        ll = ll * c1 + c2;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = acc[e] * c1 + vnew[e] * c2;
        mm = mn;
    }
    float lse_v, inv;
    if (ll > 0.f) {
        lse_v = (mm + log2f(ll)) * kLn2;
        inv = 1.f / ll;
    } else {
        // every position masked: uniform average over the -FLT_MAX-biased positions
        float c1 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = 0.f;
        for (int j = 0; j < n; ++j) {
            const float bj = (j == nold) ? bnew : (L.bias.ok() ? L.bias.scalar(b, h, j) : 0.f);
            if (bias_class(bj) != 1) continue;
            c1 += 1.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = lane + 64 * e;
                if (d >= dim) continue;
                float v;
                if (j == nold) v = vnew[e];
                else {
                    v = to_f(L.v.row<T>(b, h, j)[d]);
                    if (L.vmul.ok()) v = round_to<T>(v * to_f(L.vmul.row<T>(b, h, j)[d]));
                }
                acc[e] += v;
            }
        }
        lse_v = c1 > 0.f ? -FLT_MAX : -INFINITY;
        inv = c1 > 0.f ? 1.f / c1 : NAN;
    }
    // write the step result (replicated over the view heads) and keep it in LDS
    const int slot = (D.n_dev && !final_level) ? nold : 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d >= dim) continue;
        const float o = acc[e] * inv;
        for (int r = 0; r < L.out_rep; ++r) L.out.wrow<T>(b, h * L.out_rep + r, slot)[d] = from_f<T>(o);
        s_msg2[hh * dim + d] = round_to<T>(o);
    }
    // the value the lse slot now holds (its dtype's rounding; every lane computes it), which
    // the next level's cached bias will hold
    float stored = lse_v;
    if (L.lse.ok())
        stored = L.lse.dtype == PA_F32 ? lse_v
                 : L.lse.dtype == PA_F16 ? (float)(f16)lse_v : (float)(bf16)lse_v;
    if (lane == 0) {
        if (L.lse.ok())
            for (int r = 0; r < L.lse_rep; ++r)
                store_any(L.lse.p, L.lse.dtype, L.lse.idx(b, h * L.lse_rep + r, slot), lse_v);
        s_lse2[hh] = stored;
    }
    return stored;
}

// merge the chunk partials of one (level, head): running max, sum and sum p v.  The chunk
// weights come from one load per lane (lane c holds chunk c); the value rows are then summed
// with loads that do not depend on each other (four chunks per step).
__device__ __forceinline__ void dec_merge(const DecodeDev& D, const DecLevelDev& L, int b, int h,
                                          int lane, float& mm, float& ll, float (&acc)[4]) {
    const int dim = D.dim;
    const float* recs = L.ws + ((int64_t)b * L.heads + h) * D.nchunks * D.rec;
    ll = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = 0.f;
    mm = -INFINITY;
    for (int c0 = 0; c0 < D.nchunks; c0 += 64) {
        const int c = c0 + lane;
        if (c < D.nchunks) mm = fmaxf(mm, recs[(int64_t)c * D.rec]);
    }
    for (int off = 32; off > 0; off >>= 1) mm = fmaxf(mm, __shfl_xor(mm, off));
    if (mm == -INFINITY) return;
    for (int c0 = 0; c0 < D.nchunks; c0 += 64) {
        const int c = c0 + lane;
        float wl = 0.f, lc = 0.f;
        if (c < D.nchunks) {
            const float mc = recs[(int64_t)c * D.rec];
            wl = mc == -INFINITY ? 0.f : exp2f(mc - mm);
            lc = recs[(int64_t)c * D.rec + 1];
        }
        float lsum = lc * wl;
        for (int off = 32; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off);
        ll += lsum;
        const int cn = min(64, D.nchunks - c0);
        int k = 0;
        for (; k + 4 <= cn; k += 4) {
            float wk[4], v[4][4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                wk[q] = __shfl(wl, k + q);
                const float* rc = recs + (int64_t)(c0 + k + q) * D.rec + 2;
                // a zero weight (an empty record: its vector part is never written) adds
                // nothing and is not read, so stale contents cannot turn into 0 * NaN
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int d = lane + 64 * e;
                    v[q][e] = (d < dim && wk[q] != 0.f) ? rc[d] : 0.f;
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] += v[q][e] * wk[q];
        }
        for (; k < cn; ++k) {
            const float wk = __shfl(wl, k);
            if (wk == 0.f) continue;  // uniform across the wave
            const float* rc = recs + (int64_t)(c0 + k) * D.rec + 2;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = lane + 64 * e;
                if (d < dim) acc[e] += rc[d] * wk;
            }
        }
    }
}

// One workgroup per (batch, KV group): chain the levels, deepest first.  Phase 1 merges the
// chunk partials and reads the new position's q, k (and v) for every (level, head) of the
// group at once, into LDS; phase 2 walks the levels, each needing only the deeper level's
// step result.  Items beyond the kDecCombElems budget of LDS state are merged in phase 2.
constexpr int kDecCombElems = 8192;
template <typename T>
__global__ __launch_bounds__(kDecThreads) void k_dec_combine(DecodeDev D) {
    const int b = blockIdx.x / D.kv_heads, g = blockIdx.x % D.kv_heads;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int kWaves = kDecThreads / 64;
    // per (level, head) item: [mm, ll, part, -, acc(dim), v(dim)]
    __shared__ float s_st[kDecCombElems];
    // step results of the previous (deeper) level, per level head of this group:
    // [head][dim] flattened, heads-per-group * dim <= kDecMaxGroupElems (checked on the host)
    __shared__ float s_msg[kDecMaxGroupElems];
    __shared__ float s_lse[kDecMaxHeadsPerGroup];
    __shared__ float s_msg2[kDecMaxGroupElems];
    __shared__ float s_lse2[kDecMaxHeadsPerGroup];
    const int dim = D.dim;
    const int n = step_n(D);
    const int nold = n - 1;
    const int ist = 4 + 2 * dim;  // floats per item

    // phase 1: all items in parallel, one wave per item
    int nitems = 0;
    for (int t = 0; t < D.order; ++t) nitems += D.L[t].rep;
    const int nfit = min(nitems, kDecCombElems / ist);  // items whose state fits in LDS
    for (int it = wave; it < nfit; it += kWaves) {
        int t = 0, hh = it;
        while (hh >= D.L[t].rep) hh -= D.L[t++].rep;
        const DecLevelDev& L = D.L[t];
        const int h = g * L.rep + hh;
        const bool final_level = (t == D.order - 1);
        float mm, ll, acc[4];
        dec_merge(D, L, b, h, lane, mm, ll, acc);
        float part = 0.f;
        const T* qrow = L.q.row<T>(b, h, 0);
        const T* krow = L.k.row<T>(b, h, nold);
        float* st = s_st + it * ist;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = lane + 64 * e;
            if (d < dim) {
                part += to_f(qrow[d]) * to_f(krow[d]);
                st[4 + d] = acc[e];
                st[4 + dim + d] = final_level ? 0.f : to_f(L.v.row<T>(b, h, nold)[d]);
            }
        }
        for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
        if (lane == 0) {
            st[0] = mm;
            st[1] = ll;
            st[2] = part;
        }
    }
    __syncthreads();

    // phase 2: the levels in order.  With one level head per KV group at every level (no GQA)
    // the chain is one wave's work: the deeper level's result stays in that wave (each lane
    // reads back only the features it wrote itself; the lse, uniform, is returned to every
    // lane), with no workgroup barrier or LDS copy per level.
    bool single = nitems <= nfit;
    for (int t = 0; t < D.order; ++t) single = single && D.L[t].rep == 1;
    if (single) {
        if (wave != 0) return;  // no barrier below
        float vprev[4] = {0.f, 0.f, 0.f, 0.f}, lprev = 0.f;
        for (int t = 0; t < D.order; ++t) {
            const DecLevelDev& L = D.L[t];
            const bool deepest = (t == 0), final_level = (t == D.order - 1);
            const float* st = s_st + t * ist;  // item t: level t's only head
            float acc[4], vnew[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = lane + 64 * e;
                acc[e] = d < dim ? st[4 + d] : 0.f;
                const float vr = d < dim ? st[4 + dim + d] : 0.f;
                vnew[e] = d >= dim ? 0.f
                          : deepest ? vr
                          : final_level ? vprev[e]
                          : round_to<T>(vr * vprev[e]);
            }
            lprev = dec_finish<T>(D, L, b, g, 0, lane, final_level, n, st[0], st[1], acc, st[2],
                                  vnew, deepest ? 0.f : lprev, s_msg2, s_lse2);
#pragma unroll
            for (int e = 0; e < 4; ++e) {  // this lane's own features of the result
                const int d = lane + 64 * e;
                vprev[e] = d < dim ? s_msg2[d] : 0.f;
            }
        }
        return;
    }
    int prev_rep = 1, base = 0;
    for (int t = 0; t < D.order; ++t) {
        const DecLevelDev& L = D.L[t];
        const bool deepest = (t == 0), final_level = (t == D.order - 1);
        for (int hh = wave; hh < L.rep; hh += kWaves) {
            const int h = g * L.rep + hh;
            // index of this head's deeper-level result (deeper level has prev_rep heads/group)
            const int ph = (hh * prev_rep) / L.rep;
            float mm, ll, part, acc[4], vr[4];
            if (base + hh < nfit) {
                const float* st = s_st + (base + hh) * ist;
                mm = st[0];
                ll = st[1];
                part = st[2];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int d = lane + 64 * e;
                    acc[e] = d < dim ? st[4 + d] : 0.f;
                    vr[e] = d < dim ? st[4 + dim + d] : 0.f;
                }
            } else {  // state beyond the LDS budget: merge and read here
                dec_merge(D, L, b, h, lane, mm, ll, acc);
                part = 0.f;
                const T* qrow = L.q.row<T>(b, h, 0);
                const T* krow = L.k.row<T>(b, h, nold);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int d = lane + 64 * e;
                    vr[e] = 0.f;
                    if (d < dim) {
                        part += to_f(qrow[d]) * to_f(krow[d]);
                        if (!final_level) vr[e] = to_f(L.v.row<T>(b, h, nold)[d]);
                    }
                }
                for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
            }
            float vnew[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = lane + 64 * e;
                vnew[e] = 0.f;
                if (d < dim) {
                    if (deepest) vnew[e] = vr[e];
                    else if (final_level) vnew[e] = s_msg[ph * dim + d];
                    else vnew[e] = round_to<T>(vr[e] * s_msg[ph * dim + d]);
                }
            }
            const float bnew = deepest ? 0.f : s_lse[ph];
            dec_finish<T>(D, L, b, h, hh, lane, final_level, n, mm, ll, acc, part, vnew, bnew,
                          s_msg2, s_lse2);
        }
        __syncthreads();
        for (int x = threadIdx.x; x < L.rep * dim; x += kDecThreads)
            s_msg[x] = s_msg2[x];
        for (int x = threadIdx.x; x < L.rep; x += kDecThreads) s_lse[x] = s_lse2[x];
        __syncthreads();
        prev_rep = L.rep;
        base += L.rep;
    }
}

// ---------------------------------------------------------------------------------------
// Decode prologue: q RMSNorm + rotary + cache append for every q / k / v of one layer's
// new token, one wave per (item, batch, head) row.

struct ProItemDev {
    DView src, out, cache;
    const void* w;
    int32_t wdt, rotate, heads, row0;
};

struct ProDev {
    int32_t batch, dim, count, capacity, rot_dim, pos, rows;
    float eps;
    const void* angles;
    int32_t adt;
    const int32_t* n_dev;
    int32_t* overflow;
    const float* inv_freq;  // angles from the position (when angles is null)
    float interp;
    ProItemDev it[2 * PA_MAX_ORDER];
};

constexpr int kProThreads = 256;

template <typename T>
__global__ __launch_bounds__(kProThreads) void k_dec_prologue(ProDev P) {
    // separate roundings of every product and sum, as torch's element-wise kernels do
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kProThreads / 64) + (threadIdx.x >> 6);
    if (row >= P.rows) return;  // no barriers below: whole waves leave together
    int k = 0;
    while (k + 1 < P.count && row >= P.it[k + 1].row0) ++k;
    const ProItemDev& I = P.it[k];
    const int local = row - I.row0;
    const int b = local / I.heads, h = local % I.heads;
    const int dim = P.dim;

    float x[4];
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        x[e] = d < dim ? to_f(I.src.row<T>(b, h, 0)[d]) : 0.f;
        ss += x[e] * x[e];
    }
    if (I.w) {
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
        const float r = rsqrtf(ss / (float)dim + P.eps);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = lane + 64 * e;
            const float w = d < dim ? load_any(I.w, I.wdt, d) : 0.f;
            x[e] = round_to<T>((x[e] * r) * w);
        }
    }
    const int64_t pos = P.n_dev ? (int64_t)*P.n_dev - 1 : (int64_t)P.pos;
    if (I.rotate && (P.angles || P.inv_freq)) {
        // the rotary module's own position, rounded as its get_seq_pos builds it
        const float pt = P.angles ? 0.f : round_to<T>(round_to<T>((float)pos) / P.interp);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = lane + 64 * e;
            const float partner = __shfl_xor(x[e], 1);  // feature d ^ 1 (same 64-block)
            if (d < P.rot_dim) {
                const float a = P.angles ? load_any(P.angles, P.adt, d) : pt * P.inv_freq[d >> 1];
                const float rot = (d & 1) ? partner : -partner;
                x[e] = round_to<T>(x[e] * cosf(a) + rot * sinf(a));
            }
        }
    }
    const bool in_range = pos >= 0 && pos < P.capacity;
    const bool to_cache = I.cache.ok() && in_range;
    if (!in_range && P.overflow && row == 0 && lane == 0) *P.overflow = 1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d >= dim) continue;
        const T y = from_f<T>(x[e]);
        if (I.out.ok()) I.out.wrow<T>(b, h, 0)[d] = y;
        if (to_cache) I.cache.wrow<T>(b, h, pos)[d] = y;
    }
}

int launch_prologue(const pa_prologue* p, hipStream_t s) {
    if (p->batch < 1 || p->dim < 1 || p->count < 1 || p->count > 2 * PA_MAX_ORDER)
        return PA_EINVAL;
    if (p->dim > 256) return PA_EUNSUPPORTED;
    const bool rotary = p->angles || p->inv_freq;
    if (rotary && (p->rot_dim < 0 || p->rot_dim > p->dim || p->rot_dim % 2 != 0))
        return PA_EINVAL;
    if (!p->angles && p->inv_freq && !(p->interp > 0.f)) return PA_EINVAL;
    if (p->angles && p->angles_dtype != PA_F32 && p->angles_dtype != PA_F16 && p->angles_dtype != PA_BF16)
        return PA_EINVAL;
    const int T = p->items[0].src.dtype;
    if (T != PA_F32 && T != PA_F16 && T != PA_BF16) return PA_EINVAL;
    ProDev P;
    P.batch = p->batch;
    P.dim = p->dim;
    P.count = p->count;
    P.capacity = p->capacity;
    P.rot_dim = rotary ? p->rot_dim : 0;
    P.pos = p->pos;
    P.eps = p->eps;
    P.angles = p->angles;
    P.adt = p->angles_dtype;
    P.n_dev = p->n_dev;
    P.overflow = p->overflow;
    P.inv_freq = p->angles ? nullptr : p->inv_freq;
    P.interp = p->interp;
    int rows = 0;
    for (int k = 0; k < p->count; ++k) {
        const pa_prologue_item& it = p->items[k];
        if (!it.src.ptr || it.src.heads < 1 || it.src.dtype != T) return PA_EINVAL;
        if ((it.out.ptr && (it.out.dtype != T || it.out.heads != it.src.heads)) ||
            (it.cache.ptr && (it.cache.dtype != T || it.cache.heads != it.src.heads)))
            return PA_EINVAL;
        if (it.cache.ptr && p->capacity < 1) return PA_EINVAL;
        if (it.norm_weight && it.weight_dtype != PA_F32 && it.weight_dtype != PA_F16 &&
            it.weight_dtype != PA_BF16)
            return PA_EINVAL;
        ProItemDev& I = P.it[k];
        auto mk = [&](const pa_view& v) {
            DView x;
            x.p = static_cast<char*>(v.ptr);
            x.sb = v.sb;
            x.sh = v.sh;
            x.sn = v.sn;
            x.hdiv = 1;
            x.dtype = v.dtype;
            return x;
        };
        I.src = mk(it.src);
        I.out = mk(it.out);
        I.cache = mk(it.cache);
        I.w = it.norm_weight;
        I.wdt = it.weight_dtype;
        I.rotate = it.rotate;
        I.heads = it.src.heads;
        I.row0 = rows;
        rows += p->batch * it.src.heads;
    }
    P.rows = rows;
    const dim3 grid((rows + kProThreads / 64 - 1) / (kProThreads / 64));
    ProfScope ps("dec_prologue", s);
    if (T == PA_F32) hipLaunchKernelGGL((k_dec_prologue<float>), grid, dim3(kProThreads), 0, s, P);
    else if (T == PA_F16) hipLaunchKernelGGL((k_dec_prologue<f16>), grid, dim3(kProThreads), 0, s, P);
    else hipLaunchKernelGGL((k_dec_prologue<bf16>), grid, dim3(kProThreads), 0, s, P);
    return PA_OK;
}

// ---------------------------------------------------------------------------------------

static int elem_size(int dtype) { return dtype == PA_F32 ? 4 : 2; }

static int pick_chunks(const pa_decode* d, int* chunk_out) {
    const int nold = d->n - 1;
    if (nold <= 0) {
        *chunk_out = 1;
        return 0;
    }
    // a chunk's work (level heads per KV group x positions) stays bounded
    int max_rep = 1;
    for (int t = 0; t < d->order && t < PA_MAX_ORDER; ++t)
        if (d->kv_heads > 0 && d->levels[t].heads / d->kv_heads > max_rep)
            max_rep = d->levels[t].heads / d->kv_heads;
    int cap = kDecChunkWork / max_rep;
    if (cap > 1024) cap = 1024;
    cap = cap / 64 * 64;
    if (cap < 64) cap = 64;
    int chunk = d->chunk;
    if (chunk <= 0) {
        const long units = (long)d->batch * d->kv_heads * d->order;
        long want = (2048 + units - 1) / units;  // aim for >= 2048 workgroups
        if (want < 1) want = 1;
        chunk = (int)((nold + want - 1) / want);
        chunk = (chunk + 63) / 64 * 64;
        // at least 512 positions per chunk (fewer, longer workgroups stream better)
        const int whole = (nold + 63) / 64 * 64;
        if (chunk < 512) chunk = whole < 512 ? whole : 512;
    }
    if (chunk > cap) chunk = cap;
    if (chunk < 64) chunk = 64;
    *chunk_out = chunk;
    return (nold + chunk - 1) / chunk;
}

template <typename T, int HB>
static void launch_partial_h(const DecodeDev& D, dim3 grid, hipStream_t s) {
    switch (D.lpr) {
        case 1: hipLaunchKernelGGL((k_dec_partial<T, 1, HB>), grid, dim3(kDecThreads), 0, s, D); break;
        case 2: hipLaunchKernelGGL((k_dec_partial<T, 2, HB>), grid, dim3(kDecThreads), 0, s, D); break;
        case 4: hipLaunchKernelGGL((k_dec_partial<T, 4, HB>), grid, dim3(kDecThreads), 0, s, D); break;
        case 8: hipLaunchKernelGGL((k_dec_partial<T, 8, HB>), grid, dim3(kDecThreads), 0, s, D); break;
        case 16: hipLaunchKernelGGL((k_dec_partial<T, 16, HB>), grid, dim3(kDecThreads), 0, s, D); break;
        case 32: hipLaunchKernelGGL((k_dec_partial<T, 32, HB>), grid, dim3(kDecThreads), 0, s, D); break;
        default: hipLaunchKernelGGL((k_dec_partial<T, 64, HB>), grid, dim3(kDecThreads), 0, s, D); break;
    }
}

template <typename T, bool VM>
static void launch_partial_grp_v(const DecodeDev& D, dim3 grid, hipStream_t s) {
    switch (D.lpr) {
        case 1: hipLaunchKernelGGL((k_dec_partial_grp<T, 1, VM>), grid, dim3(kDecThreads), 0, s, D); break;
        case 2: hipLaunchKernelGGL((k_dec_partial_grp<T, 2, VM>), grid, dim3(kDecThreads), 0, s, D); break;
        case 4: hipLaunchKernelGGL((k_dec_partial_grp<T, 4, VM>), grid, dim3(kDecThreads), 0, s, D); break;
        case 8: hipLaunchKernelGGL((k_dec_partial_grp<T, 8, VM>), grid, dim3(kDecThreads), 0, s, D); break;
        case 16: hipLaunchKernelGGL((k_dec_partial_grp<T, 16, VM>), grid, dim3(kDecThreads), 0, s, D); break;
        case 32: hipLaunchKernelGGL((k_dec_partial_grp<T, 32, VM>), grid, dim3(kDecThreads), 0, s, D); break;
        default: hipLaunchKernelGGL((k_dec_partial_grp<T, 64, VM>), grid, dim3(kDecThreads), 0, s, D); break;
    }
}

template <typename T>
static void launch_partial_grp(const DecodeDev& D, dim3 grid, hipStream_t s) {
    bool vm = false;
    for (int t = 0; t < D.order; ++t) vm = vm || D.L[t].vmul.ok();
    if (vm) launch_partial_grp_v<T, true>(D, grid, s);
    else launch_partial_grp_v<T, false>(D, grid, s);
}

// by the largest level head count per KV group: one or two heads stream in one pass (K, values
// and biases together); more take the grouped three-phase kernel (K rows scored for every head
// at once, then the values of one head after another)
template <typename T>
static void launch_partial_t(const DecodeDev& D, int max_rep, dim3 grid, hipStream_t s) {
    if (max_rep <= 1) launch_partial_h<T, 1>(D, grid, s);
    else if (max_rep <= 2) launch_partial_h<T, 2>(D, grid, s);
    else launch_partial_grp<T>(D, grid, s);
}

static int level_heads(const pa_decode_level& L) {
    int h = L.heads;
    return h;
}

size_t decode_workspace_bytes(const pa_decode* d, int* chunk_out, int* nchunks_out) {
    const int nchunks = pick_chunks(d, chunk_out);
    *nchunks_out = nchunks;
    const int rec = (d->dim + 2 + 3) & ~3;
    size_t total = 0;
    for (int t = 0; t < d->order && t < PA_MAX_ORDER; ++t) {
        const size_t sz = (size_t)d->batch * level_heads(d->levels[t]) * nchunks * rec * 4;
        total += (sz + 255) & ~size_t(255);
    }
    return total;
}

static bool aligned16(const pa_view& v) {
    const int es = elem_size(v.dtype);
    const int E = 16 / es;
    return ((uintptr_t)v.ptr % 16 == 0) && v.sb % E == 0 && v.sh % E == 0 && v.sn % E == 0;
}

int launch_decode(const pa_decode* d, hipStream_t s) {
    if (d->order < 2 || d->order > PA_MAX_ORDER) return PA_EINVAL;
    if (d->batch < 1 || d->kv_heads < 1 || d->n < 1 || d->dim < 1) return PA_EINVAL;
    for (int t = 0; t < d->order; ++t)
        if (!d->levels[t].q.ptr || !d->levels[t].k.ptr || !d->levels[t].v.ptr) return PA_EINVAL;
    if (d->dim > 256) return PA_EUNSUPPORTED;
    const int T = d->levels[0].q.dtype;
    if (T != PA_F32 && T != PA_F16 && T != PA_BF16) return PA_EINVAL;
    const int E = 16 / elem_size(T);
    if (d->dim % E != 0) return PA_EUNSUPPORTED;
    int lpr = 1;
    while (lpr * E < d->dim) lpr <<= 1;
    if (lpr > 64) return PA_EUNSUPPORTED;

    DecodeDev D;
    D.batch = d->batch;
    D.kv_heads = d->kv_heads;
    D.n = d->n;
    D.n_dev = d->n_dev;
    D.dim = d->dim;
    D.order = d->order;
    D.scale = d->scale;
    D.softclamp = d->softclamp;
    D.lpr = lpr;
    D.rec = (d->dim + 2 + 3) & ~3;
    int chunk = 1;
    D.nchunks = pick_chunks(d, &chunk);
    D.chunk = chunk;
    const size_t need = decode_workspace_bytes(d, &chunk, &D.nchunks);
    if (D.nchunks > 0 && (!d->workspace || d->workspace_bytes < need)) return PA_EWORKSPACE;

    char* ws = static_cast<char*>(d->workspace);
    size_t off = 0;
    for (int t = 0; t < d->order; ++t) {
        const pa_decode_level& l = d->levels[t];
        const int H = l.heads;
        if (H < 1 || H % d->kv_heads != 0) return PA_EINVAL;
        if (H / d->kv_heads > kDecMaxHeadsPerGroup) return PA_EUNSUPPORTED;
        if ((H / d->kv_heads) * d->dim > kDecMaxGroupElems) return PA_EUNSUPPORTED;
        auto chk = [&](const pa_view& v, bool required, int dt) -> bool {
            if (!v.ptr) return !required;
            if (v.heads < 1) return false;
            if (dt >= 0 && v.dtype != dt) return false;
            return true;
        };
        const bool deepest = t == 0, final_level = t == d->order - 1;
        if (!chk(l.q, true, T) || !chk(l.k, true, T) || !chk(l.v, true, T)) return PA_EINVAL;
        if (!chk(l.vmul, !deepest && !final_level, T)) return PA_EINVAL;
        if (!chk(l.bias, !deepest, -1) || !chk(l.out, true, T) || !chk(l.lse, !final_level, -1))
            return PA_EINVAL;
        // tensors read with the level's head index: their head count divides H
        const pa_view* reads[5] = {&l.q, &l.k, &l.v, &l.vmul, &l.bias};
        for (const pa_view* v : reads)
            if (v->ptr && H % v->heads != 0) return PA_EINVAL;
        if (l.k.heads != d->kv_heads) return PA_EINVAL;
        if (l.out.heads % H != 0 || (l.lse.ptr && l.lse.heads % H != 0)) return PA_EINVAL;
        const pa_view* vecs[4] = {&l.q, &l.k, &l.v, &l.vmul};
        for (const pa_view* v : vecs)
            if (v->ptr && !aligned16(*v)) return PA_EUNSUPPORTED;
        if (t > 0 && d->levels[t - 1].heads > H) return PA_EUNSUPPORTED;

        DecLevelDev& L = D.L[t];
        auto mk = [&](const pa_view& v) {
            DView x;
            x.p = static_cast<char*>(v.ptr);
            x.sb = v.sb;
            x.sh = v.sh;
            x.sn = v.sn;
            x.hdiv = (v.ptr && v.heads > 0 && v.heads <= H) ? H / v.heads : 1;
            x.dtype = v.dtype;
            return x;
        };
        L.q = mk(l.q);
        L.k = mk(l.k);
        L.v = mk(l.v);
        L.vmul = mk(l.vmul);
        L.bias = mk(l.bias);
        L.out = mk(l.out);
        L.out.hdiv = 1;
        L.lse = mk(l.lse);
        L.lse.hdiv = 1;
        L.heads = H;
        L.rep = H / d->kv_heads;
        L.out_rep = l.out.heads / H;
        L.lse_rep = l.lse.ptr ? l.lse.heads / H : 1;
        L.ws = reinterpret_cast<float*>(ws + off);
        off += (((size_t)d->batch * H * D.nchunks * D.rec * 4) + 255) & ~size_t(255);
    }
    if (D.nchunks > 0) {
        dim3 grid(D.nchunks, d->batch * d->kv_heads, d->order);
        int max_rep = 1;
        for (int t = 0; t < d->order; ++t) max_rep = std::max(max_rep, D.L[t].rep);
        ProfScope ps("dec_partial", s);
        if (T == PA_F32) launch_partial_t<float>(D, max_rep, grid, s);
        else if (T == PA_F16) launch_partial_t<f16>(D, max_rep, grid, s);
        else launch_partial_t<bf16>(D, max_rep, grid, s);
    }
    dim3 cgrid(d->batch * d->kv_heads);
    ProfScope ps("dec_combine", s);
    if (T == PA_F32) hipLaunchKernelGGL((k_dec_combine<float>), cgrid, dim3(kDecThreads), 0, s, D);
    else if (T == PA_F16) hipLaunchKernelGGL((k_dec_combine<f16>), cgrid, dim3(kDecThreads), 0, s, D);
    else hipLaunchKernelGGL((k_dec_combine<bf16>), cgrid, dim3(kDecThreads), 0, s, D);
    return PA_OK;
}

// ---------------------------------------------------------------------------------------
// Static scratch of pa_poly_decode_noalloc: the split-K partial records live in a device
// array of the library instead of a caller workspace.  Each GPU the library runs on holds its
// own copy at its own address; host code takes that address from hipGetSymbolAddress, looked
// up once per device, and never uses the array's name (a host-side stand-in) as a pointer.

static __device__ __align__(256) unsigned char scratch[PA_DECODE_SCRATCH_BYTES];

constexpr int kScratchMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kScratchMaxDevices];

// the current device's copy of `scratch`
static int scratch_address(void** out, int* hip_err) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *hip_err = static_cast<int>(e);
        return PA_EHIP;
    }
    if (dev < 0 || dev >= kScratchMaxDevices) return PA_EUNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            *hip_err = static_cast<int>(e);
            return PA_EHIP;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return PA_OK;
}

int launch_decode_noalloc(const pa_decode* d, hipStream_t s, int* hip_err) {
    if (d->order < 2 || d->order > PA_MAX_ORDER) return PA_EINVAL;
    if (d->batch < 1 || d->kv_heads < 1 || d->n < 1 || d->dim < 1) return PA_EINVAL;
    for (int t = 0; t < d->order; ++t)
        if (d->levels[t].heads < 1) return PA_EINVAL;
    int chunk = 0, nchunks = 0;
    if (decode_workspace_bytes(d, &chunk, &nchunks) > PA_DECODE_SCRATCH_BYTES) return PA_ESCRATCH;
    void* ptr = nullptr;
    const int st = scratch_address(&ptr, hip_err);
    if (st != PA_OK) return st;
    pa_decode local = *d;
    local.workspace = ptr;
    local.workspace_bytes = PA_DECODE_SCRATCH_BYTES;
    return launch_decode(&local, s);
}

}  // namespace pa
