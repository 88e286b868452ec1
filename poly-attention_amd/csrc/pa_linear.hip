// pa_linear.hip -- the projections of a single-token decode step: y = x . w^T + bias for a
// handful of rows (the batch), which is a pass over the weight matrix and nothing else.
//
// Up to four projections of the same x (the q / k / v projections of a layer) share one
// launch, each output optionally followed by GELU and a residual add, and x itself optionally
// preceded by a residual add and an RMSNorm (the feed-forward of a decode harness), so that a
// step issues fewer kernels.  A library GEMM tiles such a product
// for large M and leaves most CUs idle at M <= 16; here every wave owns R output features, streams their weight rows with 16-byte non-temporal
// loads (the first round of chunks issued before x is staged, so both latencies overlap), and
// takes the x rows from LDS, staged once per workgroup; 16-bit types multiply in packed dot
// products (v_dot2_f32_{bf16,f16}, exact products, fp32 sums).  The R x MM per-lane partial sums are reduced over the wave by a
// butterfly reduce-scatter (each exchange halves the values a lane carries), so that every
// lane ends with one finished sum.  fp32 accumulation, bias added in fp32, one rounding.
#include <algorithm>
#include <type_traits>

#include "pa_common.h"
#include "pa_launch.h"

namespace pa {

// eight waves per workgroup: x is staged once per eight output features.  Staging it per four
// cost more L2 traffic than the weights themselves at decode shapes (an 8-layer order-3 decode
// step at batch 8, dim 1024: 0.898 -> 0.866 ms); sixteen leave too few or unevenly spread
// workgroups for outputs of 1024 - 6144 features.
constexpr int kLinThreads = 512;
constexpr int kLinMaxRows = 16;
constexpr int kLinMaxLds = 64 * 1024;  // bytes of staged x rows

struct LinOut {
    const char* w;
    const char* bias;
    const char* res;
    char* y;
    int64_t ws, rs, ys;  // row strides (elements)
    int32_t n, act;
    int32_t blk0;        // first workgroup of this output
};

struct LinDev {
    const char* x;
    const char* xadd;
    char* xsum;
    const void* nw;
    int64_t xs, xas, xss;
    int32_t rows, k, count, norm, nwdt;
    float eps;
    LinOut o[PA_LINEAR_MAX_OUT];
};

template <typename T> struct LinVec { static constexpr int n = 8; };
template <> struct LinVec<float> { static constexpr int n = 4; };

// Reduce-scatter of V values over the 64 lanes: afterwards lane l holds the wave sum of value
// index idx(l) (bits of l from bit 5 down, one per halving); lanes that differ only in the
// bits below log2(V) + (6 - log2(V)) hold the same sum.  Returns that sum.
template <int V>
__device__ __forceinline__ float wave_reduce_scatter(float (&v)[V], int lane) {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "power of two up to 64");
    int cnt = V;
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        if (cnt > 1) {
            const int h = cnt / 2;
            const bool up = (lane & s) != 0;
#pragma unroll
            for (int i = 0; i < V / 2; ++i) {
                if (i < h) {
                    const float send = up ? v[i] : v[h + i];
                    const float keep = up ? v[h + i] : v[i];
                    v[i] = keep + __shfl_xor(send, s);
                }
            }
            cnt = h;
        } else {
            v[0] += __shfl_xor(v[0], s);
        }
    }
    return v[0];
}

// the value index a lane holds after wave_reduce_scatter<V>
template <int V>
__device__ __forceinline__ int reduce_scatter_index(int lane) {
    int idx = 0, cnt = V;
    for (int s = 32; s >= 1 && cnt > 1; s >>= 1) {
        const int h = cnt / 2;
        if (lane & s) idx += h;
        cnt = h;
    }
    return idx;
}

// acc + <w, x> over one 16-byte chunk: packed dot products for 16-bit types (products exact
// in fp32), FMAs for fp32
template <typename T>
__device__ __forceinline__ float chunk_dot(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                           uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3, float acc) {
    if constexpr (std::is_same<T, float>::value) {
        acc = fmaf(__uint_as_float(w0), __uint_as_float(x0), acc);
        acc = fmaf(__uint_as_float(w1), __uint_as_float(x1), acc);
        acc = fmaf(__uint_as_float(w2), __uint_as_float(x2), acc);
        return fmaf(__uint_as_float(w3), __uint_as_float(x3), acc);
    } else if constexpr (std::is_same<T, bf16>::value) {
        typedef __bf16 v2 __attribute__((ext_vector_type(2)));
        auto d = [](uint32_t a, uint32_t b, float c) {
            return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
        };
        return d(w3, x3, d(w2, x2, d(w1, x1, d(w0, x0, acc))));
    } else {
        typedef _Float16 v2 __attribute__((ext_vector_type(2)));
        auto d = [](uint32_t a, uint32_t b, float c) {
            return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
        };
        return d(w3, x3, d(w2, x2, d(w1, x1, d(w0, x0, acc))));
    }
}

// U: chunks of 16 bytes per lane and feature in flight per round (the weight row of a
// feature is in flight whole up to 64 * U chunks), chosen per launch from in_features so that
// short rows do not hold registers that lower the occupancy.
template <typename T, int MM, int R, int U>
__global__ __launch_bounds__(kLinThreads) void k_linear_small(LinDev L) {
    constexpr int E = LinVec<T>::n;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    extern __shared__ u32x4 s_x[];  // rows x (k / E) chunks
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cpr = L.k / E;
    const int rows = L.rows;
    // this workgroup's output: the last one whose first workgroup is at or before it
    int oi = 0;
#pragma unroll
    for (int j = 1; j < PA_LINEAR_MAX_OUT; ++j)
        if (j < L.count && (int)blockIdx.x >= L.o[j].blk0) oi = j;
    const LinOut O = L.o[oi];
    const int n0 = (((int)blockIdx.x - O.blk0) * (kLinThreads / 64) + wave) * R;
    const T* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
        wrow[r] = reinterpret_cast<const T*>(O.w) + (int64_t)min(n0 + r, O.n - 1) * O.ws;
    const bool live = n0 < O.n;
    u32x4 wr[U][R];
    auto load_round = [&](int c0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + 64 * u;
#pragma unroll
            for (int r = 0; r < R; ++r)
                wr[u][r] = (live && c < cpr)
                               ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[r] + c * E))
                               : u32x4{0u, 0u, 0u, 0u};
        }
    };
    // the first round of weights is in flight while x is staged (SU loads per thread in
    // flight per round of the staging loop); the RMSNorm weights, when they share x's dtype,
    // are staged behind x as one more row of chunks
    constexpr int SU = U >= 8 ? 8 : 4;
    load_round(lane);
    const int total = rows * cpr;
    u32x4* s_w = s_x + total;
    const bool wvec = L.norm && L.nw && L.nwdt == (std::is_same<T, float>::value ? PA_F32
                                                  : std::is_same<T, bf16>::value ? PA_BF16 : PA_F16);
    const int staged = total + (wvec ? cpr : 0);
    for (int i0 = tid; i0 < staged; i0 += SU * kLinThreads) {
        u32x4 t[SU], ta[SU];
#pragma unroll
        for (int j = 0; j < SU; ++j) {
            const int i = i0 + j * kLinThreads;
            const int r = i / cpr, c = i - r * cpr;
            if (i < total) {
                t[j] = *reinterpret_cast<const u32x4*>(L.x + ((int64_t)r * L.xs + (int64_t)c * E) * sizeof(T));
                if (L.xadd)
                    ta[j] = *reinterpret_cast<const u32x4*>(L.xadd + ((int64_t)r * L.xas + (int64_t)c * E) * sizeof(T));
            } else if (i < staged) {
                t[j] = *reinterpret_cast<const u32x4*>(static_cast<const char*>(L.nw) + (int64_t)(i - total) * 16);
            }
        }
#pragma unroll
        for (int j = 0; j < SU; ++j) {
            const int i = i0 + j * kLinThreads;
            if (i >= staged) continue;
            if (i >= total) {
                s_x[i] = t[j];  // a norm weight chunk
                continue;
            }
            if (L.xadd) {
                // the residual add, rounded as torch's element-wise add
                T* a = reinterpret_cast<T*>(&t[j]);
                const T* bb = reinterpret_cast<const T*>(&ta[j]);
#pragma unroll
                for (int e = 0; e < E; ++e) a[e] = (T)(to_f(a[e]) + to_f(bb[e]));
                if (L.xsum && blockIdx.x == 0) {
                    const int r = i / cpr, c = i - r * cpr;
                    *reinterpret_cast<u32x4*>(L.xsum + ((int64_t)r * L.xss + (int64_t)c * E) * sizeof(T)) = t[j];
                }
            }
            s_x[i] = t[j];
        }
    }
    __syncthreads();
    if (L.norm) {
        // torch.nn.RMSNorm over each staged row: rstd in fp32, y = round((x * rstd) * w)
        __shared__ float s_rstd[kLinMaxRows];
        for (int r = wave; r < rows; r += kLinThreads / 64) {
            float ss = 0.f;
            for (int c = lane; c < cpr; c += 64) {
                const u32x4 v = s_x[r * cpr + c];
                const T* e = reinterpret_cast<const T*>(&v);
#pragma unroll
                for (int j = 0; j < E; ++j) ss += to_f(e[j]) * to_f(e[j]);
            }
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
            if (lane == 0) s_rstd[r] = rsqrtf(ss / (float)L.k + L.eps);
        }
        __syncthreads();
#pragma unroll 4
        for (int i = tid; i < total; i += kLinThreads) {
            const int r = i / cpr, c = i - r * cpr;
            u32x4 v = s_x[i];
            T* e = reinterpret_cast<T*>(&v);
            const float rs = s_rstd[r];
            if (wvec) {
                const u32x4 wr = s_w[c];
                const T* we = reinterpret_cast<const T*>(&wr);
#pragma unroll
                for (int j = 0; j < E; ++j) e[j] = (T)((to_f(e[j]) * rs) * to_f(we[j]));
            } else {
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    const float w = L.nw ? load_any(L.nw, L.nwdt, c * E + j) : 1.f;
                    e[j] = (T)((to_f(e[j]) * rs) * w);
                }
            }
            s_x[i] = v;
        }
        __syncthreads();
    }
    if (!live) return;

    float acc[R * MM];
#pragma unroll
    for (int i = 0; i < R * MM; ++i) acc[i] = 0.f;
    for (int c0 = lane; c0 < cpr; c0 += 64 * U) {
        if (c0 != lane) load_round(c0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + 64 * u;
            if (c >= cpr) break;
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                if (m >= rows) break;
                const u32x4 xr = s_x[m * cpr + c];
#pragma unroll
                for (int r = 0; r < R; ++r)
                    acc[r * MM + m] = chunk_dot<T>(wr[u][r][0], wr[u][r][1], wr[u][r][2], wr[u][r][3],
                                                   xr[0], xr[1], xr[2], xr[3], acc[r * MM + m]);
            }
        }
    }
    const float tot = wave_reduce_scatter<R * MM>(acc, lane);
    const int idx = reduce_scatter_index<R * MM>(lane);
    const int r = idx / MM, m = idx % MM;
    // one writer per value: the lowest lane of those holding it
    constexpr int V = R * MM;
    const int dup = 64 / V;  // lanes sharing a value (adjacent in the low bits)
    if ((lane & (dup - 1)) == 0 && m < rows && n0 + r < O.n) {
        const int f = n0 + r;
        float out = tot;
        if (O.bias) out += to_f(reinterpret_cast<const T*>(O.bias)[f]);
        out = round_to<T>(out);
        // torch.nn.GELU(): 0.5 y (1 + erf(y / sqrt(2))) in fp32 on the rounded product
        if (O.act == PA_ACT_GELU) out = round_to<T>(0.5f * out * (1.f + erff(out * 0.70710678118654752f)));
        if (O.res) out = round_to<T>(out + to_f(reinterpret_cast<const T*>(O.res)[(int64_t)m * O.rs + f]));
        reinterpret_cast<T*>(O.y)[(int64_t)m * O.ys + f] = (T)out;
    }
}

template <typename T, int MM>
static void launch_lin_r(const LinDev& L, int blocks, size_t lds, hipStream_t s) {
    constexpr int E = LinVec<T>::n;
    const int rounds = (L.k / E + 63) / 64;  // chunks per lane of one weight row
    if (rounds <= 1) hipLaunchKernelGGL((k_linear_small<T, MM, 1, 1>), dim3(blocks), dim3(kLinThreads), lds, s, L);
    else if (rounds <= 2) hipLaunchKernelGGL((k_linear_small<T, MM, 1, 2>), dim3(blocks), dim3(kLinThreads), lds, s, L);
    else if (rounds <= 4) hipLaunchKernelGGL((k_linear_small<T, MM, 1, 4>), dim3(blocks), dim3(kLinThreads), lds, s, L);
    else hipLaunchKernelGGL((k_linear_small<T, MM, 1, 8>), dim3(blocks), dim3(kLinThreads), lds, s, L);
}

template <typename T>
static void launch_lin_t(const LinDev& L, int blocks, size_t lds, hipStream_t s) {
    if (L.rows <= 1) launch_lin_r<T, 1>(L, blocks, lds, s);
    else if (L.rows <= 2) launch_lin_r<T, 2>(L, blocks, lds, s);
    else if (L.rows <= 4) launch_lin_r<T, 4>(L, blocks, lds, s);
    else if (L.rows <= 8) launch_lin_r<T, 8>(L, blocks, lds, s);
    else launch_lin_r<T, 16>(L, blocks, lds, s);
}

int launch_linear_small(const pa_linear* l, hipStream_t s) {
    if (l->rows < 1 || l->in_features < 1 || l->count < 1 || l->count > PA_LINEAR_MAX_OUT) return PA_EINVAL;
    if (!l->x) return PA_EINVAL;
    const int T = l->dtype;
    if (T != PA_F32 && T != PA_F16 && T != PA_BF16) return PA_EINVAL;
    if (l->rows > kLinMaxRows) return PA_EUNSUPPORTED;
    const int es = T == PA_F32 ? 4 : 2, E = 16 / es;
    if (l->in_features % E != 0) return PA_EUNSUPPORTED;
    if ((uintptr_t)l->x % 16 != 0 || l->x_stride % E != 0) return PA_EUNSUPPORTED;
    if (l->rows > 1 && l->x_stride < l->in_features) return PA_EINVAL;
    size_t lds = (size_t)l->rows * l->in_features * es;
    if (lds > (size_t)kLinMaxLds) return PA_EUNSUPPORTED;
    if (l->norm && l->norm_weight && l->norm_dtype == T) lds += (size_t)l->in_features * es;  // staged weight

    if ((l->x_add && ((uintptr_t)l->x_add % 16 != 0 || l->x_add_stride % E != 0)) ||
        (l->x_sum && ((uintptr_t)l->x_sum % 16 != 0 || l->x_sum_stride % E != 0)))
        return PA_EUNSUPPORTED;
    if (l->x_sum && !l->x_add) return PA_EINVAL;
    if (l->norm && l->norm_weight && l->norm_dtype != PA_F32 && l->norm_dtype != PA_F16 &&
        l->norm_dtype != PA_BF16)
        return PA_EINVAL;
    if (l->norm && l->norm_weight && l->norm_dtype == T && (uintptr_t)l->norm_weight % 16 != 0)
        return PA_EUNSUPPORTED;

    LinDev L;
    L.x = static_cast<const char*>(l->x);
    L.xs = l->x_stride;
    L.xadd = static_cast<const char*>(l->x_add);
    L.xas = l->x_add_stride;
    L.xsum = static_cast<char*>(l->x_sum);
    L.xss = l->x_sum_stride;
    L.norm = l->norm ? 1 : 0;
    L.nw = l->norm ? l->norm_weight : nullptr;
    L.nwdt = l->norm_dtype;
    L.eps = l->norm_eps;
    L.rows = l->rows;
    L.k = l->in_features;
    L.count = l->count;
    constexpr int waves = kLinThreads / 64;  // one output feature per wave
    int blocks = 0;
    for (int o = 0; o < PA_LINEAR_MAX_OUT; ++o) {
        LinOut& d = L.o[o];
        d = LinOut{};
        if (o >= l->count) continue;
        const pa_linear_out& u = l->out[o];
        if (!u.w || !u.y || u.out_features < 1) return PA_EINVAL;
        if (u.activation != PA_ACT_NONE && u.activation != PA_ACT_GELU) return PA_EINVAL;
        if ((uintptr_t)u.w % 16 != 0 || u.w_stride % E != 0) return PA_EUNSUPPORTED;
        if (u.w_stride < l->in_features) return PA_EINVAL;
        if (l->rows > 1 && (u.y_stride < u.out_features || (u.residual && u.residual_stride < u.out_features)))
            return PA_EINVAL;
        if ((uintptr_t)u.y % es != 0 || (u.bias && (uintptr_t)u.bias % es != 0) ||
            (u.residual && (uintptr_t)u.residual % es != 0))
            return PA_EINVAL;
        d.w = static_cast<const char*>(u.w);
        d.bias = static_cast<const char*>(u.bias);
        d.res = static_cast<const char*>(u.residual);
        d.y = static_cast<char*>(u.y);
        d.ws = u.w_stride;
        d.rs = u.residual_stride;
        d.ys = u.y_stride;
        d.n = u.out_features;
        d.act = u.activation;
        d.blk0 = blocks;
        blocks += (u.out_features + waves - 1) / waves;
    }
    ProfScope ps("linear_small", s);
    if (T == PA_F32) launch_lin_t<float>(L, blocks, lds, s);
    else if (T == PA_F16) launch_lin_t<f16>(L, blocks, lds, s);
    else launch_lin_t<bf16>(L, blocks, lds, s);
    return PA_OK;
}

}  // namespace pa
