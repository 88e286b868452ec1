// pa_norm.hip -- row RMSNorm over the head dim of [batch, heads, n, dim] views (the q/k norms
// of the poly-attention modules), optionally followed by the rotary embedding, forward and
// backward.  HBM bound: a row group of LPR lanes
// reads a whole row with 16-byte loads, reduces with DPP inside the row group, and writes the
// row back; the backward writes dx and accumulates the weight gradient per workgroup into a
// fixed partial row, summed afterwards in a fixed order (deterministic, no atomics).
#include <algorithm>

#include "pa_common.h"
#include "pa_launch.h"

namespace pa {

// n / d for n < 2^31 by a multiply-high and a shift (d fixed per launch; l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1)
struct FastDiv {
    uint32_t d, m, l;
    __device__ __forceinline__ uint32_t div(uint32_t n) const { return (__umulhi(m, n) + n) >> l; }
};
static FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    FastDiv f;
    f.d = d;
    f.l = l;
    f.m = (uint32_t)((((1ull << 32) * ((1ull << l) - d)) / d) + 1);
    return f;
}

// a strided [batch, heads, n, dim] tensor as the norm kernels address it (element strides)
struct RView {
    char* p;
    int64_t sb, sh, sn;
    template <typename T> __device__ __forceinline__ T* at(uint32_t b, uint32_t h, uint32_t i) const {
        return reinterpret_cast<T*>(p) + ((int64_t)b * sb + (int64_t)h * sh + (int64_t)i * sn);
    }
};

struct RmsDev {
    int32_t batch, heads, n, dim, lpr;
    int32_t hfast;    // rows walk heads fastest (input laid out [B, N, H, dim])
    uint32_t rows;    // < 2^31 (checked on the host)
    FastDiv fd_n, fd_h;
    float eps, inv_dim;
    RView x, y, dy, dx;
    const void* w;
    int32_t wdt;
    float* rstd;      // [batch][heads][n]
    float* partial;   // [gridDim.x][dim] (backward)
    float* dw;        // [dim] (backward, fp32)
    const void* ang;  // rotary angles [n][astride] or null
    int32_t adt, rot_dim;
    int64_t astride;
};

// rotary embedding of the E features d0.. of one row in place (fp32 math on the rounded
// norm output t, one rounding when stored): y[2i] = t[2i] cos a[2i] - t[2i+1] sin a[2i],
// y[2i+1] = t[2i+1] cos a[2i+1] + t[2i] sin a[2i+1]
template <int E>
__device__ __forceinline__ void rope_fwd(const RmsDev& R, uint32_t pos, int d0, float (&t)[E]) {
#pragma unroll
    for (int e = 0; e < E; e += 2) {
        const int d = d0 + e;
        if (d >= R.rot_dim) break;
        const int64_t o = (int64_t)pos * R.astride + d;
        const float a0 = load_any(R.ang, R.adt, o), a1 = load_any(R.ang, R.adt, o + 1);
        const float t0 = t[e], t1 = t[e + 1];
        t[e] = t0 * cosf(a0) - t1 * sinf(a0);
        t[e + 1] = t1 * cosf(a1) + t0 * sinf(a1);
    }
}

// the gradient of t from the gradient g of the rotated row (the transposed rotation)
template <int E>
__device__ __forceinline__ void rope_bwd(const RmsDev& R, uint32_t pos, int d0, float (&g)[E]) {
#pragma unroll
    for (int e = 0; e < E; e += 2) {
        const int d = d0 + e;
        if (d >= R.rot_dim) break;
        const int64_t o = (int64_t)pos * R.astride + d;
        const float a0 = load_any(R.ang, R.adt, o), a1 = load_any(R.ang, R.adt, o + 1);
        const float g0 = g[e], g1 = g[e + 1];
        g[e] = g0 * cosf(a0) + g1 * sinf(a1);
        g[e + 1] = g1 * cosf(a1) - g0 * sinf(a0);
    }
}

constexpr int kRmsThreads = 256;
constexpr int kRmsMaxBlocks = 1024;
constexpr int kRmsU = 4;  // rows per row group and pass

template <typename T> struct RVec;
template <> struct RVec<bf16> { static constexpr int n = 8; };
template <> struct RVec<f16> { static constexpr int n = 8; };
template <> struct RVec<float> { static constexpr int n = 4; };

template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) x += __shfl_xor(x, off);
    return x;
}

template <typename T>
__device__ __forceinline__ void load_row(const T* p, bool ok, float* out) {
    constexpr int E = RVec<T>::n;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 raw = {0u, 0u, 0u, 0u};
    if (ok) raw = *reinterpret_cast<const u32x4*>(p);
    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int i = 0; i < E; ++i) out[i] = to_f(e[i]);
}

template <typename T>
__device__ __forceinline__ void store_row(T* p, const float* v) {
    constexpr int E = RVec<T>::n;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 raw;
    T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int i = 0; i < E; ++i) e[i] = from_f<T>(v[i]);
    *reinterpret_cast<u32x4*>(p) = raw;
}

// row r -> (batch, head, position) in the order that walks the input's memory sequentially
__device__ __forceinline__ void row_coords(const RmsDev& R, uint32_t r, uint32_t& b, uint32_t& h,
                                           uint32_t& i) {
    if (R.hfast) {
        const uint32_t q1 = R.fd_h.div(r);
        h = r - q1 * R.fd_h.d;
        b = R.fd_n.div(q1);
        i = q1 - b * R.fd_n.d;
    } else {
        const uint32_t q1 = R.fd_n.div(r);
        i = r - q1 * R.fd_n.d;
        b = R.fd_h.div(q1);
        h = q1 - b * R.fd_h.d;
    }
}

__device__ __forceinline__ uint32_t rstd_index(const RmsDev& R, uint32_t b, uint32_t h, uint32_t i) {
    return (b * R.fd_h.d + h) * R.fd_n.d + i;
}

// y = round(x * rsqrt(mean(x^2) + eps) * w); rstd saved per row.  Each row group handles
// kRmsU rows per pass, their loads issued together (memory-level parallelism).
template <typename T, int LPR, bool ROPE>
__device__ __forceinline__ void rms_fwd_rows(const RmsDev& R) {
    constexpr int E = RVec<T>::n;
    constexpr int RPB = kRmsThreads / LPR;  // row groups per block
    const int sub = threadIdx.x % LPR, rg = threadIdx.x / LPR;
    const int d0 = sub * E;
    const bool dok = d0 < R.dim;
    float w[E];
#pragma unroll
    for (int e = 0; e < E; ++e) w[e] = (R.w && dok) ? load_any(R.w, R.wdt, d0 + e) : 1.f;
    const uint32_t step = gridDim.x * RPB;
    for (uint32_t r0 = blockIdx.x * RPB + rg; r0 < R.rows; r0 += step * kRmsU) {
        float x[kRmsU][E];
        uint32_t b[kRmsU], h[kRmsU], i[kRmsU];
#pragma unroll
        for (int u = 0; u < kRmsU; ++u) {
            const uint32_t r = r0 + u * step;
            row_coords(R, r < R.rows ? r : 0u, b[u], h[u], i[u]);
            load_row<T>(R.x.at<T>(b[u], h[u], i[u]) + d0, dok && r < R.rows, x[u]);
        }
#pragma unroll
        for (int u = 0; u < kRmsU; ++u) {
            const uint32_t r = r0 + u * step;
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) ss += x[u][e] * x[u][e];
            ss = row_sum<LPR>(ss);
            if (r >= R.rows) continue;
            const float rs = rsqrtf(ss * R.inv_dim + R.eps);
            if (dok) {
                float y[E];
#pragma unroll
                for (int e = 0; e < E; ++e) y[e] = (x[u][e] * rs) * w[e];
                if (ROPE && d0 < R.rot_dim) {
                    // the norm output is a tensor of T before the rotation
#pragma unroll
                    for (int e = 0; e < E; ++e) y[e] = round_to<T>(y[e]);
                    rope_fwd<E>(R, i[u], d0, y);
                }
                store_row<T>(R.y.at<T>(b[u], h[u], i[u]) + d0, y);
            }
            if (sub == 0 && R.rstd) R.rstd[rstd_index(R, b[u], h[u], i[u])] = rs;
        }
    }
}

template <typename T, int LPR, bool ROPE>
__global__ __launch_bounds__(kRmsThreads) void k_rms_fwd(RmsDev R) {
    rms_fwd_rows<T, LPR, ROPE>(R);
}

// several norms in one launch (pa_rmsnorm_fwd_many): blockIdx.y selects the tensor
struct RmsMany {
    RmsDev it[PA_RMS_MAX_ITEMS];
};

template <typename T, int LPR>
__global__ __launch_bounds__(kRmsThreads) void k_rms_fwd_many(RmsMany M) {
    rms_fwd_rows<T, LPR, false>(M.it[blockIdx.y]);
}

// dx = rstd * (g - xhat * mean(g * xhat)), g = dy * w, xhat = x * rstd; the block's weight
// gradient partial sum_rows dy * xhat goes to partial[blockIdx.x]
template <typename T, int LPR, bool ROPE>
__global__ __launch_bounds__(kRmsThreads) void k_rms_bwd(RmsDev R) {
    constexpr int E = RVec<T>::n;
    constexpr int RPB = kRmsThreads / LPR;
    __shared__ float s_dw[kRmsThreads / 64][512];
    const int sub = threadIdx.x % LPR, rg = threadIdx.x / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d0 = sub * E;
    const bool dok = d0 < R.dim;
    float w[E], acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        w[e] = (R.w && dok) ? load_any(R.w, R.wdt, d0 + e) : 1.f;
        acc[e] = 0.f;
    }
    const uint32_t step = gridDim.x * RPB;
    for (uint32_t r0 = blockIdx.x * RPB + rg; r0 < R.rows; r0 += step * kRmsU) {
        float x[kRmsU][E], dy[kRmsU][E], rs[kRmsU];
        uint32_t b[kRmsU], h[kRmsU], i[kRmsU];
#pragma unroll
        for (int u = 0; u < kRmsU; ++u) {
            const uint32_t r = r0 + u * step;
            const bool ok = r < R.rows;
            row_coords(R, ok ? r : 0u, b[u], h[u], i[u]);
            load_row<T>(R.x.at<T>(b[u], h[u], i[u]) + d0, dok && ok, x[u]);
            load_row<T>(R.dy.at<T>(b[u], h[u], i[u]) + d0, dok && ok, dy[u]);
            rs[u] = ok ? R.rstd[rstd_index(R, b[u], h[u], i[u])] : 0.f;
        }
        if (ROPE && d0 < R.rot_dim) {
            // back through the rotation: the gradient of the norm output, a tensor of T
#pragma unroll
            for (int u = 0; u < kRmsU; ++u) {
                rope_bwd<E>(R, i[u], d0, dy[u]);
#pragma unroll
                for (int e = 0; e < E; ++e) dy[u][e] = round_to<T>(dy[u][e]);
            }
        }
#pragma unroll
        for (int u = 0; u < kRmsU; ++u) {
            float c = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float xh = x[u][e] * rs[u];
                c += dy[u][e] * w[e] * xh;
                acc[e] += dy[u][e] * xh;
            }
            c = row_sum<LPR>(c) * R.inv_dim;
            if (r0 + u * step < R.rows && dok) {
                float dx[E];
#pragma unroll
                for (int e = 0; e < E; ++e) dx[e] = rs[u] * (dy[u][e] * w[e] - x[u][e] * rs[u] * c);
                store_row<T>(R.dx.at<T>(b[u], h[u], i[u]) + d0, dx);
            }
        }
    }
    if (!R.partial) return;
    // reduce acc over the row groups of the wave (lanes sub, sub + LPR, ...), then the waves
#pragma unroll
    for (int e = 0; e < E; ++e)
        for (int off = LPR; off < 64; off <<= 1) acc[e] += __shfl_xor(acc[e], off);
    if (lane < LPR && dok)
#pragma unroll
        for (int e = 0; e < E; ++e) s_dw[wave][d0 + e] = acc[e];
    __syncthreads();
    for (int f = threadIdx.x; f < R.dim; f += kRmsThreads) {
        float s = 0.f;
#pragma unroll
        for (int v = 0; v < kRmsThreads / 64; ++v) s += s_dw[v][f];
        R.partial[(int64_t)blockIdx.x * R.dim + f] = s;
    }
}

// dw[f] = sum over the nparts partial rows in a fixed order: the 64 lanes of a wave stride
// the partials, then a fixed butterfly; one wave per feature
__global__ __launch_bounds__(kRmsThreads) void k_rms_dw(RmsDev R, int nparts) {
    const int lane = threadIdx.x & 63;
    const int f = blockIdx.x * (kRmsThreads / 64) + (threadIdx.x >> 6);
    if (f >= R.dim) return;
    float s[4] = {0.f, 0.f, 0.f, 0.f};  // independent chains: the loads stay in flight
    int p = lane;
    for (; p + 192 < nparts; p += 256)
#pragma unroll
        for (int k = 0; k < 4; ++k) s[k] += R.partial[(int64_t)(p + 64 * k) * R.dim + f];
    for (; p < nparts; p += 64) s[0] += R.partial[(int64_t)p * R.dim + f];
    float t = (s[0] + s[1]) + (s[2] + s[3]);
    for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off);
    if (lane == 0) R.dw[f] = t;
}

// ---------------------------------------------------------------------------------------

static int rms_blocks(const RmsDev& R) {
    const int64_t rpb = (int64_t)(kRmsThreads / R.lpr) * kRmsU;
    const int64_t need = ((int64_t)R.rows + rpb - 1) / rpb;
    return (int)(need < kRmsMaxBlocks ? need : kRmsMaxBlocks);
}

static int rms_setup(const pa_rmsnorm* p, RmsDev& R, bool bwd) {
    if (p->batch < 1 || p->heads < 1 || p->n < 1 || p->dim < 1) return PA_EINVAL;
    const int T = p->x.dtype;
    if (T != PA_F32 && T != PA_F16 && T != PA_BF16) return PA_EINVAL;
    const int es = T == PA_F32 ? 4 : 2, E = 16 / es;
    if (p->dim % E != 0 || p->dim > 512) return PA_EUNSUPPORTED;
    auto view_ok = [&](const pa_view& v) {
        if (!v.ptr || v.dtype != T || v.heads != p->heads) return false;
        return (uintptr_t)v.ptr % 16 == 0 && v.sb % E == 0 && v.sh % E == 0 && v.sn % E == 0;
    };
    if (!view_ok(p->x)) return PA_EINVAL;
    if (!bwd && !view_ok(p->y)) return PA_EINVAL;
    if (bwd && (!view_ok(p->dy) || !view_ok(p->dx))) return PA_EINVAL;
    if (bwd && !p->rstd) return PA_EINVAL;  // the forward writes it only when given
    if (p->weight && p->weight_dtype != PA_F32 && p->weight_dtype != PA_F16 &&
        p->weight_dtype != PA_BF16)
        return PA_EINVAL;
    if (p->angles && (p->rot_dim < 0 || p->rot_dim > p->dim || p->rot_dim % 2 != 0 ||
                      p->angles_stride < 0 ||
                      (p->angles_dtype != PA_F32 && p->angles_dtype != PA_F16 && p->angles_dtype != PA_BF16)))
        return PA_EINVAL;
    int lpr = 1;
    while (lpr * E < p->dim) lpr <<= 1;
    const int64_t rows = (int64_t)p->batch * p->heads * p->n;
    if (rows >= ((int64_t)1 << 31)) return PA_EUNSUPPORTED;
    auto mk = [](const pa_view& v) {
        RView x;
        x.p = static_cast<char*>(v.ptr);
        x.sb = v.sb;
        x.sh = v.sh;
        x.sn = v.sn;
        return x;
    };
    R.batch = p->batch;
    R.heads = p->heads;
    R.n = p->n;
    R.dim = p->dim;
    R.lpr = lpr;
    R.rows = (uint32_t)rows;
    R.hfast = p->heads > 1 && p->n > 1 && p->x.sh < p->x.sn;
    R.fd_n = make_fastdiv((uint32_t)p->n);
    R.fd_h = make_fastdiv((uint32_t)p->heads);
    R.eps = p->eps;
    R.inv_dim = 1.f / (float)p->dim;
    R.x = mk(p->x);
    R.y = mk(p->y);
    R.dy = mk(p->dy);
    R.dx = mk(p->dx);
    R.w = p->weight;
    R.wdt = p->weight_dtype;
    R.rstd = p->rstd;
    R.partial = nullptr;
    R.dw = p->dweight;
    R.ang = (p->angles && p->rot_dim > 0) ? p->angles : nullptr;
    R.adt = p->angles_dtype;
    R.rot_dim = R.ang ? p->rot_dim : 0;
    R.astride = p->angles_stride;
    return PA_OK;
}

template <typename T, bool ROPE>
static void rms_launch_r(const RmsDev& R, bool bwd, hipStream_t s) {
    const dim3 grid(rms_blocks(R));
#define PA_RMS_CASE(L)                                                                          \
    case L:                                                                                     \
        if (bwd) hipLaunchKernelGGL((k_rms_bwd<T, L, ROPE>), grid, dim3(kRmsThreads), 0, s, R); \
        else hipLaunchKernelGGL((k_rms_fwd<T, L, ROPE>), grid, dim3(kRmsThreads), 0, s, R);     \
        break;
    switch (R.lpr) {
        PA_RMS_CASE(1)
        PA_RMS_CASE(2)
        PA_RMS_CASE(4)
        PA_RMS_CASE(8)
        PA_RMS_CASE(16)
        PA_RMS_CASE(32)
        default: PA_RMS_CASE(64)
    }
#undef PA_RMS_CASE
}

template <typename T>
static void rms_launch(const RmsDev& R, bool bwd, hipStream_t s) {
    if (R.ang) rms_launch_r<T, true>(R, bwd, s);
    else rms_launch_r<T, false>(R, bwd, s);
}

int launch_rms_fwd(const pa_rmsnorm* p, hipStream_t s) {
    RmsDev R;
    const int st = rms_setup(p, R, false);
    if (st != PA_OK) return st;
    ProfScope ps("rms_fwd", s);
    if (p->x.dtype == PA_F32) rms_launch<float>(R, false, s);
    else if (p->x.dtype == PA_F16) rms_launch<f16>(R, false, s);
    else rms_launch<bf16>(R, false, s);
    return PA_OK;
}

int launch_rms_fwd_many(const pa_rmsnorm* items, int count, hipStream_t s) {
    if (!items || count < 1 || count > PA_RMS_MAX_ITEMS) return PA_EINVAL;
    RmsMany M;
    int blocks = 1;
    for (int k = 0; k < count; ++k) {
        const pa_rmsnorm* p = items + k;
        if (p->angles) return PA_EUNSUPPORTED;  // rotary: one pa_rmsnorm_fwd per tensor
        if (p->x.dtype != items[0].x.dtype || p->dim != items[0].dim) return PA_EINVAL;
        const int st = rms_setup(p, M.it[k], false);
        if (st != PA_OK) return st;
        blocks = std::max(blocks, rms_blocks(M.it[k]));
    }
    const dim3 grid(blocks, count);
    ProfScope ps("rms_fwd_many", s);
#define PA_RMS_MANY(T)                                                                        \
    switch (M.it[0].lpr) {                                                                    \
        case 1: hipLaunchKernelGGL((k_rms_fwd_many<T, 1>), grid, dim3(kRmsThreads), 0, s, M); break;   \
        case 2: hipLaunchKernelGGL((k_rms_fwd_many<T, 2>), grid, dim3(kRmsThreads), 0, s, M); break;   \
        case 4: hipLaunchKernelGGL((k_rms_fwd_many<T, 4>), grid, dim3(kRmsThreads), 0, s, M); break;   \
        case 8: hipLaunchKernelGGL((k_rms_fwd_many<T, 8>), grid, dim3(kRmsThreads), 0, s, M); break;   \
        case 16: hipLaunchKernelGGL((k_rms_fwd_many<T, 16>), grid, dim3(kRmsThreads), 0, s, M); break; \
        case 32: hipLaunchKernelGGL((k_rms_fwd_many<T, 32>), grid, dim3(kRmsThreads), 0, s, M); break; \
        default: hipLaunchKernelGGL((k_rms_fwd_many<T, 64>), grid, dim3(kRmsThreads), 0, s, M); break; \
    }
    if (items[0].x.dtype == PA_F32) { PA_RMS_MANY(float) }
    else if (items[0].x.dtype == PA_F16) { PA_RMS_MANY(f16) }
    else { PA_RMS_MANY(bf16) }
#undef PA_RMS_MANY
    return PA_OK;
}

size_t rms_bwd_workspace(const pa_rmsnorm* p) {
    RmsDev R;
    if (rms_setup(p, R, true) != PA_OK) return 0;
    return (size_t)rms_blocks(R) * p->dim * sizeof(float);
}

int launch_rms_bwd(const pa_rmsnorm* p, hipStream_t s) {
    RmsDev R;
    const int st = rms_setup(p, R, true);
    if (st != PA_OK) return st;
    const int nb = rms_blocks(R);
    if (p->dweight) {
        const size_t need = (size_t)nb * p->dim * sizeof(float);
        if (!p->workspace || p->workspace_bytes < need) return PA_EWORKSPACE;
        R.partial = static_cast<float*>(p->workspace);
    }
    {
        ProfScope ps("rms_bwd", s);
        if (p->x.dtype == PA_F32) rms_launch<float>(R, true, s);
        else if (p->x.dtype == PA_F16) rms_launch<f16>(R, true, s);
        else rms_launch<bf16>(R, true, s);
    }
    if (p->dweight) {
        ProfScope ps("rms_dw", s);
        const dim3 grid((p->dim + kRmsThreads / 64 - 1) / (kRmsThreads / 64));
        hipLaunchKernelGGL(k_rms_dw, grid, dim3(kRmsThreads), 0, s, R, nb);
    }
    return PA_OK;
}

}  // namespace pa
