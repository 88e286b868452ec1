// pa_common.h -- device-side helpers shared by the libpolyattn kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <float.h>
#include <math.h>

#include "polyattn.h"

namespace pa {

typedef __bf16 bf16;
typedef _Float16 f16;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// A score at or below this is "masked" in the reference's finite-fill sense
// (-finfo.max, poly_attention.py:68); normal scores and lse values are far above it.
constexpr float kMaskedThreshold = -1.0e30f;

// ---------------------------------------------------------------------------------------
// element conversions (bf16 / f16 rounding is round-to-nearest-even, as torch's casts)
template <typename T> __device__ __forceinline__ float to_f(T x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }
template <typename T> __device__ __forceinline__ float round_to(float x) { return (float)(T)x; }

__device__ __forceinline__ float load_any(const void* p, int dtype, int64_t off) {
    if (dtype == PA_F32) return ((const float*)p)[off];
    if (dtype == PA_F16) return (float)((const f16*)p)[off];
    return (float)((const bf16*)p)[off];
}
__device__ __forceinline__ void store_any(void* p, int dtype, int64_t off, float v) {
    if (dtype == PA_F32) ((float*)p)[off] = v;
    else if (dtype == PA_F16) ((f16*)p)[off] = (f16)v;
    else ((bf16*)p)[off] = (bf16)v;
}

// ---------------------------------------------------------------------------------------
// A view as the kernels see it: hdiv = (pass head count) / (this tensor's head count).
struct DView {
    char* p;
    int64_t sb, sh, sn;
    int32_t hdiv;
    int32_t dtype;
    __host__ __device__ __forceinline__ bool ok() const { return p != nullptr; }
    __device__ __forceinline__ int64_t idx(int b, int h, int64_t n) const {
        return (int64_t)b * sb + (int64_t)(h / hdiv) * sh + n * sn;
    }
    template <typename T> __device__ __forceinline__ const T* row(int b, int h, int64_t n) const {
        return reinterpret_cast<const T*>(p) + idx(b, h, n);
    }
    template <typename T> __device__ __forceinline__ T* wrow(int b, int h, int64_t n) const {
        return reinterpret_cast<T*>(p) + idx(b, h, n);
    }
    __device__ __forceinline__ float scalar(int b, int h, int64_t n) const {
        return load_any(p, dtype, idx(b, h, n));
    }
};

struct DMask {
    const uint8_t* p;
    int64_t sb, sn;
    __device__ __forceinline__ bool keep(int b, int64_t n) const {
        return p == nullptr || p[(int64_t)b * sb + n * sn] != 0;
    }
};

// All the geometry of one pass, as passed to every pass kernel (by value).
struct PassDev {
    int32_t batch, heads, nq, nk, dim;
    float scale, softclamp;
    int32_t causal, flags;
    DView q, k, v, vmul, bias, out, lse;
    DMask km, qm;
    DView er, eg, ey;  // module epilogue: root, gate, y (ey absent: no epilogue)
    int32_t eflags;    // PA_EPI_*
    // RMSNorm of the queries / keys on load (PA_NORM_* in nflags; weights of the pass dtype)
    const void* qnw;
    const void* knw;
    float qeps, keps;
    int32_t nflags;
    // masked passes on the MFMA kernels: per (b, key head) [first, last + 1) of the keys that
    // can enter a normal row (kept, key bias of class 0), or null
    const int32_t* live;
};

struct GradDev {
    PassDev f;
    DView dout, dlse, dq, dk, dv, dvmul, dbias;
    DView droot, dgate;    // epilogue input gradients (with f.ey)
    int32_t accumulate;
    int32_t hk;            // key-side head count (k, v, vmul, bias share it)
    float* ws_D;           // [B, heads, nq]  rowsum(dO * O) - dlse
    float* ws_lse;         // [B, heads, nq]  lse for normal rows, +inf for degenerate rows
    float* ws_invc;        // [B, heads, nq]  1 / (#class-1 keys) for degenerate rows, else 0
    int32_t fused_pre;     // the dQ kernel computes ws_D / ws_lse for its rows (no preprocess)
    int32_t seeds;         // with fused_pre: ws_lse / ws_D hold the dK/dV kernel's accumulator
                           // seeds, -lse/scale (lse*log2e with softclamp) and -D
    // masked passes on the MFMA kernels (null otherwise)
    const int32_t* ws_kcnt;  // [B, hk, 2]: keys of bias class 0 and of bias class 1
    float* ws_part;          // [B, heads, chunks, dim + 2]: over the fully-masked rows of a
                             // chunk of kFixRowChunk rows of a head, sum dO / c1, sum D / c1
                             // and their number
};

// rows per partial sum of the masked backward's fully-masked rows (GradDev::ws_part)
constexpr int kFixRowChunk = 512;
__host__ __device__ inline int fix_row_chunks(int nq) { return (nq + kFixRowChunk - 1) / kFixRowChunk; }

__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }

// The module epilogue of one output element o (already rounded to T) from its raw root and
// gate values, in torch's order: t = round(r * o) with r = root or round(sigmoid(root)),
// y = round(t * round(sigmoid(gate))); an absent factor is skipped.
template <typename T>
__device__ __forceinline__ float epi_combine(float o, float root, float gate, bool has_r,
                                             bool has_g, bool sig) {
    float t = o;
    if (has_r) t = round_to<T>((sig ? round_to<T>(sigmoid_f(root)) : root) * t);
    if (has_g) t = round_to<T>(t * round_to<T>(sigmoid_f(gate)));
    return t;
}
template <typename T>
__device__ __forceinline__ float epi_y(const PassDev& P, int b, int h, int64_t i, int d, float o) {
    const float r = P.er.ok() ? to_f(P.er.row<T>(b, h, i)[d]) : 0.f;
    const float g = P.eg.ok() ? to_f(P.eg.row<T>(b, h, i)[d]) : 0.f;
    return epi_combine<T>(o, r, g, P.er.ok(), P.eg.ok(), (P.eflags & PA_EPI_ROOT_SIGMOID) != 0);
}

// class of a bias value in the finite-fill arithmetic: 0 normal, 1 = -FLT_MAX, 2 = -inf
__device__ __forceinline__ int bias_class(float x) {
    return x == -INFINITY ? 2 : (x <= kMaskedThreshold ? 1 : 0);
}

__device__ __forceinline__ float softclamp_f(float x, float c) {
    return c > 0.f ? c * tanhf(x / c) : x;
}
// d softclamp(x) / dx expressed through y = softclamp(x)
__device__ __forceinline__ float softclamp_grad(float y, float c) {
    if (c <= 0.f) return 1.f;
    float t = y / c;
    return 1.f - t * t;
}

}  // namespace pa
