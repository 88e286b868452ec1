// pa_mfma.h -- MFMA fragment helpers shared by the gfx950 attention kernels.
//
// All kernels use v_mfma_f32_32x32x16_{bf16,f16}: A is 32 x 16 (lane l holds row l % 32,
// k elements 8*(l/32) .. +7), B is 16 x 32 (lane l holds column l % 32, the same k
// elements), and the 32 x 32 fp32 accumulator gives lane l the column n = l % 32 and the
// rows m(i) = 8*(i/4) + 4*(l/32) + (i%4) for its 16 registers i.
//
// "Transposed-operand" trick used throughout: an accumulator block C (rows m(i) of a lane's
// column) can be fed back as the B operand of a second product over the same row index by
// splitting its 16 registers into two groups of 8 (t = 0, 1); group t then carries the row
// indices 16t + 8*(e/4) + 4*(l/32) + (e%4), e = 0..7, and the matching A operand is read from
// a transposed LDS copy as two 4-element runs at rows 16t + 4*(l/32) and 16t + 8 + 4*(l/32).
#pragma once

#include "pa_common.h"
#include "pa_order.h"

namespace pa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <typename T> struct Mma;
template <> struct Mma<bf16> {
    typedef bf16x8_t frag;
    static __device__ __forceinline__ f32x16_t run(frag a, frag b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mma<f16> {
    typedef f16x8_t frag;
    static __device__ __forceinline__ f32x16_t run(frag a, frag b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

__device__ __forceinline__ f32x16_t zero16() {
    f32x16_t z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

// two floats -> two T (round to nearest even) packed in one 32-bit word (lo = first);
// one v_cvt_pk_{bf16,f16}_f32
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef T t2 __attribute__((ext_vector_type(2)));
    const f2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, t2));
}

// the two T packed in a 32-bit word (lo = first) as floats, in registers (element access
// through a T pointer into a packed register array makes the compiler spill the array to
// scratch memory)
template <typename T>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef T t2 __attribute__((ext_vector_type(2)));
    const f2 f = __builtin_convertvector(__builtin_bit_cast(t2, w), f2);
    lo = f[0];
    hi = f[1];
}

// max / sum with the lane 32 apart (the other half of a 32x32 accumulator column) through
// v_permlane32_swap: lane l ends up with {x[l], x[l ^ 32]} in the two results
__device__ __forceinline__ float xhalf_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Marks a rarely taken uniform branch body: the side-effecting (empty) asm keeps the compiler
// from flattening the branch into unconditionally executed selects.
__device__ __forceinline__ void keep_branch() { asm volatile("" ::: "memory"); }

// the wave index as a scalar value, so conditions built from it compile to scalar branches
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// accumulator registers 8t .. 8t+7 (times `scale`) as a B-operand fragment
template <typename T>
__device__ __forceinline__ typename Mma<T>::frag acc_to_frag(const f32x16_t& c, int t) {
    u32x4_t r;
#pragma unroll
    for (int k = 0; k < 4; ++k) r[k] = pack2<T>(c[8 * t + 2 * k], c[8 * t + 2 * k + 1]);
    return __builtin_bit_cast(typename Mma<T>::frag, r);
}

// acc + lo + hi of a packed pair of T (one v_dot2c_f32_{bf16,f16} against (1, 1))
template <typename T> __device__ __forceinline__ float sum_pair(uint32_t w, float acc);
template <>
__device__ __forceinline__ float sum_pair<bf16>(uint32_t w, float acc) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, w), __builtin_bit_cast(v2, 0x3F803F80u),
                                           acc, false);
}
template <>
__device__ __forceinline__ float sum_pair<f16>(uint32_t w, float acc) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, w), __builtin_bit_cast(v2, 0x3C003C00u), acc,
                                  false);
}

// element-wise product of 8 values rounded to T (the reference multiplies in T)
template <typename T>
__device__ __forceinline__ u32x4_t mul_round8(u32x4_t v, u32x4_t m) {
    const T* pv = reinterpret_cast<const T*>(&v);
    const T* pm = reinterpret_cast<const T*>(&m);
    u32x4_t r;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        r[k] = pack2<T>((float)pv[2 * k] * (float)pm[2 * k],
                        (float)pv[2 * k + 1] * (float)pm[2 * k + 1]);
    return r;
}

// A-operand fragment read as two 4-element runs of a transposed LDS row (see header note)
template <typename T>
__device__ __forceinline__ typename Mma<T>::frag lds_runs(const T* row) {
    const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(row);
    const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(row + 8);
    const u32x4_t v = {lo[0], lo[1], hi[0], hi[1]};
    return __builtin_bit_cast(typename Mma<T>::frag, v);
}

// 16-byte fragment load (LDS or global)
template <typename T>
__device__ __forceinline__ typename Mma<T>::frag ld_frag(const T* p) {
    return __builtin_bit_cast(typename Mma<T>::frag, *reinterpret_cast<const u32x4_t*>(p));
}

// Store a 4-row x 8-column block held as four 16-byte rows (w[r] = row r) transposed:
// dst[(c0 + j) * stride + r] for j = 0..7, r = 0..3, as eight 8-byte stores.
__device__ __forceinline__ void store_block_transposed(const u32x4_t* w, uint16_t* dst,
                                                       int stride) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t w0 = w[0][m], w1 = w[1][m], w2 = w[2][m], w3 = w[3][m];
        u32x2_t even, odd;
        even[0] = (w0 & 0xffffu) | (w1 << 16);
        even[1] = (w2 & 0xffffu) | (w3 << 16);
        odd[0] = (w0 >> 16) | (w1 & 0xffff0000u);
        odd[1] = (w2 >> 16) | (w3 & 0xffff0000u);
        *reinterpret_cast<u32x2_t*>(dst + (2 * m) * stride) = even;
        *reinterpret_cast<u32x2_t*>(dst + (2 * m + 1) * stride) = odd;
    }
}

// ---------------------------------------------------------------------------------------
// Direct global -> LDS loads (buffer_load_dwordx4 ... lds) and transposing LDS reads.
//
// The loads are issued through inline assembly, so the compiler neither sees them nor
// inserts waits for them: kernels that use them count their outstanding vector-memory
// operations themselves (wait_vmcnt) and order LDS with lds_barrier.  The assembly sets M0
// (the LDS destination); no compiler-generated code in these kernels uses M0.

typedef int32_t srd_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef short s16x4_t __attribute__((ext_vector_type(4)));

// raw buffer descriptor over [base, base + bytes): offsets >= bytes read as zeros
__device__ __forceinline__ srd_t make_srd(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    srd_t r;
    r[0] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)a);
    r[1] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)(a >> 32) & 0xffff);  // stride 0
    r[2] = __builtin_amdgcn_readfirstlane((int32_t)bytes);
    r[3] = 0x00020000;  // 32-bit data format
    return r;
}

// byte address of a __shared__ object in LDS
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>((const lds_void*)p);
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// Each active lane loads 16 bytes at byte offset `voff` of the buffer; lane i's bytes land at
// LDS byte address lds + 16 * i (lds uniform across the wave).
__device__ __forceinline__ void dma16(srd_t srd, uint32_t lds, uint32_t voff) {
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds"
                 :
                 : "v"(voff), "s"(lds), "s"(srd)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// a value the compiler must treat as produced here (orders it after preceding volatile ops)
template <typename X>
__device__ __forceinline__ X opaque(X x) {
    asm volatile("" : "+v"(x));
    return x;
}

// wait until at most N vector-memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier for LDS hand-offs: waits for this wave's LDS operations, then s_barrier.
// Unlike __syncthreads it carries no release fence, which on this target would also wait for
// every outstanding global load and so drain a direct-to-LDS prefetch pipeline; the waves'
// buffer_load ... lds transfers are made complete beforehand with wait_vmcnt.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ds_read_b64_tr_b16: the 16 lanes of each quarter-wave address 16 rows R[j] of 4 16-bit
// elements (8 bytes each); lane L of the group receives R[L/4 + 4e][L%4] for e = 0..3.
// Addressing row j = 4 consecutive rows r0 + j/4 at columns c0 + 4*(j%4) therefore hands lane
// L the 4 elements of column c0 + L in rows r0 .. r0+3: a transposed read of a row-major tile.
__device__ __forceinline__ u32x2_t lds_read_tr(const void* p) {
    const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t*)(p));
    return __builtin_bit_cast(u32x2_t, v);
}

// bare v_exp_f32 (2^x; results below 2^-126 flush to 0, which softmax weights tolerate)
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

#ifndef PA_HEAVY_FIRST
#define PA_HEAVY_FIRST 1
#endif

// (unit, rank) of this workgroup (pa_order.h): causal grids heaviest blocks first
template <bool CAUSAL>
__device__ __forceinline__ void block_order(int nblk, int heads, int group, int& unit, int& rank) {
    block_map(blockIdx.x, gridDim.x, nblk, heads, group, CAUSAL && PA_HEAVY_FIRST, unit, rank);
}

static inline bool aligned_rows_host(const DView& v, int elems) {
    return ((uintptr_t)v.p % 16 == 0) && v.sb % elems == 0 && v.sh % elems == 0 &&
           v.sn % elems == 0;
}

}  // namespace pa
