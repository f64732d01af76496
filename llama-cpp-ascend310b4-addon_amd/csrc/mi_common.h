// mi_common.h -- shared device/host helpers for the gfx950 decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "ggml_mi355x_kernels.h"

namespace mi {

constexpr int kWave = 64;

// ---------------------------------------------------------------- errors
void set_error(const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);

#define MI_CHECK_ARG(cond, ...)                 \
    do {                                        \
        if (!(cond)) {                          \
            ::mi::set_error(__VA_ARGS__);       \
            return MI_ERR_ARG;                  \
        }                                       \
    } while (0)

#define MI_CHECK_LAUNCH(what)                                   \
    do {                                                        \
        hipError_t e_ = hipGetLastError();                      \
        if (e_ != hipSuccess) return ::mi::hip_fail(e_, what);  \
    } while (0)

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
inline bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// ---------------------------------------------------------------- device helpers
typedef _Float16 half_t;
typedef half_t half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h2f(uint16_t h) {
    half_t v = __builtin_bit_cast(half_t, h);
    return (float)v;
}

// fp32 -> fp16, round to nearest even, from the already rounded fp32 value: the empty asm
// keeps the compiler from folding the producing multiply or add into a mixed-precision
// v_fma_mixlo_f16 (one rounding straight to fp16, which differs from the fp32-then-fp16
// rounding of ggml's fp32 tensors converted to fp16 in rare double-rounding cases)
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    half_t v = (half_t)f;
    return __builtin_bit_cast(uint16_t, v);
}

__device__ __forceinline__ half2_t u2h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t h22u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// fp32 += a.x*b.x + a.y*b.y with exact fp16 products (v_dot2_f32_f16)
__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(u2h2(a), u2h2(b), c, false);
}

// Products rounded before the add or subtract, as C built with -ffp-contract=off computes
// them (HIP contracts a*b+c into an FMA by default, and its __fmul_rn / __fadd_rn are
// plain operators that do not prevent it).
__device__ __forceinline__ float mul_add_rn(float a, float b, float c) {
#pragma clang fp contract(off)
    return a * b + c;
}
__device__ __forceinline__ float mul_sub_mul_rn(float a, float b, float c, float d) {  // a*b - c*d
#pragma clang fp contract(off)
    return a * b - c * d;
}
__device__ __forceinline__ float mul_add_mul_rn(float a, float b, float c, float d) {  // a*b + c*d
#pragma clang fp contract(off)
    return a * b + c * d;
}
// x*x rounded to float, for sums (double)(x*x) as ggml's rms_norm forms them (a contracted
// fpext(x*x) + sum would square in double)
__device__ __forceinline__ float sq_rn(float a) {
#pragma clang fp contract(off)
    return a * a;
}

// DPP move helpers (row = 16 lanes)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}

constexpr int DPP_QUAD_1032 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_2301 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

// sum over aligned groups of G lanes (G in 1,2,4,8,16,32,64); every lane of the group gets the sum
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += dpp_f<DPP_QUAD_1032>(v);
    if constexpr (G >= 4) v += dpp_f<DPP_QUAD_2301>(v);
    if constexpr (G >= 8) v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    if constexpr (G >= 16) v += dpp_f<DPP_ROW_MIRROR>(v);
    if constexpr (G >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (G >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (G >= 2) v = fmaxf(v, dpp_f<DPP_QUAD_1032>(v));
    if constexpr (G >= 4) v = fmaxf(v, dpp_f<DPP_QUAD_2301>(v));
    if constexpr (G >= 8) v = fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
    if constexpr (G >= 16) v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    if constexpr (G >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    if constexpr (G >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// 64-bit DPP move of a double (both halves through the 32-bit DPP path)
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __builtin_amdgcn_update_dpp(0, p.x, CTRL, 0xf, 0xf, true);
    r.y = __builtin_amdgcn_update_dpp(0, p.y, CTRL, 0xf, 0xf, true);
    return __builtin_bit_cast(double, r);
}

__device__ __forceinline__ double readlane_d(double v, int lane) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __builtin_amdgcn_readlane(p.x, lane);
    r.y = __builtin_amdgcn_readlane(p.y, lane);
    return __builtin_bit_cast(double, r);
}

// Sum of one double per thread over a 256-thread workgroup, in one fixed order (every
// RMSNorm of this library sums its squares through it, so fused and standalone norms
// agree bit for bit): rows of 16 lanes by DPP, the 4 row sums of a wave by readlane,
// the 4 wave sums through s_red[4] after one barrier.  Every thread must call it.
__device__ __forceinline__ double block_sum_d256(double v, double *s_red, int tid) {
    v += dpp_d<DPP_QUAD_1032>(v);
    v += dpp_d<DPP_QUAD_2301>(v);
    v += dpp_d<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_d<DPP_ROW_MIRROR>(v);
    const double w = (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
    if ((tid & 63) == 0) s_red[tid >> 6] = w;
    __syncthreads();
    return (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
}

// Entry i of a 4-entry array member of a by-value kernel argument, indexed through its
// address: one scalar load from the kernel-argument segment (i must be wave-uniform).
// A select between the four entries would cost a compare-and-select chain per use.
template <class T>
__device__ __forceinline__ T karg_at(const T (&a)[4], int i) {
    return (&a[0])[i];
}

// streaming (read-once) 16-byte load of weights
typedef int int4v_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld_stream16(const void *p) {
    const int4v_t v = __builtin_nontemporal_load((const int4v_t *)p);
    return make_int4(v.x, v.y, v.z, v.w);
}

}  // namespace mi
