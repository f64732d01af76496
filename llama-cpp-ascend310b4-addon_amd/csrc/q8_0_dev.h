// q8_0_dev.h -- device pieces of the A8W8 (ggml Q8_0) decode kernels shared by the
// per-node launches (q8_0.hip) and the persistent layer pipeline (persist.hip): the
// planar weight layout, the Q8_0 activation quantizer with ggml's two roundings, the
// exact int32 block dot, and the one-row GEMV building blocks (first-pass weight loads,
// the activation staged in LDS, the row dot and its lane reduction).
#pragma once

#include "decode_common.h"

#include <limits.h>

namespace {

using namespace mi;

constexpr int QK = 32;

struct Q8Planes {
    size_t plane;  // bytes of one qs half-plane (256-aligned)
    size_t total;
};

inline Q8Planes q8_planes(int64_t n, int64_t k) {
    const int64_t nb = k / QK;
    Q8Planes p;
    p.plane = align_up((size_t)n * nb * 16, 256);
    p.total = 2 * p.plane + align_up((size_t)n * nb * 2, 256);
    return p;
}

// 8 lanes per 32-block, 4 consecutive values per lane.  Returns the 4 int8 values
// packed in a uint32 and the block scale d (fp32, before fp16 rounding).
__device__ __forceinline__ uint32_t quant4(float v0, float v1, float v2, float v3, int rounding, float &d) {
    float a = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
    const float amax = group_max<8>(a);
    d = amax / 127.0f;
    int q0, q1, q2, q3;
    if (rounding == MI_Q8_ROUND_X86) {
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        q0 = (int)rintf(v0 * id); q1 = (int)rintf(v1 * id);
        q2 = (int)rintf(v2 * id); q3 = (int)rintf(v3 * id);
    } else {
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        q0 = (int)roundf(v0 * id); q1 = (int)roundf(v1 * id);
        q2 = (int)roundf(v2 * id); q3 = (int)roundf(v3 * id);
    }
    return (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
           ((uint32_t)(q3 & 0xff) << 24);
}

// Lane layout (both GEMV kernels): G lanes per output row (power of two),
// RPB = 256/G rows per 256-thread workgroup.  Lane j of a row handles blocks
// b = j, j+G, ..., U of them per pass.  Weight loads use clamped addresses and
// no branches, so all of a pass is in flight at once; the int32 block dots are
// exact (v_dot4_i32_i8) and the fp32 scale d_w*d_x is applied per block.

__device__ __forceinline__ int dot_block(const int4 &l4, const int4 &h4, const int4 &x0, const int4 &x1) {
    int s = 0;
    s = __builtin_amdgcn_sdot4(l4.x, x0.x, s, false);
    s = __builtin_amdgcn_sdot4(l4.y, x0.y, s, false);
    s = __builtin_amdgcn_sdot4(l4.z, x0.z, s, false);
    s = __builtin_amdgcn_sdot4(l4.w, x0.w, s, false);
    s = __builtin_amdgcn_sdot4(h4.x, x1.x, s, false);
    s = __builtin_amdgcn_sdot4(h4.y, x1.y, s, false);
    s = __builtin_amdgcn_sdot4(h4.z, x1.z, s, false);
    s = __builtin_amdgcn_sdot4(h4.w, x1.w, s, false);
    return s;
}

// Up to four Q8_0 matrices of equal k stacked along the output rows (e.g. the
// q/k/v or gate/up projections that read one activation): one launch, one
// activation quantization per workgroup.
struct Q8Set {
    const uint8_t *qlo[4];
    const uint8_t *qhi[4];
    const uint16_t *d[4];
    float *y[4];
    const float *add[4];  // vector added to matrix i's results (bias or residual), or null
    int row_end[4];       // cumulative row counts; unused slots hold INT_MAX
};

__device__ __forceinline__ int q8set_index(const Q8Set &S, int r) {
    return (r >= S.row_end[0]) + (r >= S.row_end[1]) + (r >= S.row_end[2]);
}

__device__ __forceinline__ int q8set_row_start(const Q8Set &S, int i) {
    return i == 0 ? 0 : i == 1 ? S.row_end[0] : i == 2 ? S.row_end[1] : S.row_end[2];
}

// member `f` of slot i, selected once per workgroup with constant indices (the values
// are already in scalar registers; a load from the kernel-argument segment would put its
// latency in front of the first weight loads)
#define Q8SET_PICK(S, f, i) ((i) == 0 ? (S).f[0] : (i) == 1 ? (S).f[1] : (i) == 2 ? (S).f[2] : (S).f[3])

// RMSNorm (optional), then the SmoothQuant reciprocal, then Q8_0 quantization of each
// 32-block into LDS.  The caller puts a barrier between this and the reads of s_qs / s_d.
template <int XN, bool NORM>
__device__ __forceinline__ void xstage_quant(XStage<XN, NORM> &st, const float *__restrict__ inv_s, int k4,
                                             float scale, int rounding, int8_t *s_qs, float *s_d, int tid) {
#pragma unroll
    for (int t = 0; t < XN; t++) {
        const int f = tid + t * 256;  // float4 index; 8 consecutive threads form one 32-block
        float4 v = xstage_value(st, scale, t);
        if (inv_s) { v.x *= st.sv[t].x; v.y *= st.sv[t].y; v.z *= st.sv[t].z; v.w *= st.sv[t].w; }
        float d;
        const uint32_t q = quant4(v.x, v.y, v.z, v.w, rounding, d);
        if (f < k4) {
            *(uint32_t *)(s_qs + (size_t)f * 4) = q;
            if ((f & 7) == 0) s_d[f >> 3] = h2f(f2h(d));
        }
    }
}

// Row dot of one lane over its blocks j, j+G, ...: the first pass's weights were
// loaded by the caller (before the activation staging).
template <int G, int U>
__device__ __forceinline__ float q8_row_dot(const uint8_t *__restrict__ qlo, const uint8_t *__restrict__ qhi,
                                            const uint16_t *__restrict__ wd, size_t rbase, int nb, int j, int4 (&lo)[U],
                                            int4 (&hi)[U], uint32_t (&dw)[U], const int8_t *s_qs, const float *s_d) {
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int b = j + u * G;
        if (b < nb) {
            const int4 *xs = (const int4 *)(s_qs + (size_t)b * QK);
            const int s = dot_block(lo[u], hi[u], xs[0], xs[1]);
            acc = fmaf((float)s, h2f((uint16_t)dw[u]) * s_d[b], acc);
        }
    }
    for (int b0 = U * G; b0 < nb; b0 += U * G) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = min(b0 + j + u * G, nb - 1);
            lo[u] = ld_stream16(qlo + (rbase + b) * 16);
            hi[u] = ld_stream16(qhi + (rbase + b) * 16);
            dw[u] = wd[rbase + b];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = b0 + j + u * G;
            if (b < nb) {
                const int4 *xs = (const int4 *)(s_qs + (size_t)b * QK);
                const int s = dot_block(lo[u], hi[u], xs[0], xs[1]);
                acc = fmaf((float)s, h2f((uint16_t)dw[u]) * s_d[b], acc);
            }
        }
    }
    return group_sum<G>(acc);
}

template <int G, int U>
__device__ __forceinline__ void q8_first_pass(const uint8_t *__restrict__ qlo, const uint8_t *__restrict__ qhi,
                                              const uint16_t *__restrict__ wd, size_t rbase, int nb, int j,
                                              int4 (&lo)[U], int4 (&hi)[U], uint32_t (&dw)[U]) {
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int b = min(j + u * G, nb - 1);
        lo[u] = ld_stream16(qlo + (rbase + b) * 16);
        hi[u] = ld_stream16(qhi + (rbase + b) * 16);
        dw[u] = wd[rbase + b];
    }
}

// LDS layout of the fused kernels: [nb*32 int8 | nb fp32 scales | 4 doubles | 16 floats]
inline size_t fused_smem(int nb) { return align_up((size_t)nb * QK, 16) + align_up((size_t)nb * 4, 16) + 32 + 64; }

struct FusedLds {
    int8_t *qs;
    float *d;
    double *red;
    float *y;
};

__device__ __forceinline__ FusedLds fused_lds(uint8_t *smem, int nb) {
    FusedLds L;
    const size_t o1 = (((size_t)nb * QK + 15) / 16) * 16;
    const size_t o2 = o1 + (((size_t)nb * 4 + 15) / 16) * 16;
    L.qs = (int8_t *)smem;
    L.d = (float *)(smem + o1);
    L.red = (double *)(smem + o2);
    L.y = (float *)(smem + o2 + 32);
    return L;
}

}  // namespace
