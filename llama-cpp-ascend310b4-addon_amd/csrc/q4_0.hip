// q4_0.hip -- W4A16 decode GEMV for gfx950: ggml Q4_0 weights (int4, group 32,
// offset 8, fp16 group scale) times an fp16 activation row, fp32 accumulation.
//
// Nibbles are turned into exact fp16 values (nib - 8) with a magic-exponent
// OR (0x6400 | nib == 1024 + nib) and one packed fp16 subtract, then reduced
// with v_dot2_f32_f16 (exact fp16 products, fp32 accumulation); the group
// scale is applied once per 32-group, as the reference operator does
// (experiments/w4a16-gemv/source/w4a16_gemv_qwen.cpp:127-148).
// Replaces the add-on's add_custom W4A16 operator (same file, :24-180).
#include "mi_common.h"
#include "decode_common.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <unordered_map>

namespace {

using namespace mi;

constexpr int QK = 32;

struct Q4Planes {
    size_t plane;
    size_t total;
};

inline Q4Planes q4_planes(int64_t n, int64_t k) {
    const int64_t nb = k / QK;
    Q4Planes p;
    p.plane = align_up((size_t)n * nb * 16, 256);
    p.total = p.plane + align_up((size_t)n * nb * 2, 256);
    return p;
}

__global__ void k_prepack_q4_0(const uint8_t *__restrict__ src, uint8_t *__restrict__ qs, uint16_t *__restrict__ dpl,
                               int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint16_t *s = (const uint16_t *)(src + i * 18);
    uint16_t w[9];
#pragma unroll
    for (int t = 0; t < 9; t++) w[t] = s[t];
    *(uint4 *)(qs + i * 16) = make_uint4((uint32_t)w[1] | ((uint32_t)w[2] << 16), (uint32_t)w[3] | ((uint32_t)w[4] << 16),
                                         (uint32_t)w[5] | ((uint32_t)w[6] << 16), (uint32_t)w[7] | ((uint32_t)w[8] << 16));
    dpl[i] = w[0];
}

// dword t of a Q4_0 block holds elements 4t..4t+3 (low nibbles) and 16+4t..16+4t+3 (high nibbles)
__device__ __forceinline__ float q4_block_dot(const int4 q, const uint32_t *xs /* 16 half2 of the block */) {
    const half2_t off = {(half_t)1032.0f, (half_t)1032.0f};
    float s = 0.0f;
    const uint32_t qq[4] = {(uint32_t)q.x, (uint32_t)q.y, (uint32_t)q.z, (uint32_t)q.w};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t v = qq[t];
        const uint32_t lo01 = 0x64006400u | (v & 0xfu) | ((v & 0xf00u) << 8);
        const uint32_t lo23 = 0x64006400u | ((v >> 16) & 0xfu) | ((v >> 8) & 0xf0000u);
        const uint32_t hi01 = 0x64006400u | ((v >> 4) & 0xfu) | ((v << 4) & 0xf0000u);
        const uint32_t hi23 = 0x64006400u | ((v >> 20) & 0xfu) | ((v >> 12) & 0xf0000u);
        s = fdot2(h22u(u2h2(lo01) - off), xs[2 * t], s);
        s = fdot2(h22u(u2h2(lo23) - off), xs[2 * t + 1], s);
        s = fdot2(h22u(u2h2(hi01) - off), xs[8 + 2 * t], s);
        s = fdot2(h22u(u2h2(hi23) - off), xs[8 + 2 * t + 1], s);
    }
    return s;
}

// G lanes per output row; lane j owns blocks j, j+G, ... (U per pass, loads
// branch-free with clamped addresses); the fp16 activation rows are staged in LDS.
template <int G, int U, int M, bool F32X>
__global__ __launch_bounds__(256) void k_gemv_q4_0(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ wd,
                                                   const uint16_t *__restrict__ x16, const float *__restrict__ x32,
                                                   float *__restrict__ y, int n, int nb, int m) {
    constexpr int RPB = 256 / G;
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t *s_x = (uint16_t *)smem;  // [M][k]
    const int tid = threadIdx.x;
    const int j = tid % G;
    const int row = blockIdx.x * RPB + tid / G;
    const bool row_ok = row < n;
    const int k = nb * QK;
    const size_t rbase = (size_t)min(row, n - 1) * nb;

    int4 wq[U];
    uint32_t dw[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int b = min(j + u * G, nb - 1);
        wq[u] = ld_stream16(qs + (rbase + b) * 16);
        dw[u] = wd[rbase + b];
    }

    if constexpr (F32X) {
        for (int i = tid * 4; i < m * k; i += 256 * 4) {
            const float4 v = *(const float4 *)(x32 + i);
            *(uint2 *)(s_x + i) = make_uint2((uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16),
                                             (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16));
        }
    } else {
        for (int i = tid * 8; i < m * k; i += 256 * 8) *(int4 *)(s_x + i) = *(const int4 *)(x16 + i);
    }
    __syncthreads();

    float acc[M];
#pragma unroll
    for (int i = 0; i < M; i++) acc[i] = 0.0f;

    auto consume = [&](int b, const int4 &q4, uint32_t dbits) {
        const float d = h2f((uint16_t)dbits);
#pragma unroll
        for (int i = 0; i < M; i++) {
            if (i < m) {
                const int4 *xp = (const int4 *)(s_x + (size_t)i * k + b * QK);
                uint32_t xs[16];
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int4 t = xp[c];
                    xs[4 * c + 0] = (uint32_t)t.x; xs[4 * c + 1] = (uint32_t)t.y;
                    xs[4 * c + 2] = (uint32_t)t.z; xs[4 * c + 3] = (uint32_t)t.w;
                }
                acc[i] = fmaf(d, q4_block_dot(q4, xs), acc[i]);
            }
        }
    };

#pragma unroll
    for (int u = 0; u < U; u++) {
        const int b = j + u * G;
        if (b < nb) consume(b, wq[u], dw[u]);
    }
    for (int b0 = U * G; b0 < nb; b0 += U * G) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = min(b0 + j + u * G, nb - 1);
            wq[u] = ld_stream16(qs + (rbase + b) * 16);
            dw[u] = wd[rbase + b];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = b0 + j + u * G;
            if (b < nb) consume(b, wq[u], dw[u]);
        }
    }

#pragma unroll
    for (int i = 0; i < M; i++) {
        const float s = group_sum<G>(acc[i]);
        if (row_ok && j == 0 && i < m) y[(size_t)i * n + row] = s;
    }
}

// fp16 activations read straight from global memory (2*k bytes per row, L1/L2
// resident and shared by every workgroup): no LDS staging, no barrier.  R rows per
// lane group (rows r, r + 256/G, ...) reuse each activation chunk R times.
template <int G, int U, int M, int R>
__global__ __launch_bounds__(256) void k_gemv_q4_0_gx(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ wd,
                                                      const uint16_t *__restrict__ x16, float *__restrict__ y,
                                                      const float *__restrict__ add, int n, int nb, int m) {
    constexpr int RG = 256 / G;
    const int tid = threadIdx.x;
    const int j = tid % G;
    const int row0 = blockIdx.x * RG * R + tid / G;
    const int k = nb * QK;
    size_t rb[R];
#pragma unroll
    for (int r = 0; r < R; r++) rb[r] = (size_t)min(row0 + r * RG, n - 1) * nb;

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int i = 0; i < M; i++) acc[r][i] = 0.0f;

    for (int b0 = 0; b0 < nb; b0 += U * G) {
        int4 wq[U][R];
        uint32_t dw[U][R];
        int4 xv[U][M][4];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = min(b0 + j + u * G, nb - 1);
#pragma unroll
            for (int r = 0; r < R; r++) {
                wq[u][r] = ld_stream16(qs + (rb[r] + b) * 16);
                dw[u][r] = wd[rb[r] + b];
            }
#pragma unroll
            for (int i = 0; i < M; i++) {
                const int4 *xp = (const int4 *)(x16 + (size_t)min(i, m - 1) * k + (size_t)b * QK);
#pragma unroll
                for (int c = 0; c < 4; c++) xv[u][i][c] = xp[c];
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (b0 + j + u * G < nb) {
#pragma unroll
                for (int i = 0; i < M; i++) {
                    uint32_t xs[16];
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        xs[4 * c + 0] = (uint32_t)xv[u][i][c].x; xs[4 * c + 1] = (uint32_t)xv[u][i][c].y;
                        xs[4 * c + 2] = (uint32_t)xv[u][i][c].z; xs[4 * c + 3] = (uint32_t)xv[u][i][c].w;
                    }
#pragma unroll
                    for (int r = 0; r < R; r++)
                        acc[r][i] = fmaf(h2f((uint16_t)dw[u][r]), q4_block_dot(wq[u][r], xs), acc[r][i]);
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r * RG;
#pragma unroll
        for (int i = 0; i < M; i++) {
            const float s = group_sum<G>(acc[r][i]);
            if (row < n && j == 0 && i < m) y[(size_t)i * n + row] = add ? s + add[(size_t)i * n + row] : s;
        }
    }
}

// Several activation rows (2..16: a batch of sequences) on the matrix cores:
// v_mfma_f32_16x16x16_f16 with A = 16 weight rows x 16 k and B = 16 k x the
// activation rows (columns past m are zero).  Lane (g, c) of a wave loads one dword
// of block b of weight row c: bytes 4g..4g+3 hold elements 4g..4g+3 (low nibbles,
// the first k-step) and 16+4g..16+4g+3 (high nibbles, the second), turned into exact
// fp16 (nib - 8).  The two MFMAs give the block's exact-product fp32 partial for 16
// rows x 16 columns; it is scaled by the block scale of its row and accumulated.  The
// C layout puts rows 4g..4g+3 and column c in lane (g, c).  KS waves of a workgroup
// split k (partials reduced through LDS); with KS = 1 each wave owns 16 rows.
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half4_t q4_nibbles(uint32_t v, int hi) {
    const uint32_t s = hi ? v >> 4 : v;
    const uint32_t p01 = 0x64006400u | (s & 0xfu) | ((s & 0xf00u) << 8);
    const uint32_t p23 = 0x64006400u | ((s >> 16) & 0xfu) | ((s >> 8) & 0xf0000u);
    const half2_t off = {(half_t)1032.0f, (half_t)1032.0f};
    const half2_t a = u2h2(p01) - off, b = u2h2(p23) - off;
    return half4_t{a.x, a.y, b.x, b.y};
}

template <int U>
struct Q4MStage {
    uint32_t w[U];
    uint32_t d[U][4];  // fp16 scales of the lane's 4 output rows
    half4_t x0[U], x1[U];
};

template <int KS, int U, bool XF32>
__global__ __launch_bounds__(64 * KS) void k_gemv_q4_0_mfma(const uint8_t *__restrict__ qs,
                                                             const uint16_t *__restrict__ wd,
                                                             const void *__restrict__ xin, float *__restrict__ y,
                                                             const float *__restrict__ add, int n, int nb, int m) {
    __shared__ float s_acc[KS][64][4];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int row0 = blockIdx.x * 16;
    const int k = nb * QK;
    const int per = (nb + KS - 1) / KS;  // k range of this wave, in blocks
    const int b_lo = wave * per, b_hi = min(nb, b_lo + per);
    const size_t arow = (size_t)min(row0 + c, n - 1) * nb;
    size_t drow[4];
#pragma unroll
    for (int i = 0; i < 4; i++) drow[i] = (size_t)min(row0 + 4 * g + i, n - 1) * nb;
    const bool col_ok = c < m;
    const size_t xoff = (size_t)min(c, m - 1) * k + 4 * g;

    auto load = [&](Q4MStage<U> &st, int b0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = min(b0 + u, b_hi - 1);
            st.w[u] = *(const uint32_t *)(qs + (arow + b) * 16 + 4 * g);
#pragma unroll
            for (int i = 0; i < 4; i++) st.d[u][i] = wd[drow[i] + b];
            if constexpr (XF32) {
                // fp32 activation rounded to fp16 (RNE) as ggml converts src1
                const float *xr = (const float *)xin + xoff + (size_t)b * QK;
                const float4 a0 = *(const float4 *)xr, a1 = *(const float4 *)(xr + 16);
                st.x0[u] = half4_t{(half_t)a0.x, (half_t)a0.y, (half_t)a0.z, (half_t)a0.w};
                st.x1[u] = half4_t{(half_t)a1.x, (half_t)a1.y, (half_t)a1.z, (half_t)a1.w};
            } else {
                const uint16_t *xr = (const uint16_t *)xin + xoff + (size_t)b * QK;
                st.x0[u] = __builtin_bit_cast(half4_t, *(const uint2 *)xr);
                st.x1[u] = __builtin_bit_cast(half4_t, *(const uint2 *)(xr + 16));
            }
        }
    };
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Q4MStage<U> &st, int b0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (b0 + u < b_hi) {
                float4_t t = {0.f, 0.f, 0.f, 0.f};
                const half4_t z = {0, 0, 0, 0};
                t = __builtin_amdgcn_mfma_f32_16x16x16f16(q4_nibbles(st.w[u], 0), col_ok ? st.x0[u] : z, t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x16f16(q4_nibbles(st.w[u], 1), col_ok ? st.x1[u] : z, t, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = fmaf(h2f((uint16_t)st.d[u][i]), t[i], acc[i]);
            }
        }
    };
    if (b_lo < b_hi) {
        // two register stages: the next U blocks are in flight while the current ones compute
        Q4MStage<U> sa, sb;
        load(sa, b_lo);
        for (int b0 = b_lo; b0 < b_hi; b0 += 2 * U) {
            if (b0 + U < b_hi) load(sb, b0 + U);
            compute(sa, b0);
            if (b0 + U >= b_hi) break;
            if (b0 + 2 * U < b_hi) load(sa, b0 + 2 * U);
            compute(sb, b0 + U);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) s_acc[wave][lane][i] = acc[i];
    __syncthreads();
    if (wave != 0 || !col_ok) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < KS; w++) v += s_acc[w][lane][i];
        const int row = row0 + 4 * g + i;
        if (row < n) {
            const size_t o = (size_t)c * n + row;
            y[o] = add ? v + add[o] : v;
        }
    }
}

// Selecting a matrix's pointer once at a workgroup's start: the four candidates pass
// through an empty asm statement first, so the select works on values already in scalar
// registers.  Without it the compiler turns the select into a load from a computed
// kernel-argument address, whose latency then sits in front of the first weight loads
// (karg_at makes that load on purpose where a selection repeats inside a loop).
template <class T>
__device__ __forceinline__ T opaque_s(T v) {
    if constexpr (sizeof(T) == 8) {
        uint64_t u = (uint64_t)v;
        asm volatile("" : "+s"(u));
        return (T)u;
    } else {
        uint32_t u = (uint32_t)v;
        asm volatile("" : "+s"(u));
        return (T)u;
    }
}

template <class T>
__device__ __forceinline__ T pick4(int i, T a0, T a1, T a2, T a3) {
    return i >= 3 ? a3 : i >= 2 ? a2 : i >= 1 ? a1 : a0;
}

// global-address-space accesses from integer addresses (the picked pointers are
// plain integers after the register select; a generic pointer would give flat loads,
// which also count against the LDS counter)
#define MI_GLOBAL __attribute__((address_space(1)))
__device__ __forceinline__ int4 ldg_stream16(uint64_t a) {
    const int4v_t v = __builtin_nontemporal_load((const MI_GLOBAL int4v_t *)a);
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ldg_u16(uint64_t a) { return *(const MI_GLOBAL uint16_t *)a; }
__device__ __forceinline__ float ldg_f32(uint64_t a) { return *(const MI_GLOBAL float *)a; }
__device__ __forceinline__ void stg_f32(uint64_t a, float v) { *(MI_GLOBAL float *)a = v; }
__device__ __forceinline__ void stg_u16(uint64_t a, uint16_t v) { *(MI_GLOBAL uint16_t *)a = v; }
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ldg_u4(uint64_t a) {
    const u32x4_t v = *(const MI_GLOBAL u32x4_t *)a;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldg_u2(uint64_t a) {
    const u32x2_t v = *(const MI_GLOBAL u32x2_t *)a;
    return make_uint2(v.x, v.y);
}

// Several activation rows on the matrix cores with the activation as the A operand:
// D[16 rows of x][16 weight rows] += X[16 x 32 k] . W^T[32 k x 16 weight rows], one
// v_mfma_f32_16x16x32_f16 per block.  Lane (g, c) supplies dword g of a block of weight
// row c (k slots 0..3 its low nibbles, 4..7 its high nibbles) and the activation row c's
// matching values; it receives weight row c's results for activation rows 4g..4g+3, so
// it applies one block scale (row c's) per block.  The activation comes converted to fp16 in the
// order in which a weight dword's nibbles come out (see q4_dot_xr):
//   xp[row][block][g][8] = x[4g], x[4g+2], x[4g+1], x[4g+3], x[16+4g], x[18+4g], x[17+4g], x[19+4g]
// one 16-byte load per block.  k is split over KS waves (partials reduced in LDS).
// activation sources of k_perm_f16
constexpr int PERM_F16 = 0;   // fp16 rows
constexpr int PERM_F32 = 1;   // fp32 rows, rounded to fp16 (RNE) as ggml converts src1
constexpr int PERM_GLU = 2;   // fp32 gate and up rows: fp16(silu(g) * u), ggml swiglu then the conversion
constexpr int PERM_READY = 3; // the activation arrives converted and permuted (no conversion launch)

template <int MODE>
__global__ __launch_bounds__(256) void k_perm_f16(const void *__restrict__ x, const float *__restrict__ up,
                                                  uint4 *__restrict__ xp, int m, int nb) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (row, block, g)
    if (i >= (int64_t)m * nb * 4) return;
    const int g = (int)(i & 3);
    const int64_t rb = i >> 2;  // row * nb + block
    uint16_t h[8];
    const int idx[8] = {4 * g, 4 * g + 2, 4 * g + 1, 4 * g + 3, 16 + 4 * g, 18 + 4 * g, 17 + 4 * g, 19 + 4 * g};
    if constexpr (MODE == PERM_F32) {
        const float *xb = (const float *)x + rb * QK;
#pragma unroll
        for (int j = 0; j < 8; j++) h[j] = f2h(xb[idx[j]]);
    } else if constexpr (MODE == PERM_GLU) {
        const float *gb = (const float *)x + rb * QK;
        const float *ub = up + rb * QK;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float gv = gb[idx[j]];
            h[j] = f2h((gv / (1.0f + expf(-gv))) * ub[idx[j]]);
        }
    } else {
        const uint16_t *xb = (const uint16_t *)x + rb * QK;
#pragma unroll
        for (int j = 0; j < 8; j++) h[j] = xb[idx[j]];
    }
    xp[i] = make_uint4((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16),
                       (uint32_t)h[4] | ((uint32_t)h[5] << 16), (uint32_t)h[6] | ((uint32_t)h[7] << 16));
}

// RMS_NORM -> MUL(w) of each activation row, then the permuted fp16 conversion of
// k_perm_f16: one workgroup per row forms the row's scale with the loads, order and
// reduction of the RMSNorm kernel's vector path (k <= 4096), then converts
// (x * scale) * w, as that kernel writes it and the matmul converts it.
__global__ __launch_bounds__(256) void k_perm_norm_f16(const float *__restrict__ x, const float *__restrict__ w,
                                                       float eps, uint4 *__restrict__ xp, int nb) {
    const int row = blockIdx.x, tid = threadIdx.x;
    const int ne0 = nb * QK, n4 = ne0 / 4;
    const float *xr = x + (size_t)row * ne0;
    __shared__ double s_red[4];
    __shared__ uint2 s_h[1024];  // the converted row, 4 halves per float4
    float4 xv[4], wv[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int f = min(tid + t * 256, n4 - 1);
        xv[t] = ((const float4 *)xr)[f];
        wv[t] = ((const float4 *)w)[f];
    }
    double s = 0.0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        if (tid + t * 256 < n4) {
            s += (double)sq_rn(xv[t].x);
            s += (double)sq_rn(xv[t].y);
            s += (double)sq_rn(xv[t].z);
            s += (double)sq_rn(xv[t].w);
        }
    }
    const double tot = block_sum_d256(s, s_red, tid);
    const float mean = (float)(tot / ne0);
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int f = tid + t * 256;
        if (f < n4) {
            const float4 v = xv[t];
            const uint32_t h0 = f2h((v.x * scale) * wv[t].x), h1 = f2h((v.y * scale) * wv[t].y);
            const uint32_t h2 = f2h((v.z * scale) * wv[t].z), h3 = f2h((v.w * scale) * wv[t].w);
            s_h[f] = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
        }
    }
    __syncthreads();
    // unit (block b, slot g): halves 4g, 4g+2, 4g+1, 4g+3 and the same + 16 (float4s 8b+g, 8b+4+g)
    for (int u = tid; u < nb * 4; u += 256) {
        const int g = u & 3, b = u >> 2;
        const uint2 lo = s_h[8 * b + g], hi = s_h[8 * b + 4 + g];
        xp[(size_t)row * nb * 4 + u] =
            make_uint4((lo.x & 0xffffu) | (lo.y << 16), (lo.x >> 16) | (lo.y & 0xffff0000u),
                       (hi.x & 0xffffu) | (hi.y << 16), (hi.x >> 16) | (hi.y & 0xffff0000u));
    }
}

// Matrices of one batched launch (equal k, one activation): workgroups [wg_end[i-1],
// wg_end[i]) take matrix i's tiles.  Per output row: y = W x (+ bias[row]) (+ add[r][row]),
// bias broadcast over the activation rows (ggml ADD of a bias row), add a full [m][n]
// tensor (the residual).
struct Q4BSet {
    const uint8_t *qs[4];
    const uint16_t *wd[4];
    float *y[4];
    const float *bias[4];
    const float *add[4];
    int n[4];
    int wg_end[4];  // cumulative workgroup counts; unused slots INT_MAX
    uint16_t *hxp;  // GLU pairs: the swiglu rows as the next projection's permuted fp16 activation
};

// RoPE pairs: the attention-input tail of a q/k/v set (matrices 0, 1, 2), per activation
// row r: neox rotation of q and k by pos[r], q to q_out, the rotated k and v as fp16 into
// cache row kv_idx[r]
struct Q4BRope {
    float *q_out;
    uint8_t *kc, *vc;
    const int32_t *pos;
    const void *kv_idx;
    int kv_i64;
    int hd;
    size_t k_row_bytes, v_row_bytes;
    int64_t n_cache_rows;
    float theta_scale, freq_scale, attn_factor;
};
constexpr int PAIR_NONE = 0, PAIR_GLU = 1, PAIR_ROPE = 2;

// selected once per workgroup: a register select (see opaque_s), not a kernel-argument
// load whose latency would sit in front of the first weight loads
#define Q4B_PICK(S, f, i) \
    pick4((i), opaque_s((S).f[0]), opaque_s((S).f[1]), opaque_s((S).f[2]), opaque_s((S).f[3]))

// Groups of 4 blocks: lane (g, c) loads block 4j+g of weight row c whole (16 bytes; the
// 4 g-lanes of a row read 64 contiguous bytes) and the 4 scales of row c's group (8
// bytes; with SP the 8 scales of the stage's two groups in one 16-byte load).  A 4x4
// dword transpose through the wave's LDS slot then gives lane (g, c) dword g of each of
// the group's 4 blocks, the operand the matrix core wants.
template <int UG, int TW, bool SP>
struct Q4XStage {
    uint4 w[UG][TW];   // block 4j+g of row c of each tile
    uint2 d[UG][TW];   // fp16 scales of row c, blocks 4j..4j+3, of each tile (without SP)
    uint4 dp[TW];      // fp16 scales of row c, blocks 4jp..4jp+7 (with SP)
    uint4 x[UG][4];    // activation row c, blocks 4j..4j+3, slot g (shared by the tiles)
};

// TW 16-row tiles per wave share each activation load; k is split over KS waves.  A
// matrix's tiles never straddle into the next matrix (n[i] % (16*TW) == 0 but for the
// last).  SP (two groups per stage, at least two groups per row) loads the scales of a
// stage's groups j0, j0+1 together from group jp = min(j0, ng - 2), which stays inside
// the row.  Pairs (TW = 2) put two related row tiles in one workgroup:
// - PAIR_GLU (matrices 0 and 1 of n rows each: gate and up): tile 0 is gate rows 16b..,
//   tile 1 the same up rows, and the epilogue writes fp16(silu(gate) * up), ggml's swiglu
//   then the src1 conversion, into S.hxp in the permuted block layout of the activation
//   (the next projection's input, k = n);
// - PAIR_ROPE (q, k, v of a q/k/v set, heads of hd rows): for q and k, tile 0 is dims
//   16t.. of a head and tile 1 dims hd/2 + 16t.., so a lane holds both members of its
//   rotation pairs; v takes 32 consecutive rows.  The epilogue adds the bias, rotates as
//   the rope + cache-write kernel does and writes q_out and the k / v cache rows.
template <int KS, int UG, int TW, bool SP, int PAIR = PAIR_NONE>
__global__ __launch_bounds__(64 * KS) void k_gemv_q4_0_mfma_x(const Q4BSet S, const uint4 *__restrict__ xp, int nb,
                                                              int m, const Q4BRope RP) {
    constexpr bool GLU = PAIR == PAIR_GLU, ROPE = PAIR == PAIR_ROPE;
    __shared__ float s_acc[KS][TW][64][4];
    __shared__ uint32_t s_t[KS][16][4][4];  // per wave: [row c][dword][block in group]
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int b = blockIdx.x;
    static_assert(PAIR == PAIR_NONE || TW == 2, "a pair is two tiles");
    const int mi = GLU ? 0 : (b >= S.wg_end[0]) + (b >= S.wg_end[1]) + (b >= S.wg_end[2]);
    const int wg0 = GLU ? 0 : pick4(mi, 0, opaque_s(S.wg_end[0]), opaque_s(S.wg_end[1]), opaque_s(S.wg_end[2]));
    const int n = Q4B_PICK(S, n, mi);
    uint64_t qsb[TW], wdb[TW];  // each tile's matrix (the same one but for GLU pairs)
#pragma unroll
    for (int t = 0; t < TW; t++) {
        qsb[t] = (uint64_t)(GLU ? S.qs[t] : Q4B_PICK(S, qs, mi));
        wdb[t] = (uint64_t)(GLU ? S.wd[t] : Q4B_PICK(S, wd, mi));
    }
    // first row of each tile
    int trow[TW];
    const int wi = b - wg0;
#pragma unroll
    for (int t = 0; t < TW; t++) {
        if constexpr (GLU) {
            trow[t] = b * 16;
        } else if constexpr (ROPE) {
            const int tph = RP.hd / 32;  // workgroups per head
            trow[t] = mi < 2 ? (wi / tph) * RP.hd + 16 * (wi % tph) + t * (RP.hd / 2) : wi * 32 + 16 * t;
        } else {
            trow[t] = wi * 16 * TW + 16 * t;
        }
    }
    const int ng = nb / 4;               // whole groups (nb % 4 == 0)
    const int per = (ng + KS - 1) / KS;  // groups of this wave
    const int j_lo = wave * per, j_hi = min(ng, j_lo + per);
    uint64_t wrow[TW];
#pragma unroll
    for (int t = 0; t < TW; t++) wrow[t] = (uint64_t)min(trow[t] + c, n - 1) * nb;
    // activation rows past m (lanes c >= m) re-read row m - 1: their products land only in
    // output rows >= m, which are never stored
    const uint4 *xrow = xp + (size_t)min(c, m - 1) * nb * 4 + g;
    // nibble q becomes fp16 16 + q (exponent of 16, q in the top mantissa bits); the 24
    // this adds to each weight (q - 8) leaves through one more product per block with a
    // constant -24 operand, shared by the TW tiles
    uint32_t magic = 0x4C004C00u;
    asm volatile("" : "+v"(magic));
    const uint32_t m24 = 0xCE00CE00u;  // fp16 -24, -24
    const half8_t neg24 = __builtin_bit_cast(half8_t, make_uint4(m24, m24, m24, m24));

    static_assert(!SP || UG == 2, "scale pairs cover the two groups of a stage");
    auto load = [&](Q4XStage<UG, TW, SP> &st, int j0) {
        if constexpr (SP) {
            const int jp = min(j0, ng - 2);
#pragma unroll
            for (int t = 0; t < TW; t++) st.dp[t] = ldg_u4(wdb[t] + (wrow[t] + 4 * jp) * 2);
        }
#pragma unroll
        for (int u = 0; u < UG; u++) {
            const int j = min(j0 + u, j_hi - 1);
#pragma unroll
            for (int t = 0; t < TW; t++) {
                st.w[u][t] = ldg_u4(qsb[t] + (wrow[t] + 4 * j + g) * 16);
                if constexpr (!SP) st.d[u][t] = ldg_u2(wdb[t] + (wrow[t] + 4 * j) * 2);
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++) st.x[u][jj] = xrow[(size_t)(4 * j + jj) * 4];
        }
    };
    float4_t acc[TW];
#pragma unroll
    for (int t = 0; t < TW; t++) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Q4XStage<UG, TW, SP> &st, int j0) {
        const int jp = min(j0, ng - 2);
#pragma unroll
        for (int u = 0; u < UG; u++) {
            const bool valid = j0 + u < j_hi;
            const bool hi_half = SP && j0 + u - jp >= 1;  // group j0+u is the pair's second
            uint32_t ww[TW][4];
#pragma unroll
            for (int t = 0; t < TW; t++) {
                // transpose: lane (g, c) has dwords 0..3 of block g; wants dword g of blocks 0..3.
                // One wave writes and reads its own slot: LDS executes a wave's operations in
                // order, so only the compiler needs fencing.
                s_t[wave][c][0][g] = st.w[u][t].x;
                s_t[wave][c][1][g] = st.w[u][t].y;
                s_t[wave][c][2][g] = st.w[u][t].z;
                s_t[wave][c][3][g] = st.w[u][t].w;
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_wave_barrier();
                const uint4 wt = *(const uint4 *)&s_t[wave][c][g][0];
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_wave_barrier();
                ww[t][0] = wt.x;
                ww[t][1] = wt.y;
                ww[t][2] = wt.z;
                ww[t][3] = wt.w;
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                // k slots 0..7 of lane group g: the low nibbles of bytes 0, 2, 1, 3 of dword g,
                // then the high nibbles in the same order (the activation is permuted to match)
                const half8_t x8 = __builtin_bit_cast(half8_t, st.x[u][jj]);
                const float4_t corr =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(x8, neg24, float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int t = 0; t < TW; t++) {
                    const uint32_t v = ww[t][jj];
                    const uint4 wq = make_uint4(((v << 6) & 0x03c003c0u) | magic, ((v >> 2) & 0x03c003c0u) | magic,
                                                ((v << 2) & 0x03c003c0u) | magic, ((v >> 6) & 0x03c003c0u) | magic);
                    const float4_t r =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(x8, __builtin_bit_cast(half8_t, wq), corr, 0, 0, 0);
                    uint2 d2;
                    if constexpr (SP)
                        d2 = hi_half ? make_uint2(st.dp[t].z, st.dp[t].w) : make_uint2(st.dp[t].x, st.dp[t].y);
                    else
                        d2 = st.d[u][t];
                    const uint32_t dw = jj < 2 ? d2.x : d2.y;
                    const float ds = valid ? h2f((uint16_t)(jj & 1 ? dw >> 16 : dw & 0xffffu)) : 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[t][i] = fmaf(ds, r[i], acc[t][i]);
                }
            }
        }
    };
    if (j_lo < j_hi) {
        // two register stages; the prefetches are unconditional (clamped: past the end they
        // re-read the last group, a cache hit, and its scales are zeroed), since a load
        // under a branch makes the compiler wait for every load at the join
        Q4XStage<UG, TW, SP> sa, sb;
        load(sa, j_lo);
        for (int j0 = j_lo; j0 < j_hi; j0 += 2 * UG) {
            load(sb, j0 + UG);
            __builtin_amdgcn_sched_barrier(0);
            compute(sa, j0);
            load(sa, j0 + 2 * UG);
            __builtin_amdgcn_sched_barrier(0);
            compute(sb, j0 + UG);
        }
    }
#pragma unroll
    for (int t = 0; t < TW; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) s_acc[wave][t][lane][i] = acc[t][i];
    __syncthreads();
    if constexpr (ROPE) {
        // every wave takes one of the lane's 4 activation rows (the rotation's angle loop
        // and sin / cos are the long part)
        static_assert(KS == 4, "one epilogue row per wave");
        const uint64_t bias = (uint64_t)Q4B_PICK(S, bias, mi);
        float bv[TW];
#pragma unroll
        for (int t = 0; t < TW; t++) bv[t] = bias ? ldg_f32(bias + 4 * (uint64_t)(trow[t] + c)) : 0.0f;
        const int half = RP.hd / 2;
        const int p = trow[0] % RP.hd + c;  // rotation pair (q, k): dims p and p + half of its head
        const int head = trow[0] / RP.hd;
        {
            const int i = wave;
            const int r = 4 * g + i;
            if (r >= m) return;
            float v[TW];
#pragma unroll
            for (int t = 0; t < TW; t++) {
                float a = 0.0f;
#pragma unroll
                for (int w = 0; w < KS; w++) a += s_acc[w][t][lane][i];
                v[t] = bias ? a + bv[t] : a;
            }
            const int64_t ci = RP.kv_i64 ? ((const int64_t *)RP.kv_idx)[r] : (int64_t)((const int32_t *)RP.kv_idx)[r];
            const bool ci_ok = ci >= 0 && ci < RP.n_cache_rows;
            if (mi < 2) {
                float theta = (float)RP.pos[r];
                for (int tt = 0; tt < p; tt++) theta *= RP.theta_scale;  // the rope kernel's product order
                const float th = RP.freq_scale * theta;
                const float cs = cosf(th) * RP.attn_factor;
                const float sn = sinf(th) * RP.attn_factor;
                const float y0 = mul_sub_mul_rn(v[0], cs, v[1], sn);
                const float y1 = mul_add_mul_rn(v[0], sn, v[1], cs);
                if (mi == 0) {
                    float *yr = RP.q_out + ((size_t)r * (n / RP.hd) + head) * RP.hd;
                    yr[p] = y0;
                    yr[p + half] = y1;
                } else if (ci_ok) {
                    uint16_t *kr = (uint16_t *)(RP.kc + (size_t)ci * RP.k_row_bytes) + (size_t)head * RP.hd;
                    kr[p] = f2h(y0);
                    kr[p + half] = f2h(y1);
                }
            } else if (ci_ok) {
                uint16_t *vr = (uint16_t *)(RP.vc + (size_t)ci * RP.v_row_bytes);
#pragma unroll
                for (int t = 0; t < TW; t++)
                    if (trow[t] + c < n) vr[trow[t] + c] = f2h(v[t]);
            }
        }
        return;
    }
    // the waves share the epilogue: wave w takes the lane's activation rows 4g + i, i = w (mod KS)
    if (wave >= 4) return;
    if constexpr (GLU) {
        const int row = trow[0] + c;  // h index
        if (row >= n) return;
        const int p = row & 31, q = p & 3;
        const int gp = (p & 15) >> 2, jp = (p >> 4) * 4 + (q == 1 ? 2 : q == 2 ? 1 : q);
        const size_t nbd = (size_t)n / QK;
        for (int i = wave; i < 4; i += KS) {
            const int r = 4 * g + i;
            if (r < m) {
                float gv = 0.0f, uv = 0.0f;
#pragma unroll
                for (int w = 0; w < KS; w++) {
                    gv += s_acc[w][0][lane][i];
                    uv += s_acc[w][1][lane][i];
                }
                S.hxp[(((size_t)r * nbd + row / QK) * 4 + gp) * 8 + jp] = f2h((gv / (1.0f + expf(-gv))) * uv);
            }
        }
        return;
    }
    const uint64_t y = (uint64_t)Q4B_PICK(S, y, mi);
    const uint64_t bias = (uint64_t)Q4B_PICK(S, bias, mi);
    const uint64_t add = (uint64_t)Q4B_PICK(S, add, mi);
#pragma unroll
    for (int t = 0; t < TW; t++) {
        const int row = trow[t] + c;
        if (row >= n) continue;
        const float bv = bias ? ldg_f32(bias + 4 * (uint64_t)row) : 0.0f;
        for (int i = wave; i < 4; i += KS) {
            const int r = 4 * g + i;  // activation row
            if (r < m) {
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < KS; w++) v += s_acc[w][t][lane][i];
                const uint64_t o = (uint64_t)r * n + row;
                if (bias) v = v + bv;
                if (add) v = v + ldg_f32(add + 4 * o);
                stg_f32(y + 4 * o, v);
            }
        }
    }
}

// fp32 -> fp16 (round to nearest even, as ggml's activation conversion)
__global__ __launch_bounds__(256) void k_cast_f16(const float *__restrict__ x, uint16_t *__restrict__ y, int64_t n4) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float4 v = ((const float4 *)x)[i];
    ((uint2 *)y)[i] = make_uint2((uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16),
                                 (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16));
}

// ---------------------------------------------------------------- one activation row
// The activation row lives in registers and weight rows stream past it.  Lane l of a
// wave owns the blocks l + 64*(ks + WPR*i), i < KB, of every row (WPR waves split k,
// ks = the wave's slice), so its activation blocks are loaded once per workgroup (from
// an fp16 copy of the row staged in LDS) and each row costs the lane only its weight
// loads: 16 nibble bytes and one fp16 scale per block.  The unit of work is a pair of
// rows; the next pair's weights are in flight while the current pair is reduced, and
// the grid is sized to what the GPU holds at once (each pair group walks the units
// with a grid stride).
//
// The activation pairs are kept in the order in which four nibble pairs come out of a
// weight dword with one shift and one AND-OR each (dword t holds elements 4t+b in the
// low and 16+4t+b in the high nibble of byte b):
//   xs[4t+0] = (x[4t],    x[4t+2])     <- (v      ) & 0x000f000f
//   xs[4t+1] = (x[4t+1],  x[4t+3])     <- (v >>  8) & 0x000f000f
//   xs[4t+2] = (x[16+4t], x[16+4t+2])  <- (v >>  4) & 0x000f000f
//   xs[4t+3] = (x[17+4t], x[19+4t])    <- (v >> 12) & 0x000f000f
// Shifted to mantissa bits 6..9 and ORed with 0x4C00 (16.0), each nibble becomes the
// exact fp16 16 + nib (the binade [16, 32) has a 1/64 step).  The dot runs on those
// values and the offset comes out once per block: sum (nib - 8) x = sum (16 + nib) x -
// 24 * sum x, with sum x of the lane's block formed once per kernel (q4_xr_block_sum).
// The fp16 products are exact in fp32 and the partial sums stay within ~25x the block's
// activation magnitude, so the result keeps fp32-level accuracy; per nibble pair this is
// a shift and an AND-OR, with no fp16 subtraction.  magic: 0x4C004C00 held in a VGPR by
// the caller, so that each AND-OR is one v_and_or_b32 (gfx9 VOP3 takes no literal and
// one scalar operand).
__device__ __forceinline__ float q4_dot_xr(const int4 q, const uint32_t *xs, uint32_t magic, float xsum) {
    const uint32_t qq[4] = {(uint32_t)q.x, (uint32_t)q.y, (uint32_t)q.z, (uint32_t)q.w};
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t v = qq[t];
        const uint32_t a = ((v << 6) & 0x03c003c0u) | magic;  // low nibbles of bytes 0, 2
        const uint32_t c = ((v >> 2) & 0x03c003c0u) | magic;  // low nibbles of bytes 1, 3
        const uint32_t b = ((v << 2) & 0x03c003c0u) | magic;  // high nibbles of bytes 0, 2
        const uint32_t d = ((v >> 6) & 0x03c003c0u) | magic;  // high nibbles of bytes 1, 3
        s = fdot2(a, xs[4 * t + 0], s);
        s = fdot2(c, xs[4 * t + 1], s);
        s = fdot2(b, xs[4 * t + 2], s);
        s = fdot2(d, xs[4 * t + 3], s);
    }
    return fmaf(-24.0f, xsum, s);
}

// sum of the 32 activation values of one block (the lane's 16 permuted pairs)
__device__ __forceinline__ float q4_xr_block_sum(const uint32_t *xs) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const half2_t h = u2h2(xs[j]);
        s += (float)h.x + (float)h.y;
    }
    return s;
}

// up to four weight matrices stacked along the output rows (rows [row_end[i-1],
// row_end[i]) belong to matrix i; unused entries hold INT_MAX)
struct Q4Set {
    const uint8_t *qs[4];
    const uint16_t *d[4];
    const float *add[4];  // residual or bias of the matrix's output rows, or NULL
    float *y[4];
    int row_end[4];
};

// The register kernel selects a unit's matrix once per unit inside its loop: a scalar
// load from the kernel-argument segment per pointer (hidden behind the previous unit's
// math) costs far fewer scalar instructions than a select chain.
#define Q4SET_PICK(S, f, i) karg_at((S).f, (i))

__device__ __forceinline__ int q4set_index(const Q4Set &S, int r) {
    return (r >= S.row_end[0]) + (r >= S.row_end[1]) + (r >= S.row_end[2]);
}
__device__ __forceinline__ int q4set_row_start(const Q4Set &S, int i) {
    return i == 0 ? 0 : karg_at(S.row_end, i - 1);
}

// unit modes: which two rows a unit holds and what its epilogue does
constexpr int XR_PAIRS = 0;  // rows 2u, 2u+1; y = W x (+ add)
constexpr int XR_GLU = 1;    // gate row u and up row u; h[u] = fp16(silu(g) * u)
constexpr int XR_ROPE = 2;   // q/k rotation pairs (i, i + hd/2) of one head, then v row pairs

template <int UM>
__device__ __forceinline__ void xr_rows(const Q4Set &S, const RopeKV &R, int u, int n_rows, int &r0, int &r1,
                                        bool &ok1) {
    if constexpr (UM == XR_PAIRS) {
        r0 = 2 * u;
        r1 = 2 * u + 1;
        ok1 = r1 < n_rows;
        if (!ok1) r1 = r0;
    } else if constexpr (UM == XR_GLU) {
        r0 = u;
        r1 = S.row_end[0] + u;
        ok1 = true;
    } else {
        const int half = R.hd / 2, n_pairs = (R.n_q + R.n_k) / 2;
        if (u < n_pairs) {
            r0 = (u / half) * R.hd + u % half;
            r1 = r0 + half;
        } else {
            r0 = R.n_q + R.n_k + 2 * (u - n_pairs);
            r1 = r0 + 1;
        }
        ok1 = true;
    }
}

template <int KB>
struct XrRows {
    int4 w[2][KB];
    uint32_t d[2][KB];
    float a[2];  // the rows' add / bias values (read with the weights, used in the epilogue)
};


// weights of rows r0, r1 at the lane's blocks; with dummy every lane reads block 0 of
// r0 (one cache line: keeps the instruction count, and so the wait counts, identical
// on the last step)
template <int KB>
__device__ __forceinline__ void xr_load(XrRows<KB> &W, const Q4Set &S, int r0, int r1, const int *bidx, bool dummy,
                                        int nb) {
#pragma unroll
    for (int rr = 0; rr < 2; rr++) {
        const int r = rr ? r1 : r0;
        const int mi = q4set_index(S, r);
        const uint64_t base = (uint64_t)(r - q4set_row_start(S, mi)) * (uint64_t)nb;
        const uint64_t qs = (uint64_t)Q4SET_PICK(S, qs, mi) + base * 16;
        const uint64_t dp = (uint64_t)Q4SET_PICK(S, d, mi) + base * 2;
        const uint64_t ap = (uint64_t)Q4SET_PICK(S, add, mi);
        // without an add vector the load reads the row's first weight bytes (unused)
        W.a[rr] = ldg_f32(ap ? ap + 4 * (uint64_t)(r - q4set_row_start(S, mi)) : qs);
#pragma unroll
        for (int i = 0; i < KB; i++) {
            const uint64_t b = dummy ? 0 : (uint64_t)bidx[i];
            W.w[rr][i] = ldg_stream16(qs + b * 16);
            W.d[rr][i] = ldg_u16(dp + b * 2);
        }
    }
}

template <int KB>
__device__ __forceinline__ void xr_dot(const XrRows<KB> &W, const uint32_t (*xr)[16], const float *xsum,
                                       const bool *bval, float &s0, float &s1, uint32_t magic) {
    s0 = 0.0f;
    s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < KB; i++) {
        const float a = q4_dot_xr(W.w[0][i], xr[i], magic, xsum[i]);
        const float b = q4_dot_xr(W.w[1][i], xr[i], magic, xsum[i]);
        const float t0 = fmaf(h2f((uint16_t)W.d[0][i]), a, s0);
        const float t1 = fmaf(h2f((uint16_t)W.d[1][i]), b, s1);
        s0 = bval[i] ? t0 : s0;
        s1 = bval[i] ? t1 : s1;
    }
}

struct XrRope {
    const float *tab;  // LDS [2][64]: cos and sin of rotation pair p < hd/2 <= 64
    int64_t ci;
    bool ci_ok;
};

// epilogue of one unit with its two row sums (lane 0 of the reducing wave writes; every
// lane of that wave calls it, for the shuffles)
template <int UM>
__device__ __forceinline__ void xr_store(const Q4Set &S, const RopeKV &R, const XrRope &rp, uint16_t *h_out, int u,
                                         int r0, int r1, bool ok1, float s0, float s1, float av0, float av1,
                                         int lane) {
    const int m0 = q4set_index(S, r0), m1 = q4set_index(S, r1);
    const int l0 = r0 - q4set_row_start(S, m0), l1 = r1 - q4set_row_start(S, m1);
    const bool a0 = Q4SET_PICK(S, add, m0) != nullptr;
    const bool a1 = Q4SET_PICK(S, add, m1) != nullptr;
    if constexpr (UM == XR_ROPE) {
        const int half = R.hd / 2, n_pairs = (R.n_q + R.n_k) / 2;
        if (lane != 0) return;
        const float cs = rp.tab[u % half], sn = rp.tab[64 + u % half];
        const float x0 = a0 ? s0 + av0 : s0;
        const float x1 = a1 ? s1 + av1 : s1;
        if (u < n_pairs) {
            const float y0 = mul_sub_mul_rn(x0, cs, x1, sn);
            const float y1 = mul_add_mul_rn(x0, sn, x1, cs);
            if (r0 < R.n_q) {
                R.q_out[r0] = y0;
                R.q_out[r1] = y1;
            } else if (rp.ci_ok) {
                uint16_t *kr = (uint16_t *)(R.k_cache + (size_t)rp.ci * R.k_row_bytes);
                kr[r0 - R.n_q] = f2h(y0);
                kr[r1 - R.n_q] = f2h(y1);
            }
        } else if (rp.ci_ok) {
            uint16_t *vr = (uint16_t *)(R.v_cache + (size_t)rp.ci * R.v_row_bytes);
            vr[r0 - R.n_q - R.n_k] = f2h(x0);
            vr[r1 - R.n_q - R.n_k] = f2h(x1);
        }
    } else if constexpr (UM == XR_GLU) {
        if (lane != 0) return;
        const float g = a0 ? s0 + av0 : s0;
        const float v = a1 ? s1 + av1 : s1;
        h_out[u] = f2h((g / (1.0f + expf(-g))) * v);
    } else {
        if (lane != 0) return;
        const uint64_t y0 = (uint64_t)Q4SET_PICK(S, y, m0), y1 = (uint64_t)Q4SET_PICK(S, y, m1);
        stg_f32(y0 + 4 * (uint64_t)l0, a0 ? s0 + av0 : s0);
        if (ok1) stg_f32(y1 + 4 * (uint64_t)l1, a1 ? s1 + av1 : s1);
    }
}

// KB blocks per lane and WPR waves per row pair (k <= 64*32*WPR*KB); XF32: the
// activation is fp32 (rounded to fp16 RNE, as ggml converts src1), else fp16; XN > 0:
// the fp32 activation (k <= 1024*XN) is loaded into registers before the weights, so
// that staging it (with the RMSNorm by norm_w when NORM) waits only for those loads.
template <int KB, int WPR, bool XF32, int XN, bool NORM, int UM>
__global__ __launch_bounds__(256) void k_gemv_q4_0_xr(const Q4Set S, const void *__restrict__ xin,
                                                      const float *__restrict__ norm_w, float eps, int nb,
                                                      int n_units, int n_rows, const RopeKV R,
                                                      uint16_t *__restrict__ h_out) {
    constexpr int PG = 4 / WPR;  // pair groups per workgroup
    extern __shared__ __align__(16) uint8_t smem[];
    const int k = nb * QK;
    uint16_t *s_x = (uint16_t *)smem;                              // the fp16 row (fp32 input only)
    float *s_red = (float *)(smem + (XF32 ? (size_t)k * 2 : 0));  // [2][4][2]
    double *s_nred = (double *)(s_red + 16);        // [4]
    float *s_rope = (float *)(s_nred + 4);          // [2][64]: cos, sin of rotation pair p
    const int tid = threadIdx.x, lane = tid & 63;
    // the unit, row and matrix indices are wave-uniform: scalar registers and scalar selects
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint32_t magic = 0x4C004C00u;
    asm volatile("" : "+v"(magic));
    const int pg = wave / WPR, ks = wave % WPR;
    int bidx[KB];
    bool bval[KB];
#pragma unroll
    for (int i = 0; i < KB; i++) {
        const int b = lane + 64 * (ks + WPR * i);
        bval[i] = b < nb;
        bidx[i] = min(b, nb - 1);
    }
    const int stride = gridDim.x * PG;
    const int u_first = blockIdx.x * PG + pg;

    const int k4 = k / 4;
    // The rotation's position and cache row, then a short activation, are loaded before
    // the weights: loads retire in order, so their consumers wait only for them.  The
    // index z is an opaque per-lane zero: the values stay in vector registers (a uniform
    // load would be moved to scalar registers at once, waiting for it there).
    int z = 0;
    asm volatile("" : "+v"(z));
    int pos0 = 0;
    int32_t ci_lo = 0, ci_hi = 0;
    float tab_cs = 0.0f, tab_sn = 0.0f;
    if constexpr (UM == XR_ROPE) {
        // branch-free: the high word's load reads word 0 again for an int32 index
        pos0 = R.pos[z];
        ci_lo = ((const int32_t *)R.kv_idx)[z];
        ci_hi = ((const int32_t *)R.kv_idx)[z + (R.kv_idx_i64 ? 1 : 0)];
        rope_tab_prefetch(R, lane + z, tab_cs, tab_sn);
    }
    // An fp32 row is staged once per workgroup as fp16 in LDS (XN > 0: through registers,
    // with the RMSNorm when NORM); an fp16 row is not staged: each lane loads its own
    // blocks straight into registers.
    XStage<(XN > 0 ? XN : 1), NORM> st;
    if constexpr (XN > 0) xstage_load(st, (const float *)xin, norm_w, nullptr, k4, tid);
    constexpr int KH = XF32 ? 1 : KB;
    uint4 xh[KH][4];
    if constexpr (!XF32) {
#pragma unroll
        for (int i = 0; i < KB; i++)
#pragma unroll
            for (int c = 0; c < 4; c++) xh[i][c] = ((const uint4 *)xin)[(size_t)bidx[i] * 4 + c];
    }

    // the first unit's weights go out before the activation is staged
    XrRows<KB> wa, wb;
    int r0, r1;
    bool ok1;
    xr_rows<UM>(S, R, min(u_first, n_units - 1), n_rows, r0, r1, ok1);
    xr_load<KB>(wa, S, r0, r1, bidx, false, nb);
    __builtin_amdgcn_sched_barrier(0);  // nothing that waits on a load moves above the weight loads

    if constexpr (XN > 0) {
        const float scale = xstage_scale(st, k4, eps, s_nred, tid);  // 1 without NORM
#pragma unroll
        for (int t = 0; t < XN; t++) {
            const int f = tid + t * 256;
            const float4 v = xstage_value(st, scale, t);
            if (f < k4)
                ((uint2 *)s_x)[f] = make_uint2((uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16),
                                               (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16));
        }
    } else if constexpr (XF32) {
        for (int f = tid; f < k4; f += 256) {
            const float4 v = ((const float4 *)xin)[f];
            ((uint2 *)s_x)[f] = make_uint2((uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16),
                                           (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16));
        }
    }

    XrRope rp;
    if constexpr (UM == XR_ROPE) {
        // the rotation table, once per workgroup (wave 0, lane p): theta_p by p repeated
        // multiplications, as the CPU rope cache forms it
        if (wave == 0) {
            if (R.tab) {
                s_rope[lane] = tab_cs;
                s_rope[64 + lane] = tab_sn;
            } else {
                float theta = (float)pos0;
                for (int i = 0; i < lane && i < R.hd / 2; i++) theta *= R.theta_scale;
                const float th = R.freq_scale * theta;
                s_rope[lane] = cosf(th) * R.attn_factor;
                s_rope[64 + lane] = sinf(th) * R.attn_factor;
            }
        }
        const int64_t ci =
            R.kv_idx_i64 ? (int64_t)(((uint64_t)(uint32_t)ci_hi << 32) | (uint32_t)ci_lo) : (int64_t)ci_lo;
        rp.tab = s_rope;
        rp.ci = ci;
        rp.ci_ok = ci >= 0 && ci < R.n_cache_rows;
    }
    if constexpr (XF32 || UM == XR_ROPE) __syncthreads();

    uint32_t xr[KB][16];
#pragma unroll
    for (int i = 0; i < KB; i++) {
        uint4 q0, q1, q2, q3;
        if constexpr (XF32) {
            const uint4 *p = (const uint4 *)(s_x + (size_t)bidx[i] * QK);
            q0 = p[0]; q1 = p[1]; q2 = p[2]; q3 = p[3];
        } else {
            q0 = xh[i][0]; q1 = xh[i][1]; q2 = xh[i][2]; q3 = xh[i][3];
        }
        const uint32_t w[16] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w,
                                q2.x, q2.y, q2.z, q2.w, q3.x, q3.y, q3.z, q3.w};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            xr[i][4 * t + 0] = (w[2 * t] & 0xffffu) | (w[2 * t + 1] << 16);
            xr[i][4 * t + 1] = (w[2 * t] >> 16) | (w[2 * t + 1] & 0xffff0000u);
            xr[i][4 * t + 2] = (w[8 + 2 * t] & 0xffffu) | (w[9 + 2 * t] << 16);
            xr[i][4 * t + 3] = (w[8 + 2 * t] >> 16) | (w[9 + 2 * t] & 0xffff0000u);
        }
    }
    float xsum[KB];
#pragma unroll
    for (int i = 0; i < KB; i++) xsum[i] = q4_xr_block_sum(xr[i]);

    if constexpr (WPR == 1) {
        // one pair group per wave, no workgroup barriers past this point
        if (u_first >= n_units) return;
        int u = u_first;
        for (;;) {
            const int ub = u + stride;
            const bool more_b = ub < n_units;
            int q0, q1;
            bool qok;
            xr_rows<UM>(S, R, more_b ? ub : u, n_rows, q0, q1, qok);
            xr_load<KB>(wb, S, q0, q1, bidx, !more_b, nb);
            __builtin_amdgcn_sched_barrier(0);  // the next pair's loads issue before this pair's math
            float s0, s1;
            xr_dot<KB>(wa, xr, xsum, bval, s0, s1, magic);
            s0 = group_sum<64>(s0);
            s1 = group_sum<64>(s1);
            xr_store<UM>(S, R, rp, h_out, u, r0, r1, ok1, s0, s1, wa.a[0], wa.a[1], lane);
            if (!more_b) break;
            u = ub;
            r0 = q0; r1 = q1; ok1 = qok;

            const int ua = u + stride;
            const bool more_a = ua < n_units;
            xr_rows<UM>(S, R, more_a ? ua : u, n_rows, q0, q1, qok);
            xr_load<KB>(wa, S, q0, q1, bidx, !more_a, nb);
            __builtin_amdgcn_sched_barrier(0);  // the next pair's loads issue before this pair's math
            xr_dot<KB>(wb, xr, xsum, bval, s0, s1, magic);
            s0 = group_sum<64>(s0);
            s1 = group_sum<64>(s1);
            xr_store<UM>(S, R, rp, h_out, u, r0, r1, ok1, s0, s1, wb.a[0], wb.a[1], lane);
            if (!more_a) break;
            u = ua;
            r0 = q0; r1 = q1; ok1 = qok;
        }
    } else {
        // WPR waves share a unit: the trip count is uniform over the workgroup (units past
        // the end are computed on a clamped unit and not stored), partial sums meet in LDS
        int base = blockIdx.x * PG;
        int par = 0;
        auto finish = [&](int u, int a0, int a1, bool aok, float s0, float s1, float av0, float av1) {
            s0 = group_sum<64>(s0);
            s1 = group_sum<64>(s1);
            if (lane == 0) {
                s_red[(par * 4 + wave) * 2 + 0] = s0;
                s_red[(par * 4 + wave) * 2 + 1] = s1;
            }
            __syncthreads();
            if (ks == 0 && u < n_units) {
                float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
                for (int w = 0; w < WPR; w++) {
                    t0 += s_red[(par * 4 + pg * WPR + w) * 2 + 0];
                    t1 += s_red[(par * 4 + pg * WPR + w) * 2 + 1];
                }
                xr_store<UM>(S, R, rp, h_out, u, a0, a1, aok, t0, t1, av0, av1, lane);
            }
            par ^= 1;
        };
        if (base >= n_units) return;  // uniform over the workgroup
        for (;;) {
            const int u = base + pg;
            const int nbase = base + stride;
            const bool more_b = nbase < n_units;  // uniform
            int q0, q1;
            bool qok;
            xr_rows<UM>(S, R, min(more_b ? nbase + pg : u, n_units - 1), n_rows, q0, q1, qok);
            xr_load<KB>(wb, S, q0, q1, bidx, !more_b, nb);
            __builtin_amdgcn_sched_barrier(0);  // the next pair's loads issue before this pair's math
            float s0, s1;
            xr_dot<KB>(wa, xr, xsum, bval, s0, s1, magic);
            finish(u, r0, r1, ok1, s0, s1, wa.a[0], wa.a[1]);
            if (!more_b) break;
            base = nbase;
            r0 = q0; r1 = q1; ok1 = qok;

            const int u2 = base + pg;
            const int nbase2 = base + stride;
            const bool more_a = nbase2 < n_units;
            xr_rows<UM>(S, R, min(more_a ? nbase2 + pg : u2, n_units - 1), n_rows, q0, q1, qok);
            xr_load<KB>(wa, S, q0, q1, bidx, !more_a, nb);
            __builtin_amdgcn_sched_barrier(0);  // the next pair's loads issue before this pair's math
            xr_dot<KB>(wb, xr, xsum, bval, s0, s1, magic);
            finish(u2, r0, r1, ok1, s0, s1, wb.a[0], wb.a[1]);
            if (!more_a) break;
            base = nbase2;
            r0 = q0; r1 = q1; ok1 = qok;
        }
    }
}

inline int q4_pick_u(int64_t nb, int g) {
    int64_t u = (nb + g - 1) / g;
    if (u > 8) u = (u + 1) / 2 > 8 ? 8 : (u + 1) / 2;
    return (int)u;
}

// activation staged in LDS as fp16 from fp32 (m*k*2 <= 64 KB)
template <int G, int U, int M>
int launch_lds_gu(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const float *x32, float *y) {
    const Q4Planes p = q4_planes(n, k);
    constexpr int RPB = 256 / G;
    const size_t smem = (size_t)M * k * 2;
    hipLaunchKernelGGL((k_gemv_q4_0<G, U, M, true>), dim3((unsigned)((n + RPB - 1) / RPB)), dim3(256), smem, st, base,
                       (const uint16_t *)(base + p.plane), nullptr, x32, y, (int)n, (int)(k / QK), (int)m);
    MI_CHECK_LAUNCH("k_gemv_q4_0");
    return MI_OK;
}

template <int G, int M>
int launch_lds_g(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const float *x32, float *y) {
#define MI_U_CASE(UU) case UU: return launch_lds_gu<G, UU, M>(st, base, n, k, m, x32, y);
    switch (q4_pick_u(k / QK, G)) {
        MI_U_CASE(1) MI_U_CASE(2) MI_U_CASE(3) MI_U_CASE(4) MI_U_CASE(5) MI_U_CASE(6) MI_U_CASE(7) MI_U_CASE(8)
    }
#undef MI_U_CASE
    return MI_ERR_ARG;
}

template <int M>
int launch_lds_m(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const float *x32, float *y) {
    const int64_t nb = k / QK;
    if (nb <= 128) return launch_lds_g<16, M>(st, base, n, k, m, x32, y);
    if (nb <= 256) return launch_lds_g<32, M>(st, base, n, k, m, x32, y);
    return launch_lds_g<64, M>(st, base, n, k, m, x32, y);
}

int launch_lds(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const float *x32, float *y) {
    if ((size_t)m * k * 2 > 64 * 1024) {
        set_error("gemv_q4_0: activation of %lld x %lld does not fit in LDS", (long long)m, (long long)k);
        return MI_ERR_UNSUPPORTED;
    }
    if (m == 1) return launch_lds_m<1>(st, base, n, k, m, x32, y);
    if (m == 2) return launch_lds_m<2>(st, base, n, k, m, x32, y);
    if (m >= 3 && m <= 4) return launch_lds_m<4>(st, base, n, k, m, x32, y);
    if (m >= 5 && m <= 8) return launch_lds_m<8>(st, base, n, k, m, x32, y);
    set_error("gemv_q4_0: m=%lld not in 1..16", (long long)m);
    return MI_ERR_ARG;
}

// fp16 activation in global memory: 64 lanes per row, two rows per lane group for
// tall matrices (each activation chunk then feeds two weight blocks)
template <int U, int M, int R>
int launch_gx_ur(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const uint16_t *x16, float *y,
                 const float *add) {
    constexpr int G = 64, RPW = (256 / G) * R;
    const Q4Planes p = q4_planes(n, k);
    hipLaunchKernelGGL((k_gemv_q4_0_gx<G, U, M, R>), dim3((unsigned)((n + RPW - 1) / RPW)), dim3(256), 0, st, base,
                       (const uint16_t *)(base + p.plane), x16, y, add, (int)n, (int)(k / QK), (int)m);
    MI_CHECK_LAUNCH("k_gemv_q4_0_gx");
    return MI_OK;
}

template <int M, int R>
int launch_gx_mr(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const uint16_t *x16, float *y,
                 const float *add) {
#define MI_U_CASE(UU) case UU: return launch_gx_ur<UU, M, R>(st, base, n, k, m, x16, y, add);
    switch (q4_pick_u(k / QK, 64)) {
        MI_U_CASE(1) MI_U_CASE(2) MI_U_CASE(3) MI_U_CASE(4) MI_U_CASE(5) MI_U_CASE(6) MI_U_CASE(7) MI_U_CASE(8)
    }
#undef MI_U_CASE
    return MI_ERR_ARG;
}

// one 16-row tile per workgroup, k split over 4 (short rows) or 8 waves
template <bool XF32>
int launch_mfma(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const void *x, float *y,
                const float *add) {
    const Q4Planes p = q4_planes(n, k);
    const int nb = (int)(k / QK);
    const unsigned tiles = (unsigned)((n + 15) / 16);
    if (nb <= 128)
        hipLaunchKernelGGL((k_gemv_q4_0_mfma<4, 8, XF32>), dim3(tiles), dim3(256), 0, st, base,
                           (const uint16_t *)(base + p.plane), x, y, add, (int)n, nb, (int)m);
    else
        hipLaunchKernelGGL((k_gemv_q4_0_mfma<8, 8, XF32>), dim3(tiles), dim3(512), 0, st, base,
                           (const uint16_t *)(base + p.plane), x, y, add, (int)n, nb, (int)m);
    MI_CHECK_LAUNCH("k_gemv_q4_0_mfma");
    return MI_OK;
}

// ---- one activation row: launch of k_gemv_q4_0_xr
struct XrShape {
    int kb, wpr;
};

// blocks per lane and waves per row pair for nb blocks per row (nb <= 64*wpr*kb)
inline bool xr_shape(int64_t nb, XrShape &s) {
    if (nb <= 64) s = {1, 1};
    else if (nb <= 128) s = {2, 1};
    else if (nb <= 256) s = {2, 2};
    else if (nb <= 384) s = {3, 2};
    else if (nb <= 512) s = {2, 4};
    else if (nb <= 768) s = {3, 4};
    else if (nb <= 1024) s = {4, 4};
    else return false;
    return true;
}

inline size_t xr_smem(int64_t k, bool f32_row) {
    return (f32_row ? (size_t)k * 2 : 0) + 16 * sizeof(float) + 4 * sizeof(double) + 128 * sizeof(float);
}

// workgroups resident at once on the current device for this kernel and LDS size
int xr_resident(const void *fn, size_t smem) {
    static std::mutex mu;
    static std::unordered_map<uint64_t, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const uint64_t key = ((uint64_t)(uintptr_t)fn * 31 + smem) * 64 + (uint64_t)dev;
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = cache.find(key);
        if (it != cache.end()) return it->second;
    }
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, smem) != hipSuccess || per_cu < 1) per_cu = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    int r = per_cu * cus;
    if (const char *e = getenv("MI_Q4_XR_GRID")) r = (int)(r * atof(e));  // experiments: resident multiple
    if (r < 1) r = 1;
    std::lock_guard<std::mutex> lk(mu);
    cache[key] = r;
    return r;
}

template <int KB, int WPR, bool XF32, int XN, bool NORM, int UM>
int launch_xr(hipStream_t st, const Q4Set &S, const void *x, const float *norm_w, float eps, int nb, int n_units,
              int n_rows, const RopeKV &R, uint16_t *h) {
    constexpr int PG = 4 / WPR;
    const size_t smem = xr_smem((int64_t)nb * QK, XF32);
    auto fn = k_gemv_q4_0_xr<KB, WPR, XF32, XN, NORM, UM>;
    const int want = (n_units + PG - 1) / PG;
    const int grid = std::min(want, xr_resident((const void *)fn, smem));
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(256), smem, st, S, x, norm_w, eps, nb, n_units, n_rows, R, h);
    MI_CHECK_LAUNCH("k_gemv_q4_0_xr");
    return MI_OK;
}

// shapes for any k up to 32768 (fp16 or fp32 activation, no norm)
template <bool XF32, int UM>
int launch_xr_any(hipStream_t st, const XrShape &sh, const Q4Set &S, const void *x, int nb, int n_units, int n_rows,
                  const RopeKV &R, uint16_t *h) {
#define MI_XR_CASE(KB, WPR)           \
    if (sh.kb == KB && sh.wpr == WPR) \
        return launch_xr<KB, WPR, XF32, 0, false, UM>(st, S, x, nullptr, 0.0f, nb, n_units, n_rows, R, h);
    MI_XR_CASE(1, 1) MI_XR_CASE(2, 1) MI_XR_CASE(2, 2) MI_XR_CASE(3, 2) MI_XR_CASE(2, 4) MI_XR_CASE(3, 4)
    MI_XR_CASE(4, 4)
#undef MI_XR_CASE
    set_error("gemv_q4_0: no kernel for %d blocks per row", nb);
    return MI_ERR_UNSUPPORTED;
}

// short fp32 rows (k <= 4096: one wave per row pair, the activation through registers)
// with the optional RMSNorm
template <int XN, bool NORM, int UM>
int launch_xr_short_xn(hipStream_t st, const Q4Set &S, const void *x, const float *norm_w, float eps, int nb,
                       int n_units, int n_rows, const RopeKV &R, uint16_t *h) {
    if (nb <= 64) return launch_xr<1, 1, true, XN, NORM, UM>(st, S, x, norm_w, eps, nb, n_units, n_rows, R, h);
    return launch_xr<2, 1, true, XN, NORM, UM>(st, S, x, norm_w, eps, nb, n_units, n_rows, R, h);
}

template <int UM>
int launch_xr_short(hipStream_t st, const Q4Set &S, const void *x, const float *norm_w, float eps, int nb,
                    int n_units, int n_rows, const RopeKV &R, uint16_t *h) {
    const int k4 = nb * QK / 4;
#define MI_XR_CASE(XN)                                                                                    \
    if (k4 <= 256 * XN) {                                                                                 \
        if (norm_w) return launch_xr_short_xn<XN, true, UM>(st, S, x, norm_w, eps, nb, n_units, n_rows, R, h); \
        return launch_xr_short_xn<XN, false, UM>(st, S, x, nullptr, eps, nb, n_units, n_rows, R, h);      \
    }
    MI_XR_CASE(1) MI_XR_CASE(2) MI_XR_CASE(4)
#undef MI_XR_CASE
    set_error("gemv_q4_0: k=%d too long for the one-wave kernel", nb * QK);
    return MI_ERR_UNSUPPORTED;
}

// stacks n_mats matrices (packed Q4_0, n[i] rows of k) into a Q4Set
int make_q4set(Q4Set &S, int n_mats, const void *const *w, const int64_t *n, float *const *y,
               const float *const *add, int64_t k, int &n_total) {
    MI_CHECK_ARG(n_mats >= 1 && n_mats <= 4, "gemv_q4_0: %d matrices (1..4)", n_mats);
    int64_t tot = 0;
    for (int i = 0; i < 4; i++) {
        if (i < n_mats) {
            MI_CHECK_ARG(w[i] && n[i] > 0 && mi::aligned(w[i], 256), "gemv_q4_0: matrix %d: null, empty or misaligned", i);
            const Q4Planes p = q4_planes(n[i], k);
            S.qs[i] = (const uint8_t *)w[i];
            S.d[i] = (const uint16_t *)((const uint8_t *)w[i] + p.plane);
            S.add[i] = add ? add[i] : nullptr;
            S.y[i] = y ? y[i] : nullptr;
            tot += n[i];
            MI_CHECK_ARG(tot < (1ll << 30), "gemv_q4_0: too many rows");
            S.row_end[i] = (int)tot;
        } else {
            S.qs[i] = S.qs[0];
            S.d[i] = S.d[0];
            S.add[i] = nullptr;
            S.y[i] = nullptr;
            S.row_end[i] = INT_MAX;
        }
    }
    n_total = (int)tot;
    return MI_OK;
}

// y = W x (+ add) for one activation row through the register-resident kernel
int launch_xr_gemv(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, const void *x, bool xf32, float *y,
                   const float *add) {
    XrShape sh;
    if (!xr_shape(k / QK, sh)) return MI_ERR_UNSUPPORTED;
    Q4Set S;
    int n_total = 0;
    const void *w[1] = {base};
    const int64_t nn[1] = {n};
    float *ys[1] = {y};
    const float *as[1] = {add};
    if (int r = make_q4set(S, 1, w, nn, ys, as, k, n_total)) return r;
    RopeKV R{};
    const int units = (n_total + 1) / 2;
    if (xf32 && k <= 4096) return launch_xr_short<XR_PAIRS>(st, S, x, nullptr, 0.0f, (int)(k / QK), units, n_total, R,
                                                             nullptr);
    if (xf32) return launch_xr_any<true, XR_PAIRS>(st, sh, S, x, (int)(k / QK), units, n_total, R, nullptr);
    return launch_xr_any<false, XR_PAIRS>(st, sh, S, x, (int)(k / QK), units, n_total, R, nullptr);
}

inline bool xr_enabled() {
    static const bool on = [] {
        const char *e = getenv("MI_Q4_XR");
        return !(e && e[0] == '0');
    }();
    return on;
}

// Activation rows converted into ws as permuted fp16 (once for the whole set), then
// the A-operand matrix-core kernel over every matrix of the set in one launch.  mode:
// PERM_F32 / PERM_F16 / PERM_GLU (x the gate rows, up the up rows).
int launch_mfma_set(hipStream_t st, int count, const uint8_t *const *base, const int64_t *n, float *const *y,
                    const float *const *bias, const float *const *add, int64_t k, int64_t m, const void *x, int mode,
                    const float *up, void *ws, const float *norm_w = nullptr, float eps = 0.0f) {
    const int nb = (int)(k / QK);
    const int64_t units = m * nb * 4;
    const dim3 pg((unsigned)((units + 255) / 256));
    if (mode == PERM_READY)
        ws = const_cast<void *>(x);
    else if (norm_w)
        hipLaunchKernelGGL(k_perm_norm_f16, dim3((unsigned)m), dim3(256), 0, st, (const float *)x, norm_w, eps,
                           (uint4 *)ws, nb);
    else if (mode == PERM_F32)
        hipLaunchKernelGGL((k_perm_f16<PERM_F32>), pg, dim3(256), 0, st, x, up, (uint4 *)ws, (int)m, nb);
    else if (mode == PERM_GLU)
        hipLaunchKernelGGL((k_perm_f16<PERM_GLU>), pg, dim3(256), 0, st, x, up, (uint4 *)ws, (int)m, nb);
    else
        hipLaunchKernelGGL((k_perm_f16<PERM_F16>), pg, dim3(256), 0, st, x, up, (uint4 *)ws, (int)m, nb);
    if (mode != PERM_READY) MI_CHECK_LAUNCH("k_perm_f16");
    static const int tw_env = [] {
        const char *e = getenv("MI_Q4_MFMA_TW");
        return e ? atoi(e) : 0;
    }();
    static const int ks_env = [] {
        const char *e = getenv("MI_Q4_MFMA_KS");
        return e ? atoi(e) : 0;
    }();
    // two tiles per wave when the set has at least 4096 rows (gate / up, q/k/v), where the
    // shared activation load pays; below that, one tile keeps enough workgroups
    int64_t rows = 0;
    for (int i = 0; i < count; i++) rows += n[i];
    int tw = tw_env == 1 || tw_env == 2 ? tw_env : (rows >= 4096 ? 2 : 1);
    for (int i = 0; i + 1 < count; i++)
        if (n[i] % (16 * tw)) tw = 1;  // a tile must not straddle two matrices
    const int ks = ks_env == 2 || ks_env == 4 || ks_env == 8 || ks_env == 16 ? ks_env : 4;
    const bool sp = nb / 4 >= 2;  // scale pairs need two groups per row
    Q4BSet S;
    S.hxp = nullptr;
    int wgs = 0;
    for (int i = 0; i < 4; i++) {
        if (i < count) {
            const Q4Planes p = q4_planes(n[i], k);
            S.qs[i] = base[i];
            S.wd[i] = (const uint16_t *)(base[i] + p.plane);
            S.y[i] = y[i];
            S.bias[i] = bias ? bias[i] : nullptr;
            S.add[i] = add ? add[i] : nullptr;
            S.n[i] = (int)n[i];
            wgs += (int)((n[i] + 16 * tw - 1) / (16 * tw));
            S.wg_end[i] = wgs;
        } else {
            S.qs[i] = S.qs[0];
            S.wd[i] = S.wd[0];
            S.y[i] = S.y[0];
            S.bias[i] = nullptr;
            S.add[i] = nullptr;
            S.n[i] = S.n[0];
            S.wg_end[i] = INT_MAX;
        }
    }
#define MI_MX(KS, TW, SPV)                                                                                      \
    hipLaunchKernelGGL((k_gemv_q4_0_mfma_x<KS, 2, TW, SPV>), dim3((unsigned)wgs), dim3(64 * KS), 0, st, S,        \
                       (const uint4 *)ws, nb, (int)m, Q4BRope{})
#define MI_MX_TW(KS, TW)              \
    {                                 \
        if (sp) MI_MX(KS, TW, true);  \
        else MI_MX(KS, TW, false);    \
    }
#define MI_MX_KS(KS)                               \
    if (ks == KS) {                                \
        if (tw == 2) MI_MX_TW(KS, 2) else MI_MX_TW(KS, 1) \
    }
    MI_MX_KS(2) else MI_MX_KS(4) else MI_MX_KS(8) else MI_MX_KS(16)
#undef MI_MX_KS
#undef MI_MX_TW
#undef MI_MX
    MI_CHECK_LAUNCH("k_gemv_q4_0_mfma_x");
    return MI_OK;
}

// Gate and up (n rows each) of m activation rows, optionally after RMSNorm * norm_w, with
// the swiglu in the epilogue: hxp gets the down projection's permuted fp16 activation
// (k = n).  The activation's own conversion goes to ws (m * k * 2 bytes).
int launch_mfma_glu(hipStream_t st, const uint8_t *gate, const uint8_t *up, int64_t n, int64_t k, int64_t m,
                    const float *x, const float *norm_w, float eps, void *ws, uint16_t *hxp) {
    const int nb = (int)(k / QK);
    if (norm_w)
        hipLaunchKernelGGL(k_perm_norm_f16, dim3((unsigned)m), dim3(256), 0, st, x, norm_w, eps, (uint4 *)ws, nb);
    else
        hipLaunchKernelGGL((k_perm_f16<PERM_F32>), dim3((unsigned)((m * nb * 4 + 255) / 256)), dim3(256), 0, st,
                           (const void *)x, nullptr, (uint4 *)ws, (int)m, nb);
    MI_CHECK_LAUNCH("k_perm_f16");
    Q4BSet S;
    const Q4Planes p = q4_planes(n, k);
    const uint8_t *base[2] = {gate, up};
    for (int i = 0; i < 4; i++) {
        const uint8_t *b = base[i < 2 ? i : 0];
        S.qs[i] = b;
        S.wd[i] = (const uint16_t *)(b + p.plane);
        S.y[i] = nullptr;
        S.bias[i] = nullptr;
        S.add[i] = nullptr;
        S.n[i] = (int)n;
        S.wg_end[i] = INT_MAX;
    }
    S.hxp = hxp;
    const dim3 grid((unsigned)((n + 15) / 16));
    if (nb / 4 >= 2)
        hipLaunchKernelGGL((k_gemv_q4_0_mfma_x<4, 2, 2, true, PAIR_GLU>), grid, dim3(256), 0, st, S,
                           (const uint4 *)ws, nb, (int)m, Q4BRope{});
    else
        hipLaunchKernelGGL((k_gemv_q4_0_mfma_x<4, 2, 2, false, PAIR_GLU>), grid, dim3(256), 0, st, S,
                           (const uint4 *)ws, nb, (int)m, Q4BRope{});
    MI_CHECK_LAUNCH("k_gemv_q4_0_mfma_x");
    return MI_OK;
}

// q/k/v (+ bias) of m activation rows after RMSNorm * norm_w (or not), then RoPE of q and
// k and the k / v cache writes in the epilogue (PAIR_ROPE).  n[0], n[1] multiples of
// the head size hd (a multiple of 32, <= 256), n[2] of 32.
int launch_mfma_rope(hipStream_t st, const uint8_t *const *base, const int64_t *n, const float *const *bias,
                     int64_t k, int64_t m, const float *x, const float *norm_w, float eps, void *ws,
                     const Q4BRope &RP) {
    const int nb = (int)(k / QK);
    if (norm_w)
        hipLaunchKernelGGL(k_perm_norm_f16, dim3((unsigned)m), dim3(256), 0, st, x, norm_w, eps, (uint4 *)ws, nb);
    else
        hipLaunchKernelGGL((k_perm_f16<PERM_F32>), dim3((unsigned)((m * nb * 4 + 255) / 256)), dim3(256), 0, st,
                           (const void *)x, nullptr, (uint4 *)ws, (int)m, nb);
    MI_CHECK_LAUNCH("k_perm_f16");
    Q4BSet S;
    int wgs = 0;
    for (int i = 0; i < 4; i++) {
        const int j = i < 3 ? i : 0;
        const Q4Planes p = q4_planes(n[j], k);
        S.qs[i] = base[j];
        S.wd[i] = (const uint16_t *)(base[j] + p.plane);
        S.y[i] = nullptr;
        S.bias[i] = i < 3 && bias ? bias[i] : nullptr;
        S.add[i] = nullptr;
        S.n[i] = (int)n[j];
        if (i < 3) wgs += (int)(n[i] / 32);
        S.wg_end[i] = i < 3 ? wgs : INT_MAX;
    }
    S.hxp = nullptr;
    if (nb / 4 >= 2)
        hipLaunchKernelGGL((k_gemv_q4_0_mfma_x<4, 2, 2, true, PAIR_ROPE>), dim3((unsigned)wgs), dim3(256), 0, st, S,
                           (const uint4 *)ws, nb, (int)m, RP);
    else
        hipLaunchKernelGGL((k_gemv_q4_0_mfma_x<4, 2, 2, false, PAIR_ROPE>), dim3((unsigned)wgs), dim3(256), 0, st, S,
                           (const uint4 *)ws, nb, (int)m, RP);
    MI_CHECK_LAUNCH("k_gemv_q4_0_mfma_x");
    return MI_OK;
}

int launch_mfma_x(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const void *x, bool xf32,
                  float *y, const float *add, void *ws) {
    return launch_mfma_set(st, 1, &base, &n, &y, nullptr, add ? &add : nullptr, k, m, x, xf32 ? PERM_F32 : PERM_F16,
                           nullptr, ws);
}

inline bool mfma_x_enabled() {
    static const bool on = [] {
        const char *e = getenv("MI_Q4_MFMA_X");
        return !(e && e[0] == '0');
    }();
    return on;
}

// the grouped kernel needs whole groups of 4 blocks per row
inline bool mfma_x_ok(int64_t k) { return mfma_x_enabled() && (k / QK) % 4 == 0; }

// One fp16 row, few rows (n <= 2048) and short rows (at most 512 blocks): a workgroup
// of NW waves owns RW consecutive rows, and lane t owns block t of every one of them.
// The lane loads its 32 activation values once and uses them for all RW rows, so the
// activation crosses L2 -> L1 once per workgroup (the row-per-wave kernel reads it once
// per row: 17.5 KB per row at k = 8960, 3.5x the row's weights).  The activation loads
// go first and the rows' weights after them in row order (a wave's loads return in
// order), so row r's dot starts as soon as row r has arrived.  The dot is the register
// kernel's (q4_dot_xr: nibbles made fp16 16 + q with one shift and one AND-OR per pair,
// the activation pairs permuted to match once per lane).  Each row's lane partials
// reduce within the wave, then over the NW waves through LDS.
template <int RW, int NW>
__global__ __launch_bounds__(NW * 64) void k_gemv_q4_0_kb(const uint8_t *__restrict__ qs,
                                                          const uint16_t *__restrict__ wd,
                                                          const uint16_t *__restrict__ x16, float *__restrict__ y,
                                                          int n, int nb) {
    __shared__ float s_part[NW][RW];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.x * RW;
    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) acc[r] = 0.0f;
    if (tid < nb) {
        const int b = tid;
        const int4 *xp = (const int4 *)(x16 + (size_t)b * QK);
        int4 xv[4];
#pragma unroll
        for (int c = 0; c < 4; c++) xv[c] = xp[c];
        int4 wq[RW];
        uint16_t dw[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const size_t rb = (size_t)min(row0 + r, n - 1) * nb + b;
            wq[r] = ld_stream16(qs + rb * 16);
            dw[r] = wd[rb];
        }
        // xs[i] = (x[2i], x[2i+1]) -> the pair order of q4_dot_xr
        uint32_t xs[16], xq[16];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            xs[4 * c + 0] = (uint32_t)xv[c].x; xs[4 * c + 1] = (uint32_t)xv[c].y;
            xs[4 * c + 2] = (uint32_t)xv[c].z; xs[4 * c + 3] = (uint32_t)xv[c].w;
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t a = xs[2 * t], bb = xs[2 * t + 1], c = xs[8 + 2 * t], d = xs[9 + 2 * t];
            xq[4 * t + 0] = (a & 0xffffu) | (bb << 16);
            xq[4 * t + 1] = (a >> 16) | (bb & 0xffff0000u);
            xq[4 * t + 2] = (c & 0xffffu) | (d << 16);
            xq[4 * t + 3] = (c >> 16) | (d & 0xffff0000u);
        }
        uint32_t magic = 0x4C004C00u;
        asm volatile("" : "+v"(magic));
        float xsum = 0.0f;  // the block's activation sum: one dot2 with (1, 1) per pair
#pragma unroll
        for (int i = 0; i < 16; i++) xsum = fdot2(xq[i], 0x3C003C00u, xsum);
#pragma unroll
        for (int r = 0; r < RW; r++) acc[r] = fmaf(h2f(dw[r]), q4_dot_xr(wq[r], xq, magic, xsum), acc[r]);
    }
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const float v = group_sum<64>(acc[r]);
        if (lane == 0) s_part[wave][r] = v;
    }
    __syncthreads();
    if (tid < RW && row0 + tid < n) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) v += s_part[w][tid];
        y[row0 + tid] = v;
    }
}

template <int NW>
int launch_kb_nw(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, const uint16_t *x16, float *y) {
    const Q4Planes p = q4_planes(n, k);
    // rows per workgroup: about two workgroups per CU (at 1536 x 8960: 3 rows, 512
    // workgroups measured 4.24 us against 4.31 for 2 rows, 4.46 for 6 and 4.86 for 1)
    const int rw = (int)((n + 511) / 512);
    const unsigned grid = (unsigned)((n + rw - 1) / rw);
    const uint16_t *wd = (const uint16_t *)(base + p.plane);
#define MI_RW_CASE(R)                                                                                          \
    case R:                                                                                                    \
        hipLaunchKernelGGL((k_gemv_q4_0_kb<R, NW>), dim3(grid), dim3(NW * 64), 0, st, base, wd, x16, y, (int)n, \
                           (int)(k / QK));                                                                     \
        break;
    switch (rw) {
        MI_RW_CASE(1) MI_RW_CASE(2) MI_RW_CASE(3) MI_RW_CASE(4) MI_RW_CASE(5) MI_RW_CASE(6) MI_RW_CASE(7)
        MI_RW_CASE(8)
        default: set_error("gemv_q4_0_kb: %lld rows", (long long)n); return MI_ERR_ARG;
    }
#undef MI_RW_CASE
    MI_CHECK_LAUNCH("k_gemv_q4_0_kb");
    return MI_OK;
}

// one fp16 row, n <= 2048 rows of at most 512 blocks (3584 x 3584 measured 4.83 us here
// against 4.73 for the row-per-wave kernel): 4 waves up to 256 blocks, 5 up to
// 320, else 8
inline bool kb_fits(int64_t n, int64_t k) { return n <= 2048 && k / QK <= 512; }
int launch_kb(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, const uint16_t *x16, float *y) {
    const int64_t nb = k / QK;
    if (nb <= 256) return launch_kb_nw<4>(st, base, n, k, x16, y);
    if (nb <= 320) return launch_kb_nw<5>(st, base, n, k, x16, y);
    return launch_kb_nw<8>(st, base, n, k, x16, y);
}

int launch_gx(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const uint16_t *x16, float *y,
              const float *add = nullptr) {
    if (m >= 2 && m <= 16) return launch_mfma<false>(st, base, n, k, m, x16, y, add);
    // One fp16 row: with an add vector (the fused chains' residual launch, which must
    // match the node-by-node path bit for bit) always the register kernel; without,
    // the register kernel for long rows and the fp16-from-global kernel below 512 blocks
    // per row, where it measured faster.
    if (m == 1 && xr_enabled() && k / QK <= 1024 && (add || k / QK >= 512))
        return launch_xr_gemv(st, base, n, k, x16, false, y, add);
    if (m == 1 && !add && kb_fits(n, k)) return launch_kb(st, base, n, k, x16, y);
    const bool tall = n >= 2048;
    if (m == 1) return tall ? launch_gx_mr<1, 2>(st, base, n, k, m, x16, y, add)
                            : launch_gx_mr<1, 1>(st, base, n, k, m, x16, y, add);
    if (m == 2) return launch_gx_mr<2, 1>(st, base, n, k, m, x16, y, add);
    if (m >= 3 && m <= 4) return launch_gx_mr<4, 1>(st, base, n, k, m, x16, y, add);
    if (m >= 5 && m <= 8) return launch_gx_mr<8, 1>(st, base, n, k, m, x16, y, add);
    set_error("gemv_q4_0: m=%lld not in 1..16", (long long)m);
    return MI_ERR_ARG;
}

int check_shape(const char *what, int64_t n, int64_t k) {
    MI_CHECK_ARG(n > 0 && k > 0 && k % QK == 0, "%s: bad shape n=%lld k=%lld (k must be a multiple of 32)", what,
                 (long long)n, (long long)k);
    MI_CHECK_ARG(n < (1ll << 31) && k < (1ll << 24), "%s: shape too large", what);
    return MI_OK;
}

}  // namespace

extern "C" {

size_t mi_q4_0_packed_size(int64_t n, int64_t k) { return q4_planes(n, k).total; }

int mi_prepack_q4_0(void *stream, const void *src_blocks, void *dst_packed, int64_t n, int64_t k) {
    if (int r = check_shape("prepack_q4_0", n, k)) return r;
    MI_CHECK_ARG(src_blocks && dst_packed, "prepack_q4_0: null pointer");
    MI_CHECK_ARG(mi::aligned(src_blocks, 2) && mi::aligned(dst_packed, 256), "prepack_q4_0: src must be 2-byte, dst 256-byte aligned");
    const Q4Planes p = q4_planes(n, k);
    const int64_t nblocks = n * (k / QK);
    uint8_t *base = (uint8_t *)dst_packed;
    hipLaunchKernelGGL(k_prepack_q4_0, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t *)src_blocks, base, (uint16_t *)(base + p.plane), nblocks);
    MI_CHECK_LAUNCH("k_prepack_q4_0");
    return MI_OK;
}

int mi_prepack_q4_0_host(const void *src_blocks, void *dst_packed, int64_t n, int64_t k) {
    if (int r = check_shape("prepack_q4_0_host", n, k)) return r;
    const Q4Planes p = q4_planes(n, k);
    const int64_t nblocks = n * (k / QK);
    const uint8_t *s = (const uint8_t *)src_blocks;
    uint8_t *base = (uint8_t *)dst_packed;
    memset(base, 0, p.total);
    for (int64_t i = 0; i < nblocks; i++) {
        memcpy(base + i * 16, s + i * 18 + 2, 16);
        memcpy(base + p.plane + i * 2, s + i * 18, 2);
    }
    return MI_OK;
}

int mi_unpack_q4_0_host(const void *packed, void *dst_blocks, int64_t n, int64_t k) {
    if (int r = check_shape("unpack_q4_0_host", n, k)) return r;
    const Q4Planes p = q4_planes(n, k);
    const int64_t nblocks = n * (k / QK);
    const uint8_t *base = (const uint8_t *)packed;
    uint8_t *d = (uint8_t *)dst_blocks;
    for (int64_t i = 0; i < nblocks; i++) {
        memcpy(d + i * 18, base + p.plane + i * 2, 2);
        memcpy(d + i * 18 + 2, base + i * 16, 16);
    }
    return MI_OK;
}

int mi_gemv_q4_0_f16(void *stream, const void *w_packed, const uint16_t *x_f16, float *y, int64_t n, int64_t k,
                     int64_t m) {
    if (int r = check_shape("gemv_q4_0_f16", n, k)) return r;
    MI_CHECK_ARG(w_packed && x_f16 && y, "gemv_q4_0_f16: null pointer");
    MI_CHECK_ARG(mi::aligned(w_packed, 256) && mi::aligned(x_f16, 16), "gemv_q4_0_f16: w_packed must be 256-byte, x 16-byte aligned");
    return launch_gx((hipStream_t)stream, (const uint8_t *)w_packed, n, k, m, x_f16, y);
}

int mi_gemv_q4_0_f16_add(void *stream, const void *w_packed, const uint16_t *x_f16, const float *add, float *y,
                         int64_t n, int64_t k, int64_t m) {
    if (int r = check_shape("gemv_q4_0_f16_add", n, k)) return r;
    MI_CHECK_ARG(w_packed && x_f16 && y, "gemv_q4_0_f16_add: null pointer");
    MI_CHECK_ARG(mi::aligned(w_packed, 256) && mi::aligned(x_f16, 16), "gemv_q4_0_f16_add: w_packed must be 256-byte, x 16-byte aligned");
    return launch_gx((hipStream_t)stream, (const uint8_t *)w_packed, n, k, m, x_f16, y, add);
}

size_t mi_mul_mat_q4_0_workspace_size(int64_t m, int64_t k) {
    if (m > 1) return mfma_x_ok(k) ? mi::align_up((size_t)m * k * 2, 256) : 0;  // permuted fp16 rows
    if (k * 2 <= 64 * 1024) return 0;
    return mi::align_up((size_t)m * k * 2, 256);
}

int mi_mul_mat_q4_0_f32(void *stream, const void *w_packed, const float *x, float *y, int64_t n, int64_t k,
                        int64_t m, void *ws, size_t ws_bytes) {
    if (int r = check_shape("mul_mat_q4_0_f32", n, k)) return r;
    MI_CHECK_ARG(w_packed && x && y, "mul_mat_q4_0_f32: null pointer");
    MI_CHECK_ARG(m >= 1 && m <= 16, "mul_mat_q4_0_f32: m=%lld not in 1..16", (long long)m);
    MI_CHECK_ARG(mi::aligned(w_packed, 256) && mi::aligned(x, 16), "mul_mat_q4_0_f32: w_packed must be 256-byte, x 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (m > 1) {
        if (!mfma_x_ok(k)) return launch_mfma<true>(st, (const uint8_t *)w_packed, n, k, m, x, y, nullptr);
        const size_t need = mi_mul_mat_q4_0_workspace_size(m, k);
        if (!ws || ws_bytes < need || !mi::aligned(ws, 16)) {
            mi::set_error("mul_mat_q4_0_f32: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
            return MI_ERR_WORKSPACE;
        }
        return launch_mfma_x(st, (const uint8_t *)w_packed, n, k, m, x, true, y, nullptr, ws);
    }
    // one fp32 row: the register kernel (the fused chains' arithmetic, so that fused and
    // node-by-node graphs agree bit for bit) while the fp16 row fits 64 KB of LDS
    if (xr_enabled() && k / QK <= 1008) return launch_xr_gemv(st, (const uint8_t *)w_packed, n, k, x, true, y, nullptr);
    const size_t need = mi_mul_mat_q4_0_workspace_size(m, k);
    if (need == 0) return launch_lds(st, (const uint8_t *)w_packed, n, k, m, x, y);
    if (!ws || ws_bytes < need || !mi::aligned(ws, 16)) {
        mi::set_error("mul_mat_q4_0_f32: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    if (int r = mi_cast_f32_f16(stream, x, (uint16_t *)ws, m * k)) return r;
    return launch_gx(st, (const uint8_t *)w_packed, n, k, m, (const uint16_t *)ws, y);
}

int mi_mul_mat_q4_0_f32_batch(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, const float *const *bias, const float *const *add, int64_t k,
                              int64_t m, const float *x, const float *up, const float *norm_w, float eps, void *ws,
                              size_t ws_bytes) {
    MI_CHECK_ARG(n_mats >= 1 && n_mats <= 4, "mul_mat_q4_0_f32_batch: %d matrices (1..4)", n_mats);
    MI_CHECK_ARG(w_packed && n && y && x, "mul_mat_q4_0_f32_batch: null pointer");
    MI_CHECK_ARG(m >= 1 && m <= 16, "mul_mat_q4_0_f32_batch: m=%lld not in 1..16", (long long)m);
    MI_CHECK_ARG(k % (4 * QK) == 0, "mul_mat_q4_0_f32_batch: k=%lld not a multiple of 128", (long long)k);
    int64_t rows = 0;
    const uint8_t *base[4];
    for (int i = 0; i < n_mats; i++) {
        if (int r = check_shape("mul_mat_q4_0_f32_batch", n[i], k)) return r;
        MI_CHECK_ARG(w_packed[i] && y[i], "mul_mat_q4_0_f32_batch: matrix %d: null pointer", i);
        MI_CHECK_ARG(mi::aligned(w_packed[i], 256), "mul_mat_q4_0_f32_batch: packed weight %d not 256-byte aligned",
                     i);
        base[i] = (const uint8_t *)w_packed[i];
        rows += n[i];
    }
    MI_CHECK_ARG(rows < (1ll << 31), "mul_mat_q4_0_f32_batch: too many rows");
    MI_CHECK_ARG(mi::aligned(x, 4) && (!up || mi::aligned(up, 4)), "mul_mat_q4_0_f32_batch: misaligned activation");
    MI_CHECK_ARG(!(up && norm_w), "mul_mat_q4_0_f32_batch: up and norm_w are exclusive");
    MI_CHECK_ARG(!norm_w || (k <= 4096 && mi::aligned(x, 16) && mi::aligned(norm_w, 16)),
                 "mul_mat_q4_0_f32_batch: the fused RMSNorm needs k <= 4096 and 16-byte aligned x / norm_w");
    const size_t need = (size_t)m * k * 2;
    if (!ws || ws_bytes < need || !mi::aligned(ws, 16)) {
        mi::set_error("mul_mat_q4_0_f32_batch: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    return launch_mfma_set((hipStream_t)stream, n_mats, base, n, y, bias, add, k, m, x, up ? PERM_GLU : PERM_F32, up,
                           ws, norm_w, eps);
}

int mi_mul_mat_q4_0_batch_xp(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                             float *const *y, const float *const *bias, const float *const *add, int64_t k,
                             int64_t m, const void *xp) {
    MI_CHECK_ARG(n_mats >= 1 && n_mats <= 4, "mul_mat_q4_0_batch_xp: %d matrices (1..4)", n_mats);
    MI_CHECK_ARG(w_packed && n && y && xp, "mul_mat_q4_0_batch_xp: null pointer");
    MI_CHECK_ARG(m >= 1 && m <= 16, "mul_mat_q4_0_batch_xp: m=%lld not in 1..16", (long long)m);
    MI_CHECK_ARG(k % (4 * QK) == 0, "mul_mat_q4_0_batch_xp: k=%lld not a multiple of 128", (long long)k);
    MI_CHECK_ARG(mi::aligned(xp, 16), "mul_mat_q4_0_batch_xp: xp not 16-byte aligned");
    int64_t rows = 0;
    const uint8_t *base[4];
    for (int i = 0; i < n_mats; i++) {
        if (int r = check_shape("mul_mat_q4_0_batch_xp", n[i], k)) return r;
        MI_CHECK_ARG(w_packed[i] && y[i], "mul_mat_q4_0_batch_xp: matrix %d: null pointer", i);
        MI_CHECK_ARG(mi::aligned(w_packed[i], 256), "mul_mat_q4_0_batch_xp: packed weight %d not 256-byte aligned", i);
        base[i] = (const uint8_t *)w_packed[i];
        rows += n[i];
    }
    MI_CHECK_ARG(rows < (1ll << 31), "mul_mat_q4_0_batch_xp: too many rows");
    return launch_mfma_set((hipStream_t)stream, n_mats, base, n, y, bias, add, k, m, xp, PERM_READY, nullptr,
                           nullptr);
}

int mi_mul_mat_q4_0_gate_up_glu_batch(void *stream, const void *w_gate, const void *w_up, int64_t n, int64_t k,
                                      int64_t m, const float *x, const float *norm_w, float eps, void *ws,
                                      size_t ws_bytes, void *hxp) {
    MI_CHECK_ARG(w_gate && w_up && x && hxp, "mul_mat_q4_0_gate_up_glu_batch: null pointer");
    if (int r = check_shape("mul_mat_q4_0_gate_up_glu_batch", n, k)) return r;
    MI_CHECK_ARG(m >= 1 && m <= 16, "mul_mat_q4_0_gate_up_glu_batch: m=%lld not in 1..16", (long long)m);
    MI_CHECK_ARG(k % (4 * QK) == 0 && n % (4 * QK) == 0,
                 "mul_mat_q4_0_gate_up_glu_batch: k=%lld and n=%lld must be multiples of 128", (long long)k,
                 (long long)n);
    MI_CHECK_ARG(mi::aligned(w_gate, 256) && mi::aligned(w_up, 256),
                 "mul_mat_q4_0_gate_up_glu_batch: packed weights not 256-byte aligned");
    MI_CHECK_ARG(mi::aligned(x, 16) && mi::aligned(hxp, 16) && (!norm_w || (k <= 4096 && mi::aligned(norm_w, 16))),
                 "mul_mat_q4_0_gate_up_glu_batch: x, hxp (and norm_w, k <= 4096) must be 16-byte aligned");
    const size_t need = (size_t)m * k * 2;
    if (!ws || ws_bytes < need || !mi::aligned(ws, 16)) {
        mi::set_error("mul_mat_q4_0_gate_up_glu_batch: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    const uint8_t *wsb = (const uint8_t *)ws, *hb = (const uint8_t *)hxp;
    MI_CHECK_ARG(hb + (size_t)m * n * 2 <= wsb || wsb + need <= hb,
                 "mul_mat_q4_0_gate_up_glu_batch: hxp overlaps the workspace");
    return launch_mfma_glu((hipStream_t)stream, (const uint8_t *)w_gate, (const uint8_t *)w_up, n, k, m, x, norm_w,
                           eps, ws, (uint16_t *)hxp);
}

int mi_qkv_rope_kv_q4_0_batch(void *stream, const void *const *w_packed, const int64_t *n, const float *const *bias,
                              int64_t k, int64_t m, const float *x, const float *norm_w, float eps, void *ws,
                              size_t ws_bytes, int64_t head_dim, const int32_t *pos, float freq_base,
                              float freq_scale, float attn_factor, float *q_out, void *k_cache, size_t k_row_bytes,
                              void *v_cache, size_t v_row_bytes, const void *kv_idx, int kv_idx_is_i64,
                              int64_t n_cache_rows) {
    MI_CHECK_ARG(w_packed && n && x && pos && q_out && k_cache && v_cache && kv_idx,
                 "qkv_rope_kv_q4_0_batch: null pointer");
    MI_CHECK_ARG(m >= 1 && m <= 16, "qkv_rope_kv_q4_0_batch: m=%lld not in 1..16", (long long)m);
    MI_CHECK_ARG(k % (4 * QK) == 0, "qkv_rope_kv_q4_0_batch: k=%lld not a multiple of 128", (long long)k);
    MI_CHECK_ARG(head_dim >= 32 && head_dim <= 256 && head_dim % 32 == 0 && n[0] % head_dim == 0 &&
                     n[1] % head_dim == 0 && n[2] % 32 == 0,
                 "qkv_rope_kv_q4_0_batch: head_dim %lld / rows %lld %lld %lld not supported", (long long)head_dim,
                 (long long)n[0], (long long)n[1], (long long)n[2]);
    const uint8_t *base[3];
    for (int i = 0; i < 3; i++) {
        if (int r = check_shape("qkv_rope_kv_q4_0_batch", n[i], k)) return r;
        MI_CHECK_ARG(w_packed[i] && mi::aligned(w_packed[i], 256),
                     "qkv_rope_kv_q4_0_batch: packed weight %d null or not 256-byte aligned", i);
        base[i] = (const uint8_t *)w_packed[i];
    }
    MI_CHECK_ARG(k_row_bytes >= (size_t)n[1] * 2 && v_row_bytes >= (size_t)n[2] * 2,
                 "qkv_rope_kv_q4_0_batch: cache rows too short");
    MI_CHECK_ARG(mi::aligned(x, 16) && (!norm_w || (k <= 4096 && mi::aligned(norm_w, 16))),
                 "qkv_rope_kv_q4_0_batch: x (and norm_w, k <= 4096) must be 16-byte aligned");
    const size_t need = (size_t)m * k * 2;
    if (!ws || ws_bytes < need || !mi::aligned(ws, 16)) {
        mi::set_error("qkv_rope_kv_q4_0_batch: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    Q4BRope RP;
    RP.q_out = q_out;
    RP.kc = (uint8_t *)k_cache;
    RP.vc = (uint8_t *)v_cache;
    RP.pos = pos;
    RP.kv_idx = kv_idx;
    RP.kv_i64 = kv_idx_is_i64;
    RP.hd = (int)head_dim;
    RP.k_row_bytes = k_row_bytes;
    RP.v_row_bytes = v_row_bytes;
    RP.n_cache_rows = n_cache_rows;
    RP.theta_scale = powf(freq_base, -2.0f / (float)head_dim);
    RP.freq_scale = freq_scale;
    RP.attn_factor = attn_factor;
    return launch_mfma_rope((hipStream_t)stream, base, n, bias, k, m, x, norm_w, eps, ws, RP);
}

int mi_mul_mat_q4_0_f32_fused(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, const float *const *add, int64_t k, const float *x,
                              const float *norm_w, float eps) {
    MI_CHECK_ARG(w_packed && n && y && x, "mul_mat_q4_0_f32_fused: null pointer");
    if (int r = check_shape("mul_mat_q4_0_f32_fused", 1, k)) return r;
    // the fp16 copy of the row and the reduction slots fit 64 KB of LDS up to 1008 blocks
    MI_CHECK_ARG(k <= (norm_w ? 4096 : 1008 * QK), "mul_mat_q4_0_f32_fused: k=%lld too long", (long long)k);
    MI_CHECK_ARG(mi::aligned(x, 16) && (!norm_w || mi::aligned(norm_w, 16)),
                 "mul_mat_q4_0_f32_fused: x/norm_w must be 16-byte aligned");
    for (int i = 0; i < n_mats && i < 4; i++) MI_CHECK_ARG(y[i], "mul_mat_q4_0_f32_fused: y[%d] is NULL", i);
    Q4Set S;
    int n_total = 0;
    if (int r = make_q4set(S, n_mats, w_packed, n, y, add, k, n_total)) return r;
    RopeKV R{};
    if (!norm_w && k > 4096) {
        XrShape sh;
        xr_shape(k / QK, sh);
        return launch_xr_any<true, XR_PAIRS>((hipStream_t)stream, sh, S, x, (int)(k / QK), (n_total + 1) / 2, n_total,
                                             R, nullptr);
    }
    return launch_xr_short<XR_PAIRS>((hipStream_t)stream, S, x, norm_w, eps, (int)(k / QK), (n_total + 1) / 2,
                                     n_total, R, nullptr);
}

int mi_gate_up_swiglu_q4_0(void *stream, const void *w_gate, const void *w_up, int64_t n, int64_t k, const float *x,
                           const float *norm_w, float eps, uint16_t *h_out) {
    MI_CHECK_ARG(w_gate && w_up && x && h_out, "gate_up_swiglu_q4_0: null pointer");
    if (int r = check_shape("gate_up_swiglu_q4_0", n, k)) return r;
    MI_CHECK_ARG(k <= 4096, "gate_up_swiglu_q4_0: k=%lld > 4096", (long long)k);
    MI_CHECK_ARG(mi::aligned(x, 16) && (!norm_w || mi::aligned(norm_w, 16)),
                 "gate_up_swiglu_q4_0: x/norm_w must be 16-byte aligned");
    Q4Set S;
    int n_total = 0;
    const void *w[2] = {w_gate, w_up};
    const int64_t nn[2] = {n, n};
    if (int r = make_q4set(S, 2, w, nn, nullptr, nullptr, k, n_total)) return r;
    RopeKV R{};
    return launch_xr_short<XR_GLU>((hipStream_t)stream, S, x, norm_w, eps, (int)(k / QK), (int)n, n_total, R, h_out);
}

int mi_qkv_rope_kv_q4_0(void *stream, const void *const *w_packed, const int64_t *n, const float *const *bias,
                        int64_t k, const float *x, const float *norm_w, float eps, int64_t head_dim,
                        const int32_t *pos, float freq_base, float freq_scale, float attn_factor, float *q_out,
                        void *k_cache, size_t k_row_bytes, void *v_cache, size_t v_row_bytes, const void *kv_idx,
                        int kv_idx_is_i64, int64_t n_cache_rows, const float *rope_table) {
    MI_CHECK_ARG(w_packed && n && bias && x && pos && q_out && k_cache && v_cache && kv_idx,
                 "qkv_rope_kv_q4_0: null pointer");
    if (int r = check_shape("qkv_rope_kv_q4_0", 1, k)) return r;
    MI_CHECK_ARG(k <= 4096, "qkv_rope_kv_q4_0: k=%lld > 4096", (long long)k);
    MI_CHECK_ARG(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 128, "qkv_rope_kv_q4_0: head_dim %lld (even, <= 128)",
                 (long long)head_dim);
    MI_CHECK_ARG(n[0] > 0 && n[1] > 0 && n[2] > 0 && n[0] % head_dim == 0 && n[1] % head_dim == 0 && n[2] % 2 == 0,
                 "qkv_rope_kv_q4_0: q/k rows must be whole heads, v rows even");
    MI_CHECK_ARG(k_row_bytes >= (size_t)n[1] * 2 && v_row_bytes >= (size_t)n[2] * 2 && n_cache_rows > 0,
                 "qkv_rope_kv_q4_0: cache rows too short");
    MI_CHECK_ARG(mi::aligned(x, 16) && (!norm_w || mi::aligned(norm_w, 16)),
                 "qkv_rope_kv_q4_0: x/norm_w must be 16-byte aligned");
    Q4Set S;
    int n_total = 0;
    if (int r = make_q4set(S, 3, w_packed, n, nullptr, bias, k, n_total)) return r;
    RopeKV R{};
    R.q_out = q_out;
    R.k_cache = (uint8_t *)k_cache;
    R.v_cache = (uint8_t *)v_cache;
    R.k_row_bytes = k_row_bytes;
    R.v_row_bytes = v_row_bytes;
    R.pos = pos;
    R.kv_idx = kv_idx;
    R.kv_idx_i64 = kv_idx_is_i64;
    R.n_cache_rows = n_cache_rows;
    R.hd = (int)head_dim;
    R.n_q = (int)n[0];
    R.n_k = (int)n[1];
    R.n_v = (int)n[2];
    // theta_scale on the host with the C library powf, as the CPU rope cache does
    R.theta_scale = powf(freq_base, -2.0f / (float)head_dim);
    R.freq_scale = freq_scale;
    R.attn_factor = attn_factor;
    R.tab = rope_table;
    const int units = (R.n_q + R.n_k) / 2 + R.n_v / 2;
    return launch_xr_short<XR_ROPE>((hipStream_t)stream, S, x, norm_w, eps, (int)(k / QK), units, n_total, R,
                                    nullptr);
}

int mi_cast_f32_f16(void *stream, const float *x, uint16_t *y, int64_t n) {
    MI_CHECK_ARG(x && y && n > 0 && n % 4 == 0, "cast_f32_f16: bad arguments");
    MI_CHECK_ARG(mi::aligned(x, 16) && mi::aligned(y, 8), "cast_f32_f16: x must be 16-byte, y 8-byte aligned");
    const int64_t n4 = n / 4;
    hipLaunchKernelGGL(k_cast_f16, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, y, n4);
    MI_CHECK_LAUNCH("k_cast_f16");
    return MI_OK;
}

}  // extern "C"
