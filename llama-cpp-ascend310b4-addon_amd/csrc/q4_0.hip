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

#include <string.h>

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

// fp32 -> fp16 (round to nearest even, as ggml's activation conversion)
__global__ __launch_bounds__(256) void k_cast_f16(const float *__restrict__ x, uint16_t *__restrict__ y, int64_t n4) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float4 v = ((const float4 *)x)[i];
    ((uint2 *)y)[i] = make_uint2((uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16),
                                 (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16));
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

int launch_gx(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const uint16_t *x16, float *y,
              const float *add = nullptr) {
    if (m >= 2 && m <= 16) return launch_mfma<false>(st, base, n, k, m, x16, y, add);
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
    if (m > 1 || k * 2 <= 64 * 1024) return 0;  // matrix cores read fp32 rows directly
    return mi::align_up((size_t)m * k * 2, 256);
}

int mi_mul_mat_q4_0_f32(void *stream, const void *w_packed, const float *x, float *y, int64_t n, int64_t k,
                        int64_t m, void *ws, size_t ws_bytes) {
    if (int r = check_shape("mul_mat_q4_0_f32", n, k)) return r;
    MI_CHECK_ARG(w_packed && x && y, "mul_mat_q4_0_f32: null pointer");
    MI_CHECK_ARG(m >= 1 && m <= 16, "mul_mat_q4_0_f32: m=%lld not in 1..16", (long long)m);
    MI_CHECK_ARG(mi::aligned(w_packed, 256) && mi::aligned(x, 16), "mul_mat_q4_0_f32: w_packed must be 256-byte, x 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (m > 1) return launch_mfma<true>(st, (const uint8_t *)w_packed, n, k, m, x, y, nullptr);
    const size_t need = mi_mul_mat_q4_0_workspace_size(m, k);
    if (need == 0) return launch_lds(st, (const uint8_t *)w_packed, n, k, m, x, y);
    if (!ws || ws_bytes < need || !mi::aligned(ws, 16)) {
        mi::set_error("mul_mat_q4_0_f32: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    if (int r = mi_cast_f32_f16(stream, x, (uint16_t *)ws, m * k)) return r;
    return launch_gx(st, (const uint8_t *)w_packed, n, k, m, (const uint16_t *)ws, y);
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
