// f16.hip -- F16 decode GEMV for gfx950 (the tied fp16 output head).
//
// ggml's F16 mul_mat converts the fp32 activation to fp16 (its vec_dot type)
// and accumulates exact fp16 x fp16 products in fp32; this kernel does the same
// with v_dot2_f32_f16.  The ggml ND layout (each row contiguous along K) is
// already the streaming layout a wavefront wants (16 B per lane, whole 128 B
// lines per 8 lanes), so F16 weights need no side copy.  Replaces the
// cast + aclnnMatmul(FRACTAL_NZ) + cast chain of patch:1286-1309 and the
// tied-output NZ side copy of patch:1451-1464.
#include "mi_common.h"

#include <stdlib.h>

#include <algorithm>

namespace {

using namespace mi;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

template <int G, int U, int M>
__global__ __launch_bounds__(256) void k_gemv_f16(const uint16_t *__restrict__ w, int64_t ldw,
                                                  const float *__restrict__ x, float *__restrict__ y, int n, int k,
                                                  int m) {
    constexpr int RPB = 256 / G;
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t *s_x = (uint16_t *)smem;  // [M][k] fp16
    const int tid = threadIdx.x;
    const int j = tid % G;
    const int row = blockIdx.x * RPB + tid / G;
    const bool row_ok = row < n;
    const int nc = k / 8;  // 16-byte chunks per row
    const uint16_t *wr = w + (size_t)min(row, n - 1) * ldw;

    int4 wv[U];
#pragma unroll
    for (int u = 0; u < U; u++) wv[u] = ld_stream16(wr + (size_t)min(j + u * G, nc - 1) * 8);

    for (int i = tid * 4; i < m * k; i += 256 * 4) {
        const float4 v = *(const float4 *)(x + i);
        *(uint2 *)(s_x + i) = make_uint2((uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16),
                                         (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16));
    }
    __syncthreads();

    float acc[M];
#pragma unroll
    for (int i = 0; i < M; i++) acc[i] = 0.0f;

    auto consume = [&](int c, const int4 &wq) {
#pragma unroll
        for (int i = 0; i < M; i++) {
            if (i < m) {
                const int4 xv = *(const int4 *)(s_x + (size_t)i * k + c * 8);
                float s = acc[i];
                s = fdot2((uint32_t)wq.x, (uint32_t)xv.x, s);
                s = fdot2((uint32_t)wq.y, (uint32_t)xv.y, s);
                s = fdot2((uint32_t)wq.z, (uint32_t)xv.z, s);
                s = fdot2((uint32_t)wq.w, (uint32_t)xv.w, s);
                acc[i] = s;
            }
        }
    };

#pragma unroll
    for (int u = 0; u < U; u++) {
        const int c = j + u * G;
        if (c < nc) consume(c, wv[u]);
    }
    for (int c0 = U * G; c0 < nc; c0 += U * G) {
#pragma unroll
        for (int u = 0; u < U; u++) wv[u] = ld_stream16(wr + (size_t)min(c0 + j + u * G, nc - 1) * 8);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = c0 + j + u * G;
            if (c < nc) consume(c, wv[u]);
        }
    }

#pragma unroll
    for (int i = 0; i < M; i++) {
        const float s = group_sum<G>(acc[i]);
        if (row_ok && j == 0 && i < m) y[(size_t)i * n + row] = s;
    }
}

// Several activation rows (2..8) on the matrix cores: D[16 x rows][16 weight rows] +=
// X[16 x 32 k] . W^T[32 k x 16 weight rows], one v_mfma_f32_16x16x32_f16 per 32-k step.
// Lane (g, c) loads 16 bytes of weight row n0 + c at k 32s + 8g (a row's 4 lanes read 64
// contiguous bytes) and the x fragment of row c at the same k from LDS; it receives x rows
// 4g..4g+3 against weight row n0 + c.  The activation is staged once per workgroup as
// fp16 (RNE, as ggml converts src1 to the F16 vec-dot type), rows padded by 16 bytes
// (LDS banks); rows past m read row m - 1, whose products land in output rows that are
// never stored.  Each wave owns whole 16-row tiles (all of k: no cross-wave reduction)
// and walks them with a stride of the grid; two register stages of U steps each.  The
// B-operand loads cover 16 rows x 64 bytes per instruction; the same bytes read as 4 rows
// x 256 contiguous bytes measured 20% faster (a cross-lane exchange would be needed, and
// its LDS does not fit beside the activation within 64 KB), while deeper stages, 8- or
// 16-wave workgroups and fewer rows (less LDS, more residency) measured no faster.
template <int U, int NW>
__global__ __launch_bounds__(64 * NW) void k_gemv_f16_mfma(const uint16_t *__restrict__ w, int64_t ldw,
                                                       const float *__restrict__ x, float *__restrict__ y, int n,
                                                       int k, int m, int n_tiles) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t *s_x = (uint16_t *)smem;  // [m][k + 8] fp16
    const int kp = k + 8;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int k4 = k / 4;
    for (int i = tid; i < m * k4; i += 64 * NW) {
        const int r = i / k4, f = i - r * k4;
        const float4 v = ((const float4 *)x)[i];
        *(uint2 *)(s_x + (size_t)r * kp + 4 * f) = make_uint2((uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16),
                                                              (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16));
    }
    __syncthreads();
    const uint16_t *xs = s_x + (size_t)min(c, m - 1) * kp + 8 * g;
    const int ns = k / 32;  // 32-k steps
    for (int t = blockIdx.x * NW + wave; t < n_tiles; t += gridDim.x * NW) {
        const uint16_t *wr = w + (size_t)min(16 * t + c, n - 1) * ldw + 8 * g;
        int4 wa[U], wb[U];
        auto load = [&](int4 (&wv)[U], int s0) {
#pragma unroll
            for (int u = 0; u < U; u++) wv[u] = ld_stream16(wr + 32 * (size_t)min(s0 + u, ns - 1));
        };
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
        auto compute = [&](const int4 (&wv)[U], int s0) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u < ns) {  // uniform
                    const half8_t xf = __builtin_bit_cast(half8_t, *(const uint4 *)(xs + 32 * (s0 + u)));
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf, __builtin_bit_cast(half8_t, wv[u]), acc, 0, 0, 0);
                }
            }
        };
        // the prefetches are unconditional (clamped to the last step, a cache hit)
        load(wa, 0);
        for (int s0 = 0; s0 < ns; s0 += 2 * U) {
            load(wb, s0 + U);
            __builtin_amdgcn_sched_barrier(0);
            compute(wa, s0);
            load(wa, s0 + 2 * U);
            __builtin_amdgcn_sched_barrier(0);
            compute(wb, s0 + U);
        }
        const int col = 16 * t + c;
        if (col < n) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (4 * g + i < m) y[(size_t)(4 * g + i) * n + col] = acc[i];
        }
    }
}

// workgroups of a kernel resident at once for a block size and LDS size
int f16_resident(const void *fn, int threads, size_t smem) {
    int per_cu = 0, cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, smem) != hipSuccess || per_cu < 1)
        per_cu = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    return per_cu * cus;
}

// the matrix-core kernel takes 2..8 rows when k is whole 32-k steps and the fp16 rows fit in LDS
inline bool f16_mfma_ok(int64_t k, int64_t m) {
    static const bool on = [] {
        const char *e = getenv("MI_F16_MFMA");
        return !(e && e[0] == '0');
    }();
    return on && m >= 2 && m <= 8 && k % 32 == 0 && (size_t)m * (k + 8) * 2 <= 64 * 1024;
}

int launch_f16_mfma(hipStream_t st, const uint16_t *w, int64_t ldw, const float *x, float *y, int64_t n, int64_t k,
                    int64_t m) {
    const size_t smem = (size_t)m * (k + 8) * 2;
    const int n_tiles = (int)((n + 15) / 16);
    auto fn = k_gemv_f16_mfma<4, 4>;
    const int grid = std::min((n_tiles + 3) / 4, f16_resident((const void *)fn, 256, smem));
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(256), smem, st, w, ldw, x, y, (int)n, (int)k, (int)m, n_tiles);
    MI_CHECK_LAUNCH("k_gemv_f16_mfma");
    return MI_OK;
}

template <int G, int U, int M>
int launch_gu(hipStream_t st, const uint16_t *w, int64_t ldw, const float *x, float *y, int64_t n, int64_t k,
              int64_t m) {
    constexpr int RPB = 256 / G;
    const size_t smem = (size_t)M * k * 2;
    if (smem > 64 * 1024) {
        set_error("gemv_f16: activation of %d x %lld does not fit in LDS", M, (long long)k);
        return MI_ERR_UNSUPPORTED;
    }
    hipLaunchKernelGGL((k_gemv_f16<G, U, M>), dim3((unsigned)((n + RPB - 1) / RPB)), dim3(256), smem, st, w, ldw, x,
                       y, (int)n, (int)k, (int)m);
    MI_CHECK_LAUNCH("k_gemv_f16");
    return MI_OK;
}

template <int G, int M>
int launch_g(hipStream_t st, const uint16_t *w, int64_t ldw, const float *x, float *y, int64_t n, int64_t k,
             int64_t m) {
    const int64_t nc = k / 8;
    int64_t u = (nc + G - 1) / G;
    if (u > 8) u = (u + 1) / 2 > 8 ? 8 : (u + 1) / 2;
#define MI_U_CASE(UU) case UU: return launch_gu<G, UU, M>(st, w, ldw, x, y, n, k, m);
    switch (u) {
        MI_U_CASE(1) MI_U_CASE(2) MI_U_CASE(3) MI_U_CASE(4) MI_U_CASE(5) MI_U_CASE(6) MI_U_CASE(7) MI_U_CASE(8)
    }
#undef MI_U_CASE
    return MI_ERR_ARG;
}

template <int M>
int launch_m(hipStream_t st, const uint16_t *w, int64_t ldw, const float *x, float *y, int64_t n, int64_t k,
             int64_t m) {
    const int64_t nc = k / 8;
    if (nc <= 128) return launch_g<16, M>(st, w, ldw, x, y, n, k, m);
    if (nc <= 256) return launch_g<32, M>(st, w, ldw, x, y, n, k, m);
    return launch_g<64, M>(st, w, ldw, x, y, n, k, m);
}

}  // namespace

extern "C" int mi_gemv_f16(void *stream, const uint16_t *w, int64_t ldw, const float *x, float *y, int64_t n,
                           int64_t k, int64_t m) {
    MI_CHECK_ARG(w && x && y, "gemv_f16: null pointer");
    MI_CHECK_ARG(n > 0 && k > 0 && k % 8 == 0 && ldw >= k && ldw % 8 == 0,
                 "gemv_f16: bad shape n=%lld k=%lld ldw=%lld (k, ldw multiples of 8)", (long long)n, (long long)k,
                 (long long)ldw);
    MI_CHECK_ARG(mi::aligned(w, 16) && mi::aligned(x, 16), "gemv_f16: w and x must be 16-byte aligned");
    MI_CHECK_ARG(n < (1ll << 31) && k < (1ll << 24), "gemv_f16: shape too large");
    hipStream_t st = (hipStream_t)stream;
    if (f16_mfma_ok(k, m)) return launch_f16_mfma(st, w, ldw, x, y, n, k, m);
    if (m == 1) return launch_m<1>(st, w, ldw, x, y, n, k, m);
    if (m == 2) return launch_m<2>(st, w, ldw, x, y, n, k, m);
    if (m >= 3 && m <= 4) return launch_m<4>(st, w, ldw, x, y, n, k, m);
    if (m >= 5 && m <= 8) return launch_m<8>(st, w, ldw, x, y, n, k, m);
    mi::set_error("gemv_f16: m=%lld not in 1..8", (long long)m);
    return MI_ERR_ARG;
}
