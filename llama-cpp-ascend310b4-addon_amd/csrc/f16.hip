// f16.hip -- F16 decode GEMV for gfx950 (the tied fp16 output head).
//
// ggml's F16 mul_mat converts the fp32 activation to fp16 (its vec_dot type)
// and accumulates exact fp16 x fp16 products in fp32; this kernel does the same
// with v_dot2_f32_f16.  The ggml ND layout (each row contiguous along K) is
// already the streaming layout a wavefront wants (16 B per lane, whole 128 B
// lines per 8 lanes), so F16 weights need no side copy.  Replaces the
// cast + aclnnMatmul(FRACTAL_NZ) + cast chain of patch:1286-1309 and the
// tied-output NZ side copy of patch:1451-1464.
#include "decode_common.h"
#include "mi_common.h"

#include <limits.h>
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

constexpr int kHeadRI = 2;  // row groups per head workgroup (4 measured slower: 69.9 / 156.6 us)

// The tied output head of a decode token with its neighbours in the graph folded in:
// the output RMSNorm ((x*scale)*norm_w, as k_rms_norm then MUL compute it; XStage)
// converted to fp16 into LDS as k_gemv_f16 converts its activation, k_gemv_f16<G,U,1>'s
// row dot (same lanes, same order: the logits are bit-identical), and per workgroup the
// first maximum of its rows, ARGMAX's first pass (strict >, so NaN is never taken and
// ties keep the lower row; -inf rows leave the workgroup's first row).
template <int G, int U, int XN>
__global__ __launch_bounds__(256) void k_head_f16(const uint16_t *__restrict__ w, int64_t ldw,
                                                  const float *__restrict__ x, const float *__restrict__ norm_w,
                                                  float eps, float *__restrict__ y, float2 *__restrict__ part, int n,
                                                  int k) {
    constexpr int RPB = 256 / G;          // rows per pass of the workgroup
    constexpr int RPW = RPB * kHeadRI;    // rows per workgroup (one norm prologue for all)
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t *s_x = (uint16_t *)smem;  // [k] fp16
    __shared__ double s_red[4];
    __shared__ float s_v[RPW];
    __shared__ int s_i[RPW];
    const int tid = threadIdx.x;
    const int j = tid % G;
    const int row0 = blockIdx.x * RPW + tid / G;  // this thread's rows: row0 + ri * RPB
    const int nc = k / 8, k4 = k / 4;

    // the first pass of two row groups in flight (the first two during the norm prologue,
    // each later one while the group two before it is consumed)
    constexpr int NBUF = kHeadRI < 2 ? kHeadRI : 2;
    int4 wv[NBUF][U];
    auto first_pass = [&](int ri, int4 (&dst)[U]) {
        const uint16_t *wr = w + (size_t)min(row0 + ri * RPB, n - 1) * ldw;
#pragma unroll
        for (int u = 0; u < U; u++) dst[u] = ld_stream16(wr + (size_t)min(j + u * G, nc - 1) * 8);
    };
#pragma unroll
    for (int ri = 0; ri < NBUF; ri++) first_pass(ri, wv[ri]);

    XStage<XN, true> st;
    xstage_load(st, x, norm_w, nullptr, k4, tid);
    const float scale = xstage_scale(st, k4, eps, s_red, tid);
#pragma unroll
    for (int t = 0; t < XN; t++) {
        const int f = tid + t * 256;
        if (f < k4) {
            const float4 v = xstage_value(st, scale, t);
            *(uint2 *)(s_x + (size_t)f * 4) = make_uint2((uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16),
                                                         (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16));
        }
    }
    __syncthreads();

#pragma unroll
    for (int ri = 0; ri < kHeadRI; ri++) {
        const int row = row0 + ri * RPB;
        const uint16_t *wr = w + (size_t)min(row, n - 1) * ldw;
        float acc = 0.0f;
        auto consume = [&](int c, const int4 &wq) {
            const int4 xv = *(const int4 *)(s_x + (size_t)c * 8);
            float s = acc;
            s = fdot2((uint32_t)wq.x, (uint32_t)xv.x, s);
            s = fdot2((uint32_t)wq.y, (uint32_t)xv.y, s);
            s = fdot2((uint32_t)wq.z, (uint32_t)xv.z, s);
            s = fdot2((uint32_t)wq.w, (uint32_t)xv.w, s);
            acc = s;
        };
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = j + u * G;
            if (c < nc) consume(c, wv[ri % NBUF][u]);
        }
        if (ri + NBUF < kHeadRI) first_pass(ri + NBUF, wv[ri % NBUF]);
        for (int c0 = U * G; c0 < nc; c0 += U * G) {
            int4 wq[U];
#pragma unroll
            for (int u = 0; u < U; u++) wq[u] = ld_stream16(wr + (size_t)min(c0 + j + u * G, nc - 1) * 8);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = c0 + j + u * G;
                if (c < nc) consume(c, wq[u]);
            }
        }
        const float v = group_sum<G>(acc);
        if (j == 0) {
            if (row < n) y[row] = v;
            s_v[ri * RPB + tid / G] = row < n ? v : -INFINITY;
            s_i[ri * RPB + tid / G] = row;
        }
    }
    __syncthreads();
    if (tid == 0) {  // the rows in ascending order
        float best = -INFINITY;
        int bi = blockIdx.x * RPW;
#pragma unroll
        for (int r = 0; r < RPW; r++)
            if (s_v[r] > best) {
                best = s_v[r];
                bi = s_i[r];
            }
        part[blockIdx.x] = make_float2(best, __int_as_float(bi));
    }
}

// ARGMAX's final pass over the head's per-workgroup partials (one per 8..32 rows: ~9.5K
// for a 152K vocabulary): the first maximum (equal values keep the lower index).  1024
// threads, each with 8 partials' loads in flight per step: one thread walking its share
// with one load at a time took ~24 us.
__global__ __launch_bounds__(1024) void k_head_argmax_final(const float2 *__restrict__ part, int n_parts,
                                                            int32_t *__restrict__ out) {
    constexpr int B = 8;
    __shared__ float sv[16];
    __shared__ int si[16];
    auto merge = [](float &v, int &i, float v2, int i2) {
        if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    };
    float best = -INFINITY;
    int bi = INT_MAX;
    for (int c0 = threadIdx.x; c0 < n_parts; c0 += 1024 * B) {
        float2 p[B];
#pragma unroll
        for (int b = 0; b < B; b++) {
            const int c = c0 + b * 1024;
            p[b] = c < n_parts ? part[c] : make_float2(-INFINITY, __int_as_float(INT_MAX));
        }
#pragma unroll
        for (int b = 0; b < B; b++) merge(best, bi, p[b].x, __float_as_int(p[b].y));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) merge(best, bi, __shfl_xor(best, o, 64), __shfl_xor(bi, o, 64));
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = best; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        best = sv[0];
        bi = si[0];
#pragma unroll
        for (int w = 1; w < 16; w++) merge(best, bi, sv[w], si[w]);
        out[0] = bi == INT_MAX ? 0 : bi;
    }
}

// the lanes per row and the rows per pass of k_gemv_f16<G, U, 1> at this k
int head_g(int64_t k) { return k / 8 <= 128 ? 16 : (k / 8 <= 256 ? 32 : 64); }
int head_u(int64_t k, int g) {
    int64_t u = (k / 8 + g - 1) / g;
    if (u > 8) u = (u + 1) / 2 > 8 ? 8 : (u + 1) / 2;
    return (int)u;
}

template <int G, int U, int XN>
int launch_head_gux(hipStream_t st, const uint16_t *w, int64_t ldw, const float *x, const float *norm_w, float eps,
                    float *y, float2 *part, int64_t n, int64_t k) {
    constexpr int RPW = 256 / G * kHeadRI;
    hipLaunchKernelGGL((k_head_f16<G, U, XN>), dim3((unsigned)((n + RPW - 1) / RPW)), dim3(256), (size_t)k * 2, st, w,
                       ldw, x, norm_w, eps, y, part, (int)n, (int)k);
    MI_CHECK_LAUNCH("k_head_f16");
    return MI_OK;
}

template <int G, int XN>
int launch_head_gx(hipStream_t st, const uint16_t *w, int64_t ldw, const float *x, const float *norm_w, float eps,
                   float *y, float2 *part, int64_t n, int64_t k) {
#define MI_U_CASE(UU) case UU: return launch_head_gux<G, UU, XN>(st, w, ldw, x, norm_w, eps, y, part, n, k);
    switch (head_u(k, G)) {
        MI_U_CASE(1) MI_U_CASE(2) MI_U_CASE(3) MI_U_CASE(4) MI_U_CASE(5) MI_U_CASE(6) MI_U_CASE(7) MI_U_CASE(8)
    }
#undef MI_U_CASE
    return MI_ERR_ARG;
}

template <int XN>
int launch_head_x(hipStream_t st, const uint16_t *w, int64_t ldw, const float *x, const float *norm_w, float eps,
                  float *y, float2 *part, int64_t n, int64_t k) {
    switch (head_g(k)) {
        case 16: return launch_head_gx<16, XN>(st, w, ldw, x, norm_w, eps, y, part, n, k);
        case 32: return launch_head_gx<32, XN>(st, w, ldw, x, norm_w, eps, y, part, n, k);
        default: return launch_head_gx<64, XN>(st, w, ldw, x, norm_w, eps, y, part, n, k);
    }
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

extern "C" size_t mi_head_f16_argmax_workspace_size(int64_t n, int64_t k) {
    if (n <= 0 || k <= 0) return 0;
    const int64_t rpw = 256 / head_g(k) * kHeadRI;
    return mi::align_up((size_t)((n + rpw - 1) / rpw) * sizeof(float2), 256);
}

extern "C" int mi_head_f16_argmax(void *stream, const uint16_t *w, int64_t ldw, const float *x, const float *norm_w,
                                  float eps, float *y, int32_t *out, int64_t n, int64_t k, void *ws,
                                  size_t ws_bytes) {
    MI_CHECK_ARG(w && x && norm_w && y && out, "head_f16_argmax: null pointer");
    MI_CHECK_ARG(n > 0 && k > 0 && k % 32 == 0 && k <= 4096 && ldw >= k && ldw % 8 == 0 && n < (1ll << 31),
                 "head_f16_argmax: bad shape n=%lld k=%lld ldw=%lld (k a multiple of 32, <= 4096)", (long long)n,
                 (long long)k, (long long)ldw);
    MI_CHECK_ARG(mi::aligned(w, 16) && mi::aligned(x, 16) && mi::aligned(norm_w, 16),
                 "head_f16_argmax: w, x and norm_w must be 16-byte aligned");
    const size_t need = mi_head_f16_argmax_workspace_size(n, k);
    if (!ws || ws_bytes < need || !mi::aligned(ws, 8)) {
        mi::set_error("head_f16_argmax: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    hipStream_t st = (hipStream_t)stream;
    float2 *part = (float2 *)ws;
    const int r = k <= 2048 ? launch_head_x<2>(st, w, ldw, x, norm_w, eps, y, part, n, k)
                            : launch_head_x<4>(st, w, ldw, x, norm_w, eps, y, part, n, k);
    if (r) return r;
    const int64_t rpw = 256 / head_g(k) * kHeadRI;
    hipLaunchKernelGGL(k_head_argmax_final, dim3(1), dim3(1024), 0, st, (const float2 *)part,
                       (int)((n + rpw - 1) / rpw), out);
    MI_CHECK_LAUNCH("k_head_argmax_final");
    return MI_OK;
}

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
