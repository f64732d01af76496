// q8_0.hip -- A8W8 (ggml Q8_0 x Q8_0) decode path for gfx950:
//   * weight prepack into the planar layout (qlo / qhi / d planes),
//   * per-token activation quantization (ggml Q8_0, SmoothQuant divisor folded in),
//   * the GEMV: one lane owns whole 32-blocks, exact int32 block dots with
//     v_dot4_i32_i8, fp32 scaling d_w*d_x fused in the epilogue, split-K over a
//     power-of-two lane group per output row reduced with DPP row ops.
//
// Replaces, on the reference side: the A8W8 weight transform at set_tensor
// (patch:1674-1695, 1700-1809), W8a8QuantizeCustom
// (experiments/a8w8/w8a8_quantize_custom_vector.cpp:20-64), MatmulW8a8I32Custom
// (experiments/a8w8/custom_ops_nz/op_kernel/matmul_w8a8_i32_custom.cpp:15-48)
// and W8a8DequantCustom (called at patch:1269-1270) with its casts.
#include "q8_0_dev.h"

#include <limits.h>
#include <atomic>
#include <math.h>
#include <string.h>

namespace {

using namespace mi;

// ------------------------------------------------------------------ prepack

__global__ void k_prepack_q8_0(const uint8_t *__restrict__ src, uint8_t *__restrict__ qlo,
                               uint8_t *__restrict__ qhi, uint16_t *__restrict__ dpl, int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint16_t *s = (const uint16_t *)(src + i * 34);  // 2-byte aligned block
    uint16_t w[17];
#pragma unroll
    for (int t = 0; t < 17; t++) w[t] = s[t];
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        lo[t] = (uint32_t)w[1 + 2 * t] | ((uint32_t)w[2 + 2 * t] << 16);
        hi[t] = (uint32_t)w[9 + 2 * t] | ((uint32_t)w[10 + 2 * t] << 16);
    }
    *(uint4 *)(qlo + i * 16) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *(uint4 *)(qhi + i * 16) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    dpl[i] = w[0];
}

// ------------------------------------------------------------------ A8W8 weight quantization

// An F16 weight [n][k] (the ggml rows the loader wrote) times the SmoothQuant factors
// s[k] (NULL = none), quantized per 32-block to Q8_0 with ggml's quantize_row_q8_0_ref
// rounding (what llama-quantize writes for Q8_0 weights), straight into the planar side
// copy.  8 lanes per block, 4 values per lane: lanes 0..3 fill the qlo plane's 16 bytes,
// lanes 4..7 the qhi plane's.  grid: ceil(n*nb / 32) x 256.
__global__ __launch_bounds__(256) void k_quantize_f16_q8_0(const uint16_t *__restrict__ w, const float *__restrict__ s,
                                                           uint8_t *__restrict__ qlo, uint8_t *__restrict__ qhi,
                                                           uint16_t *__restrict__ dpl, int64_t k,
                                                           int64_t total_blocks) {
    const int64_t blk = (int64_t)blockIdx.x * 32 + threadIdx.x / 8;
    const int sub = threadIdx.x % 8;
    const bool valid = blk < total_blocks;
    const int64_t nb = k / QK;
    const int64_t b = valid ? blk % nb : 0;
    float v0 = 0.f, v1 = 0.f, v2 = 0.f, v3 = 0.f;
    if (valid) {
        // block blk starts at element blk*32 of the row-major [n][k] weight
        const uint2 h = *(const uint2 *)(w + blk * QK + sub * 4);
        v0 = h2f((uint16_t)(h.x & 0xffff)); v1 = h2f((uint16_t)(h.x >> 16));
        v2 = h2f((uint16_t)(h.y & 0xffff)); v3 = h2f((uint16_t)(h.y >> 16));
        if (s) {
            const float4 sv = *(const float4 *)(s + b * QK + sub * 4);
            v0 *= sv.x; v1 *= sv.y; v2 *= sv.z; v3 *= sv.w;
        }
    }
    float d;
    const uint32_t q = quant4(v0, v1, v2, v3, MI_Q8_ROUND_REF, d);
    if (valid) {
        *(uint32_t *)((sub < 4 ? qlo : qhi) + blk * 16 + (sub & 3) * 4) = q;
        if (sub == 0) dpl[blk] = f2h(d);
    }
}

// ------------------------------------------------------------------ activation quant

// grid: ceil(m*nb / 32) x 256 threads
__global__ __launch_bounds__(256) void k_act_quant_q8_0(const float *__restrict__ x, const float *__restrict__ inv_s,
                                                        int8_t *__restrict__ qs, uint16_t *__restrict__ dout,
                                                        int64_t k, int64_t total_blocks, int rounding,
                                                        const float *__restrict__ up = nullptr) {
    const int64_t blk = (int64_t)blockIdx.x * 32 + threadIdx.x / 8;
    const int sub = threadIdx.x % 8;
    const bool valid = blk < total_blocks;
    const int64_t nb = k / QK;
    const int64_t row = valid ? blk / nb : 0;
    const int64_t b = valid ? blk % nb : 0;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) {
        v = *(const float4 *)(x + row * k + b * QK + sub * 4);
        if (up) {  // ggml's silu(g) * u (k_swiglu)
            const float4 u = *(const float4 *)(up + row * k + b * QK + sub * 4);
            v.x = (v.x / (1.0f + expf(-v.x))) * u.x;
            v.y = (v.y / (1.0f + expf(-v.y))) * u.y;
            v.z = (v.z / (1.0f + expf(-v.z))) * u.z;
            v.w = (v.w / (1.0f + expf(-v.w))) * u.w;
        }
        if (inv_s) {
            const float4 s = *(const float4 *)(inv_s + b * QK + sub * 4);
            v.x *= s.x; v.y *= s.y; v.z *= s.z; v.w *= s.w;
        }
    }
    float d;
    const uint32_t q = quant4(v.x, v.y, v.z, v.w, rounding, d);
    if (valid) {
        *(uint32_t *)(qs + row * k + b * QK + sub * 4) = q;
        if (sub == 0) dout[row * nb + b] = f2h(d);
    }
}

// ------------------------------------------------------------------ GEMV

// Pre-quantized activations (planar xq) read straight from global memory: the
// m*k bytes are shared by every workgroup and stay resident in L1/L2, so no LDS
// staging and no barrier sit between the weight loads and the math.
template <int G, int U, int M>
__global__ __launch_bounds__(256) void k_gemv_q8_0_xq(const uint8_t *__restrict__ qlo, const uint8_t *__restrict__ qhi,
                                                      const uint16_t *__restrict__ wd,
                                                      const int8_t *__restrict__ xq_qs,
                                                      const uint16_t *__restrict__ xq_d, float *__restrict__ y,
                                                      const float *__restrict__ add, int n, int nb, int m) {
    constexpr int RPB = 256 / G;
    const int tid = threadIdx.x;
    const int j = tid % G;
    const int row = blockIdx.x * RPB + tid / G;
    const bool row_ok = row < n;
    const int k = nb * QK;
    const size_t rbase = (size_t)min(row, n - 1) * nb;

    float acc[M];
#pragma unroll
    for (int i = 0; i < M; i++) acc[i] = 0.0f;

    for (int b0 = 0; b0 < nb; b0 += U * G) {
        int4 lo[U], hi[U], xa[U][M], xb[U][M];
        uint32_t dw[U], dx[U][M];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = min(b0 + j + u * G, nb - 1);
            lo[u] = ld_stream16(qlo + (rbase + b) * 16);
            hi[u] = ld_stream16(qhi + (rbase + b) * 16);
            dw[u] = wd[rbase + b];
#pragma unroll
            for (int i = 0; i < M; i++) {
                const int ii = min(i, m - 1);
                const int4 *xs = (const int4 *)(xq_qs + (size_t)ii * k + (size_t)b * QK);
                xa[u][i] = xs[0];
                xb[u][i] = xs[1];
                dx[u][i] = xq_d[(size_t)ii * nb + b];
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (b0 + j + u * G < nb) {
                const float dwf = h2f((uint16_t)dw[u]);
#pragma unroll
                for (int i = 0; i < M; i++) {
                    const int s = dot_block(lo[u], hi[u], xa[u][i], xb[u][i]);
                    acc[i] = fmaf((float)s, dwf * h2f((uint16_t)dx[u][i]), acc[i]);
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < M; i++) {
        const float s = group_sum<G>(acc[i]);
        if (row_ok && j == 0 && i < m) y[(size_t)i * n + row] = add ? s + add[(size_t)i * n + row] : s;
    }
}

// Fused activation quantization (optionally after RMSNorm * norm weight), one
// activation row (m == 1), k <= 1024*XN; results plus the optional add vector.
template <int G, int U, int XN, bool NORM>
__global__ __launch_bounds__(256) void k_gemv_q8_0_fused1(const Q8Set S, const float *__restrict__ x,
                                                          const float *__restrict__ norm_w, float eps,
                                                          const float *__restrict__ inv_s, int n_total, int nb,
                                                          int rounding) {
    constexpr int RPB = 256 / G;
    extern __shared__ __align__(16) uint8_t smem[];
    const FusedLds L = fused_lds(smem, nb);
    const int tid = threadIdx.x;
    const int j = tid % G;
    const int grow = blockIdx.x * RPB + tid / G;
    const bool row_ok = grow < n_total;
    const int rc = min(grow, n_total - 1);
    const int mi = q8set_index(S, rc);
    const int row = rc - q8set_row_start(S, mi);
    const uint8_t *qlo = Q8SET_PICK(S, qlo, mi);
    const uint8_t *qhi = Q8SET_PICK(S, qhi, mi);
    const uint16_t *wd = Q8SET_PICK(S, d, mi);
    const int k4 = nb * (QK / 4);
    const size_t rbase = (size_t)row * nb;

    XStage<XN, NORM> st;
    xstage_load(st, x, norm_w, inv_s, k4, tid);
    int4 lo[U], hi[U];
    uint32_t dw[U];
    q8_first_pass<G, U>(qlo, qhi, wd, rbase, nb, j, lo, hi, dw);
    const float scale = xstage_scale(st, k4, eps, L.red, tid);  // 1 without NORM
    xstage_quant(st, inv_s, k4, scale, rounding, L.qs, L.d, tid);
    __syncthreads();
    const float s = q8_row_dot<G, U>(qlo, qhi, wd, rbase, nb, j, lo, hi, dw, L.qs, L.d);
    if (row_ok && j == 0) {
        const float *add = Q8SET_PICK(S, add, mi);
        Q8SET_PICK(S, y, mi)[row] = add ? s + add[row] : s;
    }
}

// Gate and up projections of one activation row (RMSNorm and SmoothQuant fused as in
// fused1) with the swiglu and the down projection's Q8_0 activation quantization in the
// epilogue.  A workgroup owns 32 consecutive h indices: gate rows 32b.. and up rows 32b..,
// as four passes of 16 row slots, so the quantization block is whole.  Each row's dot
// is fused1's (G = 16 lanes, same block order and reduction), so h and its quantization
// equal the unfused GEMVs followed by the swiglu-quantize kernel bit for bit.
template <int U, int XN, bool NORM>
__global__ __launch_bounds__(256) void k_gemv_q8_0_gu_swiglu(const Q8Set S, const float *__restrict__ x,
                                                             const float *__restrict__ norm_w, float eps,
                                                             const float *__restrict__ inv_s,
                                                             const float *__restrict__ inv_s_down,
                                                             int8_t *__restrict__ xq_qs, uint16_t *__restrict__ xq_d,
                                                             int nb, int rounding) {
    constexpr int G = 16;
    extern __shared__ __align__(16) uint8_t smem[];
    const FusedLds L = fused_lds(smem, nb);
    __shared__ float s_gu[64];  // gate h 0..31, then up h 0..31
    const int tid = threadIdx.x;
    const int j = tid % G, slot = tid / G;
    const int hb = blockIdx.x;  // h indices 32hb .. 32hb+31
    const int k4 = nb * (QK / 4);

    XStage<XN, NORM> st;
    xstage_load(st, x, norm_w, inv_s, k4, tid);
    int4 lo[4][U], hi[4][U];
    uint32_t dw[4][U];
    size_t rbase[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        rbase[p] = (size_t)(32 * hb + 16 * (p & 1) + slot) * nb;
        if (p < 2) q8_first_pass<G, U>(S.qlo[0], S.qhi[0], S.d[0], rbase[p], nb, j, lo[p], hi[p], dw[p]);
        else q8_first_pass<G, U>(S.qlo[1], S.qhi[1], S.d[1], rbase[p], nb, j, lo[p], hi[p], dw[p]);
    }
    const float scale = xstage_scale(st, k4, eps, L.red, tid);  // 1 without NORM
    xstage_quant(st, inv_s, k4, scale, rounding, L.qs, L.d, tid);
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const float s = p < 2 ? q8_row_dot<G, U>(S.qlo[0], S.qhi[0], S.d[0], rbase[p], nb, j, lo[p], hi[p], dw[p],
                                                 L.qs, L.d)
                              : q8_row_dot<G, U>(S.qlo[1], S.qhi[1], S.d[1], rbase[p], nb, j, lo[p], hi[p], dw[p],
                                                 L.qs, L.d);
        if (j == 0) s_gu[16 * p + slot] = s;
    }
    __syncthreads();
    if (tid < 8) {  // 4 consecutive h values per lane, 8 lanes per 32-block (as the swiglu-quantize kernel)
        const int i = 4 * tid;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float gv = s_gu[i + e], uv = s_gu[32 + i + e];
            v[e] = (gv / (1.0f + expf(-gv))) * uv;
        }
        if (inv_s_down) {
            const float4 sv = ((const float4 *)inv_s_down)[8 * hb + tid];
            v[0] *= sv.x; v[1] *= sv.y; v[2] *= sv.z; v[3] *= sv.w;
        }
        float d;
        const uint32_t q = quant4(v[0], v[1], v[2], v[3], rounding, d);
        *(uint32_t *)(xq_qs + (size_t)32 * hb + i) = q;
        if (tid == 0) xq_d[hb] = f2h(d);
    }
}

// Gate and up projections of one activation row with the swiglu in the epilogue: a
// workgroup pairs gate rows 8t..8t+7 (row slots 0..7) with the same up rows (slots
// 8..15) and forms h[8t + i] = silu(g) * u times the down projection's SmoothQuant
// reciprocal.  Each row's dot is fused1's (G = 16 lanes, same block order and reduction)
// and the swiglu is k_swiglu_quant_q8_0's expression, so h and its quantization equal
// the unfused chain's bit for bit; the 1120 workgroups of the Qwen2.5-1.5B shape keep the
// gate+up launch's grid.
//   QUANT = false: h is written in fp32 (the down launch quantizes it in its prologue).
//   QUANT = true: h is quantized to Q8_0 in this launch.  The four workgroups of a
//   32-block publish their 8 values (agent-scope stores, completed before the count) and
//   count themselves on the block's counter; the one that brings it to 4 reads the block
//   back, quantizes it (quant4 over 8 lanes, as k_swiglu_quant_q8_0) and zeroes the
//   counter for the next launch.  Nothing waits: the last arrival does the work.
template <int U, int XN, bool NORM, bool QUANT>
__global__ __launch_bounds__(256) void k_gemv_q8_0_gu_pair(const Q8Set S, const float *__restrict__ x,
                                                           const float *__restrict__ norm_w, float eps,
                                                           const float *__restrict__ inv_s,
                                                           const float *__restrict__ inv_s_down, float *h,
                                                           unsigned *counters, int8_t *__restrict__ xq_qs,
                                                           uint16_t *__restrict__ xq_d, int nb, int rounding) {
    constexpr int G = 16;
    extern __shared__ __align__(16) uint8_t smem[];
    const FusedLds L = fused_lds(smem, nb);
    __shared__ float s_gu[16];  // gate rows 0..7, then up rows 0..7
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int j = tid % G, slot = tid / G;
    const int t = blockIdx.x;  // h indices 8t .. 8t+7
    const int k4 = nb * (QK / 4);
    const bool up = slot >= 8;
    const uint8_t *qlo = up ? S.qlo[1] : S.qlo[0];
    const uint8_t *qhi = up ? S.qhi[1] : S.qhi[0];
    const uint16_t *wd = up ? S.d[1] : S.d[0];
    const size_t rbase = (size_t)(8 * t + (slot & 7)) * nb;

    XStage<XN, NORM> st;
    xstage_load(st, x, norm_w, inv_s, k4, tid);
    int4 lo[U], hi[U];
    uint32_t dw[U];
    q8_first_pass<G, U>(qlo, qhi, wd, rbase, nb, j, lo, hi, dw);
    float sd = 1.0f;  // the down divisor of this thread's h index, loaded with the weights
    if (tid < 8 && inv_s_down) sd = inv_s_down[8 * t + tid];
    const float scale = xstage_scale(st, k4, eps, L.red, tid);  // 1 without NORM
    xstage_quant(st, inv_s, k4, scale, rounding, L.qs, L.d, tid);
    __syncthreads();
    const float s = q8_row_dot<G, U>(qlo, qhi, wd, rbase, nb, j, lo, hi, dw, L.qs, L.d);
    if (j == 0) s_gu[slot] = s;
    __syncthreads();
    if constexpr (!QUANT) {
        if (tid < 8) {
            const float gv = s_gu[tid], uv = s_gu[8 + tid];
            float v = (gv / (1.0f + expf(-gv))) * uv;
            if (inv_s_down) v *= sd;
            h[8 * t + tid] = v;
        }
    } else {
        if (tid < 8) {
            const float gv = s_gu[tid], uv = s_gu[8 + tid];
            float v = (gv / (1.0f + expf(-gv))) * uv;
            if (inv_s_down) v *= sd;
            __hip_atomic_store(h + 8 * t + tid, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);  // this workgroup's values are written through
        __syncthreads();
        const int blk = t / 4;
        if (tid == 0) {
            const unsigned prev =
                __hip_atomic_fetch_add(counters + blk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = prev == 3u;
        }
        __syncthreads();
        if (s_last && tid < 8) {  // 4 consecutive h values per lane, 8 lanes per block
            const float *hb = h + 32 * blk + 4 * tid;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = __hip_atomic_load(hb + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float d;
            const uint32_t q = quant4(v[0], v[1], v[2], v[3], rounding, d);
            *(uint32_t *)(xq_qs + (size_t)32 * blk + 4 * tid) = q;
            if (tid == 0) {
                xq_d[blk] = f2h(d);
                __hip_atomic_store(counters + blk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// The projection of an attention output still in flash-decoding split form: every
// workgroup merges the splits' records (log-sum-exp combine) for the whole row in its
// prologue, then scales by the SmoothQuant reciprocal and quantizes as fused1 does.
// x[h*hd + i] = (sum_s w_s o_s[i]) / (sum_s w_s l_s), w_s = 2^(m_s - max_s m_s), 0 for a
// split with no position (m_s = -inf), and x = 0 when the weight sum is 0.  One kernel
// boundary replaces the combine launch; up to MAXS splits, k <= 1024*XN.
template <int G, int U, int XN, int MAXS>
__global__ __launch_bounds__(256) void k_gemv_q8_0_lse(const Q8Set S, const float *__restrict__ part, int n_splits,
                                                       int hd, const float *__restrict__ inv_s, int n_total, int nb,
                                                       int rounding) {
    constexpr int RPB = 256 / G;
    extern __shared__ __align__(16) uint8_t smem[];
    const FusedLds L = fused_lds(smem, nb);
    const int tid = threadIdx.x;
    const int j = tid % G;
    const int grow = blockIdx.x * RPB + tid / G;
    const bool row_ok = grow < n_total;
    const int rc = min(grow, n_total - 1);
    const int mi = q8set_index(S, rc);
    const int row = rc - q8set_row_start(S, mi);
    const uint8_t *qlo = Q8SET_PICK(S, qlo, mi);
    const uint8_t *qhi = Q8SET_PICK(S, qhi, mi);
    const uint16_t *wd = Q8SET_PICK(S, d, mi);
    const int k4 = nb * (QK / 4);
    const size_t rbase = (size_t)row * nb;
    const int hd4 = hd / 4, ps = hd + 4;

    // every split's record for this thread's float4s, loaded before the weights
    float4 os[XN][MAXS], sv[XN];
    float ms[XN][MAXS], ls[XN][MAXS];
#pragma unroll
    for (int t = 0; t < XN; t++) {
        const int f = min(tid + t * 256, k4 - 1);
        const float *ph = part + (size_t)(f / hd4) * n_splits * ps;
#pragma unroll
        for (int s = 0; s < MAXS; s++) {
            const float *r = ph + (size_t)min(s, n_splits - 1) * ps;
            os[t][s] = ((const float4 *)r)[f % hd4];
            ms[t][s] = r[hd];
            ls[t][s] = r[hd + 1];
        }
        if (inv_s) sv[t] = ((const float4 *)inv_s)[f];
    }
    int4 lo[U], hi[U];
    uint32_t dw[U];
    q8_first_pass<G, U>(qlo, qhi, wd, rbase, nb, j, lo, hi, dw);

#pragma unroll
    for (int t = 0; t < XN; t++) {
        const int f = tid + t * 256;  // 8 consecutive threads form one 32-block
        float mx = -INFINITY;
#pragma unroll
        for (int s = 0; s < MAXS; s++)
            if (s < n_splits) mx = fmaxf(mx, ms[t][s]);
        float l = 0.0f;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int s = 0; s < MAXS; s++) {
            const float w = (s < n_splits && ms[t][s] != -INFINITY && mx != -INFINITY)
                                ? __builtin_amdgcn_exp2f(ms[t][s] - mx) : 0.0f;
            l = fmaf(ls[t][s], w, l);
            a.x = fmaf(os[t][s].x, w, a.x);
            a.y = fmaf(os[t][s].y, w, a.y);
            a.z = fmaf(os[t][s].z, w, a.z);
            a.w = fmaf(os[t][s].w, w, a.w);
        }
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (l != 0.0f) v = make_float4(a.x / l, a.y / l, a.z / l, a.w / l);
        if (inv_s) { v.x *= sv[t].x; v.y *= sv[t].y; v.z *= sv[t].z; v.w *= sv[t].w; }
        float d;
        const uint32_t q = quant4(v.x, v.y, v.z, v.w, rounding, d);
        if (f < k4) {
            *(uint32_t *)(L.qs + (size_t)f * 4) = q;
            if ((f & 7) == 0) L.d[f >> 3] = h2f(f2h(d));
        }
    }
    __syncthreads();
    const float s = q8_row_dot<G, U>(qlo, qhi, wd, rbase, nb, j, lo, hi, dw, L.qs, L.d);
    if (row_ok && j == 0) {
        const float *add = Q8SET_PICK(S, add, mi);
        Q8SET_PICK(S, y, mi)[row] = add ? s + add[row] : s;
    }
}

// q/k/v projections with the rest of the attention-input chain fused in (bias add,
// neox RoPE of q and k, q written fp32, k and v converted to fp16 into their cache
// row); the row mapping and epilogue are shared with the W4A16 kernel (RopeKV).
template <int G, int U, int XN, bool NORM>
__global__ __launch_bounds__(256) void k_gemv_q8_0_qkv_rope(const Q8Set S, const RopeKV R, const float *__restrict__ x,
                                                            const float *__restrict__ norm_w, float eps,
                                                            const float *__restrict__ inv_s, int nb, int rounding) {
    constexpr int RPB = 256 / G;  // rows per workgroup
    extern __shared__ __align__(16) uint8_t smem[];
    const FusedLds L = fused_lds(smem, nb);
    const int tid = threadIdx.x;
    const int j = tid % G;
    const int t = tid / G;
    const int n_total = R.n_q + R.n_k + R.n_v;
    const int b = blockIdx.x;
    RopeKVPlace pl;
    const int rc = min(rope_kv_row<RPB>(R, b, t, pl), n_total - 1);
    float tab_cs, tab_sn;
    rope_tab_prefetch(R, pl.chunk * (RPB / 2) + tid % (RPB / 2), tab_cs, tab_sn);
    const int mi = q8set_index(S, rc);
    const int row = rc - q8set_row_start(S, mi);
    const uint8_t *qlo = Q8SET_PICK(S, qlo, mi);
    const uint8_t *qhi = Q8SET_PICK(S, qhi, mi);
    const uint16_t *wd = Q8SET_PICK(S, d, mi);
    const int k4 = nb * (QK / 4);
    const size_t rbase = (size_t)row * nb;

    XStage<XN, NORM> st;
    xstage_load(st, x, norm_w, inv_s, k4, tid);
    int4 lo[U], hi[U];
    uint32_t dw[U];
    q8_first_pass<G, U>(qlo, qhi, wd, rbase, nb, j, lo, hi, dw);
    const float scale = xstage_scale(st, k4, eps, L.red, tid);  // 1 without NORM
    xstage_quant(st, inv_s, k4, scale, rounding, L.qs, L.d, tid);
    __syncthreads();
    const float s = q8_row_dot<G, U>(qlo, qhi, wd, rbase, nb, j, lo, hi, dw, L.qs, L.d);
    if (j == 0) {
        const float *bias = mi == 0 ? R.bias[0] : mi == 1 ? R.bias[1] : R.bias[2];
        L.y[t] = bias ? s + bias[row] : s;
    }
    __syncthreads();
    rope_kv_epilogue<RPB>(R, L.y, b, tid, pl, tab_cs, tab_sn);
}

// silu(g) * u (ggml swiglu: silu(x) = x / (1 + expf(-x))), times the SmoothQuant
// reciprocal of the next projection, quantized to Q8_0: the GLU node and the down
// projection's activation quantization in one pass.  grid: ceil(nblocks / 32) x 256.
__global__ __launch_bounds__(256) void k_swiglu_quant_q8_0(const float *__restrict__ g, const float *__restrict__ u,
                                                           const float *__restrict__ inv_s, int8_t *__restrict__ qs,
                                                           uint16_t *__restrict__ dout, int64_t total_blocks,
                                                           int rounding) {
    const int64_t blk = (int64_t)blockIdx.x * 32 + threadIdx.x / 8;
    const int sub = threadIdx.x % 8;
    const bool valid = blk < total_blocks;
    const int64_t e = (valid ? blk : 0) * QK + sub * 4;
    float4 gv = make_float4(0.f, 0.f, 0.f, 0.f), uv = gv, sv = make_float4(1.f, 1.f, 1.f, 1.f);
    if (valid) {
        gv = *(const float4 *)(g + e);
        uv = *(const float4 *)(u + e);
        if (inv_s) sv = *(const float4 *)(inv_s + e);
    }
    float4 v;
    v.x = (gv.x / (1.0f + expf(-gv.x))) * uv.x;
    v.y = (gv.y / (1.0f + expf(-gv.y))) * uv.y;
    v.z = (gv.z / (1.0f + expf(-gv.z))) * uv.z;
    v.w = (gv.w / (1.0f + expf(-gv.w))) * uv.w;
    if (inv_s) { v.x *= sv.x; v.y *= sv.y; v.z *= sv.z; v.w *= sv.w; }
    float d;
    const uint32_t q = quant4(v.x, v.y, v.z, v.w, rounding, d);
    if (valid) {
        *(uint32_t *)(qs + e) = q;
        if (sub == 0) dout[blk] = f2h(d);
    }
}

// exact per-block int32 dots (bit-exactness check), activation row 0: the same dot_block
// every GEMV kernel above uses on the same two 16-byte weight chunks and activation halves
__global__ void k_q8_0_block_dots(const uint8_t *__restrict__ qlo, const uint8_t *__restrict__ qhi,
                                  const int8_t *__restrict__ xq_qs, int32_t *__restrict__ out, int64_t n, int nb) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * nb) return;
    const int b = (int)(i % nb);
    const int4 lo = *(const int4 *)(qlo + i * 16);
    const int4 hi = *(const int4 *)(qhi + i * 16);
    const int4 x0 = *(const int4 *)(xq_qs + (size_t)b * QK);
    const int4 x1 = *(const int4 *)(xq_qs + (size_t)b * QK + 16);
    out[i] = dot_block(lo, hi, x0, x1);
}

// ------------------------------------------------------------------ launch helpers

inline int pick_u(int64_t nb, int g) {
    int64_t u = (nb + g - 1) / g;
    if (u > 8) u = (u + 1) / 2 > 8 ? 8 : (u + 1) / 2;  // several passes of U blocks
    return (int)u;
}

inline int pick_g(int64_t nb) { return nb <= 128 ? 16 : (nb <= 256 ? 32 : 64); }

// Lanes per row for a launch of n_rows rows: with MI_GEMV_MIN_WG=<n> set, wider rows
// (fewer rows per workgroup) until the grid has n workgroups.  Off by default: the
// small decode projections are bound by the latency chain of each workgroup (the
// activation staging is repeated per workgroup), not by the number of CUs in use.
inline int gemv_min_wg() {
    static const int v = [] {
        const char *e = getenv("MI_GEMV_MIN_WG");
        return e ? atoi(e) : 0;
    }();
    return v;
}

inline int pick_g_rows(int64_t nb, int64_t n_rows) {
    int g = pick_g(nb);
    while (g < 64 && (n_rows + 256 / g - 1) / (256 / g) < gemv_min_wg()) g *= 2;
    return g;
}

template <int G, int U, int M>
int launch_xq_gu(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const int8_t *xq_qs,
                 const uint16_t *xq_d, float *y, const float *add) {
    const Q8Planes p = q8_planes(n, k);
    constexpr int RPB = 256 / G;
    hipLaunchKernelGGL((k_gemv_q8_0_xq<G, U, M>), dim3((unsigned)((n + RPB - 1) / RPB)), dim3(256), 0, st, base,
                       base + p.plane, (const uint16_t *)(base + 2 * p.plane), xq_qs, xq_d, y, add, (int)n,
                       (int)(k / QK), (int)m);
    MI_CHECK_LAUNCH("k_gemv_q8_0_xq");
    return MI_OK;
}

template <int G, int M>
int launch_xq_g(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const int8_t *xq_qs,
                const uint16_t *xq_d, float *y, const float *add) {
#define MI_U_CASE(UU) case UU: return launch_xq_gu<G, UU, M>(st, base, n, k, m, xq_qs, xq_d, y, add);
    switch (pick_u(k / QK, G)) {
        MI_U_CASE(1) MI_U_CASE(2) MI_U_CASE(3) MI_U_CASE(4) MI_U_CASE(5) MI_U_CASE(6) MI_U_CASE(7) MI_U_CASE(8)
    }
#undef MI_U_CASE
    return MI_ERR_ARG;
}

template <int M>
int launch_xq_m(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const int8_t *xq_qs,
                const uint16_t *xq_d, float *y, const float *add) {
    switch (pick_g(k / QK)) {
        case 16: return launch_xq_g<16, M>(st, base, n, k, m, xq_qs, xq_d, y, add);
        case 32: return launch_xq_g<32, M>(st, base, n, k, m, xq_qs, xq_d, y, add);
        default: return launch_xq_g<64, M>(st, base, n, k, m, xq_qs, xq_d, y, add);
    }
}

int launch_xq(hipStream_t st, const uint8_t *base, int64_t n, int64_t k, int64_t m, const int8_t *xq_qs,
              const uint16_t *xq_d, float *y, const float *add = nullptr) {
    if (m == 1) return launch_xq_m<1>(st, base, n, k, m, xq_qs, xq_d, y, add);
    if (m == 2) return launch_xq_m<2>(st, base, n, k, m, xq_qs, xq_d, y, add);
    if (m >= 3 && m <= 4) return launch_xq_m<4>(st, base, n, k, m, xq_qs, xq_d, y, add);
    if (m >= 5 && m <= 8) return launch_xq_m<8>(st, base, n, k, m, xq_qs, xq_d, y, add);
    set_error("gemv_q8_0: m=%lld not in 1..8", (long long)m);
    return MI_ERR_ARG;
}

// ---- several activation rows (2..8: a ubatch) through up to four matrices

// The Q8_0 blocks of m activation rows with their RMSNorm folded in, one workgroup per
// row (k <= 1024*XN): RMSNorm(x) * norm_w, then * inv_s and the quantization.  The float
// operations are those of k_rms_norm + MUL (XStage) then k_act_quant_q8_0, so the bytes
// equal what those launches write in sequence.  (Without a norm, k_act_quant_q8_0 takes
// the rows 32 blocks per workgroup, the swiglu folded in when given.)
template <int XN>
__global__ __launch_bounds__(256) void k_act_quant_rows_q8_0(const float *__restrict__ x,
                                                             const float *__restrict__ norm_w, float eps,
                                                             const float *__restrict__ inv_s, int8_t *__restrict__ qs,
                                                             uint16_t *__restrict__ dout, int k, int rounding) {
    __shared__ double s_red[4];
    const int row = blockIdx.x, tid = threadIdx.x, k4 = k / 4, nb = k / QK;
    int8_t *qr = qs + (size_t)row * k;
    uint16_t *dr = dout + (size_t)row * nb;
    XStage<XN, true> st;
    xstage_load(st, x + (size_t)row * k, norm_w, nullptr, k4, tid);
    const float scale = xstage_scale(st, k4, eps, s_red, tid);
#pragma unroll
    for (int t = 0; t < XN; t++) {
        const int f = tid + t * 256;  // float4 index; 8 consecutive threads form one 32-block
        float4 v = xstage_value(st, scale, t);
        if (inv_s) {
            const float4 sv = ((const float4 *)inv_s)[min(f, k4 - 1)];
            v.x *= sv.x; v.y *= sv.y; v.z *= sv.z; v.w *= sv.w;
        }
        float d;
        const uint32_t q = quant4(v.x, v.y, v.z, v.w, rounding, d);  // whole 8-lane groups (k4 % 8 == 0)
        if (f < k4) {
            *(uint32_t *)(qr + (size_t)f * 4) = q;
            if ((f & 7) == 0) dr[f >> 3] = f2h(d);
        }
    }
}

// The several-row GEMV over a stacked set of up to four matrices (Q8Set).  The m rows'
// activation blocks are staged in LDS once per workgroup, so only the weights sit in
// registers; each row's lanes walk their blocks in k_gemv_q8_0_xq's order with the same
// products, so the results are bit-identical to it (and to the one-row kernels).
// Epilogue per matrix: + add[row] (a bias row) or, with bit t of add_rows set,
// + add[i*n + row] (a residual of the output's shape).
template <int G, int U, int M>
__global__ __launch_bounds__(256) void k_gemv_q8_0_xs(const Q8Set S, unsigned add_rows, const int8_t *__restrict__ xq_qs,
                                                      const uint16_t *__restrict__ xq_d, int n_total, int nb, int m) {
    constexpr int RPB = 256 / G;
    extern __shared__ __align__(16) uint8_t smem[];
    const int k = nb * QK;
    int8_t *s_qs = (int8_t *)smem;
    uint16_t *s_d = (uint16_t *)(smem + (size_t)m * k);
    const int tid = threadIdx.x;
    const int j = tid % G;
    const int grow = blockIdx.x * RPB + tid / G;
    const bool row_ok = grow < n_total;
    const int rc = min(grow, n_total - 1);
    const int mi = q8set_index(S, rc);
    const int r = rc - q8set_row_start(S, mi);
    const uint8_t *qlo = S.qlo[mi], *qhi = S.qhi[mi];
    const uint16_t *wd = S.d[mi];
    const size_t rbase = (size_t)r * nb;
    int4 lo[U], hi[U];
    uint32_t dw[U];
    q8_first_pass<G, U>(qlo, qhi, wd, rbase, nb, j, lo, hi, dw);  // in flight during the staging
    {
        const int qn = m * k / 16, dn = (m * nb + 1) / 2;  // int4 / uint32 words (xs_lds_bytes rounds up)
        for (int o = tid; o < qn; o += 256) ((int4 *)s_qs)[o] = ((const int4 *)xq_qs)[o];
        for (int o = tid; o < dn; o += 256) ((uint32_t *)s_d)[o] = ((const uint32_t *)xq_d)[o];
    }
    __syncthreads();
    float acc[M];
#pragma unroll
    for (int i = 0; i < M; i++) acc[i] = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += U * G) {
        if (b0) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int b = min(b0 + j + u * G, nb - 1);
                lo[u] = ld_stream16(qlo + (rbase + b) * 16);
                hi[u] = ld_stream16(qhi + (rbase + b) * 16);
                dw[u] = wd[rbase + b];
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int b = b0 + j + u * G;
            if (b < nb) {
                const float dwf = h2f((uint16_t)dw[u]);
#pragma unroll
                for (int i = 0; i < M; i++) {
                    const int ii = min(i, m - 1);
                    const int4 *xs = (const int4 *)(s_qs + (size_t)ii * k + (size_t)b * QK);
                    const int s = dot_block(lo[u], hi[u], xs[0], xs[1]);
                    acc[i] = fmaf((float)s, dwf * h2f(s_d[ii * nb + b]), acc[i]);
                }
            }
        }
    }
    const int n_mi = S.row_end[mi] - q8set_row_start(S, mi);
    const float *add = S.add[mi];
    const bool full = (add_rows >> mi) & 1u;
#pragma unroll
    for (int i = 0; i < M; i++) {
        const float v = group_sum<G>(acc[i]);
        if (row_ok && j == 0 && i < m) {
            const size_t o = (size_t)i * n_mi + r;
            S.y[mi][o] = add ? v + add[full ? o : (size_t)r] : v;
        }
    }
}

constexpr int kMaxDevices = 64;

size_t xs_lds_bytes(int64_t m, int64_t k) { return (size_t)(m * k + (m * (k / QK) + 1) / 2 * 4); }

template <int G, int U, int M>
int launch_xs_gum(hipStream_t st, const Q8Set &S, unsigned add_rows, int n_total, int64_t k, int64_t m,
                  const int8_t *xq_qs, const uint16_t *xq_d) {
    constexpr int RPB = 256 / G;
    const size_t lds = xs_lds_bytes(m, k);
    auto kern = k_gemv_q8_0_xs<G, U, M>;
    // dynamic LDS allowed so far per device for this instantiation (64 KB by default)
    static std::atomic<size_t> raised[kMaxDevices];
    int dev = 0;
    if (lds > 65536 && (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices ||
                        lds > raised[dev].load(std::memory_order_relaxed))) {
        if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess) {
            (void)hipGetLastError();
            set_error("gemv_q8_0_xs: %zu bytes of LDS per workgroup not available", lds);
            return MI_ERR_UNSUPPORTED;
        }
        if (dev >= 0 && dev < kMaxDevices) {
            size_t cur = raised[dev].load(std::memory_order_relaxed);
            while (cur < lds && !raised[dev].compare_exchange_weak(cur, lds)) {
            }
        }
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)((n_total + RPB - 1) / RPB)), dim3(256), lds, st, S, add_rows, xq_qs, xq_d,
                       n_total, (int)(k / QK), (int)m);
    MI_CHECK_LAUNCH("k_gemv_q8_0_xs");
    return MI_OK;
}

template <int G, int M>
int launch_xs_gm(hipStream_t st, const Q8Set &S, unsigned add_rows, int n_total, int64_t k, int64_t m,
                 const int8_t *xq_qs, const uint16_t *xq_d) {
#define MI_U_CASE(UU) case UU: return launch_xs_gum<G, UU, M>(st, S, add_rows, n_total, k, m, xq_qs, xq_d);
    switch (pick_u(k / QK, G)) {
        MI_U_CASE(1) MI_U_CASE(2) MI_U_CASE(3) MI_U_CASE(4) MI_U_CASE(5) MI_U_CASE(6) MI_U_CASE(7) MI_U_CASE(8)
    }
#undef MI_U_CASE
    return MI_ERR_ARG;
}

template <int M>
int launch_xs_m(hipStream_t st, const Q8Set &S, unsigned add_rows, int n_total, int64_t k, int64_t m,
                const int8_t *xq_qs, const uint16_t *xq_d) {
    switch (pick_g(k / QK)) {  // the lane layout of k_gemv_q8_0_xq at this k
        case 16: return launch_xs_gm<16, M>(st, S, add_rows, n_total, k, m, xq_qs, xq_d);
        case 32: return launch_xs_gm<32, M>(st, S, add_rows, n_total, k, m, xq_qs, xq_d);
        default: return launch_xs_gm<64, M>(st, S, add_rows, n_total, k, m, xq_qs, xq_d);
    }
}

int launch_xs(hipStream_t st, const Q8Set &S, unsigned add_rows, int n_total, int64_t k, int64_t m,
              const int8_t *xq_qs, const uint16_t *xq_d) {
    if (m == 2) return launch_xs_m<2>(st, S, add_rows, n_total, k, m, xq_qs, xq_d);
    if (m >= 3 && m <= 4) return launch_xs_m<4>(st, S, add_rows, n_total, k, m, xq_qs, xq_d);
    if (m >= 5 && m <= 8) return launch_xs_m<8>(st, S, add_rows, n_total, k, m, xq_qs, xq_d);
    set_error("gemv_q8_0_xs: m=%lld not in 2..8", (long long)m);
    return MI_ERR_ARG;
}

template <int G, int U, int XN, bool NORM>
int launch_fused_gux(hipStream_t st, const Q8Set &S, int n_total, int64_t k, const float *x, const float *norm_w,
                     float eps, const float *inv_s, int rounding) {
    constexpr int RPB = 256 / G;
    const int nb = (int)(k / QK);
    hipLaunchKernelGGL((k_gemv_q8_0_fused1<G, U, XN, NORM>), dim3((unsigned)((n_total + RPB - 1) / RPB)), dim3(256),
                       fused_smem(nb), st, S, x, norm_w, eps, inv_s, n_total, nb, rounding);
    MI_CHECK_LAUNCH("k_gemv_q8_0_fused1");
    return MI_OK;
}

template <int G, int XN, bool NORM>
int launch_fused_gx(hipStream_t st, const Q8Set &S, int n_total, int64_t k, const float *x, const float *norm_w,
                    float eps, const float *inv_s, int rounding) {
#define MI_U_CASE(UU) \
    case UU: return launch_fused_gux<G, UU, XN, NORM>(st, S, n_total, k, x, norm_w, eps, inv_s, rounding);
    switch (pick_u(k / QK, G)) {
        MI_U_CASE(1) MI_U_CASE(2) MI_U_CASE(3) MI_U_CASE(4) MI_U_CASE(5) MI_U_CASE(6) MI_U_CASE(7) MI_U_CASE(8)
    }
#undef MI_U_CASE
    return MI_ERR_ARG;
}

template <int XN, bool NORM>
int launch_fused_x(hipStream_t st, const Q8Set &S, int n_total, int64_t k, const float *x, const float *norm_w,
                   float eps, const float *inv_s, int rounding) {
    switch (pick_g_rows(k / QK, n_total)) {
        case 16: return launch_fused_gx<16, XN, NORM>(st, S, n_total, k, x, norm_w, eps, inv_s, rounding);
        case 32: return launch_fused_gx<32, XN, NORM>(st, S, n_total, k, x, norm_w, eps, inv_s, rounding);
        default: return launch_fused_gx<64, XN, NORM>(st, S, n_total, k, x, norm_w, eps, inv_s, rounding);
    }
}

template <bool NORM>
int launch_fused_n(hipStream_t st, const Q8Set &S, int n_total, int64_t k, const float *x, const float *norm_w,
                   float eps, const float *inv_s, int rounding) {
    const int64_t xn = (k / 4 + 255) / 256;
    if (xn <= 1) return launch_fused_x<1, NORM>(st, S, n_total, k, x, norm_w, eps, inv_s, rounding);
    if (xn <= 2) return launch_fused_x<2, NORM>(st, S, n_total, k, x, norm_w, eps, inv_s, rounding);
    if (xn <= 4) return launch_fused_x<4, NORM>(st, S, n_total, k, x, norm_w, eps, inv_s, rounding);
    // up to 12288 floats (the down projection's row): 32 or 64 lanes per row, no norm
    if constexpr (!NORM) {
        if (xn <= 12) {
            const int g = pick_g_rows(k / QK, n_total);
            if (g == 32) return launch_fused_gx<32, 12, false>(st, S, n_total, k, x, nullptr, eps, inv_s, rounding);
            if (g == 64) return launch_fused_gx<64, 12, false>(st, S, n_total, k, x, nullptr, eps, inv_s, rounding);
        }
    }
    set_error("mul_mat_q8_0_f32_fused: k=%lld not supported%s", (long long)k, NORM ? " with a norm" : "");
    return MI_ERR_ARG;
}

// one activation row with k <= 4096 (16 floats per thread): single fused launch
int launch_fused(hipStream_t st, const Q8Set &S, int n_total, int64_t k, const float *x, const float *norm_w,
                 float eps, const float *inv_s, int rounding) {
    if (norm_w) return launch_fused_n<true>(st, S, n_total, k, x, norm_w, eps, inv_s, rounding);
    return launch_fused_n<false>(st, S, n_total, k, x, nullptr, eps, inv_s, rounding);
}

template <int U, int XN, int MAXS>
int launch_lse_u(hipStream_t st, const Q8Set &S, int n_total, int64_t k, const float *part, int n_splits, int hd,
                 const float *inv_s, int rounding) {
    constexpr int G = 16, RPB = 256 / G;
    const int nb = (int)(k / QK);
    hipLaunchKernelGGL((k_gemv_q8_0_lse<G, U, XN, MAXS>), dim3((unsigned)((n_total + RPB - 1) / RPB)), dim3(256),
                       fused_smem(nb), st, S, part, n_splits, hd, inv_s, n_total, nb, rounding);
    MI_CHECK_LAUNCH("k_gemv_q8_0_lse");
    return MI_OK;
}

template <int XN, int MAXS>
int launch_lse_x(hipStream_t st, const Q8Set &S, int n_total, int64_t k, const float *part, int n_splits, int hd,
                 const float *inv_s, int rounding) {
    switch (pick_u(k / QK, 16)) {  // k <= 2048: at most 4 blocks per lane
        case 1: return launch_lse_u<1, XN, MAXS>(st, S, n_total, k, part, n_splits, hd, inv_s, rounding);
        case 2: return launch_lse_u<2, XN, MAXS>(st, S, n_total, k, part, n_splits, hd, inv_s, rounding);
        case 3: return launch_lse_u<3, XN, MAXS>(st, S, n_total, k, part, n_splits, hd, inv_s, rounding);
        default: return launch_lse_u<4, XN, MAXS>(st, S, n_total, k, part, n_splits, hd, inv_s, rounding);
    }
}

int launch_lse(hipStream_t st, const Q8Set &S, int n_total, int64_t k, const float *part, int n_splits, int hd,
               const float *inv_s, int rounding) {
    const bool x1 = k <= 1024;
    if (n_splits <= 4)
        return x1 ? launch_lse_x<1, 4>(st, S, n_total, k, part, n_splits, hd, inv_s, rounding)
                  : launch_lse_x<2, 4>(st, S, n_total, k, part, n_splits, hd, inv_s, rounding);
    return x1 ? launch_lse_x<1, 16>(st, S, n_total, k, part, n_splits, hd, inv_s, rounding)
              : launch_lse_x<2, 16>(st, S, n_total, k, part, n_splits, hd, inv_s, rounding);
}

template <int G, int U, int XN, bool NORM>
int launch_qkv_gu(hipStream_t st, const Q8Set &S, const RopeKV &R, int64_t k, const float *x, const float *norm_w,
                  float eps, const float *inv_s, int rounding) {
    constexpr int RPB = 256 / G;
    const int nb = (int)(k / QK);
    const int n_rope = R.n_q + R.n_k;
    const unsigned grid = (unsigned)(n_rope / RPB + (R.n_v + RPB - 1) / RPB);
    hipLaunchKernelGGL((k_gemv_q8_0_qkv_rope<G, U, XN, NORM>), dim3(grid), dim3(256), fused_smem(nb), st, S, R, x,
                       norm_w, eps, inv_s, nb, rounding);
    MI_CHECK_LAUNCH("k_gemv_q8_0_qkv_rope");
    return MI_OK;
}

template <int G, int XN, bool NORM>
int launch_qkv_gx(hipStream_t st, const Q8Set &S, const RopeKV &R, int64_t k, const float *x, const float *norm_w,
                  float eps, const float *inv_s, int rounding) {
#define MI_U_CASE(UU) case UU: return launch_qkv_gu<G, UU, XN, NORM>(st, S, R, k, x, norm_w, eps, inv_s, rounding);
    switch (pick_u(k / QK, G)) {
        MI_U_CASE(1) MI_U_CASE(2) MI_U_CASE(3) MI_U_CASE(4) MI_U_CASE(5) MI_U_CASE(6) MI_U_CASE(7) MI_U_CASE(8)
    }
#undef MI_U_CASE
    return MI_ERR_ARG;
}

template <int XN, bool NORM>
int launch_qkv_x(hipStream_t st, int g, const Q8Set &S, const RopeKV &R, int64_t k, const float *x,
                 const float *norm_w, float eps, const float *inv_s, int rounding) {
    switch (g) {
        case 16: return launch_qkv_gx<16, XN, NORM>(st, S, R, k, x, norm_w, eps, inv_s, rounding);
        case 32: return launch_qkv_gx<32, XN, NORM>(st, S, R, k, x, norm_w, eps, inv_s, rounding);
        default: return launch_qkv_gx<64, XN, NORM>(st, S, R, k, x, norm_w, eps, inv_s, rounding);
    }
}

template <bool NORM>
int launch_qkv_n(hipStream_t st, int g, const Q8Set &S, const RopeKV &R, int64_t k, const float *x,
                 const float *norm_w, float eps, const float *inv_s, int rounding) {
    const int64_t xn = (k / 4 + 255) / 256;
    if (xn <= 1) return launch_qkv_x<1, NORM>(st, g, S, R, k, x, norm_w, eps, inv_s, rounding);
    if (xn <= 2) return launch_qkv_x<2, NORM>(st, g, S, R, k, x, norm_w, eps, inv_s, rounding);
    return launch_qkv_x<4, NORM>(st, g, S, R, k, x, norm_w, eps, inv_s, rounding);
}

int make_set(Q8Set &S, int count, const void *const *w, const int64_t *n, float *const *y, int64_t k, int &n_total,
             const float *const *add = nullptr) {
    MI_CHECK_ARG(count >= 1 && count <= 4, "mul_mat_q8_0: %d matrices (1..4 supported)", count);
    int64_t acc = 0;
    for (int i = 0; i < 4; i++) {
        if (i < count) {
            MI_CHECK_ARG(w[i] && y[i] && n[i] > 0, "mul_mat_q8_0: bad matrix %d", i);
            MI_CHECK_ARG(mi::aligned(w[i], 256), "mul_mat_q8_0: packed weight %d not 256-byte aligned", i);
            const Q8Planes p = q8_planes(n[i], k);
            const uint8_t *base = (const uint8_t *)w[i];
            S.qlo[i] = base;
            S.qhi[i] = base + p.plane;
            S.d[i] = (const uint16_t *)(base + 2 * p.plane);
            S.y[i] = y[i];
            S.add[i] = add ? add[i] : nullptr;
            acc += n[i];
            S.row_end[i] = (int)acc;
        } else {
            S.qlo[i] = S.qlo[0];
            S.qhi[i] = S.qhi[0];
            S.d[i] = S.d[0];
            S.y[i] = S.y[0];
            S.add[i] = nullptr;
            S.row_end[i] = INT_MAX;
        }
    }
    MI_CHECK_ARG(acc < (1ll << 31), "mul_mat_q8_0: too many rows");
    n_total = (int)acc;
    return MI_OK;
}

int check_shape(const char *what, int64_t n, int64_t k) {
    MI_CHECK_ARG(n > 0 && k > 0 && k % QK == 0, "%s: bad shape n=%lld k=%lld (k must be a multiple of 32)", what,
                 (long long)n, (long long)k);
    MI_CHECK_ARG(n < (1ll << 31) && k < (1ll << 24), "%s: shape too large n=%lld k=%lld", what, (long long)n,
                 (long long)k);
    return MI_OK;
}

}  // namespace

extern "C" {

size_t mi_q8_0_packed_size(int64_t n, int64_t k) { return q8_planes(n, k).total; }

size_t mi_xq_d_offset(int64_t m, int64_t k) { return mi::align_up((size_t)m * k, 256); }
size_t mi_xq_size(int64_t m, int64_t k) { return mi_xq_d_offset(m, k) + mi::align_up((size_t)m * (k / QK) * 2, 256); }

int mi_prepack_q8_0(void *stream, const void *src_blocks, void *dst_packed, int64_t n, int64_t k) {
    if (int r = check_shape("prepack_q8_0", n, k)) return r;
    MI_CHECK_ARG(src_blocks && dst_packed, "prepack_q8_0: null pointer");
    MI_CHECK_ARG(mi::aligned(src_blocks, 2) && mi::aligned(dst_packed, 256), "prepack_q8_0: src must be 2-byte, dst 256-byte aligned");
    const Q8Planes p = q8_planes(n, k);
    const int64_t nblocks = n * (k / QK);
    uint8_t *base = (uint8_t *)dst_packed;
    hipLaunchKernelGGL(k_prepack_q8_0, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t *)src_blocks, base, base + p.plane, (uint16_t *)(base + 2 * p.plane), nblocks);
    MI_CHECK_LAUNCH("k_prepack_q8_0");
    return MI_OK;
}

int mi_quantize_f16_q8_0(void *stream, const uint16_t *w_f16, const float *s, void *dst_packed, int64_t n,
                         int64_t k) {
    if (int r = check_shape("quantize_f16_q8_0", n, k)) return r;
    MI_CHECK_ARG(w_f16 && dst_packed, "quantize_f16_q8_0: null pointer");
    MI_CHECK_ARG(mi::aligned(w_f16, 8) && mi::aligned(dst_packed, 256) && (!s || mi::aligned(s, 16)),
                 "quantize_f16_q8_0: w must be 8-byte, s 16-byte, dst 256-byte aligned");
    const Q8Planes p = q8_planes(n, k);
    const int64_t nblocks = n * (k / QK);
    uint8_t *base = (uint8_t *)dst_packed;
    hipLaunchKernelGGL(k_quantize_f16_q8_0, dim3((unsigned)((nblocks + 31) / 32)), dim3(256), 0, (hipStream_t)stream,
                       w_f16, s, base, base + p.plane, (uint16_t *)(base + 2 * p.plane), k, nblocks);
    MI_CHECK_LAUNCH("k_quantize_f16_q8_0");
    return MI_OK;
}

int mi_prepack_q8_0_host(const void *src_blocks, void *dst_packed, int64_t n, int64_t k) {
    if (int r = check_shape("prepack_q8_0_host", n, k)) return r;
    const Q8Planes p = q8_planes(n, k);
    const int64_t nblocks = n * (k / QK);
    const uint8_t *s = (const uint8_t *)src_blocks;
    uint8_t *base = (uint8_t *)dst_packed;
    memset(base, 0, p.total);
    for (int64_t i = 0; i < nblocks; i++) {
        memcpy(base + i * 16, s + i * 34 + 2, 16);
        memcpy(base + p.plane + i * 16, s + i * 34 + 18, 16);
        memcpy(base + 2 * p.plane + i * 2, s + i * 34, 2);
    }
    return MI_OK;
}

int mi_unpack_q8_0_host(const void *packed, void *dst_blocks, int64_t n, int64_t k) {
    if (int r = check_shape("unpack_q8_0_host", n, k)) return r;
    const Q8Planes p = q8_planes(n, k);
    const int64_t nblocks = n * (k / QK);
    const uint8_t *base = (const uint8_t *)packed;
    uint8_t *d = (uint8_t *)dst_blocks;
    for (int64_t i = 0; i < nblocks; i++) {
        memcpy(d + i * 34, base + 2 * p.plane + i * 2, 2);
        memcpy(d + i * 34 + 2, base + i * 16, 16);
        memcpy(d + i * 34 + 18, base + p.plane + i * 16, 16);
    }
    return MI_OK;
}

int mi_act_quant_q8_0(void *stream, const float *x, const float *inv_s, int64_t m, int64_t k, void *xq,
                      int rounding) {
    if (int r = check_shape("act_quant_q8_0", m, k)) return r;
    MI_CHECK_ARG(x && xq, "act_quant_q8_0: null pointer");
    MI_CHECK_ARG(mi::aligned(x, 16) && mi::aligned(xq, 16) && (!inv_s || mi::aligned(inv_s, 16)),
                 "act_quant_q8_0: pointers must be 16-byte aligned");
    const int64_t total = m * (k / QK);
    uint8_t *base = (uint8_t *)xq;
    hipLaunchKernelGGL(k_act_quant_q8_0, dim3((unsigned)((total + 31) / 32)), dim3(256), 0, (hipStream_t)stream, x,
                       inv_s, (int8_t *)base, (uint16_t *)(base + mi_xq_d_offset(m, k)), k, total, rounding,
                       (const float *)nullptr);
    MI_CHECK_LAUNCH("k_act_quant_q8_0");
    return MI_OK;
}

int mi_gemv_q8_0(void *stream, const void *w_packed, const void *xq, float *y, int64_t n, int64_t k, int64_t m) {
    if (int r = check_shape("gemv_q8_0", n, k)) return r;
    MI_CHECK_ARG(w_packed && xq && y, "gemv_q8_0: null pointer");
    MI_CHECK_ARG(mi::aligned(w_packed, 256) && mi::aligned(xq, 16), "gemv_q8_0: w_packed must be 256-byte, xq 16-byte aligned");
    const uint8_t *xb = (const uint8_t *)xq;
    return launch_xq((hipStream_t)stream, (const uint8_t *)w_packed, n, k, m, (const int8_t *)xb,
                     (const uint16_t *)(xb + mi_xq_d_offset(m, k)), y);
}

size_t mi_mul_mat_q8_0_workspace_size(int64_t m, int64_t k) {
    if (m == 1 && k <= 4096) return 0;
    return mi_xq_size(m, k);
}

int mi_mul_mat_q8_0_f32_multi(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, int64_t k, const float *x, const float *inv_s, int rounding, void *ws,
                              size_t ws_bytes) {
    MI_CHECK_ARG(w_packed && n && y && x, "mul_mat_q8_0_f32_multi: null pointer");
    if (int r = check_shape("mul_mat_q8_0_f32_multi", 1, k)) return r;
    MI_CHECK_ARG(mi::aligned(x, 16) && (!inv_s || mi::aligned(inv_s, 16)),
                 "mul_mat_q8_0_f32_multi: x/inv_s must be 16-byte aligned");
    Q8Set S;
    int n_total = 0;
    if (int r = make_set(S, n_mats, w_packed, n, y, k, n_total)) return r;
    hipStream_t st = (hipStream_t)stream;
    if (k <= 4096) return launch_fused(st, S, n_total, k, x, nullptr, 0.0f, inv_s, rounding);
    const size_t need = mi_xq_size(1, k);
    if (!ws || ws_bytes < need || !mi::aligned(ws, 16)) {
        mi::set_error("mul_mat_q8_0_f32_multi: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    if (int r = mi_act_quant_q8_0(stream, x, inv_s, 1, k, ws, rounding)) return r;
    for (int i = 0; i < n_mats; i++)
        if (int r = mi_gemv_q8_0(stream, w_packed[i], ws, y[i], n[i], k, 1)) return r;
    return MI_OK;
}

int mi_mul_mat_q8_0_f32(void *stream, const void *w_packed, const float *x, const float *inv_s, float *y,
                        int64_t n, int64_t k, int64_t m, int rounding, void *ws, size_t ws_bytes) {
    if (int r = check_shape("mul_mat_q8_0_f32", n, k)) return r;
    MI_CHECK_ARG(w_packed && x && y, "mul_mat_q8_0_f32: null pointer");
    MI_CHECK_ARG(m >= 1 && m <= 8, "mul_mat_q8_0_f32: m=%lld not in 1..8", (long long)m);
    MI_CHECK_ARG(mi::aligned(w_packed, 256) && mi::aligned(x, 16) && (!inv_s || mi::aligned(inv_s, 16)),
                 "mul_mat_q8_0_f32: w_packed must be 256-byte, x/inv_s 16-byte aligned");
    if (m == 1) return mi_mul_mat_q8_0_f32_multi(stream, 1, &w_packed, &n, &y, k, x, inv_s, rounding, ws, ws_bytes);
    const size_t need = mi_xq_size(m, k);
    if (!ws || ws_bytes < need || !mi::aligned(ws, 16)) {
        mi::set_error("mul_mat_q8_0_f32: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    if (int r = mi_act_quant_q8_0(stream, x, inv_s, m, k, ws, rounding)) return r;
    return mi_gemv_q8_0(stream, w_packed, ws, y, n, k, m);
}

int mi_mul_mat_q8_0_f32_batch(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, const float *const *bias, const float *const *add, int64_t k, int64_t m,
                              const float *x, const float *x_up, const float *norm_w, float eps, const float *inv_s,
                              int rounding, void *ws, size_t ws_bytes) {
    if (int r = check_shape("mul_mat_q8_0_f32_batch", m, k)) return r;
    MI_CHECK_ARG(w_packed && n && y && x, "mul_mat_q8_0_f32_batch: null pointer");
    MI_CHECK_ARG(m >= 2 && m <= 8, "mul_mat_q8_0_f32_batch: m=%lld not in 2..8", (long long)m);
    MI_CHECK_ARG(!(norm_w && x_up), "mul_mat_q8_0_f32_batch: a norm and a swiglu partner together");
    MI_CHECK_ARG(!norm_w || k <= 4096, "mul_mat_q8_0_f32_batch: k=%lld > 4096 with a norm", (long long)k);
    MI_CHECK_ARG(mi::aligned(x, 16) && (!x_up || mi::aligned(x_up, 16)) && (!norm_w || mi::aligned(norm_w, 16)) &&
                     (!inv_s || mi::aligned(inv_s, 16)),
                 "mul_mat_q8_0_f32_batch: x/x_up/norm_w/inv_s must be 16-byte aligned");
    const size_t need = mi_xq_size(m, k);
    if (!ws || ws_bytes < need || !mi::aligned(ws, 16)) {
        mi::set_error("mul_mat_q8_0_f32_batch: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    Q8Set S;
    int n_total = 0;
    const float *adds[4] = {};
    unsigned add_rows = 0;
    for (int i = 0; i < n_mats && i < 4; i++) {
        MI_CHECK_ARG(!(bias && bias[i] && add && add[i]), "mul_mat_q8_0_f32_batch: matrix %d has a bias and a residual", i);
        adds[i] = bias && bias[i] ? bias[i] : add ? add[i] : nullptr;
        if (add && add[i]) add_rows |= 1u << i;
    }
    if (int r = make_set(S, n_mats, w_packed, n, y, k, n_total, adds)) return r;
    hipStream_t st = (hipStream_t)stream;
    uint8_t *xb = (uint8_t *)ws;
    int8_t *qs = (int8_t *)xb;
    uint16_t *qd = (uint16_t *)(xb + mi_xq_d_offset(m, k));
    if (norm_w) {
        hipLaunchKernelGGL(k_act_quant_rows_q8_0<4>, dim3((unsigned)m), dim3(256), 0, st, x, norm_w, eps, inv_s, qs, qd,
                           (int)k, rounding);
        MI_CHECK_LAUNCH("k_act_quant_rows_q8_0");
    } else {
        const int64_t total = m * (k / QK);
        hipLaunchKernelGGL(k_act_quant_q8_0, dim3((unsigned)((total + 31) / 32)), dim3(256), 0, st, x, inv_s, qs, qd, k,
                           total, rounding, x_up);
        MI_CHECK_LAUNCH("k_act_quant_q8_0");
    }
    return launch_xs(st, S, add_rows, n_total, k, m, qs, qd);
}

int mi_mul_mat_q8_0_f32_fused(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, const float *const *add, int64_t k, const float *x,
                              const float *norm_w, float eps, const float *inv_s, int rounding) {
    MI_CHECK_ARG(w_packed && n && y && x, "mul_mat_q8_0_f32_fused: null pointer");
    if (int r = check_shape("mul_mat_q8_0_f32_fused", 1, k)) return r;
    MI_CHECK_ARG(k <= 4096 || (!norm_w && k <= 12288), "mul_mat_q8_0_f32_fused: k=%lld > %s", (long long)k,
                 norm_w ? "4096 with a norm" : "12288");
    MI_CHECK_ARG(mi::aligned(x, 16) && (!inv_s || mi::aligned(inv_s, 16)) && (!norm_w || mi::aligned(norm_w, 16)),
                 "mul_mat_q8_0_f32_fused: x/norm_w/inv_s must be 16-byte aligned");
    Q8Set S;
    int n_total = 0;
    if (int r = make_set(S, n_mats, w_packed, n, y, k, n_total, add)) return r;
    return launch_fused((hipStream_t)stream, S, n_total, k, x, norm_w, eps, inv_s, rounding);
}

int mi_gate_up_swiglu_q8_0(void *stream, const void *w_gate, const void *w_up, int64_t n_ff, int64_t k,
                           const float *x, const float *norm_w, float eps, const float *inv_s,
                           const float *inv_s_down, int rounding, void *xq) {
    MI_CHECK_ARG(w_gate && w_up && x && xq, "gate_up_swiglu_q8_0: null pointer");
    if (int r = check_shape("gate_up_swiglu_q8_0", n_ff, k)) return r;
    MI_CHECK_ARG(n_ff % QK == 0, "gate_up_swiglu_q8_0: n_ff=%lld not a multiple of 32", (long long)n_ff);
    MI_CHECK_ARG(k <= 2048, "gate_up_swiglu_q8_0: k=%lld > 2048", (long long)k);
    MI_CHECK_ARG(mi::aligned(w_gate, 256) && mi::aligned(w_up, 256), "gate_up_swiglu_q8_0: packed weights not 256-byte aligned");
    MI_CHECK_ARG(mi::aligned(x, 16) && (!norm_w || mi::aligned(norm_w, 16)) && (!inv_s || mi::aligned(inv_s, 16)) &&
                     (!inv_s_down || mi::aligned(inv_s_down, 16)) && mi::aligned(xq, 4),
                 "gate_up_swiglu_q8_0: misaligned vectors");
    const Q8Planes p = q8_planes(n_ff, k);
    Q8Set S;
    const uint8_t *wb[2] = {(const uint8_t *)w_gate, (const uint8_t *)w_up};
    for (int i = 0; i < 4; i++) {
        const uint8_t *b = wb[i < 2 ? i : 0];
        S.qlo[i] = b;
        S.qhi[i] = b + p.plane;
        S.d[i] = (const uint16_t *)(b + 2 * p.plane);
        S.y[i] = nullptr;
        S.add[i] = nullptr;
        S.row_end[i] = INT_MAX;
    }
    const int nb = (int)(k / QK);
    const int xn = (int)((k / 4 + 255) / 256);
    int8_t *qs = (int8_t *)xq;
    uint16_t *dq = (uint16_t *)((uint8_t *)xq + mi_xq_d_offset(1, n_ff));
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(n_ff / QK));
#define MI_GUS(UU, XX, NN)                                                                                         \
    hipLaunchKernelGGL((k_gemv_q8_0_gu_swiglu<UU, XX, NN>), grid, dim3(256), fused_smem(nb), st, S, x, norm_w, eps, \
                       inv_s, inv_s_down, qs, dq, nb, rounding)
#define MI_GUS_U(XX, NN)                        \
    switch (pick_u(nb, 16)) {                   \
        case 1: MI_GUS(1, XX, NN); break;       \
        case 2: MI_GUS(2, XX, NN); break;       \
        case 3: MI_GUS(3, XX, NN); break;       \
        default: MI_GUS(4, XX, NN); break;      \
    }
    if (norm_w) {
        if (xn <= 1) { MI_GUS_U(1, true) } else { MI_GUS_U(2, true) }
    } else {
        if (xn <= 1) { MI_GUS_U(1, false) } else { MI_GUS_U(2, false) }
    }
#undef MI_GUS_U
#undef MI_GUS
    MI_CHECK_LAUNCH("k_gemv_q8_0_gu_swiglu");
    return MI_OK;
}

namespace {
// the gate/up pair launch of both forms (QUANT: counters and xq given)
int launch_gu_pair(hipStream_t st, const void *w_gate, const void *w_up, int64_t n_ff, int64_t k, const float *x,
                   const float *norm_w, float eps, const float *inv_s, const float *inv_s_down, int rounding,
                   float *h, unsigned *counters, void *xq) {
    const Q8Planes p = q8_planes(n_ff, k);
    Q8Set S;
    const uint8_t *wb[2] = {(const uint8_t *)w_gate, (const uint8_t *)w_up};
    for (int i = 0; i < 4; i++) {
        const uint8_t *b = wb[i < 2 ? i : 0];
        S.qlo[i] = b;
        S.qhi[i] = b + p.plane;
        S.d[i] = (const uint16_t *)(b + 2 * p.plane);
        S.y[i] = nullptr;
        S.add[i] = nullptr;
        S.row_end[i] = INT_MAX;
    }
    const int nb = (int)(k / QK);
    const int xn = (int)((k / 4 + 255) / 256);
    int8_t *qs = xq ? (int8_t *)xq : nullptr;
    uint16_t *dq = xq ? (uint16_t *)((uint8_t *)xq + mi_xq_d_offset(1, n_ff)) : nullptr;
    const dim3 grid((unsigned)(n_ff / 8));
#define MI_GUP(UU, XX, NN, QQ)                                                                                     \
    hipLaunchKernelGGL((k_gemv_q8_0_gu_pair<UU, XX, NN, QQ>), grid, dim3(256), fused_smem(nb), st, S, x, norm_w,  \
                       eps, inv_s, inv_s_down, h, counters, qs, dq, nb, rounding)
#define MI_GUP_U(XX, NN, QQ)                        \
    switch (pick_u(nb, 16)) {                       \
        case 1: MI_GUP(1, XX, NN, QQ); break;       \
        case 2: MI_GUP(2, XX, NN, QQ); break;       \
        case 3: MI_GUP(3, XX, NN, QQ); break;       \
        default: MI_GUP(4, XX, NN, QQ); break;      \
    }
#define MI_GUP_X(NN, QQ)                                  \
    if (xn <= 1) { MI_GUP_U(1, NN, QQ) } else { MI_GUP_U(2, NN, QQ) }
    if (xq) {
        if (norm_w) { MI_GUP_X(true, true) } else { MI_GUP_X(false, true) }
    } else {
        if (norm_w) { MI_GUP_X(true, false) } else { MI_GUP_X(false, false) }
    }
#undef MI_GUP_X
#undef MI_GUP_U
#undef MI_GUP
    MI_CHECK_LAUNCH("k_gemv_q8_0_gu_pair");
    return MI_OK;
}

int check_gu_pair(const char *fn, const void *w_gate, const void *w_up, int64_t n_ff, int64_t k, const float *x,
                  const float *norm_w, const float *inv_s, int n_ff_multiple) {
    MI_CHECK_ARG(w_gate && w_up && x, "%s: null pointer", fn);
    if (int r = check_shape(fn, n_ff, k)) return r;
    MI_CHECK_ARG(n_ff % n_ff_multiple == 0, "%s: n_ff=%lld not a multiple of %d", fn, (long long)n_ff, n_ff_multiple);
    MI_CHECK_ARG(k <= 2048, "%s: k=%lld > 2048", fn, (long long)k);
    MI_CHECK_ARG(mi::aligned(w_gate, 256) && mi::aligned(w_up, 256), "%s: packed weights not 256-byte aligned", fn);
    MI_CHECK_ARG(mi::aligned(x, 16) && (!norm_w || mi::aligned(norm_w, 16)) && (!inv_s || mi::aligned(inv_s, 16)),
                 "%s: misaligned vectors", fn);
    return MI_OK;
}
}  // namespace

int mi_gate_up_swiglu_f32_q8_0(void *stream, const void *w_gate, const void *w_up, int64_t n_ff, int64_t k,
                               const float *x, const float *norm_w, float eps, const float *inv_s,
                               const float *inv_s_down, int rounding, float *h) {
    if (int r = check_gu_pair("gate_up_swiglu_f32_q8_0", w_gate, w_up, n_ff, k, x, norm_w, inv_s, 8)) return r;
    MI_CHECK_ARG(h && mi::aligned(h, 4), "gate_up_swiglu_f32_q8_0: bad h");
    return launch_gu_pair((hipStream_t)stream, w_gate, w_up, n_ff, k, x, norm_w, eps, inv_s, inv_s_down, rounding, h,
                          nullptr, nullptr);
}

int mi_gate_up_pair_q8_0(void *stream, const void *w_gate, const void *w_up, int64_t n_ff, int64_t k, const float *x,
                         const float *norm_w, float eps, const float *inv_s, const float *inv_s_down, int rounding,
                         void *xq, float *h_tmp, unsigned *counters) {
    if (int r = check_gu_pair("gate_up_pair_q8_0", w_gate, w_up, n_ff, k, x, norm_w, inv_s, 32)) return r;
    MI_CHECK_ARG(xq && mi::aligned(xq, 4) && h_tmp && mi::aligned(h_tmp, 16) && counters,
                 "gate_up_pair_q8_0: bad xq / h_tmp / counters");
    return launch_gu_pair((hipStream_t)stream, w_gate, w_up, n_ff, k, x, norm_w, eps, inv_s, inv_s_down, rounding,
                          h_tmp, counters, xq);
}

int mi_mul_mat_q8_0_f32_lse(void *stream, const void *w_packed, int64_t n, float *y, const float *add,
                            const float *part, int64_t n_splits, int64_t n_heads, int64_t head_dim,
                            const float *inv_s, int rounding) {
    MI_CHECK_ARG(w_packed && y && part, "mul_mat_q8_0_f32_lse: null pointer");
    MI_CHECK_ARG(n_heads > 0 && head_dim > 0 && head_dim % 4 == 0 && head_dim <= 1024,
                 "mul_mat_q8_0_f32_lse: bad heads %lld x %lld", (long long)n_heads, (long long)head_dim);
    const int64_t k = n_heads * head_dim;
    if (int r = check_shape("mul_mat_q8_0_f32_lse", n, k)) return r;
    MI_CHECK_ARG(k <= 2048, "mul_mat_q8_0_f32_lse: k=%lld > 2048", (long long)k);
    MI_CHECK_ARG(n_splits >= 1 && n_splits <= 16, "mul_mat_q8_0_f32_lse: %lld splits not in 1..16",
                 (long long)n_splits);
    MI_CHECK_ARG(mi::aligned(part, 16) && (!inv_s || mi::aligned(inv_s, 16)),
                 "mul_mat_q8_0_f32_lse: part/inv_s must be 16-byte aligned");
    Q8Set S;
    int n_total = 0;
    const float *adds[1] = {add};
    if (int r = make_set(S, 1, &w_packed, &n, &y, k, n_total, adds)) return r;
    return launch_lse((hipStream_t)stream, S, n_total, k, part, (int)n_splits, (int)head_dim, inv_s, rounding);
}

int mi_qkv_rope_kv_q8_0(void *stream, const void *const *w_packed, const int64_t *n, const float *const *bias,
                        int64_t k, const float *x, const float *norm_w, float eps, const float *inv_s, int rounding,
                        int64_t head_dim, const int32_t *pos, float freq_base, float freq_scale, float attn_factor,
                        float *q_out, void *k_cache, size_t k_row_bytes, void *v_cache, size_t v_row_bytes,
                        const void *kv_idx, int kv_idx_is_i64, int64_t n_cache_rows, const float *rope_table) {
    MI_CHECK_ARG(w_packed && n && bias && x && pos && q_out && k_cache && v_cache && kv_idx,
                 "qkv_rope_kv_q8_0: null pointer");
    if (int r = check_shape("qkv_rope_kv_q8_0", 1, k)) return r;
    MI_CHECK_ARG(k <= 4096, "qkv_rope_kv_q8_0: k=%lld > 4096", (long long)k);
    MI_CHECK_ARG(head_dim >= 16 && head_dim % 16 == 0 && head_dim <= 1024, "qkv_rope_kv_q8_0: head_dim %lld",
                 (long long)head_dim);
    MI_CHECK_ARG(n[0] > 0 && n[1] > 0 && n[2] > 0 && n[0] % head_dim == 0 && n[1] % head_dim == 0,
                 "qkv_rope_kv_q8_0: q/k rows must be whole heads");
    MI_CHECK_ARG(k_row_bytes >= (size_t)n[1] * 2 && v_row_bytes >= (size_t)n[2] * 2 && n_cache_rows > 0,
                 "qkv_rope_kv_q8_0: cache rows too short");
    MI_CHECK_ARG(mi::aligned(x, 16) && (!inv_s || mi::aligned(inv_s, 16)) && (!norm_w || mi::aligned(norm_w, 16)),
                 "qkv_rope_kv_q8_0: x/norm_w/inv_s must be 16-byte aligned");
    float *ys[3] = {q_out, q_out, q_out};  // unused by the kernel: results go through the epilogue
    Q8Set S;
    int n_total = 0;
    if (int r = make_set(S, 3, w_packed, n, ys, k, n_total)) return r;
    RopeKV R;
    for (int i = 0; i < 3; i++) R.bias[i] = bias[i];
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
    hipStream_t st = (hipStream_t)stream;
    int g = pick_g_rows(k / QK, n_total);
    while (g > 16 && head_dim % (256 / g) != 0) g /= 2;  // a workgroup's rows must tile the heads
    if (norm_w) return launch_qkv_n<true>(st, g, S, R, k, x, norm_w, eps, inv_s, rounding);
    return launch_qkv_n<false>(st, g, S, R, k, x, nullptr, eps, inv_s, rounding);
}

int mi_swiglu_quant_q8_0(void *stream, const float *g, const float *u, const float *inv_s, int64_t k, void *xq,
                         int rounding) {
    if (int r = check_shape("swiglu_quant_q8_0", 1, k)) return r;
    MI_CHECK_ARG(g && u && xq, "swiglu_quant_q8_0: null pointer");
    MI_CHECK_ARG(mi::aligned(g, 16) && mi::aligned(u, 16) && mi::aligned(xq, 16) && (!inv_s || mi::aligned(inv_s, 16)),
                 "swiglu_quant_q8_0: pointers must be 16-byte aligned");
    const int64_t nb = k / QK;
    uint8_t *base = (uint8_t *)xq;
    hipLaunchKernelGGL(k_swiglu_quant_q8_0, dim3((unsigned)((nb + 31) / 32)), dim3(256), 0, (hipStream_t)stream, g, u,
                       inv_s, (int8_t *)base, (uint16_t *)(base + mi_xq_d_offset(1, k)), nb, rounding);
    MI_CHECK_LAUNCH("k_swiglu_quant_q8_0");
    return MI_OK;
}

int mi_gemv_q8_0_add(void *stream, const void *w_packed, const void *xq, const float *add, float *y, int64_t n,
                     int64_t k, int64_t m) {
    if (int r = check_shape("gemv_q8_0_add", n, k)) return r;
    MI_CHECK_ARG(w_packed && xq && y, "gemv_q8_0_add: null pointer");
    MI_CHECK_ARG(mi::aligned(w_packed, 256) && mi::aligned(xq, 16), "gemv_q8_0_add: w_packed must be 256-byte, xq 16-byte aligned");
    const uint8_t *xb = (const uint8_t *)xq;
    return launch_xq((hipStream_t)stream, (const uint8_t *)w_packed, n, k, m, (const int8_t *)xb,
                     (const uint16_t *)(xb + mi_xq_d_offset(m, k)), y, add);
}

int mi_q8_0_block_dots(void *stream, const void *w_packed, const void *xq, int32_t *out, int64_t n, int64_t k) {
    if (int r = check_shape("q8_0_block_dots", n, k)) return r;
    MI_CHECK_ARG(w_packed && xq && out, "q8_0_block_dots: null pointer");
    const Q8Planes p = q8_planes(n, k);
    const int64_t total = n * (k / QK);
    const uint8_t *base = (const uint8_t *)w_packed;
    hipLaunchKernelGGL(k_q8_0_block_dots, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       base, base + p.plane, (const int8_t *)xq, out, n, (int)(k / QK));
    MI_CHECK_LAUNCH("k_q8_0_block_dots");
    return MI_OK;
}

}  // extern "C"
