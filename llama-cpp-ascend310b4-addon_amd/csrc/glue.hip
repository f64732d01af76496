// glue.hip -- the small decode-graph ops around the hot path (one token, fp32
// activations): RMSNorm (+ the following MUL by the norm weight), broadcast
// ADD / MUL, neox RoPE, SET_ROWS into an fp16 KV cache, GET_ROWS from an fp16
// or fp32 table, SwiGLU, ARGMAX.  Semantics follow the ggml-CPU ops
// (ggml/src/ggml-cpu/ops.cpp of llama.cpp @ 37b3a9e0): rms_norm sums x*x in
// double, rope builds theta by repeated multiplication with
// powf(freq_base, -2/n_dims), argmax keeps the first maximum.
#include "mi_common.h"

#include <limits.h>
#include <math.h>

namespace {

using namespace mi;

// one workgroup per row; y = x / sqrt(mean(x^2) + eps) [* w].  Rows of up to 4096
// floats are held in registers (4 float4 per thread, all loads issued before the
// first add), the x*x terms summed in double as ggml does; longer rows loop.
__global__ __launch_bounds__(256) void k_rms_norm(const float *__restrict__ x, const float *__restrict__ w,
                                                  float *__restrict__ y, int ne0, float eps) {
    const int row = blockIdx.x;
    const float *xr = x + (size_t)row * ne0;
    float *yr = y + (size_t)row * ne0;
    const int tid = threadIdx.x;
    __shared__ double s_red[4];
    double s = 0.0;
    const bool vec = (ne0 % 4) == 0 && ne0 <= 4096 && (((uintptr_t)xr | (uintptr_t)yr | (uintptr_t)w) & 15) == 0;
    float4 xv[4], wv[4];
    if (vec) {
        const int n4 = ne0 / 4;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int f = min(tid + t * 256, n4 - 1);
            xv[t] = ((const float4 *)xr)[f];
            if (w) wv[t] = ((const float4 *)w)[f];
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (tid + t * 256 < n4) {
                s += (double)sq_rn(xv[t].x);
                s += (double)sq_rn(xv[t].y);
                s += (double)sq_rn(xv[t].z);
                s += (double)sq_rn(xv[t].w);
            }
        }
    } else {
        for (int i = tid; i < ne0; i += 256) s += (double)sq_rn(xr[i]);
    }
    const double tot = block_sum_d256(s, s_red, tid);
    const float mean = (float)(tot / ne0);
    const float scale = 1.0f / sqrtf(mean + eps);
    if (vec) {
        const int n4 = ne0 / 4;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int f = tid + t * 256;
            if (f < n4) {
                float4 v = xv[t];
                v.x = v.x * scale; v.y = v.y * scale; v.z = v.z * scale; v.w = v.w * scale;
                if (w) { v.x *= wv[t].x; v.y *= wv[t].y; v.z *= wv[t].z; v.w *= wv[t].w; }
                ((float4 *)yr)[f] = v;
            }
        }
    } else {
        for (int i = tid; i < ne0; i += 256) {
            const float v = xr[i] * scale;
            yr[i] = w ? v * w[i] : v;
        }
    }
}

// dst[i] = a[i] (op) b[i % nb], contiguous rows of a; b broadcast along rows
template <int OP>
__global__ void k_binary_bcast(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ d,
                               int64_t n, int64_t nb) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float bv = b[i % nb];
    d[i] = OP == 0 ? a[i] + bv : a[i] * bv;
}

// neox RoPE on [ne0 = head_dim][ne1 = heads][ne2 = tokens] fp32, pos[ne2]
__global__ void k_rope_neox(const float *__restrict__ x, float *__restrict__ y, const int32_t *__restrict__ pos,
                            int ne0, int ne1, int n_dims, float theta_scale, float freq_scale, float attn_factor,
                            size_t nb1, size_t nb2, size_t ob1, size_t ob2) {
    const int i = threadIdx.x;  // pair index < n_dims/2
    const int h = blockIdx.x;
    const int t = blockIdx.y;
    const char *xr = (const char *)x + (size_t)t * nb2 + (size_t)h * nb1;
    char *yr = (char *)y + (size_t)t * ob2 + (size_t)h * ob1;
    const int half = n_dims / 2;
    if (i < half) {
        float theta = (float)pos[t];
        for (int k = 0; k < i; k++) theta *= theta_scale;  // same product order as the CPU cache
        const float th = freq_scale * theta;
        const float c = cosf(th) * attn_factor;
        const float s = sinf(th) * attn_factor;
        const float x0 = ((const float *)xr)[i];
        const float x1 = ((const float *)xr)[i + half];
        ((float *)yr)[i] = mul_sub_mul_rn(x0, c, x1, s);  // unfused, as the CPU loop
        ((float *)yr)[i + half] = mul_add_mul_rn(x0, s, x1, c);
    }
    for (int j = n_dims + i; j < ne0; j += blockDim.x) ((float *)yr)[j] = ((const float *)xr)[j];
}

// The neox rotation table of one position: tab[p] = cos(theta_p) * attn_factor,
// tab[n_pairs + p] = sin(theta_p) * attn_factor, theta_p = freq_scale * (pos * theta_scale^p)
// with the power formed by p repeated multiplications (the CPU rope cache's order): one
// thread walks the chain into LDS, then every thread converts its pairs.
__global__ __launch_bounds__(256) void k_rope_table(const int32_t *__restrict__ pos, float *__restrict__ tab,
                                                    int n_pairs, float theta_scale, float freq_scale,
                                                    float attn_factor) {
    __shared__ float s_theta[512];
    if (threadIdx.x == 0) {
        float t = (float)pos[0];
        for (int p = 0; p < n_pairs; p++) {
            s_theta[p] = t;
            t *= theta_scale;
        }
    }
    __syncthreads();
    for (int p = threadIdx.x; p < n_pairs; p += 256) {
        const float th = freq_scale * s_theta[p];
        tab[p] = cosf(th) * attn_factor;
        tab[n_pairs + p] = sinf(th) * attn_factor;
    }
}

// dst rows idx[r] (fp16 table, row stride dnb1 bytes) = fp16(src row r)
template <typename IDX>
__global__ void k_set_rows_f16(const float *__restrict__ src, const IDX *__restrict__ idx, uint16_t *__restrict__ dst,
                               int ne0, size_t snb1, size_t dnb1, int64_t n_dst_rows) {
    const int r = blockIdx.x;
    const int64_t dr = (int64_t)idx[r];
    if (dr < 0 || dr >= n_dst_rows) return;
    const float *s = (const float *)((const char *)src + (size_t)r * snb1);
    uint16_t *d = (uint16_t *)((char *)dst + (size_t)dr * dnb1);
    for (int i = threadIdx.x; i < ne0; i += blockDim.x) d[i] = f2h(s[i]);
}

// ROPE q and ROPE k (neox over all hd dims, position pos[r] for activation row r), then
// SET_ROWS of the rotated k and of v into their fp16 cache rows kv_idx[r]: the four nodes
// after the q/k/v projections in one launch for m rows.  Per element the arithmetic of
// k_rope_neox and k_set_rows_f16.  grid (n_hq + n_hk + ceil(n_v / 128), m), 128 threads.
template <typename IDX>
__global__ __launch_bounds__(128) void k_rope_kv_rows(const float *__restrict__ q, const float *__restrict__ k,
                                                      const float *__restrict__ v, float *__restrict__ q_out,
                                                      uint8_t *__restrict__ kc, uint8_t *__restrict__ vc,
                                                      const int32_t *__restrict__ pos, const IDX *__restrict__ kv_idx,
                                                      int hd, int n_hq, int n_hk, int n_v, size_t k_row_bytes,
                                                      size_t v_row_bytes, int64_t n_cache_rows, float theta_scale,
                                                      float freq_scale, float attn_factor) {
    const int b = blockIdx.x, r = blockIdx.y, i = threadIdx.x;
    const int64_t ci = (int64_t)kv_idx[r];
    const bool ci_ok = ci >= 0 && ci < n_cache_rows;
    if (b < n_hq + n_hk) {
        const int half = hd / 2;
        if (i >= half) return;
        const bool is_q = b < n_hq;
        const float *xr = is_q ? q + ((size_t)r * n_hq + b) * hd : k + ((size_t)r * n_hk + (b - n_hq)) * hd;
        float theta = (float)pos[r];
        for (int t = 0; t < i; t++) theta *= theta_scale;  // same product order as the CPU cache
        const float th = freq_scale * theta;
        const float c = cosf(th) * attn_factor;
        const float s = sinf(th) * attn_factor;
        const float x0 = xr[i], x1 = xr[i + half];
        const float y0 = mul_sub_mul_rn(x0, c, x1, s);
        const float y1 = mul_add_mul_rn(x0, s, x1, c);
        if (is_q) {
            float *yr = q_out + ((size_t)r * n_hq + b) * hd;
            yr[i] = y0;
            yr[i + half] = y1;
        } else if (ci_ok) {
            uint16_t *kr = (uint16_t *)(kc + (size_t)ci * k_row_bytes) + (size_t)(b - n_hq) * hd;
            kr[i] = f2h(y0);
            kr[i + half] = f2h(y1);
        }
    } else {
        const int j = (b - n_hq - n_hk) * 128 + i;
        if (j < n_v && ci_ok) ((uint16_t *)(vc + (size_t)ci * v_row_bytes))[j] = f2h(v[(size_t)r * n_v + j]);
    }
}

template <typename T, typename IDX>
__global__ void k_get_rows(const T *__restrict__ src, const IDX *__restrict__ idx, float *__restrict__ dst, int ne0,
                           size_t snb1, int64_t n_src_rows) {
    const int r = blockIdx.x;
    int64_t sr = (int64_t)idx[r];
    sr = sr < 0 ? 0 : (sr >= n_src_rows ? n_src_rows - 1 : sr);
    const T *s = (const T *)((const char *)src + (size_t)sr * snb1);
    float *d = dst + (size_t)r * ne0;
    for (int i = threadIdx.x; i < ne0; i += blockDim.x) {
        if constexpr (sizeof(T) == 2) d[i] = h2f(s[i]);
        else d[i] = s[i];
    }
}

// silu(g) * u with ggml's silu: x / (1 + exp(-x))
__global__ void k_swiglu(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ d, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = g[i];
    d[i] = (x / (1.0f + expf(-x))) * u[i];
}

// ARGMAX in two passes: per chunk of a row the first maximum (strict >, so NaN is
// never taken and ties keep the lower index), then one workgroup per row over the
// chunk results.  Partials are (value, index) pairs in the workspace.
__device__ __forceinline__ void argmax_merge(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

__device__ __forceinline__ void argmax_block(float &best, int &bi) {
    __shared__ float sv[4];
    __shared__ int si[4];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) argmax_merge(best, bi, __shfl_xor(best, o, 64), __shfl_xor(bi, o, 64));
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = best; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    best = sv[0];
    bi = si[0];
#pragma unroll
    for (int w = 1; w < 4; w++) argmax_merge(best, bi, sv[w], si[w]);
}

__global__ __launch_bounds__(256) void k_argmax_part(const float *__restrict__ x, float2 *__restrict__ part, int ne0,
                                                     int chunk, int nchunks) {
    const int row = blockIdx.y, c = blockIdx.x;
    const float *xr = x + (size_t)row * ne0;
    const int start = c * chunk, end = min(start + chunk, ne0);
    float best = -INFINITY;
    int bi = start;
#pragma unroll 8
    for (int i = start + (int)threadIdx.x; i < end; i += 256) {
        const float v = xr[i];
        if (v > best) { best = v; bi = i; }
    }
    argmax_block(best, bi);
    if (threadIdx.x == 0) part[(size_t)row * nchunks + c] = make_float2(best, __int_as_float(bi));
}

__global__ __launch_bounds__(256) void k_argmax_final(const float2 *__restrict__ part, int32_t *__restrict__ out,
                                                      int nchunks) {
    const int row = blockIdx.x;
    float best = -INFINITY;
    int bi = INT_MAX;
    for (int c = threadIdx.x; c < nchunks; c += 256) {
        const float2 p = part[(size_t)row * nchunks + c];
        argmax_merge(best, bi, p.x, __float_as_int(p.y));
    }
    argmax_block(best, bi);
    if (threadIdx.x == 0) out[row] = bi == INT_MAX ? 0 : bi;
}

inline int64_t argmax_chunk(int64_t ne0) {
    int64_t c = (ne0 + 255) / 256;
    c = (c + 1023) / 1024 * 1024;
    return c < 2048 ? 2048 : c;
}

// fp16 decode mask row from the effective length: 0 for pos < len, -inf beyond
__global__ void k_fill_mask(uint16_t *__restrict__ mask, const int32_t *__restrict__ len, int n_kv) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n_kv) mask[i] = i < *len ? (uint16_t)0 : (uint16_t)0xfc00u;
}

// rows of fp16 values uniform in [-scale, scale) from a counter-based hash (SplitMix64
// finalizer of seed + element index): synthetic KV-cache contents of a given length
__global__ void k_fill_f16_uniform(uint8_t *__restrict__ dst, int64_t rows, int64_t row_elems, size_t row_stride,
                                   uint64_t seed, float scale) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * row_elems) return;
    const int64_t r = i / row_elems, e = i % row_elems;
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(i + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const float u = (float)(z >> 40) * (1.0f / 16777216.0f);  // [0, 1)
    ((uint16_t *)(dst + (size_t)r * row_stride))[e] = f2h((2.0f * u - 1.0f) * scale);
}

unsigned grid1(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

}  // namespace

extern "C" {

int mi_rms_norm(void *stream, const float *x, const float *w, float *y, int64_t ne0, int64_t nrows, float eps) {
    MI_CHECK_ARG(x && y && ne0 > 0 && nrows > 0, "rms_norm: bad arguments");
    hipLaunchKernelGGL(k_rms_norm, dim3((unsigned)nrows), dim3(256), 0, (hipStream_t)stream, x, w, y, (int)ne0, eps);
    MI_CHECK_LAUNCH("k_rms_norm");
    return MI_OK;
}

int mi_add_bcast(void *stream, const float *a, const float *b, float *d, int64_t n, int64_t nb) {
    MI_CHECK_ARG(a && b && d && n > 0 && nb > 0, "add: bad arguments");
    hipLaunchKernelGGL((k_binary_bcast<0>), dim3(grid1(n, 256)), dim3(256), 0, (hipStream_t)stream, a, b, d, n, nb);
    MI_CHECK_LAUNCH("k_add");
    return MI_OK;
}

int mi_mul_bcast(void *stream, const float *a, const float *b, float *d, int64_t n, int64_t nb) {
    MI_CHECK_ARG(a && b && d && n > 0 && nb > 0, "mul: bad arguments");
    hipLaunchKernelGGL((k_binary_bcast<1>), dim3(grid1(n, 256)), dim3(256), 0, (hipStream_t)stream, a, b, d, n, nb);
    MI_CHECK_LAUNCH("k_mul");
    return MI_OK;
}

int mi_rope_neox(void *stream, const float *x, float *y, const int32_t *pos, int64_t ne0, int64_t ne1, int64_t ne2,
                 int64_t n_dims, float freq_base, float freq_scale, float attn_factor, size_t nb1, size_t nb2,
                 size_t ob1, size_t ob2) {
    // theta_scale on the host with the C library powf, as the CPU rope cache does
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    MI_CHECK_ARG(x && y && pos && n_dims > 0 && n_dims % 2 == 0 && n_dims <= ne0 && n_dims <= 1024,
                 "rope: bad arguments");
    const int threads = (int)((n_dims / 2 + 63) / 64 * 64);
    hipLaunchKernelGGL(k_rope_neox, dim3((unsigned)ne1, (unsigned)ne2), dim3(threads), 0, (hipStream_t)stream, x, y,
                       pos, (int)ne0, (int)ne1, (int)n_dims, theta_scale, freq_scale, attn_factor, nb1, nb2, ob1, ob2);
    MI_CHECK_LAUNCH("k_rope_neox");
    return MI_OK;
}

int mi_rope_kv_rows(void *stream, const float *q, const float *k, const float *v, float *q_out, void *k_cache,
                    size_t k_row_bytes, void *v_cache, size_t v_row_bytes, const int32_t *pos, const void *kv_idx,
                    int kv_idx_is_i64, int64_t n_cache_rows, int64_t m, int64_t head_dim, int64_t n_head_q,
                    int64_t n_head_k, int64_t n_v, float freq_base, float freq_scale, float attn_factor) {
    MI_CHECK_ARG(q && k && v && q_out && k_cache && v_cache && pos && kv_idx, "rope_kv_rows: null pointer");
    MI_CHECK_ARG(m >= 1 && m <= 65535 && head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 256 && n_head_q > 0 &&
                     n_head_k > 0 && n_v > 0 && n_head_q + n_head_k + (n_v + 127) / 128 < (1 << 30),
                 "rope_kv_rows: bad shape");
    MI_CHECK_ARG(k_row_bytes >= (size_t)(n_head_k * head_dim * 2) && v_row_bytes >= (size_t)(n_v * 2),
                 "rope_kv_rows: cache rows too short");
    const float theta_scale = powf(freq_base, -2.0f / (float)head_dim);
    const dim3 grid((unsigned)(n_head_q + n_head_k + (n_v + 127) / 128), (unsigned)m);
#define MI_RKV(IDX)                                                                                                \
    hipLaunchKernelGGL((k_rope_kv_rows<IDX>), grid, dim3(128), 0, (hipStream_t)stream, q, k, v, q_out,             \
                       (uint8_t *)k_cache, (uint8_t *)v_cache, pos, (const IDX *)kv_idx, (int)head_dim,            \
                       (int)n_head_q, (int)n_head_k, (int)n_v, k_row_bytes, v_row_bytes, n_cache_rows, theta_scale, \
                       freq_scale, attn_factor)
    if (kv_idx_is_i64) MI_RKV(int64_t);
    else MI_RKV(int32_t);
#undef MI_RKV
    MI_CHECK_LAUNCH("k_rope_kv_rows");
    return MI_OK;
}

int mi_rope_table(void *stream, const int32_t *pos, int64_t head_dim, float freq_base, float freq_scale,
                  float attn_factor, float *table) {
    MI_CHECK_ARG(pos && table && head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 1024, "rope_table: bad arguments");
    const float theta_scale = powf(freq_base, -2.0f / (float)head_dim);
    hipLaunchKernelGGL(k_rope_table, dim3(1), dim3(256), 0, (hipStream_t)stream, pos, table, (int)(head_dim / 2),
                       theta_scale, freq_scale, attn_factor);
    MI_CHECK_LAUNCH("k_rope_table");
    return MI_OK;
}

int mi_set_rows_f16(void *stream, const float *src, const void *idx, int idx_is_i64, uint16_t *dst, int64_t ne0,
                    int64_t nrows, size_t snb1, size_t dnb1, int64_t n_dst_rows) {
    MI_CHECK_ARG(src && idx && dst && ne0 > 0 && nrows > 0, "set_rows: bad arguments");
    if (idx_is_i64)
        hipLaunchKernelGGL((k_set_rows_f16<int64_t>), dim3((unsigned)nrows), dim3(256), 0, (hipStream_t)stream, src,
                           (const int64_t *)idx, dst, (int)ne0, snb1, dnb1, n_dst_rows);
    else
        hipLaunchKernelGGL((k_set_rows_f16<int32_t>), dim3((unsigned)nrows), dim3(256), 0, (hipStream_t)stream, src,
                           (const int32_t *)idx, dst, (int)ne0, snb1, dnb1, n_dst_rows);
    MI_CHECK_LAUNCH("k_set_rows_f16");
    return MI_OK;
}

int mi_get_rows(void *stream, const void *src, int src_is_f16, const int32_t *idx, float *dst, int64_t ne0,
                int64_t nrows, size_t snb1, int64_t n_src_rows) {
    MI_CHECK_ARG(src && idx && dst && ne0 > 0 && nrows > 0, "get_rows: bad arguments");
    if (src_is_f16)
        hipLaunchKernelGGL((k_get_rows<uint16_t, int32_t>), dim3((unsigned)nrows), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t *)src, idx, dst, (int)ne0, snb1, n_src_rows);
    else
        hipLaunchKernelGGL((k_get_rows<float, int32_t>), dim3((unsigned)nrows), dim3(256), 0, (hipStream_t)stream,
                           (const float *)src, idx, dst, (int)ne0, snb1, n_src_rows);
    MI_CHECK_LAUNCH("k_get_rows");
    return MI_OK;
}

int mi_swiglu(void *stream, const float *g, const float *u, float *d, int64_t n) {
    MI_CHECK_ARG(g && u && d && n > 0, "swiglu: bad arguments");
    hipLaunchKernelGGL(k_swiglu, dim3(grid1(n, 256)), dim3(256), 0, (hipStream_t)stream, g, u, d, n);
    MI_CHECK_LAUNCH("k_swiglu");
    return MI_OK;
}

size_t mi_argmax_workspace_size(int64_t ne0, int64_t nrows) {
    if (ne0 <= 0 || nrows <= 0) return 0;
    const int64_t nchunks = (ne0 + argmax_chunk(ne0) - 1) / argmax_chunk(ne0);
    return mi::align_up((size_t)(nchunks * nrows) * sizeof(float2), 256);
}

int mi_argmax(void *stream, const float *x, int32_t *out, int64_t ne0, int64_t nrows, void *ws, size_t ws_bytes) {
    MI_CHECK_ARG(x && out && ne0 > 0 && nrows > 0 && ne0 < (1ll << 31) && nrows < 65536, "argmax: bad arguments");
    const size_t need = mi_argmax_workspace_size(ne0, nrows);
    if (!ws || ws_bytes < need || !mi::aligned(ws, 8)) {
        mi::set_error("argmax: workspace %zu < %zu bytes (or misaligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    const int64_t chunk = argmax_chunk(ne0);
    const int nchunks = (int)((ne0 + chunk - 1) / chunk);
    hipLaunchKernelGGL(k_argmax_part, dim3((unsigned)nchunks, (unsigned)nrows), dim3(256), 0, (hipStream_t)stream, x,
                       (float2 *)ws, (int)ne0, (int)chunk, nchunks);
    MI_CHECK_LAUNCH("k_argmax_part");
    hipLaunchKernelGGL(k_argmax_final, dim3((unsigned)nrows), dim3(256), 0, (hipStream_t)stream, (const float2 *)ws,
                       out, nchunks);
    MI_CHECK_LAUNCH("k_argmax_final");
    return MI_OK;
}

int mi_fill_f16_uniform(void *stream, void *dst, int64_t rows, int64_t row_elems, size_t row_stride, uint64_t seed,
                        float scale) {
    MI_CHECK_ARG(dst && rows >= 0 && row_elems > 0 && row_stride >= (size_t)row_elems * 2 && mi::aligned(dst, 2) &&
                     row_stride % 2 == 0,
                 "fill_f16_uniform: bad arguments");
    if (rows == 0) return MI_OK;
    hipLaunchKernelGGL(k_fill_f16_uniform, dim3(grid1(rows * row_elems, 256)), dim3(256), 0, (hipStream_t)stream,
                       (uint8_t *)dst, rows, row_elems, row_stride, seed, scale);
    MI_CHECK_LAUNCH("k_fill_f16_uniform");
    return MI_OK;
}

int mi_fill_mask_f16(void *stream, uint16_t *mask, const int32_t *len, int64_t n_kv) {
    MI_CHECK_ARG(mask && len && n_kv > 0, "fill_mask: bad arguments");
    hipLaunchKernelGGL(k_fill_mask, dim3(grid1(n_kv, 256)), dim3(256), 0, (hipStream_t)stream, mask, len, (int)n_kv);
    MI_CHECK_LAUNCH("k_fill_mask");
    return MI_OK;
}

}  // extern "C"
