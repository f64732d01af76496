// decode_common.h -- device pieces shared by the Q8_0 (A8W8) and Q4_0 (W4A16) fused
// decode kernels: the activation row staged through registers with an optional
// RMSNorm, and the q/k/v epilogue (bias, neox RoPE, KV-cache write).
#pragma once

#include "mi_common.h"

namespace mi {

// One activation row staged by a 256-thread workgroup: XN float4 per thread
// (k <= 1024*XN), loaded before the weights so that the activation step waits only
// for the cache-resident activation while the weight loads are in flight.  sv holds
// the SmoothQuant reciprocal (A8W8 only), nv the RMSNorm weight.
template <int XN, bool NORM>
struct XStage {
    float4 xv[XN], sv[XN], nv[XN];
};

template <int XN, bool NORM>
__device__ __forceinline__ void xstage_load(XStage<XN, NORM> &st, const float *__restrict__ x,
                                            const float *__restrict__ norm_w, const float *__restrict__ inv_s, int k4,
                                            int tid) {
#pragma unroll
    for (int t = 0; t < XN; t++) {
        const int f = min(tid + t * 256, k4 - 1);
        st.xv[t] = ((const float4 *)x)[f];
        if constexpr (NORM) st.nv[t] = ((const float4 *)norm_w)[f];
        if (inv_s) st.sv[t] = ((const float4 *)inv_s)[f];
    }
}

// RMSNorm scale of the staged row, as ggml's CPU rms_norm computes it:
// scale = 1/sqrtf(mean + eps), mean = (float)(sum of (double)(x*x) / k).  1 without
// NORM.  With NORM it contains a workgroup barrier (every thread must call it).
template <int XN, bool NORM>
__device__ __forceinline__ float xstage_scale(const XStage<XN, NORM> &st, int k4, float eps, double *s_red, int tid) {
    if constexpr (!NORM) {
        return 1.0f;
    } else {
        double ss = 0.0;
#pragma unroll
        for (int t = 0; t < XN; t++) {
            if (tid + t * 256 < k4) {
                const float4 v = st.xv[t];
                ss += (double)sq_rn(v.x);
                ss += (double)sq_rn(v.y);
                ss += (double)sq_rn(v.z);
                ss += (double)sq_rn(v.w);
            }
        }
        const double tot = block_sum_d256(ss, s_red, tid);
        const float mean = (float)(tot / (double)(k4 * 4));
        return 1.0f / sqrtf(mean + eps);
    }
}

// Staged value t after the norm (ggml rms_norm then mul: (x*scale)*w).
template <int XN, bool NORM>
__device__ __forceinline__ float4 xstage_value(const XStage<XN, NORM> &st, float scale, int t) {
    float4 v = st.xv[t];
    if constexpr (NORM) {
        v.x = (v.x * scale) * st.nv[t].x; v.y = (v.y * scale) * st.nv[t].y;
        v.z = (v.z * scale) * st.nv[t].z; v.w = (v.w * scale) * st.nv[t].w;
    }
    return v;
}

// The attention-input chain after the q/k/v projections: bias add, neox RoPE of q
// and k (theta_i = pos * theta_scale^i by repeated multiplication, products unfused
// as in ggml's CPU loop), q written fp32, k and v converted to fp16 into the cache row
// kv_idx[0] (ggml set_rows).  Rows are numbered in the stacked q|k|v space.
struct RopeKV {
    const float *bias[3];
    float *q_out;
    uint8_t *k_cache, *v_cache;
    size_t k_row_bytes, v_row_bytes;
    const int32_t *pos;
    const void *kv_idx;
    int kv_idx_i64;
    int64_t n_cache_rows;
    int hd, n_q, n_k, n_v;
    float theta_scale, freq_scale, attn_factor;
    const float *tab;  // [2][hd/2] cos, sin (mi_rope_table), or NULL: formed per launch
};

// The table entries (cos, sin) of rotation pair p, loaded early: branch-free (without a
// table the loads read pos[0], and the values are not used).
__device__ __forceinline__ void rope_tab_prefetch(const RopeKV &R, int p, float &cs, float &sn) {
    const int half = R.hd / 2;
    p = min(max(p, 0), half - 1);
    const float *c = R.tab ? R.tab + p : (const float *)R.pos;
    const float *s = R.tab ? R.tab + half + p : (const float *)R.pos;
    cs = *c;
    sn = *s;
}

// Row mapping of a workgroup of RPB rows.  A workgroup on the rotated rows (q and k)
// owns HALF = RPB/2 rotation pairs (i, i + hd/2) of one head, so each pair's two
// results meet in LDS; slot t < HALF holds element i, slot t >= HALF element i + hd/2.
// V workgroups take RPB consecutive rows.  Returns the stacked row of slot t (may be
// >= n_q + n_k + n_v in the last V workgroup: the caller clamps its loads).
struct RopeKVPlace {
    bool rope;
    int head, chunk;
};

template <int RPB>
__device__ __forceinline__ int rope_kv_row(const RopeKV &R, int b, int t, RopeKVPlace &pl) {
    constexpr int HALF = RPB / 2;
    const int n_rope = R.n_q + R.n_k;
    const int wg_per_head = R.hd / RPB;
    pl.rope = b < n_rope / RPB;
    pl.head = b / wg_per_head;
    pl.chunk = b % wg_per_head;
    return pl.rope ? pl.head * R.hd + (t / HALF) * (R.hd / 2) + pl.chunk * HALF + (t % HALF) : b * RPB + t;
}

// Epilogue over the workgroup's RPB biased projections y[0..RPB) in LDS (the caller
// has synchronised after writing them).
template <int RPB>
__device__ __forceinline__ void rope_kv_epilogue(const RopeKV &R, const float *y, int b, int tid,
                                                 const RopeKVPlace &pl, float tab_cs, float tab_sn) {
    constexpr int HALF = RPB / 2;
    const int n_rope = R.n_q + R.n_k;
    const int64_t ci = R.kv_idx_i64 ? ((const int64_t *)R.kv_idx)[0] : (int64_t)((const int32_t *)R.kv_idx)[0];
    const bool ci_ok = ci >= 0 && ci < R.n_cache_rows;
    if (pl.rope) {
        if (tid < HALF) {
            const int p = pl.chunk * HALF + tid;  // rotation pair index < hd/2
            float cs = tab_cs, sn = tab_sn;
            if (!R.tab) {
                float theta = (float)R.pos[0];
                for (int i = 0; i < p; i++) theta *= R.theta_scale;
                const float th = R.freq_scale * theta;
                cs = cosf(th) * R.attn_factor;
                sn = sinf(th) * R.attn_factor;
            }
            const float x0 = y[tid], x1 = y[tid + HALF];
            const float y0 = mul_sub_mul_rn(x0, cs, x1, sn);
            const float y1 = mul_add_mul_rn(x0, sn, x1, cs);
            const int r0 = pl.head * R.hd + p;  // row in the stacked q|k space
            if (r0 < R.n_q) {
                R.q_out[r0] = y0;
                R.q_out[r0 + R.hd / 2] = y1;
            } else if (ci_ok) {
                uint16_t *kr = (uint16_t *)(R.k_cache + (size_t)ci * R.k_row_bytes);
                kr[r0 - R.n_q] = f2h(y0);
                kr[r0 - R.n_q + R.hd / 2] = f2h(y1);
            }
        }
    } else if (tid < RPB) {
        const int vr = b * RPB + tid - n_rope;
        if (vr < R.n_v && ci_ok) ((uint16_t *)(R.v_cache + (size_t)ci * R.v_row_bytes))[vr] = f2h(y[tid]);
    }
}

}  // namespace mi
