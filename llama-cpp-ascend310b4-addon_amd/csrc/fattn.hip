// fattn.hip -- single-token GQA flash-decoding for gfx950.
//
// Replaces AttentionStepCustom
// (experiments/attention-step-custom/custom_ops/op_kernel/attention_step_custom.cpp:60-597):
// instead of one core per q head streaming the whole KV length, the KV length is
// split across workgroups (one per (split, kv head)); every K/V row is read once
// and shared by all q heads of its GQA group; each workgroup keeps an online
// softmax state (m, l, o) per q head and a parallel log-sum-exp combine kernel
// merges the splits.  (An in-kernel merge by the last workgroup of a kv head exists
// behind MI_FA_MERGE=1 / MI_FA_FUSED_COMBINE=1; it measured slower, so it is off by
// default.)  Score order follows the reference and ggml: q rounded to fp16,
// s = (q.k) * scale, s += mask, online softmax, one final divide.
#include "fattn_dev.h"

#include <math.h>
#include <stdlib.h>

#include <mutex>

#include <type_traits>

namespace {

using namespace mi;

template <int LPR>
__device__ __forceinline__ void merge_state(float &m, float &l, float *o, int xor_mask) {
    const float mo = __shfl_xor(m, xor_mask, 64);
    const float lo = __shfl_xor(l, xor_mask, 64);
    float oo[8];
#pragma unroll
    for (int i = 0; i < 8; i++) oo[i] = __shfl_xor(o[i], xor_mask, 64);
    const float mn = fmaxf(m, mo);
    if (mn == -INFINITY) return;
    const float a = fexp2(m - mn);
    const float b = fexp2(mo - mn);
    l = l * a + lo * b;
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = o[i] * a + oo[i] * b;
    m = mn;
}

template <int D, int GQ, bool MASK, int kT>
__global__ __launch_bounds__(256) void k_fa_split(const float *__restrict__ q, const uint8_t *__restrict__ kc,
                                                  const uint8_t *__restrict__ vc, const uint16_t *__restrict__ mask,
                                                  const int32_t *__restrict__ kv_len_p, int n_kv, size_t k_nb1,
                                                  size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, int chunk,
                                                  int n_splits, float *__restrict__ part, float *__restrict__ out,
                                                  unsigned *__restrict__ counters, const FaSeq sq) {
    {
        const int seq = blockIdx.z;
        q += (size_t)seq * sq.q;
        kc += (size_t)seq * sq.k;
        vc += (size_t)seq * sq.v;
        if (MASK) mask += (size_t)seq * sq.mask;
        if (kv_len_p) kv_len_p += (size_t)seq * sq.kvl;
        out += (size_t)seq * sq.out;
        part += (size_t)seq * gridDim.y * GQ * n_splits * part_stride<D>();
        if (counters) counters += (size_t)seq * gridDim.y;
    }
    constexpr int LPR = D / 8;     // lanes per position row (16 B = 8 halves per lane)
    constexpr int PPW = 64 / LPR;  // positions per wave step
    constexpr int NG = kNW * PPW;  // lane groups per workgroup
    constexpr int PS = part_stride<D>();
    __shared__ float s_m[kNW][GQ];
    __shared__ float s_l[kNW][GQ];
    __shared__ __align__(16) float s_o[kNW][GQ][D];

    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid % 64;
    const int wave = tid / 64;
    const int c = lane % LPR;
    const int g = wave * PPW + lane / LPR;

    // The effective length (ggml src[5]) bounds the tiles after the first: the first
    // tile's K/V loads are issued against the physical length so that they do not
    // wait for the kv_len load (the KV view handed in is at most a little longer
    // than the used cache, so the speculative rows are few).
    const int kl = kv_len_p ? *kv_len_p : n_kv;
    const int eff = (kl > 0 && kl < n_kv) ? kl : n_kv;
    const int start = split * chunk;
    const int end_phys = min(start + chunk, n_kv);

    uint32_t qh[GQ][4];
#pragma unroll
    for (int h = 0; h < GQ; h++) {
        const float4 *qp = (const float4 *)(q + (size_t)(kvh * GQ + h) * D + 8 * c);
        const float4 a = qp[0], b = qp[1];
        qh[h][0] = (uint32_t)f2h(a.x) | ((uint32_t)f2h(a.y) << 16);
        qh[h][1] = (uint32_t)f2h(a.z) | ((uint32_t)f2h(a.w) << 16);
        qh[h][2] = (uint32_t)f2h(b.x) | ((uint32_t)f2h(b.y) << 16);
        qh[h][3] = (uint32_t)f2h(b.z) | ((uint32_t)f2h(b.w) << 16);
    }

    float m[GQ], l[GQ], o[GQ][8];
#pragma unroll
    for (int h = 0; h < GQ; h++) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) o[h][i] = 0.0f;
    }

    const uint8_t *kb = kc + (size_t)kvh * k_nb2 + (size_t)c * 16;
    const uint8_t *vb = vc + (size_t)kvh * v_nb2 + (size_t)c * 16;

    // first tile: speculative (physical bound); later tiles stop at the effective length
    const int end_eff = min(end_phys, eff);
    for (int p0 = start + g, it = 0; p0 < (it == 0 ? end_phys : end_eff); p0 += NG * kT, it++) {
        int4 kr[kT], vr[kT];
        float mk[kT];
        bool val[kT];
#pragma unroll
        for (int t = 0; t < kT; t++) {  // branch-free loads (clamped rows) keep all 2*kT loads in flight
            const int p = p0 + t * NG;
            const int pc = min(p, end_phys - 1);
            kr[t] = *(const int4 *)(kb + (size_t)pc * k_nb1);
            vr[t] = *(const int4 *)(vb + (size_t)pc * v_nb1);
            mk[t] = MASK ? h2f(mask[pc]) : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < kT; t++) val[t] = p0 + t * NG < min(end_phys, eff);
        float s[GQ][kT];
#pragma unroll
        for (int t = 0; t < kT; t++) {
#pragma unroll
            for (int h = 0; h < GQ; h++) {
                float dsum = 0.0f;
                dsum = fdot2(qh[h][0], (uint32_t)kr[t].x, dsum);
                dsum = fdot2(qh[h][1], (uint32_t)kr[t].y, dsum);
                dsum = fdot2(qh[h][2], (uint32_t)kr[t].z, dsum);
                dsum = fdot2(qh[h][3], (uint32_t)kr[t].w, dsum);
                dsum = group_sum<LPR>(dsum);
                // ggml order: s = (q.k)*scale; s += mask; kept in log2 units for v_exp_f32
                const float sc = mul_add_rn(dsum, scale, mk[t]) * kLog2e;
                s[h][t] = val[t] ? sc : -INFINITY;
            }
        }
#pragma unroll
        for (int h = 0; h < GQ; h++) {
            float mt = s[h][0];
#pragma unroll
            for (int t = 1; t < kT; t++) mt = fmaxf(mt, s[h][t]);
            const float mn = fmaxf(m[h], mt);
            // nothing unmasked yet (uniform in the lane group): keep the empty state
            const float alpha = mn == -INFINITY ? 1.0f : fexp2(m[h] - mn);
            l[h] *= alpha;
#pragma unroll
            for (int i = 0; i < 8; i++) o[h][i] *= alpha;
#pragma unroll
            for (int t = 0; t < kT; t++) s[h][t] = mn == -INFINITY ? 0.0f : fexp2(s[h][t] - mn);
            m[h] = mn;
        }
#pragma unroll
        for (int t = 0; t < kT; t++) {
            const uint32_t w4[4] = {(uint32_t)vr[t].x, (uint32_t)vr[t].y, (uint32_t)vr[t].z, (uint32_t)vr[t].w};
            float vf[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                vf[2 * i] = h2f((uint16_t)(w4[i] & 0xffffu));
                vf[2 * i + 1] = h2f((uint16_t)(w4[i] >> 16));
            }
#pragma unroll
            for (int h = 0; h < GQ; h++) {
                l[h] += s[h][t];
#pragma unroll
                for (int i = 0; i < 8; i++) o[h][i] = fmaf(s[h][t], vf[i], o[h][i]);
            }
        }
    }

    // merge the lane groups of this wave
#pragma unroll
    for (int x = LPR; x < 64; x *= 2) {
#pragma unroll
        for (int h = 0; h < GQ; h++) merge_state<LPR>(m[h], l[h], o[h], x);
    }
    // every lane group of the wave now holds the wave state; group 0 publishes it
    if (lane < LPR) {
#pragma unroll
        for (int h = 0; h < GQ; h++) {
            *(float4 *)&s_o[wave][h][8 * c] = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
            *(float4 *)&s_o[wave][h][8 * c + 4] = make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
            if (c == 0) {
                s_m[wave][h] = m[h];
                s_l[wave][h] = l[h];
            }
        }
    }
    __syncthreads();

    // final merge across waves: thread (h, dim) for GQ*D threads, strided over the block
    for (int idx = tid; idx < GQ * D; idx += 256) {
        const int h = idx / D;
        const int dd = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kNW; w++) M = fmaxf(M, s_m[w][h]);
        float L = 0.0f, acc = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kNW; w++) {
                const float e = fexp2(s_m[w][h] - M);
                L += s_l[w][h] * e;
                acc += s_o[w][h][dd] * e;
            }
        }
        const int qh_idx = kvh * GQ + h;
        if (n_splits == 1 && out) {
            out[(size_t)qh_idx * D + dd] = L == 0.0f ? 0.0f : acc / L;
        } else {
            float *rec = part + ((size_t)qh_idx * n_splits + split) * PS;
            rec[dd] = acc;
            if (dd == 0) {
                rec[D] = M;
                rec[D + 1] = L;
            }
        }
    }
    if (n_splits == 1 || counters == nullptr) return;

    // Fused combine: the last workgroup of this kv head to finish merges all splits.
    // Release the partials device-wide, count arrivals, and acquire before reading.
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(&counters[kvh], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (unsigned)(n_splits - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // every (head, split) m and l in one round of loads, then the weights
    __shared__ float s_cm[GQ][kFusedMaxSplits];
    __shared__ float s_cl[GQ][kFusedMaxSplits];
    if (tid < GQ * n_splits) {
        const int h = tid / n_splits, sp = tid % n_splits;
        const float *rec = part + ((size_t)(kvh * GQ + h) * n_splits + sp) * PS;
        s_cm[h][sp] = rec[D];
        s_cl[h][sp] = rec[D + 1];
    }
    __syncthreads();
    // all o loads of this thread's outputs issued together (clamped, branch-free)
    constexpr int OPT = (GQ * D + 255) / 256;
    float ov[OPT][kFusedMaxSplits];
#pragma unroll
    for (int oi = 0; oi < OPT; oi++) {
        const int idx = min(tid + oi * 256, GQ * D - 1);
        const float *ph = part + (size_t)(kvh * GQ + idx / D) * n_splits * PS + idx % D;
#pragma unroll
        for (int sp = 0; sp < kFusedMaxSplits; sp++) ov[oi][sp] = ph[(size_t)min(sp, n_splits - 1) * PS];
    }
#pragma unroll
    for (int oi = 0; oi < OPT; oi++) {
        const int idx = tid + oi * 256;
        if (idx >= GQ * D) break;
        const int h = idx / D;
        float M = -INFINITY;
        for (int sp = 0; sp < n_splits; sp++) M = fmaxf(M, s_cm[h][sp]);
        float L = 0.0f, acc = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int sp = 0; sp < kFusedMaxSplits; sp++) {
                const float ms = sp < n_splits ? s_cm[h][sp] : -INFINITY;
                const float e = ms == -INFINITY ? 0.0f : fexp2(ms - M);
                L += (sp < n_splits ? s_cl[h][sp] : 0.0f) * e;
                acc += ov[oi][sp] * e;
            }
        }
        out[(size_t)(kvh * GQ + h) * D + idx % D] = L == 0.0f ? 0.0f : acc / L;
    }
    if (tid == 0) __hip_atomic_store(&counters[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Last-arrival merge for the MFMA kernel, without an L2 write-back: every workgroup
// writes its partial record with agent-scope atomic stores (written through to the
// device coherence point), waits for them, then counts its arrival; the workgroup that
// arrives last reads all records with agent-scope atomic loads and merges them.  The
// counter goes back to zero for the next launch.
template <int D, int GQ>
__device__ __forceinline__ void fa_merge_last(const float *part, float *out, unsigned *counter, int kvh, int n_splits,
                                              int tid) {
    constexpr int PS = part_stride<D>();
    __shared__ int s_last;
    __shared__ float s_cm[GQ][kFusedMaxSplits];
    __shared__ float s_cl[GQ][kFusedMaxSplits];
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // this workgroup's record stores are complete
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (unsigned)(n_splits - 1);
    }
    __syncthreads();
    if (!s_last) return;
    if (tid < GQ * n_splits) {
        const int h = tid / n_splits, sp = tid % n_splits;
        const float *rec = part + ((size_t)(kvh * GQ + h) * n_splits + sp) * PS;
        s_cm[h][sp] = ld_coherent(rec + D);
        s_cl[h][sp] = ld_coherent(rec + D + 1);
    }
    __syncthreads();
    constexpr int OPT = (GQ * D + 255) / 256;
    float ov[OPT][kFusedMaxSplits];
#pragma unroll
    for (int oi = 0; oi < OPT; oi++) {
        const int idx = min(tid + oi * 256, GQ * D - 1);
        const float *ph = part + (size_t)(kvh * GQ + idx / D) * n_splits * PS + idx % D;
#pragma unroll
        for (int sp = 0; sp < kFusedMaxSplits; sp++) ov[oi][sp] = ld_coherent(ph + (size_t)min(sp, n_splits - 1) * PS);
    }
#pragma unroll
    for (int oi = 0; oi < OPT; oi++) {
        const int idx = tid + oi * 256;
        if (idx >= GQ * D) break;
        const int h = idx / D;
        float M = -INFINITY;
        for (int sp = 0; sp < n_splits; sp++) M = fmaxf(M, s_cm[h][sp]);
        float L = 0.0f, acc = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int sp = 0; sp < kFusedMaxSplits; sp++) {
                const float ms = sp < n_splits ? s_cm[h][sp] : -INFINITY;
                const float e = ms == -INFINITY ? 0.0f : fexp2(ms - M);
                L += (sp < n_splits ? s_cl[h][sp] : 0.0f) * e;
                acc += ov[oi][sp] * e;
            }
        }
        out[(size_t)(kvh * GQ + h) * D + idx % D] = L == 0.0f ? 0.0f : acc / L;
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- MFMA flash-decoding
//
// One workgroup per (split, kv head); each of its 4 waves walks its own run of
// 16-position blocks with v_mfma_f32_16x16x16_f16:
//   S^T[16 pos x 16 heads] = K[16 pos x D] . Q^T      (A = K rows, B = q, fp16 like ggml)
//   O[16 heads x 16 dims] += P^T[heads x pos] . V      (8 tiles at D = 128)
// The C layout of the score MFMA (lane (g, c): positions 4g..4g+3 of head c) is the A
// layout P^T needs, so probabilities go from the softmax straight into the PV MFMA.
// The k index of both products is permuted so that every load instruction reads
// contiguous bytes: lane (g, c) reads K row c in 16-byte chunks at dims 32i + 8g .. +7
// (the 4 g-lanes of a row cover 64 contiguous bytes per instruction) and V rows
// 4g..4g+3 at dims [D/16*c, D/16*(c+1)); output tile t column c is dim D/16*c + t.
// P is split into fp16 hi + lo parts (two MFMAs) so the PV product keeps fp32-level
// accuracy.  Online softmax per head in log2 units; the waves merge through LDS.
template <int D, int GQ, bool MASK, int NBW, int NW = 4>
__global__ __launch_bounds__(64 * NW) void k_fa_mfma(const float *__restrict__ q, const uint8_t *__restrict__ kc,
                                                 const uint8_t *__restrict__ vc, const uint16_t *__restrict__ mask,
                                                 const int32_t *__restrict__ kv_len_p, int n_kv, size_t k_nb1,
                                                 size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, int chunk,
                                                 int n_splits, float *__restrict__ part, float *__restrict__ out,
                                                 unsigned *__restrict__ counters, const FaSeq sq) {
    const int seq = blockIdx.z;
    fa_mfma_tile<D, GQ, MASK, NBW, NW>(q, kc, vc, mask, kv_len_p, n_kv, k_nb1, k_nb2, v_nb1, v_nb2, scale, chunk,
                                       n_splits, part, out, counters != nullptr, sq, blockIdx.x, blockIdx.y, seq,
                                       gridDim.y);
    if constexpr (NW == 4) {
        if (n_splits > 1 && counters)
            fa_merge_last<D, GQ>(part + (size_t)seq * gridDim.y * GQ * n_splits * part_stride<D>(),
                                 out + (size_t)seq * sq.out, counters + (size_t)seq * gridDim.y + blockIdx.y,
                                 blockIdx.y, n_splits, threadIdx.x);
    }
}

// Parallel log-sum-exp combine: grid (q head, D/32 dim slices, sequence), 256 threads =
// 32 dims x 8 split groups.  A thread merges splits g, g+8, ... of its group itself
// (online: running maximum, rescaled sums), loading every split's m, l and output value
// of an 8U-split chunk at once, so a chunk costs one round trip (U = 16 above 64 splits,
// U = 32 above 128: up to 256 splits, 128 positions each at 32K, take one round trip,
// not two in a dependent loop; at most 64 splits keep U = 8 and its merge order); the 8 groups then merge
// through LDS.  w_s = 2^(m_s - M), 0 for a split with no position; out = sum w_s o_s /
// sum w_s l_s, 0 when no split has a position.
//
// XP: the result goes out as the fp16 activation of a several-row W4A16 projection
// (rounded RNE, as ggml converts src1), permuted within each 32-element block into the
// nibble order of a weight dword: xp[seq][block][g][8] = x[4g], x[4g+2], x[4g+1], x[4g+3],
// x[16+4g], x[18+4g], x[17+4g], x[19+4g] (out_seq is then the blocks per row).  The 32
// dims of a workgroup are one whole block.
template <int D, bool XP, int U>
__global__ __launch_bounds__(256) void k_fa_combine(const float *__restrict__ part, void *__restrict__ out_v,
                                                    int n_splits, size_t out_seq) {
    constexpr int PS = part_stride<D>();
    part += (size_t)blockIdx.z * gridDim.x * n_splits * PS;
    float *out = (float *)out_v + (XP ? 0 : (size_t)blockIdx.z * out_seq);
    __shared__ float s_m[8][32], s_l[8][32], s_a[8][32];
    const int h = blockIdx.x;
    const int d0 = blockIdx.y * 32;
    const int tid = threadIdx.x;
    const int dd = tid % 32, sg = tid / 32;
    const float *ph = part + (size_t)h * n_splits * PS;
    float M = -INFINITY, L = 0.0f, A = 0.0f;
    for (int base = 0; base < n_splits; base += 8 * U) {
        float mv[U], lv[U], ov[U];
#pragma unroll
        for (int u = 0; u < U; u++) {  // clamped, branch-free: all loads of the chunk in flight
            const int sp = base + sg + 8 * u;
            const float *rec = ph + (size_t)min(sp, n_splits - 1) * PS;
            mv[u] = sp < n_splits ? rec[D] : -INFINITY;
            lv[u] = rec[D + 1];
            ov[u] = rec[d0 + dd];
        }
        float cm = M;
#pragma unroll
        for (int u = 0; u < U; u++) cm = fmaxf(cm, mv[u]);
        if (cm == -INFINITY) continue;
        const float r = M == -INFINITY ? 0.0f : fexp2(M - cm);
        L *= r;
        A *= r;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float w = mv[u] == -INFINITY ? 0.0f : fexp2(mv[u] - cm);
            L = fmaf(lv[u], w, L);
            A = fmaf(ov[u], w, A);
        }
        M = cm;
    }
    s_m[sg][dd] = M;
    s_l[sg][dd] = L;
    s_a[sg][dd] = A;
    __syncthreads();
    if (tid < 32) {
        float mm = -INFINITY;
#pragma unroll
        for (int g = 0; g < 8; g++) mm = fmaxf(mm, s_m[g][tid]);
        float ll = 0.0f, aa = 0.0f;
        if (mm != -INFINITY) {
#pragma unroll
            for (int g = 0; g < 8; g++) {
                const float w = s_m[g][tid] == -INFINITY ? 0.0f : fexp2(s_m[g][tid] - mm);
                ll = fmaf(s_l[g][tid], w, ll);
                aa = fmaf(s_a[g][tid], w, aa);
            }
        }
        const float r = ll == 0.0f ? 0.0f : aa / ll;
        if constexpr (XP) {
            const int g = (tid & 15) >> 2, q = tid & 3;
            const int j = (tid >> 4) * 4 + (q == 1 ? 2 : q == 2 ? 1 : q);
            const size_t blk = ((size_t)h * D + d0) / 32;
            ((uint16_t *)out_v)[(((size_t)blockIdx.z * out_seq + blk) * 4 + g) * 8 + j] = f2h(r);
        } else {
            out[(size_t)h * D + d0 + tid] = r;
        }
    }
}

// The last-workgroup combine needs an agent-scope release/acquire (an L2
// write-back and invalidate on this cache hierarchy) in every workgroup, so it
// is opt-in (MI_FA_FUSED_COMBINE=1); by default a second, parallel kernel combines.
inline bool fused_combine_enabled() {
    static const bool on = [] {
        const char *e = getenv("MI_FA_FUSED_COMBINE");
        return e && e[0] == '1';
    }();
    return on;
}

// MI_FA_MERGE=1: the MFMA kernel merges its splits itself (last arrival) when they fit.
// Off by default: the serial tail of the last workgroup (arrival atomic, then the
// partials' loads) measured slower than the separate combine launch (Qwen2.5-1.5B shape,
// 512 positions: 951 vs 995 tokens/s).
inline bool mfma_merge_enabled() {
    static const bool on = [] {
        const char *e = getenv("MI_FA_MERGE");
        return e && e[0] == '1';
    }();
    return on;
}

struct FaArgs {
    const float *q;
    const void *k, *v;
    const uint16_t *mask;
    const int32_t *kv_len;
    int64_t n_kv, n_kv_heads, n_seq;
    size_t k_nb1, k_nb2, v_nb1, v_nb2;
    float scale;
    float *out, *part;
    unsigned *counters;
    FaSeq sq;
    bool partials_only;  // write every split's (o, m, l) record, no combine, out unused
    uint16_t *xp;        // non-null: the combine writes the permuted fp16 activation here, out unused
    int xp_nb;           // its 32-element blocks per sequence
};

template <int D, int GQ, bool MASK>
int launch_split_m(hipStream_t st, const FaArgs &a, const FaPlan &p) {
    const dim3 grid((unsigned)p.n_splits, (unsigned)a.n_kv_heads, (unsigned)a.n_seq);
    const uint8_t *kb = (const uint8_t *)a.k, *vb = (const uint8_t *)a.v;
    float *const out = a.partials_only || a.xp ? nullptr : a.out;
    if (p.mfma) {
        const bool merged = !a.partials_only && !a.xp && p.n_splits <= kFusedMaxSplits && a.counters &&
                            mfma_merge_enabled();
#define MI_FA_NBW(NB)                                                                                          \
    hipLaunchKernelGGL((k_fa_mfma<D, GQ, MASK, NB>), grid, dim3(256), 0, st, a.q, kb, vb, a.mask, a.kv_len,      \
                       (int)a.n_kv, a.k_nb1, a.k_nb2, a.v_nb1, a.v_nb2, a.scale, p.chunk, p.n_splits, a.part, out,   \
                       merged ? a.counters : nullptr, a.sq)
        switch (p.nbw) {
            case 1: MI_FA_NBW(1); break;
            case 2: MI_FA_NBW(2); break;
            case 4: MI_FA_NBW(4); break;
            case 8: MI_FA_NBW(8); break;
            case 16: MI_FA_NBW(16); break;
            default: MI_FA_NBW(32); break;
        }
#undef MI_FA_NBW
        MI_CHECK_LAUNCH("k_fa_mfma");
        if (merged) return MI_OK;
    } else {
        const bool fused = !a.partials_only && !a.xp && p.n_splits <= kFusedMaxSplits && fused_combine_enabled();
#define MI_FA_KT(KT)                                                                                           \
    hipLaunchKernelGGL((k_fa_split<D, GQ, MASK, KT>), grid, dim3(256), 0, st, a.q, kb, vb, a.mask, a.kv_len,     \
                       (int)a.n_kv, a.k_nb1, a.k_nb2, a.v_nb1, a.v_nb2, a.scale, p.chunk, p.n_splits, a.part, out,   \
                       fused ? a.counters : nullptr, a.sq)
        switch (p.kt) {
            case 1: MI_FA_KT(1); break;
            case 2: MI_FA_KT(2); break;
            case 4: MI_FA_KT(4); break;
            default: MI_FA_KT(8); break;
        }
#undef MI_FA_KT
        MI_CHECK_LAUNCH("k_fa_split");
        if (fused) return MI_OK;
    }
    if ((p.n_splits > 1 || a.xp) && !a.partials_only) {
        const dim3 cg((unsigned)(a.n_kv_heads * GQ), D / 32, (unsigned)a.n_seq);
        const bool wide = p.n_splits > 64;
        if (!a.xp && p.n_splits > 128)  // one round trip for up to 256 splits
            hipLaunchKernelGGL((k_fa_combine<D, false, 32>), cg, dim3(256), 0, st, a.part, (void *)a.out,
                               p.n_splits, a.sq.out);
        else if (a.xp && wide)
            hipLaunchKernelGGL((k_fa_combine<D, true, 16>), cg, dim3(256), 0, st, a.part, (void *)a.xp, p.n_splits,
                               (size_t)a.xp_nb);
        else if (a.xp)
            hipLaunchKernelGGL((k_fa_combine<D, true, 8>), cg, dim3(256), 0, st, a.part, (void *)a.xp, p.n_splits,
                               (size_t)a.xp_nb);
        else if (wide)
            hipLaunchKernelGGL((k_fa_combine<D, false, 16>), cg, dim3(256), 0, st, a.part, (void *)a.out,
                               p.n_splits, a.sq.out);
        else
            hipLaunchKernelGGL((k_fa_combine<D, false, 8>), cg, dim3(256), 0, st, a.part, (void *)a.out, p.n_splits,
                               a.sq.out);
        MI_CHECK_LAUNCH("k_fa_combine");
    }
    return MI_OK;
}

template <int D, int GQ>
int launch_split(hipStream_t st, const FaArgs &a, const FaPlan &p) {
    if (a.mask) return launch_split_m<D, GQ, true>(st, a, p);
    return launch_split_m<D, GQ, false>(st, a, p);
}

template <int D>
int launch_d(hipStream_t st, int gq, const FaArgs &a, const FaPlan &p) {
#define MI_FA_CASE(G) \
    case G: return launch_split<D, G>(st, a, p);
    switch (gq) {
        MI_FA_CASE(1)
        MI_FA_CASE(2)
        MI_FA_CASE(3)
        MI_FA_CASE(4)
        MI_FA_CASE(5)
        MI_FA_CASE(6)
        MI_FA_CASE(7)
        MI_FA_CASE(8)
        default: set_error("fa_decode: GQA group size %d not in 1..8", gq); return MI_ERR_UNSUPPORTED;
    }
#undef MI_FA_CASE
}

// kv_lengths: one workgroup per mask row
__global__ __launch_bounds__(256) void k_kv_lengths(const void *__restrict__ mask, int is_f16, int64_t n_kv,
                                                    int32_t *__restrict__ out) {
    const int64_t r = blockIdx.x;
    int64_t last = -1;
    for (int64_t i = threadIdx.x; i < n_kv; i += 256) {
        const float v = is_f16 ? h2f(((const uint16_t *)mask)[r * n_kv + i]) : ((const float *)mask)[r * n_kv + i];
        if (isfinite(v)) last = i;
    }
    __shared__ int64_t s_last[256];
    s_last[threadIdx.x] = last;
    __syncthreads();
    for (int s = 128; s > 0; s /= 2) {
        if ((int)threadIdx.x < s) s_last[threadIdx.x] = max(s_last[threadIdx.x], s_last[threadIdx.x + s]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int64_t len = s_last[0] + 1;
        out[r] = (int32_t)(len > 1 ? len : 1);
    }
}

}  // namespace

// Split partials of mi_fa_decode_noalloc: the workspace of callers that cannot allocate,
// one copy per device (held until the process ends).  In host code this name is only a
// stand-in for the symbol: kernels get the device address hipGetSymbolAddress returns.
constexpr size_t kFaNoAllocScratchBytes = 4u << 20;
static __device__ __align__(256) unsigned char scratch[kFaNoAllocScratchBytes];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mtx;
void *g_scratch_ptr[kScratchDevices] = {};

// the device address of the current device's scratch array, looked up once per device
int fa_scratch_current_device(void **ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        mi::set_error("fa_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
        return (int)e;
    }
    MI_CHECK_ARG(dev >= 0 && dev < kScratchDevices, "fa_decode_noalloc: device %d beyond %d", dev, kScratchDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mtx);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            mi::set_error("fa_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                          hipGetErrorString(e));
            return e != hipSuccess ? (int)e : MI_ERR_NODEVICE;
        }
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return MI_OK;
}

}  // namespace

extern "C" {


size_t mi_fa_decode_batch_workspace_size(int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                                         int64_t n_seq) {
    if (n_kv <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || d <= 0 || n_seq <= 0) return 0;
    const FaPlan p = fa_plan(n_kv, n_kv_heads, d, n_q_heads / n_kv_heads, n_seq);
    return fa_part_bytes(n_q_heads * n_seq, p.n_splits, d) +
           mi::align_up((size_t)(n_kv_heads * n_seq) * sizeof(unsigned), 256);
}

size_t mi_fa_decode_workspace_size(int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d) {
    return mi_fa_decode_batch_workspace_size(n_kv, n_q_heads, n_kv_heads, d, 1);
}

static int fa_decode_run(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                         const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                         size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, float *out,
                         int64_t n_seq, size_t q_seq, size_t k_seq, size_t v_seq, size_t mask_seq, size_t out_seq,
                         void *ws, size_t ws_bytes, bool partials_only, uint16_t *xp = nullptr,
                         bool use_counters = true, size_t kvl_seq = 1) {
    MI_CHECK_ARG(q && k && v && (out || partials_only || xp), "fa_decode: null pointer");
    MI_CHECK_ARG(n_kv > 0 && n_kv < (1ll << 31) && n_q_heads > 0 && n_kv_heads > 0 && n_q_heads % n_kv_heads == 0,
                 "fa_decode: bad heads/length n_kv=%lld nq=%lld nkv=%lld", (long long)n_kv, (long long)n_q_heads,
                 (long long)n_kv_heads);
    MI_CHECK_ARG(n_seq >= 1 && n_seq <= 65535, "fa_decode: n_seq=%lld", (long long)n_seq);
    MI_CHECK_ARG(d == 64 || d == 128, "fa_decode: head dim %lld not supported (64, 128)", (long long)d);
    MI_CHECK_ARG(mi::aligned(k, 16) && mi::aligned(v, 16) && k_nb1 % 16 == 0 && k_nb2 % 16 == 0 && v_nb1 % 16 == 0 &&
                     v_nb2 % 16 == 0 && mi::aligned(q, 16) && mi::aligned(out, 16) && k_seq % 16 == 0 &&
                     v_seq % 16 == 0 && q_seq % 4 == 0 && out_seq % 4 == 0,
                 "fa_decode: K/V base and strides must be 16-byte aligned");
    const FaPlan p = fa_plan(n_kv, n_kv_heads, d, n_q_heads / n_kv_heads, n_seq);
    const size_t need = mi_fa_decode_batch_workspace_size(n_kv, n_q_heads, n_kv_heads, d, n_seq);
    if ((p.n_splits > 1 || partials_only || xp) && (!ws || ws_bytes < need || !mi::aligned(ws, 256))) {
        mi::set_error("fa_decode: workspace %zu < %zu bytes (or not 256-byte aligned)", ws_bytes, need);
        return MI_ERR_WORKSPACE;
    }
    FaArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.mask = mask;
    a.kv_len = kv_len;
    a.n_kv = n_kv;
    a.n_kv_heads = n_kv_heads;
    a.n_seq = n_seq;
    a.k_nb1 = k_nb1;
    a.k_nb2 = k_nb2;
    a.v_nb1 = v_nb1;
    a.v_nb2 = v_nb2;
    a.scale = scale;
    a.out = out;
    a.part = (float *)ws;
    a.counters = ws && use_counters ? (unsigned *)((uint8_t *)ws + fa_part_bytes(n_q_heads * n_seq, p.n_splits, d))
                                    : nullptr;
    a.sq.q = q_seq;
    a.sq.k = k_seq;
    a.sq.v = v_seq;
    a.sq.mask = mask_seq;
    a.sq.out = out_seq;
    a.sq.kvl = kvl_seq;
    a.partials_only = partials_only;
    a.xp = xp;
    a.xp_nb = (int)(n_q_heads * d / 32);
    const int gq = (int)(n_q_heads / n_kv_heads);
    hipStream_t st = (hipStream_t)stream;
    if (d == 128) return launch_d<128>(st, gq, a, p);
    return launch_d<64>(st, gq, a, p);
}

int mi_fa_decode_batch(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                       const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                       size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, float *out,
                       int64_t n_seq, size_t q_seq, size_t k_seq, size_t v_seq, size_t mask_seq, size_t out_seq,
                       void *ws, size_t ws_bytes) {
    return fa_decode_run(stream, q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1, v_nb2,
                         scale, out, n_seq, q_seq, k_seq, v_seq, mask_seq, out_seq, ws, ws_bytes, false);
}

int mi_fa_decode_batch_q4act(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                             const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                             size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, void *xp,
                             int64_t n_seq, size_t q_seq, size_t k_seq, size_t v_seq, size_t mask_seq, void *ws,
                             size_t ws_bytes) {
    MI_CHECK_ARG(xp && mi::aligned(xp, 16), "fa_decode_batch_q4act: xp must be a 16-byte aligned pointer");
    return fa_decode_run(stream, q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1, v_nb2,
                         scale, nullptr, n_seq, q_seq, k_seq, v_seq, mask_seq, 0, ws, ws_bytes, false,
                         (uint16_t *)xp);
}

int mi_fa_decode_rows(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                      const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                      size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, float *out, int64_t n_rows,
                      size_t q_row, size_t mask_row, size_t out_row, void *ws, size_t ws_bytes) {
    MI_CHECK_ARG(n_rows >= 1 && n_rows <= kFaMaxRows, "fa_decode_rows: %lld query rows (1..%d)", (long long)n_rows,
                 kFaMaxRows);
    // every row reads the same cache and length; row r takes mask row r
    return fa_decode_run(stream, q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1, v_nb2,
                         scale, out, n_rows, q_row, 0, 0, mask ? mask_row : 0, out_row, ws, ws_bytes, false, nullptr,
                         true, 0);
}

int64_t mi_fa_decode_num_splits(int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d) {
    if (n_kv <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || d <= 0 || n_q_heads % n_kv_heads) return 0;
    return fa_plan(n_kv, n_kv_heads, d, n_q_heads / n_kv_heads).n_splits;
}

int mi_fa_decode_partials(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                          const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                          size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, void *ws,
                          size_t ws_bytes) {
    return fa_decode_run(stream, q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1, v_nb2,
                         scale, nullptr, 1, 0, 0, 0, 0, 0, ws, ws_bytes, true);
}

int mi_fa_decode(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                 const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                 size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, float *out, void *ws,
                 size_t ws_bytes) {
    return mi_fa_decode_batch(stream, q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1,
                              v_nb2, scale, out, 1, 0, 0, 0, 0, 0, ws, ws_bytes);
}

int mi_kv_lengths(void *stream, const void *mask, int mask_is_f16, int64_t n_kv, int64_t n_rows, int32_t *out) {
    MI_CHECK_ARG(mask && out && n_kv > 0 && n_rows > 0, "kv_lengths: bad arguments");
    hipLaunchKernelGGL(k_kv_lengths, dim3((unsigned)n_rows), dim3(256), 0, (hipStream_t)stream, mask, mask_is_f16,
                       n_kv, out);
    MI_CHECK_LAUNCH("k_kv_lengths");
    return MI_OK;
}

size_t mi_fa_decode_noalloc_max_workspace(void) { return kFaNoAllocScratchBytes; }

int mi_fa_decode_noalloc(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                         const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                         size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, float *out) {
    MI_CHECK_ARG(n_kv > 0 && n_q_heads > 0 && n_kv_heads > 0 && n_q_heads % n_kv_heads == 0,
                 "fa_decode_noalloc: bad heads/length n_kv=%lld nq=%lld nkv=%lld", (long long)n_kv,
                 (long long)n_q_heads, (long long)n_kv_heads);
    const size_t need = mi_fa_decode_workspace_size(n_kv, n_q_heads, n_kv_heads, d);
    if (need > kFaNoAllocScratchBytes) {
        mi::set_error("fa_decode_noalloc: %lld positions x %lld heads need %zu bytes of split partials, more than "
                      "the %zu-byte scratch (use mi_fa_decode with a workspace)",
                      (long long)n_kv, (long long)n_q_heads, need, kFaNoAllocScratchBytes);
        return MI_ERR_WORKSPACE;
    }
    void *ws = nullptr;
    if (int r = fa_scratch_current_device(&ws)) return r;
    // no arrival counters (they would have to start at zero): the split kernel writes every
    // record the combine reads in this call
    return fa_decode_run(stream, q, k, v, mask, kv_len, n_kv, n_q_heads, n_kv_heads, d, k_nb1, k_nb2, v_nb1, v_nb2,
                         scale, out, 1, 0, 0, 0, 0, 0, ws, kFaNoAllocScratchBytes, false, nullptr, false);
}

}  // extern "C"
