// persist.hip -- the decoder layers of one A8W8 (Q8_0) decode token as one persistent
// launch.
//
// The per-node path runs 7 launches per layer; each kernel boundary costs ~2.4 us on
// gfx950 (dispatch, drain, cache write-back) plus the tail of its last workgroups.  Here
// one grid of resident workgroups (one per CU) walks every layer through five phases
// separated by dependency hops instead of kernel boundaries:
//
//   1. q/k/v:  RMSNorm, SmoothQuant, Q8_0 quantization of x, the q/k/v rows, bias, neox
//              RoPE, q written, k and v written into the cache row
//   2. attn:   the MFMA flash-decoding split tiles (one per (split, kv head))
//   3. o:      the splits' log-sum-exp merge (in the combine kernel's exact order), the
//              o rows, + residual x -> x1
//   4. gate/up: RMSNorm(x1), SmoothQuant, quantization, the gate and up rows (each
//              tile pairs 8 gate rows with the same 8 up rows), swiglu(gate, up) and the
//              down projection's SmoothQuant divisor
//   5. down:   Q8_0 quantization of that product (every workgroup, into LDS), the down
//              rows, + residual x1 -> the layer output
//
// Every phase computes what the per-node kernels compute, with the same lane layout,
// block order and reductions, so a token's logits are bit-identical to the per-node
// path's.  A workgroup issues the first weight loads of its next phase before it waits
// on that phase's hop, so the weight stream overlaps the synchronisation.
//
// Hops: only the workgroups that produce a phase's outputs arrive (an agent-scope add
// to one of 8 counters, by workgroup id mod 8, in each of the kReps replicas of the hop's
// counter set, after their outputs are written through with agent-scope stores); only
// the consumers wait (lanes 0..7 of wave 0 poll the 8 counters of the replica of their
// workgroup id mod kReps, so few workgroups poll any one line).  Every produced buffer is distinct per layer and written once per launch,
// so a consumer's plain loads after the hop can only miss to memory or hit lines filled
// after the producers finished.  Every wait is bounded (spin_limit polls): on a timeout
// the workgroup raises the error word, every later wait returns at once, and all
// workgroups still reach the exit.  Launches alternate between two counter sets: each
// workgroup clears its share of the previous launch's set in the first layer, and the
// last one to exit flips the parity word that names the next launch's set (one workgroup
// zeroing 17,920 counter lines at the exit held the launch 23 us).  The host reads the
// error from pinned memory.
#include "q8_0_dev.h"
#include "fattn_dev.h"
#include "persist_plan.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

namespace {

using persist_plan::kCtrStride;
using persist_plan::kHops;
using persist_plan::Layout;
constexpr int kPersistMaxSplits = persist_plan::kMaxSplits;
constexpr int kTraceEvents = 24;  // timestamps per (layer, workgroup); see trace_mark below

struct PArgs {
    const mi_persist_layer *layers;
    int n_layer, n_embd, n_head_kv, hd, n_ff;
    const int32_t *pos;
    const void *kv_idx;
    int kv_idx_i64;
    int64_t n_cache_rows;
    size_t kv_row_bytes;
    int n_kv;
    const int32_t *kv_len;
    const uint16_t *mask;  // F16 [n_kv] KQ mask, or null
    float kq_scale, eps, theta_scale, freq_scale, attn_factor;
    int rounding;
    long spin_limit;
    int stall_hop;
    int fa_chunk, fa_splits;
    Layout lo;
    const float *x_in;    // the first layer's input, or null: then row tok[0] of embd
    const uint16_t *embd;  // F16 token-embedding table, rows embd_ld elements apart
    size_t embd_ld;
    const int32_t *tok;
    float *x_out;         // the last layer's output
    uint64_t *trace;      // phase timestamps [layer][workgroup][kTraceEvents], or null
    float *scratch;
    unsigned *sync;       // hop counters, exit counter, error word (device)
    unsigned *err_host;   // pinned host word, written on error
};

__device__ __forceinline__ unsigned ld_u(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_h(uint16_t *p, uint16_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// All of this workgroup's writes done, then one arrival in each counter replica (threads
// 0 .. kReps-1 of wave 0).
__device__ __forceinline__ void hop_arrive(const PArgs &a, unsigned *ctrs, int layer, int hop) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < persist_plan::kReps)  // one arrival in every replica of the counter set
        __hip_atomic_fetch_add(ctrs + persist_plan::hop_ctr_word(layer, hop, blockIdx.x & 7, threadIdx.x), 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until every producer of the hop arrived, polling the 8 counters of this
// workgroup's replica (bounded; see the file comment).
__device__ __forceinline__ void hop_wait(const PArgs &a, const unsigned *ctrs, int layer, int hop) {
    if (threadIdx.x < 64) {
        const int j = threadIdx.x & 7;
        const unsigned want = persist_plan::hop_want(a.lo, hop, j) + (layer == 0 && hop == a.stall_hop && j == 0);
        const unsigned *ctr = ctrs + persist_plan::hop_ctr_word(layer, hop, j, blockIdx.x % persist_plan::kReps);
        unsigned *err = a.sync + persist_plan::err_word(a.n_layer);
        long spins = 0;
        for (;;) {
            if (__all(ld_u(ctr) >= want)) break;
            bool stop = false;
            if (threadIdx.x == 0) {
                stop = ld_u(err) != 0u;
                if (!stop && ++spins > a.spin_limit) {
                    st_u(err, 1u);
                    if (a.err_host) __hip_atomic_store(a.err_host, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    stop = true;
                }
            }
            if (__any(stop)) break;
            // a short pause between polls: the poll period bounds how late a workgroup sees
            // a completed hop (2 measured ~3% faster decode than 20 on the C4 step)
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
}

// Exit: the last workgroup to arrive flips the parity word (the next launch counts on the
// set this launch cleared) and zeroes the exit counter and the device error word.
__device__ __forceinline__ void persist_exit(const PArgs &a, unsigned par) {
    __shared__ int s_last;
    unsigned *exit_ctr = a.sync + persist_plan::exit_word(a.n_layer);
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(exit_ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last || threadIdx.x != 0) return;
    st_u(a.sync + persist_plan::err_word(a.n_layer), 0u);
    st_u(a.sync + persist_plan::parity_word(a.n_layer), par ^ 1u);
    st_u(exit_ctr, 0u);
}

// xstage_load of a row of fp16 values (the token's embedding row, GET_ROWS folded in: the
// fp16 -> fp32 conversion is exact, so the staged values are GET_ROWS' output)
template <int XN, bool NORM>
__device__ __forceinline__ void xstage_load_h(XStage<XN, NORM> &st, const uint16_t *__restrict__ x,
                                              const float *__restrict__ norm_w, const float *__restrict__ inv_s,
                                              int k4, int tid) {
#pragma unroll
    for (int t = 0; t < XN; t++) {
        const int f = min(tid + t * 256, k4 - 1);
        const uint2 h = *(const uint2 *)(x + (size_t)f * 4);
        st.xv[t] = make_float4(h2f((uint16_t)(h.x & 0xffffu)), h2f((uint16_t)(h.x >> 16)),
                               h2f((uint16_t)(h.y & 0xffffu)), h2f((uint16_t)(h.y >> 16)));
        if constexpr (NORM) st.nv[t] = ((const float4 *)norm_w)[f];
        if (inv_s) st.sv[t] = ((const float4 *)inv_s)[f];
    }
}

// the attention tile's wait on hop 0 (q and the new cache row written), and its stage
// timestamps (events 3, 19, 20, 21)
template <class Mark>
struct FaHop {
    const PArgs &a;
    const unsigned *ctrs;
    int layer;
    Mark &mark_fn;
    __device__ void operator()() const {
        hop_wait(a, ctrs, layer, 0);
        mark_fn(layer, 3);
    }
    __device__ void mark(int k) const { mark_fn(layer, 19 + k); }
};

__device__ __forceinline__ int opaque_int(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// the matrix / row of a tile row of a set of matrices stacked along the rows
struct Mat {
    const uint8_t *qlo, *qhi;
    const uint16_t *d;
};
__device__ __forceinline__ Mat mat_of(const void *packed, int n, int nb) {
    const size_t plane = ((size_t)n * nb * 16 + 255) / 256 * 256;
    Mat m;
    m.qlo = (const uint8_t *)packed;
    m.qhi = m.qlo + plane;
    m.d = (const uint16_t *)(m.qlo + 2 * plane);
    return m;
}

// LDS of one workgroup: the k = n_embd activation stage of the fused GEMVs, the down
// projection's activation (n_ff int8 + n_ff/32 scales), the RoPE tile's 16 results.
template <int NB_E, int NF, int NH, int NGU>
struct PLds {
    int8_t qs[NB_E * 32];
    float d[NB_E];
    double red[4];
    float y[16];
    int8_t fqs[NF];
    float fd[NF / 32];
    // the attention merge's per-(head, split group) weights
    float mw[NH][8][kPersistMaxSplits / 8];  // split weights within a group
    float mg[NH][8], ml[NH][8];              // group maximum and sum
    float mwg[NH][8];                        // group weights
    float mll[NH];                           // the head's total sum
    float gu[NGU][16];                       // gate (slots 0..7) and up (8..15) rows per tile
};

template <int XN, int GE, int UE, int GF, int UF, int D, int GQ, int NBW, int NB_E, int NF, int NGU, int NDN,
          bool MASK>
__global__ __launch_bounds__(256) void k_persist_q8_0(const PArgs a) {
    constexpr int RPB = 256 / GE;     // rows per k = n_embd tile (16)
    constexpr int HALF = RPB / 2;     // RoPE pairs per rotated tile
    constexpr int RPBF = 256 / GF;    // rows per down tile (4)
    constexpr int NBF = NF / 32;      // down blocks
    // NGU / NDN: gate/up and down tiles per workgroup (all prefetched before the hop)
    constexpr int NH = NB_E * 32 / D;  // query heads (o projection input = NH x D)
    __shared__ __align__(16) PLds<NB_E, NF, NH, NGU> L;
    const int tid = threadIdx.x;
    const int wg = blockIdx.x;
    const int nwg = gridDim.x;
    const Layout &lo = a.lo;
    const int E = a.n_embd;
    const int k4 = E / 4;
    const int j = tid % GE;
    const int slot = tid / GE;

    // ---- this workgroup's q/k/v tile (at most one): its rows and RoPE angles, per token
    RopeKV R;
    R.hd = a.hd;
    R.n_q = lo.n_q;
    R.n_k = lo.n_k;
    R.n_v = lo.n_v;
    RopeKVPlace pl;
    const bool has_qkv = persist_plan::is_qkv(lo, wg);
    const int qkv_b = has_qkv ? wg : 0;
    const int qkv_n = lo.n_q + lo.n_k + lo.n_v;
    const int qkv_rc = min(rope_kv_row<RPB>(R, qkv_b, slot, pl), qkv_n - 1);
    const int qkv_mi = qkv_rc < lo.n_q ? 0 : qkv_rc < lo.n_q + lo.n_k ? 1 : 2;
    const int qkv_row = qkv_rc - (qkv_mi == 0 ? 0 : qkv_mi == 1 ? lo.n_q : lo.n_q + lo.n_k);
    float tab_cs = 0.0f, tab_sn = 0.0f;
    if (has_qkv && pl.rope && tid < HALF) {  // the angles of rope_kv_epilogue / k_rope_table
        const int p = pl.chunk * HALF + tid;
        float theta = (float)a.pos[0];
        for (int i = 0; i < p; i++) theta *= a.theta_scale;
        const float th = a.freq_scale * theta;
        tab_cs = cosf(th) * a.attn_factor;
        tab_sn = sinf(th) * a.attn_factor;
    }
    const int64_t ci = a.kv_idx_i64 ? ((const int64_t *)a.kv_idx)[0] : (int64_t)((const int32_t *)a.kv_idx)[0];
    const bool ci_ok = ci >= 0 && ci < a.n_cache_rows;

    const int fa_t = persist_plan::fa_tile(lo, wg);  // attention tile of this workgroup (if < n_fa)
    const int o_t = persist_plan::o_tile(lo, wg);    // o tile (if < n_o_tiles)

    // wall-clock timestamps of one workgroup's phase boundaries (thread 0, when tracing):
    // 0 layer start, 1 q/k/v waited, 2 q/k/v done, 3 attention waited, 4 attention done,
    // 5 o waited, 6 o done, 7 gate/up start, 8 gate/up waited, 9 gate/up done,
    // 10 down start, 11 down waited, 12 down done, 13 down activation staged,
    // 14 o input staged, 15 gate/up input staged, 16 o records requested, 17 o group
    // weights, 18 o head weights, 19 attention scores formed, 20 attention waves merged,
    // 21 attention partials stored; layer 0 only: 22 kernel entry, 23 exit (after the
    // last workgroup's counter reset)
    auto trace_mark = [&](int layer, int ev) {
        if (a.trace && tid == 0) a.trace[((size_t)layer * nwg + wg) * kTraceEvents + ev] = wall_clock64();
    };
    trace_mark(0, 22);
    // the counter set of this launch (the parity word, flipped by the previous launch's
    // exit); the other set, the previous launch's, is cleared in the first layer's phase 4
    // for the next launch (there the parity load has long returned)
    const unsigned par = ld_u(a.sync + persist_plan::parity_word(a.n_layer)) & 1u;
    unsigned *const ctrs = a.sync + persist_plan::set_base(a.n_layer, (int)par);
    // the first layer's input as the token's fp16 embedding row (or null: a.x_in)
    const uint16_t *const erow = a.x_in ? nullptr : a.embd + (size_t)a.tok[0] * a.embd_ld;

    for (int layer = 0; layer < a.n_layer; layer++) {
        // the thread index, opaque to the optimizer in every iteration: the phases' address
        // arithmetic is then recomputed per layer instead of being hoisted out of the loop,
        // where it would stay live (in registers) through every other phase
        const int tid = opaque_int((int)threadIdx.x);
        const int j = tid % GE;
        const int slot = tid / GE;
        const mi_persist_layer &P = a.layers[layer];
        trace_mark(layer, 0);
        float *scr = a.scratch + (size_t)layer * lo.layer_floats;
        float *q_buf = scr + lo.q_off;
        float *part = scr + lo.part_off;
        float *x1 = scr + lo.x1_off;
        float *hbuf = scr + lo.h_off;
        // the residual stream: the caller's input and output at the ends of the stack, the
        // per-layer scratch copies in between (each written once per launch)
        const float *x = layer == 0 ? a.x_in : a.scratch + (size_t)(layer - 1) * lo.layer_floats + lo.xr_off;
        float *x_out = layer == a.n_layer - 1 ? a.x_out : scr + lo.xr_off;
        const int nbE = NB_E;

        // the gate/up weights of this workgroup's phase-4 tiles (tile t: gate rows 8t .. 8t+7
        // in slots 0..7, the same up rows in slots 8..15; tiles wg, wg + nwg, ...), loaded
        // ahead of phase 4's hop: by the o workgroups before their phase 3 (they reach
        // phase 4 just before its hop, and a poll behind in-flight loads would come back
        // late), by the others at the start of phase 4
        constexpr int HR = RPB / 2;  // rows of each matrix per gate/up tile
        const Mat mg = mat_of(P.w_gate, a.n_ff, nbE), mu = mat_of(P.w_up, a.n_ff, nbE);
        const Mat &mm = slot < HR ? mg : mu;
        int4 gwlo[NGU][UE], gwhi[NGU][UE];
        uint32_t gwdw[NGU][UE];
        auto gu_prefetch = [&]() {
#pragma unroll
            for (int i = 0; i < NGU; i++) {
                const int t = wg + i * nwg;
                if (t < lo.n_gu_tiles) {
                    const size_t rbase = (size_t)(t * HR + slot % HR) * nbE;
                    q8_first_pass<GE, UE>(mm.qlo, mm.qhi, mm.d, rbase, nbE, j, gwlo[i], gwhi[i], gwdw[i]);
                }
            }
        };
        const bool o_role = persist_plan::is_o(lo, wg);

        // ================= phase 1: q/k/v + RoPE + KV write
        if (has_qkv) {
            const Mat m = mat_of(qkv_mi == 0 ? P.wq : qkv_mi == 1 ? P.wk : P.wv,
                                 qkv_mi == 0 ? lo.n_q : qkv_mi == 1 ? lo.n_k : lo.n_v, nbE);
            const size_t rbase = (size_t)qkv_row * nbE;
            int4 wlo[UE], whi[UE];
            uint32_t wdw[UE];
            q8_first_pass<GE, UE>(m.qlo, m.qhi, m.d, rbase, nbE, j, wlo, whi, wdw);
            const float *bias = qkv_mi == 0 ? P.bq : qkv_mi == 1 ? P.bk : P.bv;
            const float bvalue = bias ? bias[qkv_row] : 0.0f;
            if (layer > 0) hop_wait(a, ctrs, layer - 1, 4);
            trace_mark(layer, 1);
            XStage<XN, true> st;
            if (layer == 0 && erow)
                xstage_load_h(st, erow, P.attn_norm, P.inv_s_attn, k4, tid);
            else
                xstage_load(st, x, P.attn_norm, P.inv_s_attn, k4, tid);
            const float scale = xstage_scale(st, k4, a.eps, L.red, tid);
            xstage_quant(st, P.inv_s_attn, k4, scale, a.rounding, L.qs, L.d, tid);
            __syncthreads();
            const float s = q8_row_dot<GE, UE>(m.qlo, m.qhi, m.d, rbase, nbE, j, wlo, whi, wdw, L.qs, L.d);
            if (j == 0) L.y[slot] = bias ? s + bvalue : s;
            __syncthreads();
            // rope_kv_epilogue with coherent stores
            if (pl.rope) {
                if (tid < HALF) {
                    const int p = pl.chunk * HALF + tid;
                    const float x0 = L.y[tid], x1v = L.y[tid + HALF];
                    const float y0 = mul_sub_mul_rn(x0, tab_cs, x1v, tab_sn);
                    const float y1 = mul_add_mul_rn(x0, tab_sn, x1v, tab_cs);
                    const int r0 = pl.head * a.hd + p;
                    if (r0 < lo.n_q) {
                        st_f(q_buf + r0, y0);
                        st_f(q_buf + r0 + a.hd / 2, y1);
                    } else if (ci_ok) {
                        uint16_t *kr = (uint16_t *)((uint8_t *)P.k_cache + (size_t)ci * a.kv_row_bytes);
                        st_h(kr + (r0 - lo.n_q), f2h(y0));
                        st_h(kr + (r0 - lo.n_q + a.hd / 2), f2h(y1));
                    }
                }
            } else if (tid < RPB) {
                const int vr = qkv_b * RPB + tid - (lo.n_q + lo.n_k);
                if (vr < lo.n_v && ci_ok)
                    st_h((uint16_t *)((uint8_t *)P.v_cache + (size_t)ci * a.kv_row_bytes) + vr, f2h(L.y[tid]));
            }
            hop_arrive(a, ctrs, layer, 0);
            trace_mark(layer, 2);
        }

        // ================= phase 2: attention split tiles
        if (persist_plan::is_fa(lo, wg)) {
            // the K / V rows of the tile load ahead of the hop, except the row this token
            // writes in phase 1 (loaded after it, so no stale copy of it is cached)
            const FaSeq sq = {0, 0, 0, 0, 0};
            fa_mfma_tile<D, GQ, MASK, NBW, 4>(q_buf, (const uint8_t *)P.k_cache, (const uint8_t *)P.v_cache, a.mask,
                                               a.kv_len, a.n_kv, a.kv_row_bytes, (size_t)a.hd * 2, a.kv_row_bytes,
                                               (size_t)a.hd * 2, a.kq_scale, a.fa_chunk, a.fa_splits, part, nullptr,
                                               true, sq, fa_t % a.fa_splits, fa_t / a.fa_splits, 0, a.n_head_kv,
                                               ci_ok ? (int)ci : -1, FaHop<decltype(trace_mark)>{a, ctrs, layer, trace_mark});
            hop_arrive(a, ctrs, layer, 1);
            trace_mark(layer, 4);
        }

        // ================= phase 3: merge + o + residual
        if (o_role) {
            gu_prefetch();
            const Mat m = mat_of(P.wo, E, nbE);
            const int row = o_t * RPB + slot;
            const size_t rbase = (size_t)row * nbE;
            int4 wlo[UE], whi[UE];
            uint32_t wdw[UE];
            q8_first_pass<GE, UE>(m.qlo, m.qhi, m.d, rbase, nbE, j, wlo, whi, wdw);
            // The attention output (the splits' merge), SmoothQuant and Q8_0 quantization of
            // the o projection's input.  The merge is fa_merge_exact4's arithmetic (that of
            // k_fa_combine<D, *, 8> for at most 16 splits) with the per-(head, split group)
            // weights computed once into LDS instead of in every element's thread: each
            // element still gets the same fmaf chain over the same operands.
            constexpr int UL = kPersistMaxSplits / 8;
            constexpr int PS = part_stride<D>();
            constexpr int NI = (NB_E * 8 + 255) / 256;  // float4 elements per thread
            const int S = a.fa_splits;
            // the SmoothQuant divisors (constants) load ahead of the hop; data of this launch
            // (the residual, the records) only after it, so no stale line is ever cached
            float4 osv[NI];
#pragma unroll
            for (int it = 0; it < NI; it++)
                osv[it] = P.inv_s_o ? ((const float4 *)P.inv_s_o)[min(tid + it * 256, k4 - 1)]
                                    : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            hop_wait(a, ctrs, layer, 1);
            trace_mark(layer, 5);
            const float xres = layer == 0 && erow ? h2f(erow[min(row, E - 1)])
                                                  : x[min(row, E - 1)];  // the residual (the layer input)
            // the records' maxima and sums first (a wave's loads return in order: the merge
            // weights are formed while the partial outputs still arrive), then this thread's
            // partial outputs; slots past the last split (weight 0 in the merge) and elements
            // past the row (whole waves) are not loaded
            const bool mw_thread = tid < NH * 8;  // group g of head h: splits g, g + 8, ...
            float mv[UL], lv[UL];
            {
                const int h = min(tid / 8, NH - 1), g = tid % 8;
                const float *ph = part + (size_t)h * S * PS;
#pragma unroll
                for (int u = 0; u < UL; u++) {
                    const int sp = g + 8 * u;
                    const float *rec = ph + (size_t)min(sp, S - 1) * PS;
                    mv[u] = mw_thread && sp < S ? rec[D] : -INFINITY;
                    lv[u] = mw_thread ? rec[D + 1] : 0.0f;
                }
            }
            float4 ov[NI][8][UL];
#pragma unroll
            for (int it = 0; it < NI; it++) {
                const int fc = min(tid + it * 256, k4 - 1);
                const float *ph = part + (size_t)(fc * 4 / D) * S * PS + (fc * 4) % D;
                const bool in_row = tid + it * 256 < k4;
#pragma unroll
                for (int g = 0; g < 8; g++)
#pragma unroll
                    for (int u = 0; u < UL; u++)
                        ov[it][g][u] = in_row && g + 8 * u < S ? *(const float4 *)(ph + (size_t)(g + 8 * u) * PS)
                                                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            trace_mark(layer, 16);
            if (mw_thread) {
                const int h = tid / 8, g = tid % 8;
                float cm = -INFINITY, sum = 0.0f;
#pragma unroll
                for (int u = 0; u < UL; u++) cm = fmaxf(cm, mv[u]);
#pragma unroll
                for (int u = 0; u < UL; u++) {
                    // an empty group keeps the weights 0: its element sums stay +0
                    const float w = cm == -INFINITY || mv[u] == -INFINITY ? 0.0f : fexp2(mv[u] - cm);
                    if (cm != -INFINITY) sum = fmaf(lv[u], w, sum);
                    L.mw[h][g][u] = w;
                }
                L.mg[h][g] = cm;
                L.ml[h][g] = sum;
            }
            __syncthreads();
            trace_mark(layer, 17);
            if (tid < NH) {
                float mm = -INFINITY, ll = 0.0f;
#pragma unroll
                for (int g = 0; g < 8; g++) mm = fmaxf(mm, L.mg[tid][g]);
#pragma unroll
                for (int g = 0; g < 8; g++) {
                    const float gm = L.mg[tid][g];
                    const float w = mm == -INFINITY || gm == -INFINITY ? 0.0f : fexp2(gm - mm);
                    if (mm != -INFINITY) ll = fmaf(L.ml[tid][g], w, ll);
                    L.mwg[tid][g] = w;
                }
                L.mll[tid] = ll;
            }
            __syncthreads();
            trace_mark(layer, 18);
#pragma unroll
            for (int it = 0; it < NI; it++) {
                const int f = tid + it * 256;  // float4 index; 8 consecutive threads form one 32-block
                if (f < k4) {  // whole waves drop out together, so the 8-lane groups stay whole
                    const int h = f * 4 / D;
                    float4 aa = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                    for (int g = 0; g < 8; g++) {
                        float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                        for (int u = 0; u < UL; u++) {
                            const float w = L.mw[h][g][u];
                            A.x = fmaf(ov[it][g][u].x, w, A.x);
                            A.y = fmaf(ov[it][g][u].y, w, A.y);
                            A.z = fmaf(ov[it][g][u].z, w, A.z);
                            A.w = fmaf(ov[it][g][u].w, w, A.w);
                        }
                        const float wg = L.mwg[h][g];
                        aa.x = fmaf(A.x, wg, aa.x);
                        aa.y = fmaf(A.y, wg, aa.y);
                        aa.z = fmaf(A.z, wg, aa.z);
                        aa.w = fmaf(A.w, wg, aa.w);
                    }
                    const float ll = L.mll[h];
                    float4 v = ll == 0.0f ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                          : make_float4(aa.x / ll, aa.y / ll, aa.z / ll, aa.w / ll);
                    if (P.inv_s_o) {
                        v.x *= osv[it].x;
                        v.y *= osv[it].y;
                        v.z *= osv[it].z;
                        v.w *= osv[it].w;
                    }
                    float d;
                    *(uint32_t *)(L.qs + (size_t)f * 4) = quant4(v.x, v.y, v.z, v.w, a.rounding, d);
                    if ((f & 7) == 0) L.d[f >> 3] = h2f(f2h(d));
                }
            }
            __syncthreads();
            trace_mark(layer, 14);
            const float s = q8_row_dot<GE, UE>(m.qlo, m.qhi, m.d, rbase, nbE, j, wlo, whi, wdw, L.qs, L.d);
            if (j == 0 && row < E) st_f(x1 + row, s + xres);
            hop_arrive(a, ctrs, layer, 2);
            trace_mark(layer, 6);
        }

        // ================= phase 4: FFN norm + gate/up + swiglu
        {
            trace_mark(layer, 7);
            if (layer == 0) {  // this workgroup's share of the other counter set
                unsigned *other = a.sync + persist_plan::set_base(a.n_layer, (int)(par ^ 1u));
                const size_t n = persist_plan::hop_counters(a.n_layer);
                for (size_t i = (size_t)wg * 256 + tid; i < n; i += (size_t)nwg * 256)
                    st_u(other + i * persist_plan::kCtrStride, 0u);
            }
            if (!o_role) gu_prefetch();
            // the down projection's SmoothQuant divisor of this thread's swiglu row
            const int sw_i = tid / HR, sw_r = tid % HR;
            const int sw_t = wg + sw_i * nwg;
            const bool sw_row = tid < NGU * HR && sw_t < lo.n_gu_tiles;
            const float sw_s = sw_row && P.inv_s_down ? P.inv_s_down[sw_t * HR + sw_r] : 1.0f;
            hop_wait(a, ctrs, layer, 2);
            trace_mark(layer, 8);
            XStage<XN, true> st;
            xstage_load(st, x1, P.ffn_norm, P.inv_s_ffn, k4, tid);
            const float scale = xstage_scale(st, k4, a.eps, L.red, tid);
            xstage_quant(st, P.inv_s_ffn, k4, scale, a.rounding, L.qs, L.d, tid);
            __syncthreads();
            trace_mark(layer, 15);
#pragma unroll
            for (int i = 0; i < NGU; i++) {
                const int t = wg + i * nwg;
                if (t < lo.n_gu_tiles) {
                    const size_t rbase = (size_t)(t * HR + slot % HR) * nbE;
                    const float sd = q8_row_dot<GE, UE>(mm.qlo, mm.qhi, mm.d, rbase, nbE, j, gwlo[i], gwhi[i],
                                                        gwdw[i], L.qs, L.d);
                    if (j == 0) L.gu[i][slot] = sd;
                }
            }
            __syncthreads();
            if (sw_row) {  // k_swiglu_quant_q8_0's product (before its quantization)
                const float g = L.gu[sw_i][sw_r], u = L.gu[sw_i][sw_r + HR];
                float v = (g / (1.0f + expf(-g))) * u;
                if (P.inv_s_down) v *= sw_s;
                st_f(hbuf + sw_t * HR + sw_r, v);
            }
            if (persist_plan::is_gu(lo, wg)) hop_arrive(a, ctrs, layer, 3);
            trace_mark(layer, 9);
        }

        // ================= phase 5: quantization (every workgroup) + down + residual
        {
            trace_mark(layer, 10);
            const Mat md = mat_of(P.w_down, E, NBF);
            const int jf = tid % GF;
            // the weights load ahead of the hop, the product after it
            int4 wlo[NDN][UF], whi[NDN][UF];
            uint32_t wdw[NDN][UF];
            auto dn_load = [&]() {
#pragma unroll
                for (int i = 0; i < NDN; i++) {
                    const int t = persist_plan::down_tile(lo, wg, i);
                    if (t >= 0) {
                        const int row = min(t * RPBF + tid / GF, E - 1);
                        const size_t rbase = (size_t)row * NBF;
#pragma unroll
                        for (int u = 0; u < UF; u++) {
                            const int b = min(jf + u * GF, NBF - 1);
                            wlo[i][u] = ld_stream16(md.qlo + (rbase + b) * 16);
                            whi[i][u] = ld_stream16(md.qhi + (rbase + b) * 16);
                            wdw[i][u] = md.d[rbase + b];
                        }
                    }
                }
            };
            dn_load();
            float xres[NDN];  // the residual x1 (complete since hop 2)
#pragma unroll
            for (int i = 0; i < NDN; i++)
                xres[i] = x1[min(max(persist_plan::down_tile(lo, wg, i), 0) * RPBF + tid / GF, E - 1)];
            hop_wait(a, ctrs, layer, 3);
            trace_mark(layer, 11);
            constexpr int NSW = (NBF + 31) / 32;  // passes of 32 blocks
            const int sub = tid % 8;
            float4 hv[NSW];
#pragma unroll
            for (int p = 0; p < NSW; p++)
                hv[p] = *(const float4 *)(hbuf + min(p * 32 + tid / 8, NBF - 1) * 32 + sub * 4);
            // k_swiglu_quant_q8_0's quantization of every 32-block of the product, into LDS
#pragma unroll
            for (int p = 0; p < NSW; p++) {
                const int blk = p * 32 + tid / 8;
                float d;
                const uint32_t qv = quant4(hv[p].x, hv[p].y, hv[p].z, hv[p].w, a.rounding, d);  // whole 8-lane groups
                if (blk < NBF) {
                    *(uint32_t *)(L.fqs + blk * 32 + sub * 4) = qv;
                    if (sub == 0) L.fd[blk] = h2f(f2h(d));
                }
            }
            __syncthreads();
            trace_mark(layer, 13);
            // k_gemv_q8_0_xq<GF, UF, 1>'s row dot (one pass covers the row: UF * GF >= NBF)
#pragma unroll
            for (int i = 0; i < NDN; i++) {
                const int t = persist_plan::down_tile(lo, wg, i);
                if (t >= 0) {
                    const int row = t * RPBF + tid / GF;
                    float acc = 0.0f;
#pragma unroll
                    for (int u = 0; u < UF; u++) {
                        const int b = jf + u * GF;
                        if (b < NBF) {
                            const int4 *xs = (const int4 *)(L.fqs + (size_t)b * 32);
                            const int s = dot_block(wlo[i][u], whi[i][u], xs[0], xs[1]);
                            acc = fmaf((float)s, h2f((uint16_t)wdw[i][u]) * L.fd[b], acc);
                        }
                    }
                    const float s = group_sum<GF>(acc);
                    if (jf == 0 && row < E) st_f(x_out + row, s + xres[i]);
                }
            }
            if (persist_plan::is_down(lo, wg)) hop_arrive(a, ctrs, layer, 4);
            trace_mark(layer, 12);
        }
    }
    persist_exit(a, par);
    trace_mark(0, 23);
}

// ---------------------------------------------------------------- host side

struct PersistCtx {
    int device = 0;
    int n_wg = 0;
    int n_layer = 0, n_embd = 0, n_head = 0, n_head_kv = 0, hd = 0, n_ff = 0;
    mi_persist_layer *layers_dev = nullptr;
    std::vector<mi_persist_layer> layers_host;
    float *scratch = nullptr;
    size_t scratch_floats = 0;
    unsigned *sync = nullptr;
    size_t sync_words = 0;
    unsigned *err_host = nullptr;  // pinned, device-visible
    uint64_t *trace = nullptr;     // phase timestamps of the last launch (when enabled)
};

Layout layout_of(const PersistCtx &c, int fa_splits) {
    return persist_plan::make_layout(c.n_wg, c.n_embd, c.n_head, c.n_head_kv, c.hd, c.n_ff, fa_splits,
                                     part_stride<128>());
}

// the one instantiated shape: Qwen2.5-1.5B-like (n_embd 1536, head_dim 128, GQA 6, n_ff 8960)
// on 256 workgroups (gate/up: 1120 tiles = 5 per workgroup; down: 384 tiles = 2)
constexpr int kNbE = 48, kNF = 8960, kWG = 256;

bool shape_supported(int n_embd, int n_head, int n_head_kv, int hd, int n_ff) {
    return n_embd == kNbE * 32 && hd == 128 && n_head_kv > 0 && n_head % n_head_kv == 0 && n_head / n_head_kv == 6 &&
           n_head * hd == n_embd && n_ff == kNF;
}

}  // namespace

extern "C" {

int mi_persist_create(void **out, int device, int n_layer, int n_embd, int n_head, int n_head_kv, int head_dim,
                      int n_ff) {
    MI_CHECK_ARG(out && n_layer > 0, "persist_create: bad arguments");
    MI_CHECK_ARG(shape_supported(n_embd, n_head, n_head_kv, head_dim, n_ff),
                 "persist_create: shape n_embd=%d heads=%d/%d hd=%d n_ff=%d not instantiated", n_embd, n_head,
                 n_head_kv, head_dim, n_ff);
    *out = nullptr;
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return mi::hip_fail(e, "persist_create: hipSetDevice");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return mi::hip_fail(e, "persist_create: hipGetDeviceProperties");
    PersistCtx *c = new PersistCtx();
    c->device = device;
    c->n_wg = prop.multiProcessorCount;  // one resident workgroup per CU
    if (c->n_wg != kWG) {
        delete c;
        mi::set_error("persist_create: %d CUs; the pipeline is instantiated for %d", prop.multiProcessorCount, kWG);
        return MI_ERR_UNSUPPORTED;
    }
    c->n_layer = n_layer;
    c->n_embd = n_embd;
    c->n_head = n_head;
    c->n_head_kv = n_head_kv;
    c->hd = head_dim;
    c->n_ff = n_ff;
    const Layout lo = layout_of(*c, kPersistMaxSplits);
    c->scratch_floats = lo.layer_floats * n_layer;
    c->sync_words = persist_plan::sync_words(n_layer);
    if ((e = hipMalloc(&c->scratch, c->scratch_floats * sizeof(float))) != hipSuccess ||
        (e = hipMalloc(&c->sync, c->sync_words * sizeof(unsigned))) != hipSuccess ||
        (e = hipMalloc(&c->layers_dev, (size_t)n_layer * sizeof(mi_persist_layer))) != hipSuccess ||
        (e = hipHostMalloc(&c->err_host, 64, hipHostMallocMapped)) != hipSuccess ||
        (e = hipMemset(c->sync, 0, c->sync_words * sizeof(unsigned))) != hipSuccess ||
        (e = hipDeviceSynchronize()) != hipSuccess) {
        mi_persist_destroy(c);
        return mi::hip_fail(e, "persist_create: allocation");
    }
    *c->err_host = 0;
    *out = c;
    return MI_OK;
}

void mi_persist_destroy(void *ctx) {
    PersistCtx *c = (PersistCtx *)ctx;
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->scratch) (void)hipFree(c->scratch);
    if (c->sync) (void)hipFree(c->sync);
    if (c->layers_dev) (void)hipFree(c->layers_dev);
    if (c->err_host) (void)hipHostFree(c->err_host);
    if (c->trace) (void)hipFree(c->trace);
    delete c;
}

int mi_persist_set_layers(void *stream, void *ctx, const mi_persist_layer *layers, int n_layer) {
    PersistCtx *c = (PersistCtx *)ctx;
    MI_CHECK_ARG(c && layers && n_layer == c->n_layer, "persist_set_layers: %d layers, context has %d", n_layer,
                 c ? c->n_layer : 0);
    for (int l = 0; l < n_layer; l++) {
        const mi_persist_layer &L = layers[l];
        MI_CHECK_ARG(L.wq && L.wk && L.wv && L.wo && L.w_gate && L.w_up && L.w_down && L.attn_norm && L.ffn_norm &&
                         L.k_cache && L.v_cache,
                     "persist_set_layers: layer %d has a null tensor", l);
        MI_CHECK_ARG(mi::aligned(L.attn_norm, 16) &&
                         mi::aligned(L.ffn_norm, 16) && (!L.inv_s_attn || mi::aligned(L.inv_s_attn, 16)) &&
                         (!L.inv_s_o || mi::aligned(L.inv_s_o, 16)) && (!L.inv_s_ffn || mi::aligned(L.inv_s_ffn, 16)) &&
                         (!L.inv_s_down || mi::aligned(L.inv_s_down, 16)) && mi::aligned(L.k_cache, 16) &&
                         mi::aligned(L.v_cache, 16),
                     "persist_set_layers: layer %d: vectors must be 16-byte aligned", l);
    }
    if (c->layers_host.size() == (size_t)n_layer &&
        memcmp(c->layers_host.data(), layers, (size_t)n_layer * sizeof(mi_persist_layer)) == 0)
        return MI_OK;  // unchanged: nothing to upload (and nothing to record under stream capture)
    hipError_t e = hipSetDevice(c->device);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
    if (e == hipSuccess)
        e = hipMemcpy(c->layers_dev, layers, (size_t)n_layer * sizeof(mi_persist_layer), hipMemcpyHostToDevice);
    if (e != hipSuccess) return mi::hip_fail(e, "persist_set_layers: upload");
    c->layers_host.assign(layers, layers + n_layer);
    return MI_OK;
}

int mi_persist_decode_q8_0(void *stream, void *ctx, const mi_persist_args *args) {
    PersistCtx *c = (PersistCtx *)ctx;
    MI_CHECK_ARG(c && args && !c->layers_host.empty(), "persist_decode: no context or no layers set");
    MI_CHECK_ARG(args->x_out && mi::aligned(args->x_out, 16) &&
                     (args->x_in ? mi::aligned(args->x_in, 16)
                                 : args->embd && args->tok && mi::aligned(args->embd, 8) && args->embd_ld >= c->n_embd &&
                                       args->embd_ld % 4 == 0),
                 "persist_decode: x_in / x_out must be 16-byte aligned device vectors (or x_in NULL and an "
                 "8-byte aligned F16 embedding table with its row index)");
    MI_CHECK_ARG(args->pos && args->kv_idx && args->kv_row_bytes >= (size_t)c->n_head_kv * c->hd * 2 &&
                     args->kv_row_bytes % 16 == 0 && args->n_kv > 0 && args->n_cache_rows > 0,
                 "persist_decode: bad position / cache arguments");
    const FaPlan p = fa_plan(args->n_kv, c->n_head_kv, c->hd, c->n_head / c->n_head_kv);
    MI_CHECK_ARG(p.mfma && p.nbw == 1 && p.n_splits <= kPersistMaxSplits,
                 "persist_decode: a %d-position view needs %d attention splits (at most %d fit the o prologue)",
                 args->n_kv, p.n_splits, kPersistMaxSplits);
    PArgs a;
    memset(&a, 0, sizeof(a));
    a.layers = c->layers_dev;
    a.n_layer = c->n_layer;
    a.n_embd = c->n_embd;
    a.n_head_kv = c->n_head_kv;
    a.hd = c->hd;
    a.n_ff = c->n_ff;
    a.pos = args->pos;
    a.kv_idx = args->kv_idx;
    a.kv_idx_i64 = args->kv_idx_is_i64;
    a.n_cache_rows = args->n_cache_rows;
    a.kv_row_bytes = args->kv_row_bytes;
    a.n_kv = args->n_kv;
    a.kv_len = args->kv_len;
    a.mask = args->mask;
    a.kq_scale = args->kq_scale;
    a.eps = args->rms_eps;
    // theta_scale on the host with the C library powf, as the CPU rope cache does
    a.theta_scale = powf(args->freq_base, -2.0f / (float)c->hd);
    a.freq_scale = args->freq_scale;
    a.attn_factor = args->attn_factor;
    a.rounding = args->rounding;
    a.spin_limit = args->spin_limit > 0 ? args->spin_limit : (1l << 22);
    a.stall_hop = args->debug_stall_hop >= 0 && args->debug_stall_hop < kHops ? args->debug_stall_hop : -1;
    a.fa_chunk = p.chunk;
    a.fa_splits = p.n_splits;
    a.lo = layout_of(*c, p.n_splits);
    constexpr int NGU = 5, NDN = 2;
    MI_CHECK_ARG(persist_plan::layout_fits(a.lo, NGU, NDN), "persist_decode: %d workgroups do not fit the tiles",
                 c->n_wg);
    a.x_in = args->x_in;
    a.embd = args->x_in ? nullptr : args->embd;
    a.embd_ld = (size_t)args->embd_ld;
    a.tok = args->tok;
    a.x_out = args->x_out;
    a.trace = c->trace;
    a.scratch = c->scratch;
    a.sync = c->sync;
    a.err_host = c->err_host;
    if (a.mask)
        hipLaunchKernelGGL((k_persist_q8_0<2, 16, 3, 64, 5, 128, 6, 1, kNbE, kNF, NGU, NDN, true>),
                           dim3((unsigned)c->n_wg), dim3(256), 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL((k_persist_q8_0<2, 16, 3, 64, 5, 128, 6, 1, kNbE, kNF, NGU, NDN, false>),
                           dim3((unsigned)c->n_wg), dim3(256), 0, (hipStream_t)stream, a);
    MI_CHECK_LAUNCH("k_persist_q8_0");
    return MI_OK;
}

int mi_persist_enable_trace(void *ctx) {
    PersistCtx *c = (PersistCtx *)ctx;
    MI_CHECK_ARG(c, "persist_enable_trace: no context");
    if (c->trace) return MI_OK;
    hipError_t e = hipSetDevice(c->device);
    const size_t n = (size_t)c->n_layer * c->n_wg * kTraceEvents;
    if (e == hipSuccess) e = hipMalloc(&c->trace, n * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMemset(c->trace, 0, n * sizeof(uint64_t));
    if (e != hipSuccess) return mi::hip_fail(e, "persist_enable_trace");
    return MI_OK;
}

int mi_persist_read_trace(void *ctx, uint64_t *dst, size_t n_words, int *n_layer, int *n_wg, int *n_events,
                          double *ticks_per_us) {
    PersistCtx *c = (PersistCtx *)ctx;
    MI_CHECK_ARG(c && c->trace, "persist_read_trace: tracing is not enabled");
    const size_t n = (size_t)c->n_layer * c->n_wg * kTraceEvents;
    if (n_layer) *n_layer = c->n_layer;
    if (n_wg) *n_wg = c->n_wg;
    if (n_events) *n_events = kTraceEvents;
    if (ticks_per_us) {
        int khz = 0;
        (void)hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, c->device);
        *ticks_per_us = khz / 1000.0;
    }
    if (!dst) return MI_OK;
    MI_CHECK_ARG(n_words >= n, "persist_read_trace: %zu words, %zu needed", n_words, n);
    hipError_t e = hipSetDevice(c->device);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(dst, c->trace, n * sizeof(uint64_t), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return mi::hip_fail(e, "persist_read_trace");
    return MI_OK;
}

int mi_persist_supported(int64_t n_kv, int n_embd, int n_head, int n_head_kv, int head_dim, int n_ff) {
    if (!shape_supported(n_embd, n_head, n_head_kv, head_dim, n_ff) || n_kv < 1) return 0;
    const FaPlan p = fa_plan(n_kv, n_head_kv, head_dim, n_head / n_head_kv);
    return p.mfma && p.nbw == 1 && p.n_splits <= kPersistMaxSplits ? 1 : 0;
}

int mi_persist_status(void *ctx) {
    PersistCtx *c = (PersistCtx *)ctx;
    if (!c || !c->err_host) return MI_ERR_ARG;
    const unsigned v = __atomic_load_n(c->err_host, __ATOMIC_ACQUIRE);
    if (v == 0) return MI_OK;
    __atomic_store_n(c->err_host, 0u, __ATOMIC_RELEASE);
    mi::set_error("persist_decode: a workgroup gave up waiting for a dependency (spin limit); that token's "
                  "results are invalid");
    return MI_ERR_UNSUPPORTED;
}

}  // extern "C"
