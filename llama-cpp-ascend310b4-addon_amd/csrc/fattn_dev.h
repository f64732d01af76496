// fattn_dev.h -- device pieces of the single-token GQA flash-decoding shared by the
// per-node launches (fattn.hip) and the persistent layer pipeline (persist.hip): the
// split plan, the MFMA split tile (scores, online softmax, P.V for one (split, kv head)
// of 16-position blocks), coherent record stores, and the log-sum-exp merge of the
// splits in the combine kernel's exact order.
#pragma once

#include "mi_common.h"

#include <math.h>
#include <stdlib.h>

#include <type_traits>

namespace {

using namespace mi;

constexpr int kNW = 4;  // waves per workgroup
constexpr float kLog2e = 1.4426950408889634f;
// lazy softmax rescaling threshold (log2 units): probabilities stay below 2^8 = 256
constexpr float kLazyLog2 = 8.0f;

// 2^x with the hardware v_exp_f32 (arguments here are <= 0; -inf gives 0)
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int D>
constexpr int part_stride() { return D + 4; }  // o[D], m, l, pad -> 16-byte aligned records

struct FaPlan {
    int chunk;     // positions per workgroup
    int n_splits;
    int kt;        // VALU kernel: positions per lane group per tile (all loads of a tile in flight together)
    int nbw;       // MFMA kernel: 16-position blocks per wave
    bool mfma;
};


// One workgroup per (split, kv head), each with 4 waves of lane groups (one KV row
// per lane group: 16 groups per workgroup at D = 128, 32 at D = 64).  A workgroup's
// time is a chain of dependent steps per tile, so short contexts get one short tile
// per workgroup and many workgroups; long contexts aim at ~512 workgroups with 8-deep
// tiles.  With at most kFusedMaxSplits splits the last workgroup of a kv head can
// merge the partials itself (opt-in).  MI_FA_CHUNK=<positions> overrides the chunk.
constexpr int kFusedMaxSplits = 16;
// query rows of one sequence in one launch (a prompt ubatch): the MUL_MAT row limit
constexpr int kFaMaxRows = 8;
constexpr int kMaxSplits = 1024;

inline int fa_chunk_override() {
    static const int v = [] {
        const char *e = getenv("MI_FA_CHUNK");
        return e ? atoi(e) : 0;
    }();
    return v;
}

inline bool fa_valu_forced() {
    static const bool v = [] {
        const char *e = getenv("MI_FA_VALU");
        return e && e[0] == '1';
    }();
    return v;
}

inline FaPlan fa_plan(int64_t n_kv, int64_t n_kv_heads, int64_t d, int64_t gq, int64_t n_seq = 1) {
    const int64_t ng = 4 * 64 / (d / 8);  // lane groups per workgroup
    const int64_t target_wg = 512;        // over all sequences of the launch
    int64_t per = (n_kv * n_kv_heads * n_seq + target_wg - 1) / target_wg;
    if (fa_chunk_override() > 0) per = fa_chunk_override();
    FaPlan p;
    p.mfma = !fa_valu_forced() && gq <= 16;
    if (p.mfma) {
        // 4 waves x nbw blocks of 16 positions per workgroup
        p.kt = 1;
        // at most 8 blocks per wave (fully unrolled, 3 waves per SIMD); longer runs (a
        // runtime loop at 2 waves per SIMD, measured slower) only when the split count
        // would exceed kMaxSplits (over 512K positions)
        p.nbw = per <= 64 ? 1 : per <= 128 ? 2 : per <= 256 ? 4 : 8;
        int64_t chunk = 64 * p.nbw;
        while ((n_kv + chunk - 1) / chunk > kMaxSplits) chunk *= 2;
        if (chunk <= 64 * 32) {  // a run of at most 32 blocks per wave (the kernel's instances)
            p.chunk = (int)chunk;
            p.nbw = (int)(chunk / 64);
            p.n_splits = (int)((n_kv + chunk - 1) / chunk);
            return p;
        }
        p.mfma = false;  // over 2M positions: the VALU kernel, whose chunk is a runtime loop
    }
    p.nbw = 0;
    if (per <= ng) p.kt = 1;
    else if (per <= 2 * ng) p.kt = 2;
    else if (per <= 4 * ng) p.kt = 4;
    else p.kt = 8;
    int64_t chunk = (per + ng * p.kt - 1) / (ng * p.kt) * (ng * p.kt);
    while ((n_kv + chunk - 1) / chunk > kMaxSplits) chunk *= 2;
    p.chunk = (int)chunk;
    p.n_splits = (int)((n_kv + chunk - 1) / chunk);
    return p;
}

inline size_t fa_part_bytes(int64_t n_q_heads, int64_t n_splits, int64_t d) {
    return align_up((size_t)n_q_heads * n_splits * (d + 4) * sizeof(float), 256);
}

// Sequences (grid z) are independent problems: per-sequence strides of q / out
// (floats), K / V (bytes) and mask (elements); kv_len and the partials are indexed by
// sequence.
// per-launch-row element strides (blockIdx.z): a row is a sequence of a batch, or one of
// the query rows of a single sequence's ubatch (then k = v = kvl = 0: one cache, one
// length, and its own mask row)
struct FaSeq {
    size_t q, k, v, mask, out;
    size_t kvl = 1;
};

__device__ __forceinline__ void st_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

template <int N>
struct U32s {
    uint32_t w[N];
};

template <int NB>  // bytes per load group: 64 / 32 (K) or 16 / 8 (V)
__device__ __forceinline__ void ld_bytes(uint32_t *dst, const uint8_t *src) {
    if constexpr (NB % 16 == 0) {
#pragma unroll
        for (int i = 0; i < NB / 16; i++) {
            const int4 v = *(const int4 *)(src + 16 * i);
            dst[4 * i] = (uint32_t)v.x; dst[4 * i + 1] = (uint32_t)v.y;
            dst[4 * i + 2] = (uint32_t)v.z; dst[4 * i + 3] = (uint32_t)v.w;
        }
    } else {
        const int2 v = *(const int2 *)src;
        dst[0] = (uint32_t)v.x; dst[1] = (uint32_t)v.y;
    }
}

// K row slice of lane group g: NC 16-byte chunks at byte offsets 64i + 16g, so that one
// load instruction covers a contiguous 64-byte piece of each of its 16 rows
template <int NC>
__device__ __forceinline__ void ld_k_chunks(uint32_t *dst, const uint8_t *src) {
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int4 v = *(const int4 *)(src + 64 * i);
        dst[4 * i] = (uint32_t)v.x; dst[4 * i + 1] = (uint32_t)v.y;
        dst[4 * i + 2] = (uint32_t)v.z; dst[4 * i + 3] = (uint32_t)v.w;
    }
}

__device__ __forceinline__ half4_t h4(uint32_t a, uint32_t b) {
    uint32_t t[2] = {a, b};
    return __builtin_bit_cast(half4_t, t);
}

struct FaNoWait {
    __device__ void operator()() const {}
    __device__ void mark(int) const {}
};

// One (split, kv head, sequence) tile of the MFMA flash-decoding kernel: a workgroup of
// NW waves (64*NW threads).  Partials go to part (coherent: written through with
// agent-scope stores, for readers on other XCDs within the same launch), or straight to
// out when there is one split.
//
// The first K / V loads are issued before q is read.  A caller whose q and newest cache
// row are produced in the same launch passes wait (called by every thread between the
// first K / V loads and the q loads) and late_row, the row written behind that wait:
// lanes whose first-block row is late_row load it after wait, so no line of it is cached
// before it was written.  (NBW == 1 only; the plain kernel passes FaNoWait and -1.)
// wait.mark(k) is called at the tile's stage boundaries (k = 0: first block's scores
// formed, 1: output merged across waves, 2: partials stored), for phase timestamps.
template <int D, int GQ, bool MASK, int NBW, int NW = 4, class Wait = FaNoWait>
__device__ __forceinline__ void fa_mfma_tile(const float *__restrict__ q, const uint8_t *__restrict__ kc,
                                             const uint8_t *__restrict__ vc, const uint16_t *__restrict__ mask,
                                             const int32_t *__restrict__ kv_len_p, int n_kv, size_t k_nb1,
                                             size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, int chunk,
                                             int n_splits, float *__restrict__ part, float *__restrict__ out,
                                             bool coherent, const FaSeq &sq, int split, int kvh, int seq,
                                             int n_kvh, int late_row = -1, Wait wait = Wait{}) {
    constexpr bool kLate = !std::is_same<Wait, FaNoWait>::value;
    static_assert(!kLate || NBW == 1, "a wait inside the tile needs NBW == 1");
    {
        q += (size_t)seq * sq.q;
        kc += (size_t)seq * sq.k;
        vc += (size_t)seq * sq.v;
        if (MASK) mask += (size_t)seq * sq.mask;
        if (kv_len_p) kv_len_p += (size_t)seq * sq.kvl;
        out += (size_t)seq * sq.out;
        part += (size_t)seq * n_kvh * GQ * n_splits * part_stride<D>();
    }
    constexpr int KS = D / 16;    // k-steps of the score product
    constexpr int KW = D / 8;     // K dwords per lane per block (D/4 halves)
    constexpr int VT = D / 16;    // output tiles = V halves per lane per row
    constexpr int VW = D / 32;    // V dwords per lane per row
    constexpr int PS = part_stride<D>();
    __shared__ float s_m[NW][16];
    __shared__ float s_l[NW][16];
    __shared__ __align__(16) float s_o[NW][GQ][D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int c = lane & 15;

    const int kl = kv_len_p ? *kv_len_p : n_kv;
    const int eff = (kl > 0 && kl < n_kv) ? kl : n_kv;
    const int start = split * chunk;
    const int end_phys = min(start + chunk, n_kv);
    const int end_eff = min(end_phys, eff);
    const int wstart = start + wave * NBW * 16;

    // q fragment (B operand): lane (g, c) holds head c, dims 32*(s/2) + 8g + 4*(s%2) .. +3
    // for step s, the dims its K chunks hold
    half4_t qf[KS];
    auto load_q = [&]() {
        const float *qh = q + (size_t)(kvh * GQ + min(c, GQ - 1)) * D + 8 * g;
#pragma unroll
        for (int s2 = 0; s2 < KS; s2++) {
            const float4 v = *(const float4 *)(qh + 32 * (s2 / 2) + 4 * (s2 % 2));
            const uint32_t a = (uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16);
            const uint32_t b = (uint32_t)f2h(v.z) | ((uint32_t)f2h(v.w) << 16);
            qf[s2] = c < GQ ? h4(a, b) : h4(0u, 0u);
        }
    };
    if constexpr (!kLate) load_q();

    const uint8_t *kb = kc + (size_t)kvh * k_nb2 + (size_t)16 * g;
    const uint8_t *vb = vc + (size_t)kvh * v_nb2 + (size_t)(D / 8) * c;
    const int last = end_phys - 1;

    float m = -INFINITY, l = 0.0f;
    float4_t o[VT];
#pragma unroll
    for (int t = 0; t < VT; t++) o[t] = float4_t{0.f, 0.f, 0.f, 0.f};

    U32s<KW> kr[2];
    U32s<VW> vr[2][4];
    auto issue = [&](int blk, int buf) {
        const int p0 = wstart + blk * 16;
        const int kro = min(p0 + c, last);
        if (!kLate || kro != late_row) ld_k_chunks<D / 32>(kr[buf].w, kb + (size_t)kro * k_nb1);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int vro = min(p0 + 4 * g + r, last);
            if (!kLate || vro != late_row) ld_bytes<D / 8>(vr[buf][r].w, vb + (size_t)vro * v_nb1);
        }
    };
    // one 16-position block: scores, online softmax, P.V (buffer buf holds its K / V)
    auto step = [&](int blk, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const int p0 = wstart + blk * 16;
        float mk[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (MASK) {
#pragma unroll
            for (int r = 0; r < 4; r++) mk[r] = h2f(mask[min(p0 + 4 * g + r, last)]);
        }
        float4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < KS; s2++)
            sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(h4(kr[buf].w[2 * s2], kr[buf].w[2 * s2 + 1]), qf[s2], sacc,
                                                         0, 0, 0);
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const bool ok = c < GQ && p0 + 4 * g + r < end_eff;
            // ggml order: s = (q.k)*scale; s += mask; kept in log2 units for v_exp_f32
            const float v = mul_add_rn(sacc[r], scale, mk[r]) * kLog2e;
            sc[r] = ok ? v : -INFINITY;
        }
        float bm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        // Lazy rescaling: the reference maximum m moves only when a score exceeds it by more
        // than kLazyLog2 (log2 units), so most blocks skip the output rescale (a read,
        // multiply and write-back of each MFMA accumulator).  p = 2^(s - m) then stays below
        // 2^kLazyLog2; l and o share the reference m, so o / l and the records' (m, l, o)
        // mean what they meant with an exact running maximum.
        const bool grow = bm > m + kLazyLog2;  // m = -inf: the first finite score
        if (__any(grow)) {
            const float mn = grow ? bm : m;
            const float alpha = mn == -INFINITY ? 1.0f : fexp2(m - mn);
            l *= alpha;
            m = mn;
            // rescale the output rows: row 4g+r belongs to head 4g+r, whose alpha sits in lane 4g+r
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float a = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
                for (int t = 0; t < VT; t++) o[t][r] *= a;
            }
        }
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; r++) p[r] = m == -INFINITY ? 0.0f : fexp2(sc[r] - m);
        l += (p[0] + p[1]) + (p[2] + p[3]);
        half_t ph[4], pl[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            ph[r] = (half_t)p[r];
            pl[r] = (half_t)(p[r] - (float)ph[r]);
        }
        const half4_t ahi = {ph[0], ph[1], ph[2], ph[3]};
        const half4_t alo = {pl[0], pl[1], pl[2], pl[3]};
#pragma unroll
        for (int t = 0; t < VT; t++) {
            // column c of tile t is dim D/16*c + t: half t of each of the lane's 4 V rows
            const int wd = t >> 1;
            uint32_t a0, a1;
            if (t & 1) {
                a0 = (vr[buf][0].w[wd] >> 16) | (vr[buf][1].w[wd] & 0xffff0000u);
                a1 = (vr[buf][2].w[wd] >> 16) | (vr[buf][3].w[wd] & 0xffff0000u);
            } else {
                a0 = (vr[buf][0].w[wd] & 0xffffu) | (vr[buf][1].w[wd] << 16);
                a1 = (vr[buf][2].w[wd] & 0xffffu) | (vr[buf][3].w[wd] << 16);
            }
            const half4_t bv = h4(a0, a1);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(ahi, bv, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(alo, bv, o[t], 0, 0, 0);
        }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    issue(0, 0);
    if constexpr (kLate) {
        wait();
        load_q();
        const int kro = min(wstart + c, last);
        if (kro == late_row) ld_k_chunks<D / 32>(kr[0].w, kb + (size_t)kro * k_nb1);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int vro = min(wstart + 4 * g + r, last);
            if (vro == late_row) ld_bytes<D / 8>(vr[0][r].w, vb + (size_t)vro * v_nb1);
        }
    }
    if constexpr (NBW == 1) {
        step(0, B0{});
        if constexpr (kLate) wait.mark(0);
    } else {
        // two register stages.  Fully unrolled (NBW <= 8) the last pair issues nothing
        // past the run; in the runtime loop (NBW > 8) the next pair's loads stay
        // unconditional (past the run they re-read its last row: cache hits, masked), so
        // no wait gathers every load
        issue(1, 1);
        if constexpr (NBW <= 8) {
#pragma unroll
            for (int blk = 0; blk < NBW; blk += 2) {
                step(blk, B0{});
                if (blk + 2 < NBW) issue(blk + 2, 0);
                step(blk + 1, B1{});
                if (blk + 3 < NBW) issue(blk + 3, 1);
            }
        } else {
            for (int blk = 0; blk < NBW; blk += 2) {
                step(blk, B0{});
                issue(blk + 2, 0);
                step(blk + 1, B1{});
                issue(blk + 3, 1);
            }
        }
    }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);

    if (g == 0) {
        s_m[wave][c] = m;
        s_l[wave][c] = l;
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int h = 4 * g + r;
        if (h < GQ) {
#pragma unroll
            for (int t = 0; t < VT; t++) s_o[wave][h][(D / 16) * c + t] = o[t][r];
        }
    }
    __syncthreads();
    if constexpr (kLate) wait.mark(1);

    for (int idx = tid; idx < GQ * D; idx += 64 * NW) {
        const int h = idx / D;
        const int dd = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, s_m[w][h]);
        float L = 0.0f, acc = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float e = fexp2(s_m[w][h] - M);
                L += s_l[w][h] * e;
                acc += s_o[w][h][dd] * e;
            }
        }
        const int qh_idx = kvh * GQ + h;
        if (n_splits == 1 && out) {
            out[(size_t)qh_idx * D + dd] = L == 0.0f ? 0.0f : acc / L;
        } else if (coherent) {
            float *rec = part + ((size_t)qh_idx * n_splits + split) * PS;
            st_coherent(rec + dd, acc);
            if (dd == 0) {
                st_coherent(rec + D, M);
                st_coherent(rec + D + 1, L);
            }
        } else {
            float *rec = part + ((size_t)qh_idx * n_splits + split) * PS;
            rec[dd] = acc;
            if (dd == 0) {
                rec[D] = M;
                rec[D + 1] = L;
            }
        }
    }
    if constexpr (kLate) wait.mark(2);
}

// The log-sum-exp merge of one output element over the splits' records, in exactly the
// floating-point order of k_fa_combine<D, *, U> (8 split groups, each an online merge of
// splits g, g+8, ... in chunks of 8U; then the 8 group states merged), so a consumer that
// merges in its own prologue gets the combine kernel's value bit for bit.
template <int D, int U>
__device__ __forceinline__ float fa_merge_exact(const float *__restrict__ ph, int n_splits, int dim) {
    constexpr int PS = part_stride<D>();
    float gm[8], gl[8], ga[8];
#pragma unroll
    for (int sg = 0; sg < 8; sg++) {
        float M = -INFINITY, L = 0.0f, A = 0.0f;
        for (int base = 0; base < n_splits; base += 8 * U) {
            float mv[U], lv[U], ov[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int sp = base + sg + 8 * u;
                const float *rec = ph + (size_t)min(sp, n_splits - 1) * PS;
                mv[u] = sp < n_splits ? rec[D] : -INFINITY;
                lv[u] = rec[D + 1];
                ov[u] = rec[dim];
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
        gm[sg] = M;
        gl[sg] = L;
        ga[sg] = A;
    }
    float mm = -INFINITY;
#pragma unroll
    for (int g = 0; g < 8; g++) mm = fmaxf(mm, gm[g]);
    float ll = 0.0f, aa = 0.0f;
    if (mm != -INFINITY) {
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const float w = gm[g] == -INFINITY ? 0.0f : fexp2(gm[g] - mm);
            ll = fmaf(gl[g], w, ll);
            aa = fmaf(ga[g], w, aa);
        }
    }
    return ll == 0.0f ? 0.0f : aa / ll;
}

// fa_merge_exact<D, U> for the four consecutive elements dim .. dim+3 (dim a multiple of
// 4) when n_splits <= 8 * UL (UL <= U): the split maxima and sums are shared, and only
// the chunk slots u < UL are loaded.  The slots u >= UL hold no split (maximum -inf,
// weight 0): their terms fmaf(v, 0, acc) leave the finite accumulators unchanged, so
// every element equals fa_merge_exact<D, U>'s (k_fa_combine<D, *, U>'s) bit for bit.
template <int D, int UL>
__device__ __forceinline__ float4 fa_merge_exact4(const float *__restrict__ ph, int n_splits, int dim) {
    constexpr int PS = part_stride<D>();
    float gm[8], gl[8];
    float4 ga[8];
#pragma unroll
    for (int sg = 0; sg < 8; sg++) {
        // the one chunk of group sg: splits sg, sg + 8, ...
        float mv[UL], lv[UL];
        float4 ov[UL];
#pragma unroll
        for (int u = 0; u < UL; u++) {
            const int sp = sg + 8 * u;
            const float *rec = ph + (size_t)min(sp, n_splits - 1) * PS;
            mv[u] = sp < n_splits ? rec[D] : -INFINITY;
            lv[u] = rec[D + 1];
            ov[u] = *(const float4 *)(rec + dim);
        }
        float cm = -INFINITY, L = 0.0f;
        float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int u = 0; u < UL; u++) cm = fmaxf(cm, mv[u]);
        if (cm != -INFINITY) {
            // the running state before the chunk is empty (M = -inf, L = A = 0): its
            // rescale by 0 leaves L and A at 0
#pragma unroll
            for (int u = 0; u < UL; u++) {
                const float w = mv[u] == -INFINITY ? 0.0f : fexp2(mv[u] - cm);
                L = fmaf(lv[u], w, L);
                A.x = fmaf(ov[u].x, w, A.x);
                A.y = fmaf(ov[u].y, w, A.y);
                A.z = fmaf(ov[u].z, w, A.z);
                A.w = fmaf(ov[u].w, w, A.w);
            }
        }
        gm[sg] = cm;
        gl[sg] = L;
        ga[sg] = A;
    }
    float mm = -INFINITY;
#pragma unroll
    for (int g = 0; g < 8; g++) mm = fmaxf(mm, gm[g]);
    float ll = 0.0f;
    float4 aa = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (mm != -INFINITY) {
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const float w = gm[g] == -INFINITY ? 0.0f : fexp2(gm[g] - mm);
            ll = fmaf(gl[g], w, ll);
            aa.x = fmaf(ga[g].x, w, aa.x);
            aa.y = fmaf(ga[g].y, w, aa.y);
            aa.z = fmaf(ga[g].z, w, aa.z);
            aa.w = fmaf(ga[g].w, w, aa.w);
        }
    }
    if (ll == 0.0f) return make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    return make_float4(aa.x / ll, aa.y / ll, aa.z / ll, aa.w / ll);
}

}  // namespace
