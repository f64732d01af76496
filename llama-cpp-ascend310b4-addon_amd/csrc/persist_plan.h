// persist_plan.h -- the work split and dependency hops of the persistent layer-stack
// decode (persist.hip), as plain functions shared by the kernel, its host launcher and
// the CPU model of the hop protocol.
//
// A grid of n_wg workgroups (a multiple of 8) walks every layer through five phases; hop
// h of layer l is the event "every producer of phase h of layer l has written its
// outputs".  Producers arrive on one of 8 counters (workgroup id mod 8), in each of
// kReps replicas of the counter set; a consumer polls the replica of its workgroup id mod
// kReps until every counter holds the arrivals expected on it (fewer pollers per line).
//
//   phase (hop)   producers                              consumers (wait before use)
//   0 q/k/v       tiles 0 .. n_qkv_tiles-1 (wg = tile)   attention tiles        (hop 0)
//   1 attention   workgroups fa0 .. fa0+n_fa-1           o tiles                (hop 1)
//   2 o           workgroups o0 .. o0+n_o_tiles-1        every workgroup        (hop 2)
//   3 gate/up     every workgroup with a tile            every workgroup        (hop 3)
//     (+ swiglu)
//   4 down        every workgroup with a tile            next layer's q/k/v     (hop 4)
//
// The three first phases run on disjoint workgroups, so the attention of layer l can
// overlap nothing but the weight prefetch of the o tiles, and every wait depends only on
// earlier phases: the walk cannot deadlock when every workgroup is resident.
#pragma once

#include <stddef.h>

#ifdef __HIPCC__
#define MI_PLAN_HD __host__ __device__
#else
#define MI_PLAN_HD
#endif

namespace persist_plan {

constexpr int kHops = 5;         // hops per layer
constexpr int kCtrStride = 64;   // unsigned words between counters (256 bytes)
constexpr int kReps = 16;        // replicas of each hop's 8 counters (16 pollers per line at 256 workgroups)
constexpr int kMaxSplits = 16;   // attention splits the o prologue merges
constexpr int kRowsE = 16;       // rows per k = n_embd tile (q/k/v, o, gate/up)
constexpr int kRowsF = 4;        // rows per k = n_ff tile (down)

struct Layout {
    int n_wg;
    int n_q, n_k, n_v;  // rows of the q, k, v projections
    int n_qkv_tiles, n_fa, n_o_tiles, n_gu_tiles, n_down_tiles;
    int fa0, o0;        // first workgroup of the attention and o tiles
    int hop_first[kHops], hop_count[kHops];  // producers: workgroups first .. first+count-1 (mod n_wg)
    // per-layer scratch (floats): q, attention split records, x1 = o + x, the swiglu
    // product (SmoothQuant-divided), layer output
    size_t q_off, part_off, x1_off, h_off, xr_off, layer_floats;
};

MI_PLAN_HD inline size_t round_up64(size_t v) { return (v + 63) / 64 * 64; }

// part_rec = floats per attention split record (head_dim + 4)
MI_PLAN_HD inline Layout make_layout(int n_wg, int n_embd, int n_head, int n_head_kv, int hd, int n_ff,
                                     int fa_splits, int part_rec) {
    Layout lo;
    lo.n_wg = n_wg;
    lo.n_q = n_head * hd;
    lo.n_k = n_head_kv * hd;
    lo.n_v = n_head_kv * hd;
    lo.n_qkv_tiles = (lo.n_q + lo.n_k + lo.n_v) / kRowsE;
    lo.n_fa = fa_splits * n_head_kv;
    lo.n_o_tiles = n_embd / kRowsE;
    lo.n_gu_tiles = 2 * n_ff / kRowsE;  // 8 gate rows + the same 8 up rows each
    lo.n_down_tiles = n_embd / kRowsF;
    lo.fa0 = lo.n_qkv_tiles % n_wg;
    lo.o0 = (lo.fa0 + lo.n_fa) % n_wg;
    const int firsts[kHops] = {0, lo.fa0, lo.o0, 0, 0};
    const int counts[kHops] = {lo.n_qkv_tiles, lo.n_fa, lo.n_o_tiles, lo.n_gu_tiles, lo.n_down_tiles};
    for (int h = 0; h < kHops; h++) {
        lo.hop_first[h] = firsts[h];
        lo.hop_count[h] = counts[h] < n_wg ? counts[h] : n_wg;
    }
    lo.q_off = 0;
    lo.part_off = round_up64((size_t)lo.n_q);
    lo.x1_off = lo.part_off + round_up64((size_t)n_head * kMaxSplits * part_rec);
    lo.h_off = lo.x1_off + round_up64((size_t)n_embd);
    lo.xr_off = lo.h_off + round_up64((size_t)n_ff);
    lo.layer_floats = lo.xr_off + round_up64((size_t)n_embd);
    return lo;
}

// the three first phases must sit on disjoint workgroups and the later ones must give
// every workgroup at most max_gu / max_down tiles
MI_PLAN_HD inline bool layout_fits(const Layout &lo, int max_gu, int max_down) {
    return lo.n_wg % 8 == 0 && lo.n_qkv_tiles + lo.n_fa + lo.n_o_tiles <= lo.n_wg &&
           lo.n_gu_tiles <= max_gu * lo.n_wg && lo.n_down_tiles <= max_down * lo.n_wg;
}

// roles of workgroup wg
MI_PLAN_HD inline bool is_qkv(const Layout &lo, int wg) { return wg < lo.n_qkv_tiles; }
MI_PLAN_HD inline int fa_tile(const Layout &lo, int wg) { return (wg - lo.fa0 + lo.n_wg) % lo.n_wg; }
MI_PLAN_HD inline int o_tile(const Layout &lo, int wg) { return (wg - lo.o0 + lo.n_wg) % lo.n_wg; }
MI_PLAN_HD inline bool is_fa(const Layout &lo, int wg) { return fa_tile(lo, wg) < lo.n_fa; }
MI_PLAN_HD inline bool is_o(const Layout &lo, int wg) { return o_tile(lo, wg) < lo.n_o_tiles; }
MI_PLAN_HD inline bool is_gu(const Layout &lo, int wg) { return wg < lo.n_gu_tiles; }
MI_PLAN_HD inline bool is_down(const Layout &lo, int wg) { return wg < lo.n_down_tiles; }

// down tile i (0 or 1) of workgroup wg, or -1: every workgroup has tile wg; the tiles
// past n_wg go to the last workgroups (wg >= 2 n_wg - n_down_tiles), whose q/k/v and
// gate/up shares are the lighter ones
MI_PLAN_HD inline int down_tile(const Layout &lo, int wg, int i) {
    if (i == 0) return wg < lo.n_down_tiles ? wg : -1;
    const int extra = lo.n_down_tiles - lo.n_wg;
    return extra > 0 && wg >= lo.n_wg - extra ? wg + extra : -1;
}

// arrivals expected on counter j (0..7) of hop h: the producers (first + t) mod n_wg,
// t < count, whose id mod 8 is j (n_wg is a multiple of 8, so (first + t) mod 8 == j)
MI_PLAN_HD inline unsigned hop_want(const Layout &lo, int h, int j) {
    const int first = lo.hop_first[h], count = lo.hop_count[h];
    return (unsigned)(count / 8 + (((j - first) & 7) < (count & 7) ? 1 : 0));
}

// word offsets in the sync area: two sets of counters, kReps x 8 per (layer, hop) each;
// a launch counts on the set the parity word names and clears the other one (the set
// of the previous launch, which nobody reads any more) for the next launch, whose set
// it becomes when the last workgroup to exit flips the parity.  Then the exit counter,
// the device error word and the parity word.  Every word on its own 256-byte line.
MI_PLAN_HD inline size_t hop_ctr_word(int layer, int hop, int j, int rep) {
    return (((size_t)(layer * kHops + hop) * kReps + rep) * 8 + j) * kCtrStride;
}
MI_PLAN_HD inline size_t hop_counters(int n_layer) { return (size_t)n_layer * kHops * kReps * 8; }
MI_PLAN_HD inline size_t set_base(int n_layer, int set) { return (size_t)set * hop_counters(n_layer) * kCtrStride; }
MI_PLAN_HD inline size_t exit_word(int n_layer) { return 2 * hop_counters(n_layer) * kCtrStride; }
MI_PLAN_HD inline size_t err_word(int n_layer) { return exit_word(n_layer) + kCtrStride; }
MI_PLAN_HD inline size_t parity_word(int n_layer) { return exit_word(n_layer) + 2 * kCtrStride; }
MI_PLAN_HD inline size_t sync_words(int n_layer) { return exit_word(n_layer) + 3 * kCtrStride; }

}  // namespace persist_plan
