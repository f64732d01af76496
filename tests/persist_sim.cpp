// CPU model of the dependency-hop protocol of the persistent layer-stack decode
// (k_persist_q8_0 in llama-cpp-ascend310b4-addon_amd/csrc/persist.hip).
//
// One std::thread per workgroup walks the kernel's sequence of phases with the roles,
// expected-arrival counts and sync-area layout of persist_plan.h (the header the kernel
// and its launcher use), on std::atomic counters: arrivals go to every replica of a hop's
// counter set, a workgroup polls its own replica.  A producer marks its output of
// (layer, hop) before it arrives; after every wait the consumer checks that every
// producer of that hop has marked, so a wait that returns early is a violation.  Waits
// are bounded like the kernel's (spin_limit polls, then the error word), threads sleep
// for random short times between steps to vary the interleaving.  Launches alternate
// between the two counter sets as the kernel's do: each thread clears its share of the
// other set in the first layer's gate/up phase, the last thread to exit flips the parity
// word.  Each run does
// several launches on one sync area.
//
// usage: persist_sim n_wg n_embd n_head n_head_kv hd n_ff n_layer fa_splits launches
//                    spin_limit stall_hop seed
// prints one line "ok violations=V timeouts=T err=E residue=R arrivals=A expected=X"
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>

#include "persist_plan.h"

using namespace persist_plan;

struct Sim {
    Layout lo{};
    int n_layer = 0;
    long spin_limit = 0;
    int stall_hop = -1;
    std::vector<std::atomic<unsigned>> sync;
    std::vector<std::atomic<int>> mark;  // [layer][hop][wg]: the producer's output is written
    std::atomic<long> violations{0}, timeouts{0}, arrivals{0};
    unsigned seed = 1;

    Sim(const Layout &l, int nl, long spin, int stall)
        : lo(l), n_layer(nl), spin_limit(spin), stall_hop(stall), sync(sync_words(nl)),
          mark((size_t)nl * kHops * l.n_wg) {
        for (auto &w : sync) w.store(0);
    }
    std::atomic<int> &mk(int layer, int hop, int wg) { return mark[((size_t)layer * kHops + hop) * lo.n_wg + wg]; }
    bool producer(int hop, int wg) const {
        switch (hop) {
            case 0: return is_qkv(lo, wg);
            case 1: return is_fa(lo, wg);
            case 2: return is_o(lo, wg);
            case 3: return is_gu(lo, wg);
            default: return is_down(lo, wg);
        }
    }
};

struct Walker {
    Sim &S;
    int wg;
    std::mt19937 rng;
    Walker(Sim &s, int w, unsigned seed) : S(s), wg(w), rng(seed * 7919u + (unsigned)w) {}

    void jitter() {
        const unsigned r = rng() % 16;
        if (r < 10) return;
        if (r < 14) std::this_thread::yield();
        else std::this_thread::sleep_for(std::chrono::microseconds(rng() % 50));
    }
    size_t base = 0;  // this launch's counter set
    unsigned par = 0;
    void arrive(int layer, int hop) {
        S.mk(layer, hop, wg).store(1, std::memory_order_release);
        for (int r = 0; r < kReps; r++)  // every replica of the counter set
            S.sync[base + hop_ctr_word(layer, hop, wg & 7, r)].fetch_add(1, std::memory_order_acq_rel);
        S.arrivals.fetch_add(1);
    }
    // the kernel's hop_wait: poll the 8 counters; give up after spin_limit polls or when
    // another workgroup raised the error word
    void wait(int layer, int hop) {
        std::atomic<unsigned> &err = S.sync[err_word(S.n_layer)];
        long spins = 0;
        for (;;) {
            bool all = true;
            for (int j = 0; j < 8; j++) {  // the replica of this workgroup
                const unsigned want = hop_want(S.lo, hop, j) + (layer == 0 && hop == S.stall_hop && j == 0);
                all = all &&
                      S.sync[base + hop_ctr_word(layer, hop, j, wg % kReps)].load(std::memory_order_acquire) >= want;
            }
            if (all) break;
            if (err.load(std::memory_order_acquire)) return;
            if (++spins > S.spin_limit) {
                err.store(1, std::memory_order_release);
                S.timeouts.fetch_add(1);
                return;
            }
            std::this_thread::yield();
        }
        // a completed wait: every producer of the hop has written its output
        for (int w = 0; w < S.lo.n_wg; w++)
            if (S.producer(hop, w) && !S.mk(layer, hop, w).load(std::memory_order_acquire)) S.violations.fetch_add(1);
    }
    // the kernel's persist_exit
    void exit() {
        std::atomic<unsigned> &ex = S.sync[exit_word(S.n_layer)];
        const unsigned prev = ex.fetch_add(1, std::memory_order_acq_rel);
        if (prev != (unsigned)S.lo.n_wg - 1) return;
        S.sync[err_word(S.n_layer)].store(0);
        S.sync[parity_word(S.n_layer)].store(par ^ 1u);
        ex.store(0);
    }
    // the walk of k_persist_q8_0: phase order, roles, which hop each phase waits on
    void run() {
        const Layout &lo = S.lo;
        par = S.sync[parity_word(S.n_layer)].load() & 1u;
        base = set_base(S.n_layer, (int)par);
        const size_t other = set_base(S.n_layer, (int)(par ^ 1u));
        for (int l = 0; l < S.n_layer; l++) {
            if (is_qkv(lo, wg)) {  // q/k/v: after the previous layer's output
                jitter();
                if (l > 0) wait(l - 1, 4);
                jitter();
                arrive(l, 0);
            }
            if (is_fa(lo, wg)) {  // attention: after q and the cache row
                wait(l, 0);
                jitter();
                arrive(l, 1);
            }
            if (is_o(lo, wg)) {  // merge + o: after every split record
                jitter();
                wait(l, 1);
                jitter();
                arrive(l, 2);
            }
            if (l == 0)  // this thread's share of the other counter set, where the kernel clears it
                for (size_t i = (size_t)wg; i < hop_counters(S.n_layer); i += (size_t)lo.n_wg) {
                    jitter();
                    S.sync[other + i * kCtrStride].store(0);
                }
            jitter();  // gate/up: after x1
            wait(l, 2);
            jitter();
            if (is_gu(lo, wg)) arrive(l, 3);
            jitter();  // down: after gate and up
            wait(l, 3);
            jitter();
            if (is_down(lo, wg)) arrive(l, 4);
        }
        exit();
    }
};

int main(int argc, char **argv) {
    if (argc != 13) {
        fprintf(stderr, "usage: %s n_wg n_embd n_head n_head_kv hd n_ff n_layer fa_splits launches spin stall seed\n",
                argv[0]);
        return 2;
    }
    const int n_wg = atoi(argv[1]), n_embd = atoi(argv[2]), n_head = atoi(argv[3]), n_head_kv = atoi(argv[4]);
    const int hd = atoi(argv[5]), n_ff = atoi(argv[6]), n_layer = atoi(argv[7]), splits = atoi(argv[8]);
    const int launches = atoi(argv[9]);
    const long spin = atol(argv[10]);
    const int stall = atoi(argv[11]);
    const unsigned seed = (unsigned)atol(argv[12]);
    const Layout lo = make_layout(n_wg, n_embd, n_head, n_head_kv, hd, n_ff, splits, hd + 4);
    if (!layout_fits(lo, 5, 2)) {
        printf("unfit\n");
        return 3;
    }
    {  // every down tile has exactly one workgroup
        std::vector<int> cover(lo.n_down_tiles, 0);
        for (int w = 0; w < n_wg; w++)
            for (int i = 0; i < 2; i++) {
                const int t = down_tile(lo, w, i);
                if (t >= lo.n_down_tiles) {
                    printf("down tile %d of workgroup %d out of range\n", t, w);
                    return 5;
                }
                if (t >= 0) cover[t]++;
            }
        for (int t = 0; t < lo.n_down_tiles; t++)
            if (cover[t] != 1) {
                printf("down tile %d covered %d times\n", t, cover[t]);
                return 5;
            }
    }
    long expected = 0;
    for (int h = 0; h < kHops; h++) {
        long sum = 0;
        for (int j = 0; j < 8; j++) sum += hop_want(lo, h, j);
        if (sum != lo.hop_count[h]) {
            printf("want-sum hop %d: %ld != %d\n", h, sum, lo.hop_count[h]);
            return 4;
        }
        expected += lo.hop_count[h];
    }
    expected *= (long)n_layer * launches;
    Sim S(lo, n_layer, spin, stall);
    S.seed = seed;
    long residue = 0, err_left = 0;
    for (int it = 0; it < launches; it++) {
        for (auto &m : S.mark) m.store(0);
        std::vector<std::thread> th;
        th.reserve(n_wg);
        for (int w = 0; w < n_wg; w++)
            th.emplace_back([&S, w, seed, it] { Walker(S, w, seed + 1000u * (unsigned)it).run(); });
        for (auto &t : th) t.join();
        // the next launch must find its counter set, the exit counter and the error word clean
        const size_t next = set_base(n_layer, (int)(S.sync[parity_word(n_layer)].load() & 1u));
        for (size_t i = 0; i < hop_counters(n_layer); i++) residue += S.sync[next + i * kCtrStride].load() != 0;
        residue += S.sync[exit_word(n_layer)].load() != 0;
        err_left += S.sync[err_word(n_layer)].load();
        S.seed++;
        if (stall >= 0) S.stall_hop = -1;  // only the first launch stalls
    }
    printf("ok violations=%ld timeouts=%ld err=%ld residue=%ld arrivals=%ld expected=%ld\n", S.violations.load(),
           S.timeouts.load(), err_left, residue, S.arrivals.load(), expected);
    return 0;
}
