// CPU model of the decode kernels' grid barrier: the protocol of
// homelab_amd/csrc/grid_barrier.hpp (the same source the device code compiles), run with
// one std::thread per block over GCC atomics on a shared barrier header.
//
// It checks the protocol's logic (bases from the exit counters, arrivals, exits, what a
// waiter waits for) across calls of different grid sizes on one header, back-to-back
// meetings, waits that give up, and blocks that start late. Threads start in whatever
// order the OS runs them; no start gate. It does not model the GPU's memory ordering.
//
//   barrier_model <scenario>    exit 0 = the scenario's expectation held
//
// Scenarios:
//   sizes      calls of 3, 256, 5, 256, 1, 300, 8, 9, 256, 2 and 512 blocks on one header,
//              each meeting the grid once: every meeting releases, none early, none gives up
//   twice      the same calls meeting twice (areas 0 and 1)
//   b2b        256 blocks, 200 meetings back to back alternating two areas (each area
//              met 100 times in the call), no work between; then 200 with random work
//   giveup     a block arrives late while the others' waits give up (tiny limit); after
//              that call the header serves a normal call of 256 blocks with no give-up
//   giveup2    the same for a kernel meeting twice, each meeting in its own area
//   late       a block starts only after all the others have arrived at its first meeting:
//              it still reads the call's bases, so nobody gives up or passes early
//   old_sizes  (expected to FAIL) the round-one protocol, which published the generation
//              to the first min(blocks, 8) words only, on the sizes sequence: a call
//              after a small one gives up
#include <array>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#define OOM_BARRIER_FN inline
#include "../homelab_amd/csrc/grid_barrier.hpp"

using namespace oom;

struct CpuOps {
    static uint32_t load(uint32_t* p) { return __atomic_load_n(p, __ATOMIC_RELAXED); }
    static void store(uint32_t* p, uint32_t v) { __atomic_store_n(p, v, __ATOMIC_RELAXED); }
    static uint32_t fetch_add(uint32_t* p, uint32_t v) { return __atomic_fetch_add(p, v, __ATOMIC_RELAXED); }
    static void add(uint32_t* p, uint32_t v) { (void)__atomic_fetch_add(p, v, __ATOMIC_RELAXED); }
    static void wait_mem() { __atomic_thread_fence(__ATOMIC_SEQ_CST); }
    static void pause() { std::this_thread::yield(); }
};

constexpr int OLD_WORDS = (2 * BAR_GROUPS + 1) * BAR_STRIDE;  // the round-one area: groups, top, generations

// The round-one protocol (group counters reset by their last arrival, a top counter, and
// generation words published by the last arrival, to the first G = min(blocks, 8) words
// only). Restated here to show the model finds the fault that partial publication caused.
static bool old_arrive_wait(uint32_t* bar, uint32_t block, uint32_t nblocks, uint32_t spin_limit) {
    const uint32_t G = nblocks < (uint32_t)BAR_GROUPS ? nblocks : (uint32_t)BAR_GROUPS, g = block % G;
    const uint32_t n_g = (nblocks - g + G - 1) / G;
    uint32_t* cnt = bar + g * BAR_STRIDE;
    uint32_t* top = bar + BAR_GROUPS * BAR_STRIDE;
    uint32_t* genw = bar + (BAR_GROUPS + 1 + g) * BAR_STRIDE;
    const uint32_t target = CpuOps::load(genw) + 1u;
    CpuOps::wait_mem();
    if (CpuOps::fetch_add(cnt, 1u) == n_g - 1) {
        CpuOps::store(cnt, 0u);
        CpuOps::wait_mem();
        if (CpuOps::fetch_add(top, 1u) == G - 1) {
            CpuOps::store(top, 0u);
            CpuOps::wait_mem();
            for (uint32_t q = 0; q < G; q++) CpuOps::store(bar + (BAR_GROUPS + 1 + q) * BAR_STRIDE, target);
            CpuOps::wait_mem();
            return true;
        }
    }
    for (uint32_t spins = 0; (int32_t)(CpuOps::load(genw) - target) < 0;) {
        CpuOps::pause();
        if (++spins > spin_limit) return false;
    }
    return true;
}

struct Header {
    std::vector<uint32_t> words = std::vector<uint32_t>(2 * OLD_WORDS, 0u);
    uint32_t* area(int i) { return words.data() + i * OLD_WORDS; }
};

struct Result {
    long gave_up = 0;      // waits that reached the spin limit
    long early = 0;        // releases before every block of the meeting had arrived
};

// One call of `n` blocks meeting `meetings` times; meeting m uses area areas[m]. Block
// `late_start` starts only after the others have arrived at the first meeting. Block
// `late` (if >= 0) sleeps `late_ms` before its first arrival. Work between meetings is a
// random spin when `work` is set. Each block exits every area it used, after its last
// meeting.
static Result call(Header& hdr, uint32_t n, int meetings, const std::vector<int>& areas, uint32_t limit, bool old,
                   int late = -1, int late_ms = 0, bool work = false, int late_start = -1) {
    std::vector<std::atomic<uint32_t>> arrived(meetings);
    for (auto& a : arrived) a.store(0);
    std::atomic<long> gave_up{0}, early{0};
    std::vector<std::thread> th;
    th.reserve(n);
    for (uint32_t b = 0; b < n; b++) {
        th.emplace_back([&, b]() {
            std::mt19937 rng(1234u + b);
            if ((int)b == late_start) {
                while (arrived[0].load() < n - 1) std::this_thread::yield();
                std::this_thread::sleep_for(std::chrono::milliseconds(5));
            }
            // each area's bases, read once at the start
            std::vector<std::array<uint32_t, BAR_GROUPS>> bases(meetings);
            for (int m = 0; m < meetings; m++) {
                int first = m;
                for (int j = 0; j < m; j++)
                    if (areas[j] == areas[m]) { first = j; break; }
                if (first == m) {
                    uint32_t tmp[BAR_GROUPS];
                    if (!old) barrier_bases<CpuOps>(hdr.area(areas[m]), tmp);
                    for (int q = 0; q < BAR_GROUPS; q++) bases[m][q] = old ? 0u : tmp[q];
                } else {
                    bases[m] = bases[first];
                }
            }
            for (int m = 0; m < meetings; m++) {
                if ((int)b == late && m == 0) std::this_thread::sleep_for(std::chrono::milliseconds(late_ms));
                if (work) {
                    volatile uint32_t s = 0;
                    const uint32_t iters = rng() % 20000;
                    for (uint32_t i = 0; i < iters; i++) s = s + i;
                }
                arrived[m].fetch_add(1);
                uint32_t* bar = hdr.area(areas[m]);
                bool ok;
                if (old) {
                    ok = old_arrive_wait(bar, b, n, limit);
                } else {
                    uint32_t base[BAR_GROUPS];
                    for (int q = 0; q < BAR_GROUPS; q++) base[q] = bases[m][q];
                    int use = 0;  // earlier meetings of this call on the same area
                    for (int j = 0; j < m; j++) use += areas[j] == areas[m];
                    ok = barrier_arrive_wait<CpuOps>(bar, base, (uint32_t)use, b, n, limit);
                }
                if (!ok) gave_up++;
                else if (arrived[m].load() != n) early++;
            }
            if (!old) {
                for (int m = 0; m < meetings; m++) {
                    int first = m, uses = 0;
                    for (int j = 0; j < m; j++)
                        if (areas[j] == areas[m]) { first = j; break; }
                    if (first != m) continue;
                    for (int j = 0; j < meetings; j++) uses += areas[j] == areas[m];
                    barrier_exit<CpuOps>(hdr.area(areas[m]), b, n, (uint32_t)uses);
                }
            }
        });
    }
    for (auto& t : th) t.join();
    return Result{gave_up.load(), early.load()};
}

static const uint32_t BIG = 20000000u;  // polls (yields): far beyond any honest wait here

static bool run_sizes(bool old, int meetings) {
    Header hdr;
    const uint32_t sizes[] = {3, 256, 5, 256, 1, 300, 8, 9, 256, 2, 512, 3, 256, 7, 256};
    std::vector<int> areas;
    for (int m = 0; m < meetings; m++) areas.push_back(m % 2);
    long bad = 0;
    for (uint32_t n : sizes) {
        const Result r = call(hdr, n, meetings, areas, old ? 200000u : BIG, old);
        if (r.gave_up || r.early) {
            std::printf("  %u blocks: %ld waits gave up, %ld early releases\n", n, r.gave_up, r.early);
            bad++;
        }
    }
    return bad == 0;
}

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    const std::string sc = argv[1];
    if (sc == "sizes") return run_sizes(false, 1) ? 0 : 1;
    if (sc == "twice") return run_sizes(false, 2) ? 0 : 1;
    if (sc == "old_sizes") return run_sizes(true, 1) ? 0 : 1;
    if (sc == "b2b") {
        Header hdr;
        std::vector<int> areas;
        for (int m = 0; m < 200; m++) areas.push_back(m % 2);
        const Result a = call(hdr, 256, 200, areas, BIG, false);
        const Result b = call(hdr, 256, 200, areas, BIG, false, -1, 0, true);
        std::printf("  no work: %ld gave up, %ld early; work: %ld gave up, %ld early\n", a.gave_up, a.early, b.gave_up,
                    b.early);
        return (a.gave_up || a.early || b.gave_up || b.early) ? 1 : 0;
    }
    if (sc == "late") {
        Header hdr;
        const Result w = call(hdr, 5, 1, {0}, BIG, false);  // earlier calls on the header
        const Result r = call(hdr, 64, 1, {0}, BIG, false, -1, 0, false, 9);
        std::printf("  call with a late starter: %ld waits gave up, %ld early\n", r.gave_up, r.early);
        if (w.gave_up || w.early || r.gave_up || r.early) return 1;
        const Result n = call(hdr, 256, 1, {0}, BIG, false);
        std::printf("  next call: %ld gave up, %ld early\n", n.gave_up, n.early);
        return (n.gave_up || n.early) ? 1 : 0;
    }
    if (sc == "giveup" || sc == "giveup2") {
        Header hdr;
        const int meetings = sc == "giveup" ? 1 : 2;
        const std::vector<int> areas = sc == "giveup2" ? std::vector<int>{0, 1} : std::vector<int>{0, 0};
        // block 5 arrives 50 ms late; the others poll 10 times, then go on
        const Result r = call(hdr, 256, meetings, areas, 10u, false, 5, 50);
        std::printf("  call with a late block: %ld waits gave up\n", r.gave_up);
        if (r.gave_up == 0) return 3;  // the scenario did not happen
        const Result n = call(hdr, 256, meetings, areas, BIG, false);
        std::printf("  next call: %ld gave up, %ld early\n", n.gave_up, n.early);
        return (n.gave_up || n.early) ? 1 : 0;
    }
    return 2;
}
