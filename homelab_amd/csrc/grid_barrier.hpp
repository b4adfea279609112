// The grid barrier's protocol over an atomics policy, run by a CPU model of it
// (tests/barrier_model.cpp, std::thread per block). The device form (grid_barrier_words
// and grid_barrier_exit in stream.hpp) takes the same steps with the same group and target
// helpers below, written lane-parallel: lane q < BAR_GROUPS of the block's first wave loads
// group q's counter and the wave ballots the lanes' conditions (the model loops over the
// groups in one thread), with a short sleep between polls, one meeting per area (use = 0)
// and an exit add of 1 (meetings = 1).
//
// A barrier area holds BAR_GROUPS arrival counters and BAR_GROUPS exit counters, each on
// a 256-byte line of its own, that only ever grow. Block b belongs to group b % G
// (G = min(blocks, 8): one group per XCD under round-robin dispatch).
//   * start: a block reads the group EXIT counters (its bases);
//   * arrive: one add to its group's arrival counter, not waited for;
//   * wait: until every group's arrival counter has reached base + the group's blocks;
//   * exit (the block's last action): one add to its group's exit counter.
// Every block of every call arrives once and exits once, so when a call starts the
// arrival and exit counters agree; an exit counter cannot move during a call until its
// block has left the barrier, which needs every block of the call to have arrived, hence
// to have started and read its bases. So every block reads the same bases, whenever it
// is dispatched, without any reset or publication: the last arrival costs one add and
// the waiters see it on their next poll. Calls of any grid size follow each other on one
// area, and a wait that gives up (a late block, a tiny spin limit) leaves the counters
// where a normal call would. Counter comparisons are modulo 2^32.
//
// An area usually serves one meeting per call (a kernel that meets twice uses two areas,
// and its blocks exit both). It can serve several: the k-th meeting (k = 0, 1, ...)
// waits for base + (k + 1) x the group's blocks, and each block's exit then adds the
// number of meetings, so the counters agree again when the call ends.
#pragma once

#include <stdint.h>

#ifndef OOM_BARRIER_FN
#define OOM_BARRIER_FN __device__ __forceinline__
#endif

namespace oom {

constexpr int BAR_GROUPS = 8;                          // groups of an area
constexpr int BAR_STRIDE = 64;                         // u32 words between counters: a 256-byte line each
constexpr int BAR_EXIT = BAR_GROUPS * BAR_STRIDE;      // word offset of the exit counters in an area
constexpr int BAR_WORDS = 2 * BAR_GROUPS * BAR_STRIDE; // one barrier area

OOM_BARRIER_FN uint32_t bar_groups(uint32_t nblocks) {
    return nblocks < (uint32_t)BAR_GROUPS ? nblocks : (uint32_t)BAR_GROUPS;
}
// Blocks of group q (q < BAR_GROUPS; 0 for a group the grid does not use).
OOM_BARRIER_FN uint32_t bar_group_size(uint32_t q, uint32_t nblocks) {
    const uint32_t G = bar_groups(nblocks);
    return q < G ? (nblocks - q + G - 1) / G : 0u;
}

// The group of block `block` and what group q's arrival counter must reach for the
// meeting `use` (0, 1, ...) of an area whose bases are `base`.
OOM_BARRIER_FN uint32_t bar_group_of(uint32_t block, uint32_t nblocks) { return block % bar_groups(nblocks); }
OOM_BARRIER_FN uint32_t bar_target(uint32_t base, uint32_t use, uint32_t q, uint32_t nblocks) {
    return base + (use + 1) * bar_group_size(q, nblocks);
}

// Ops: static load (relaxed, device-coherent), add (relaxed, no value returned),
// wait_mem (this agent's earlier memory operations complete) and pause (a short sleep
// between polls). The CPU model runs these per block; the device runs the same steps
// with lane q of one wave on group q (stream.hpp).
template <class Ops>
OOM_BARRIER_FN void barrier_bases(uint32_t* bar, uint32_t (&base)[BAR_GROUPS]) {
    for (int q = 0; q < BAR_GROUPS; q++) base[q] = Ops::load(bar + BAR_EXIT + q * BAR_STRIDE);
}

template <class Ops>
OOM_BARRIER_FN bool barrier_arrive_wait(uint32_t* bar, const uint32_t (&base)[BAR_GROUPS], uint32_t use,
                                        uint32_t block, uint32_t nblocks, uint32_t spin_limit) {
    Ops::wait_mem();  // the bases (and this block's stores) are complete before the arrival
    Ops::add(bar + bar_group_of(block, nblocks) * BAR_STRIDE, 1u);
    for (uint32_t spins = 0;;) {
        bool met = true;
        for (int q = 0; q < BAR_GROUPS; q++)
            met &= (int32_t)(Ops::load(bar + q * BAR_STRIDE) - bar_target(base[q], use, (uint32_t)q, nblocks)) >= 0;
        if (met) return true;
        Ops::pause();
        if (++spins > spin_limit) return false;
    }
}

template <class Ops>
OOM_BARRIER_FN void barrier_exit(uint32_t* bar, uint32_t block, uint32_t nblocks, uint32_t meetings) {
    Ops::add(bar + BAR_EXIT + bar_group_of(block, nblocks) * BAR_STRIDE, meetings);
}

}  // namespace oom
