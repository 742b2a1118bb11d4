// sk_arrive.h - arrival count of the parts of one stream-K tile.
//
// The parts of a tile cut along K count their arrivals on one 64-bit counter:
// the launch's 48-bit epoch in the high bits, the count in the low 16. A
// counter holding another epoch (an earlier launch's, or any scratch contents)
// counts as zero. The first arrival of a launch installs its epoch with one
// compare-exchange; every later one adds 1 with one atomic, so parts arriving
// together never retry against each other. A failed exchange can only have
// seen another part install this epoch, so the second round adds: two rounds
// always suffice on a counter only this launch's parts touch, and `tries`
// bounds the loop against a counter something else keeps changing.
//
// Written over an operations policy so the same protocol runs on the device
// (system-scope HIP atomics, streamk.h) and in a host unit test (std::atomic).
#pragma once
#include <stdint.h>

#ifndef SK_HOST_DEVICE
#define SK_HOST_DEVICE __host__ __device__
#endif

namespace spinn {

// Arrival outcome of one part: the count it completed (1-based), or -1 when
// no claim succeeded within `tries` rounds.
//   Ops::load()                      -> uint64_t
//   Ops::fetch_add(uint64_t d)       -> uint64_t (old value)
//   Ops::cas(uint64_t &exp, uint64_t desired) -> bool (exp updated on failure)
template <class Ops>
SK_HOST_DEVICE inline int sk_arrive_count(Ops &c, uint64_t epoch, int tries) {
    const uint64_t tag = epoch << 16;
    uint64_t v = c.load();
    int count = -1;
    for (int t = 0; t < tries && count < 0; ++t) {
        if ((v >> 16) == epoch) {
            count = (int)(c.fetch_add(1ull) & 0xFFFFu) + 1;
        } else if (c.cas(v, tag | 1ull)) {
            count = 1;
        }
    }
    return count;
}

// What the arriving part does with its count: 1 = it is the last part (sum the
// parts, apply the epilogue, reset the counter to `epoch << 16`), 0 = not the
// last, -1 = the protocol broke (no claim, or a count past the number of parts,
// which only a counter changed by something other than this launch's parts can
// produce): the tile cannot be finished and the launch must report an error.
SK_HOST_DEVICE inline int sk_arrive_outcome(int count, int nparts) {
    if (count < 1 || count > nparts) return -1;
    return count == nparts ? 1 : 0;
}

} // namespace spinn
