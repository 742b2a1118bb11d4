// streamk.h - data-parallel + stream-K work split of one MFMA GEMM launch.
//
// A grid of T output tiles on C compute units leaves ceil(T/C) tiles on some
// CUs and floor(T/C) on others; with ResNet-101's shapes at batch 32 that is
// 7 against 6.125 (1568 tiles) or 2 against 1.53 (392 tiles) per CU. Here the
// first floor(T/C)*C tiles run whole, one workgroup each ("data-parallel"),
// and the R = T mod C remaining tiles are cut along K into parts spread over
// the CUs, so every CU ends with nearly the same number of K slices. Two
// schemes place the parts:
//   SPLIT_WGS (at most two whole tiles per CU, R > C/4): R*S slices (S per
//     tile) in equal contiguous ranges of at most S, one range per extra
//     workgroup, one extra workgroup per CU; a range may end one tile and
//     start the next. Extra workgroups have the lowest block ids, so they are
//     dispatched, and their parts finished, first.
//   PARTS_IN_DP (otherwise): each remaining tile in p equal parts of >= 4
//     slices, one part done by each of the first R*p data-parallel workgroups
//     before its own tile, so no workgroup beyond one per slot is launched.
// The dispatcher deals workgroups to the 8 XCDs round-robin: each XCD gets a
// contiguous run of whole tiles and its own share of the remaining ones, so
// the workgroups that share an input panel or a split tile sit behind one L2.
//
// A tile cut into parts is finished by whichever part arrives last (no
// workgroup ever waits on another): each part writes its partial sums to its
// slot, then counts its arrival on the tile's counter (system-scope atomics);
// the part that completes the count reads the parts' slots back, sums them in
// K order and applies the epilogue.
// The sum order depends only on the shape, so results are deterministic. The
// first part of a tile (K offset 0) starts its accumulators from the
// epilogue's bias + residual, like a whole tile.
//
// Arrival counters are 64-bit: the launch's 48-bit epoch in the high bits and
// the arrival count in the low 16 (protocol in sk_arrive.h). A counter holding
// another epoch (left by an earlier launch, or any scratch contents) counts as
// zero, so the workspace needs no clearing; the last arrival resets the count
// to zero under its own epoch, so a graph replaying the same launch (same
// epoch) starts from zero. An arrival that cannot complete the protocol sets
// the host-visible status word instead of leaving the tile silently unwritten.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "mfma_core.h"
#include "sk_arrive.h"

namespace spinn {

constexpr int kXcds = 8;
constexpr int kSkSplitWgs = 0;  // SPLIT_WGS scheme
constexpr int kSkPartsInDp = 1; // PARTS_IN_DP scheme
constexpr int kSkMaxParts = 8;  // parts per remaining tile, at most

// Kernel-side description of the split (host side: plan_streamk).
struct SkSched {
    int tiles_m;     // tile t covers (t % tiles_m, t / tiles_m)
    int S;           // K slices per tile
    int dp_per_xcd;  // whole tiles per XCD (data-parallel workgroups)
    int R;           // tiles cut along K, after the 8 * dp_per_xcd whole ones
    int scheme;      // kSkSplitWgs or kSkPartsInDp
    int W;           // SPLIT_WGS: extra workgroups per XCD (0 for PARTS_IN_DP)
    int p;           // PARTS_IN_DP: parts per remaining tile
    int rx;          // ceil(R / 8): remaining tiles of the largest XCD share
    int local;       // 1: workgroup id % 8 is its XCD (checked at set-up), parts exchanged through that L2
    uint64_t epoch;  // 48-bit tag of this launch's counters, nonzero
    unsigned long long *cnt; // R arrival counters
    float *part;     // partial tiles in the per-thread layout, one slot per part
    unsigned *status; // host-visible status word: set to 1 when an arrival fails (may be null)
    int tries;       // arrival rounds before giving up (2 always suffice; see sk_arrive.h)
};

// Contiguous share of XCD x in the remaining tiles: [start, start + count).
__device__ __forceinline__ void sk_xcd_tiles(const SkSched &s, int x, int &start, int &count) {
    const int q = s.R / kXcds, r = s.R % kXcds;
    start = x * q + min(x, r);
    count = q + (x < r ? 1 : 0);
}

// SPLIT_WGS: first K slice (in the XCD's iteration space of I slices) of
// workgroup w out of Wx, and the workgroup owning slice i.
__device__ __forceinline__ int sk_begin(int w, int I, int Wx) { return (int)((int64_t)w * I / Wx); }
__device__ __forceinline__ int sk_owner(int i, int I, int Wx) { return (int)(((int64_t)(i + 1) * Wx - 1) / I); }

// System-scope atomics on one arrival counter (the operations sk_arrive_count needs).
struct SkDeviceCounter {
    unsigned long long *p;
    __device__ uint64_t load() const { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); }
    __device__ uint64_t fetch_add(uint64_t d) const {
        return __hip_atomic_fetch_add(p, (unsigned long long)d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __device__ bool cas(uint64_t &exp, uint64_t desired) const {
        unsigned long long e = exp;
        const bool ok = __hip_atomic_compare_exchange_strong(p, &e, (unsigned long long)desired, __ATOMIC_RELAXED,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        exp = e;
        return ok;
    }
};

// Register the arrival of one part of a tile; true for the last part, which
// resets the counter to a zero count under this epoch (so a graph replaying
// the launch starts from zero). Thread 0 only; the caller has made its partial
// stores complete before calling. A broken protocol (sk_arrive_outcome -1)
// leaves the tile unfinished, so it is reported through the status word, which
// the host reads after synchronising (spinn_hip_device_status).
__device__ __forceinline__ bool sk_arrive(const SkSched &s, int cnt_idx, int nparts) {
    SkDeviceCounter c{s.cnt + cnt_idx};
    const int outcome = sk_arrive_outcome(sk_arrive_count(c, s.epoch, s.tries), nparts);
    if (outcome < 0) {
        if (s.status) __hip_atomic_store(s.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return false;
    }
    if (outcome == 1)
        __hip_atomic_store(c.p, (unsigned long long)s.epoch << 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return outcome == 1;
}

// Partial sums move between the parts of a tile in one of two ways. All parts
// of a tile have the same block id modulo 8, so when that is the XCD (checked
// once per device at set-up, xcd_local_parts) they share one L2, the
// coherence point of an XCD: plain stores (the L1 writes through to the L2)
// and loads marked sc0 suffice. Correctness there does not rest on sc0 alone
// (the compiler's memory model counts sc0 as workgroup scope, which may hit in
// the CU's L1) but on no L1 holding a line of a part slot when the last part
// reads it: every L1 is invalidated when a launch starts, slots are 64x64x4 B
// (whole cache lines, one slot per part), and within a launch each slot's lines
// are read once, by the tile's last part, after every part's stores completed
// (s_waitcnt before the arrival); the only earlier access from any CU is the
// owning part's own store, which writes through. Otherwise system-scope stores
// and loads (sc0 + sc1: written through to / read from memory, past every L2)
// make the exchange correct whatever the placement, at a longer round trip.
constexpr int kAuxL2Load = 1;  // sc0
constexpr int kAuxSys = 17;    // sc0 + sc1
__device__ __forceinline__ void part_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 v, bool local) {
    const auto u = __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v);
    if (local) __builtin_amdgcn_raw_buffer_store_b128(u, r, (int)off, 0, 0);
    else __builtin_amdgcn_raw_buffer_store_b128(u, r, (int)off, 0, kAuxSys);
}
__device__ __forceinline__ float4 part_load4(__amdgpu_buffer_rsrc_t r, uint32_t off, bool local) {
    return __builtin_bit_cast(float4, local ? __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kAuxL2Load)
                                            : __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kAuxSys));
}

// Wait until this thread's stores have completed.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// One part of a tile is done: store it to its slot, count the arrival, and if
// it was the last, sum all parts in K order into `sf` (slot_of(q) gives the
// slot of part q) and return true. NA accumulators per thread of a TILE-float
// tile; `flag` is a workgroup-shared int. Called by every thread.
template <int NA, int TILE, class SlotOf>
__device__ __forceinline__ bool sk_finish_part(const SkSched &s, int nslots, int my_slot, int cnt_idx, int nparts,
                                               const float *accf, float *sf, int tid, int &flag,
                                               const SlotOf &slot_of) {
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(s.part, (uint32_t)nslots * (uint32_t)TILE * 4u);
    const uint32_t mine = ((uint32_t)my_slot * TILE + tid * NA) * 4u;
#pragma unroll
    for (int v = 0; v < NA / 4; ++v)
        part_store4(rp, mine + v * 16u, make_float4(accf[4 * v], accf[4 * v + 1], accf[4 * v + 2], accf[4 * v + 3]),
                    s.local);
    wait_stores();
    __syncthreads();
    if (tid == 0) flag = sk_arrive(s, cnt_idx, nparts) ? 1 : 0;
    __syncthreads();
    if (!flag) return false;
#pragma unroll
    for (int v = 0; v < NA; ++v) sf[v] = 0.f;
    // two parts' loads in flight at a time, added in K order
#pragma unroll 1
    for (int q = 0; q < nparts; q += 2) {
        const bool two = q + 1 < nparts;
        const uint32_t o0 = ((uint32_t)slot_of(q) * TILE + tid * NA) * 4u;
        const uint32_t o1 = two ? ((uint32_t)slot_of(q + 1) * TILE + tid * NA) * 4u : 0x80000000u;
        float4 p0[NA / 4], p1[NA / 4];
#pragma unroll
        for (int v = 0; v < NA / 4; ++v) {
            p0[v] = part_load4(rp, o0 + v * 16u, s.local);
            p1[v] = part_load4(rp, o1 + v * 16u, s.local); // past the end when !two: reads 0
        }
#pragma unroll
        for (int v = 0; v < NA / 4; ++v) {
            sf[4 * v] += p0[v].x;
            sf[4 * v + 1] += p0[v].y;
            sf[4 * v + 2] += p0[v].z;
            sf[4 * v + 3] += p0[v].w;
        }
        if (two) {
#pragma unroll
            for (int v = 0; v < NA / 4; ++v) {
                sf[4 * v] += p1[v].x;
                sf[4 * v + 1] += p1[v].y;
                sf[4 * v + 2] += p1[v].z;
                sf[4 * v + 3] += p1[v].w;
            }
        }
    }
    return true;
}

} // namespace spinn
