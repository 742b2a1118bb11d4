// postproc.hip - detector post-processing operators: ReduceMax, TopK,
// GatherElements, Tile, Cast and the integer forms of Div / Mod.
//
// These close the YOLOv10n graph after the decoded head (the exported
// v10 post-process: max class score per anchor, TopK 300 anchors, gather of
// their boxes and scores, TopK 300 over anchor x class, label = index mod nc,
// anchor = index / nc, final gather). All of them are small and latency-bound;
// each is one launch with coalesced loads where the layout allows.
#include "spinn_hip_internal.h"

namespace spinn {

namespace {

// ---------------------------------------------------------------------------
// ReduceMax over contiguous blocks (SPINN/run_time/ops/reduce/reduce_max.c:18-26).
// One wave per row: lanes read consecutive elements, then a shuffle tree keeps
// (value, index) with "strictly greater wins, equal values keep the lower
// index", which for NaN-free rows returns exactly the element the reference's
// in-order scan ends on (the first maximal one, -0.0 and +0.0 being equal).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void reduce_max_rows_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                              int64_t rows, int64_t block) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * block;
    float best = 0.f;
    int64_t bi = -1;
    for (int64_t j = lane; j < block; j += 64) {
        const float v = xr[j];
        if (bi < 0 || v > best) {
            best = v;
            bi = j;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int64_t oi = __shfl_xor(bi, off);
        const bool take = oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi));
        if (take) {
            best = ov;
            bi = oi;
        }
    }
    if (lane == 0) y[row] = xr[bi]; // the element itself (keeps the sign of a zero)
}

// Short rows (a detector's class scores, 80 per anchor): one thread per row,
// the reference's own scan - start from the first element, replace it by any
// later one that is strictly greater - in float4 steps when VEC.
template <bool VEC>
__global__ __launch_bounds__(256) void reduce_max_short_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                               int64_t rows, int block) {
    for (int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; row < rows;
         row += (int64_t)gridDim.x * blockDim.x) {
        const float *xr = x + row * block;
        float best = xr[0];
        if constexpr (VEC) {
            for (int j = 0; j < block; j += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(xr + j);
                if (v.x > best) best = v.x;
                if (v.y > best) best = v.y;
                if (v.z > best) best = v.z;
                if (v.w > best) best = v.w;
            }
        } else {
            for (int j = 1; j < block; ++j) {
                const float v = xr[j];
                if (v > best) best = v;
            }
        }
        y[row] = best;
    }
}

// Short rows of a multiple of 16 floats (a detector's 80 class scores): four
// lanes per row, each scanning a contiguous quarter in float4 steps with the
// reference's rule, then the quarters combined in index order (a later
// quarter's maximum replaces the running one only when strictly greater):
// for NaN-free rows the first maximal element, as the single scan finds it,
// with four times the threads (8400 rows at batch 1: 132 workgroups, not 33).
__global__ __launch_bounds__(256) void reduce_max_short4_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                                int64_t rows, int block) {
    const int64_t total = rows * 4;
    const int len = block >> 2; // a multiple of 4
    for (int64_t base = (int64_t)blockIdx.x * blockDim.x; base < total; base += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = base + threadIdx.x; // uniform trip count: every lane reaches the shuffles
        const bool live = t < total;
        const int64_t row = t >> 2;
        const int q = (int)(t & 3);
        float best = 0.f;
        if (live) {
            const float *xr = x + row * block + (int64_t)q * len;
            best = xr[0];
            for (int j = 0; j < len; j += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(xr + j);
                if (v.x > best) best = v.x;
                if (v.y > best) best = v.y;
                if (v.z > best) best = v.z;
                if (v.w > best) best = v.w;
            }
        }
        const int lead = (int)(threadIdx.x & 63) & ~3;
        const float b1 = __shfl(best, lead + 1, 64), b2 = __shfl(best, lead + 2, 64), b3 = __shfl(best, lead + 3, 64);
        if (live && q == 0) {
            float m = best;
            if (b1 > m) m = b1;
            if (b2 > m) m = b2;
            if (b3 > m) m = b3;
            y[row] = m;
        }
    }
}

// ---------------------------------------------------------------------------
// TopK (SPINN/run_time/ops/tensor/topk.c:20-89), one 1024-thread workgroup per row.
// Order: value descending, ties by ascending index - what the reference's stable
// qsort of (value, index) pairs under `a > b` produces for NaN-free rows.
//   1. radix select of the k-th largest order key, 8 bits per pass, LDS histogram;
//   2. compaction of the k winners: every key above the threshold, and the
//      lowest-index elements equal to it (block-wide prefix count in index order);
//   3. bitonic sort of the winners by (key desc, index asc), in registers and LDS.
// ---------------------------------------------------------------------------
constexpr int kTopkThreads = 1024;

__device__ __forceinline__ uint32_t order_key(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) == 0u) u = 0u;               // -0.0 == +0.0
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0u;    // NaN: below everything
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u); // larger float -> larger key
}

constexpr int kTopkWaves = kTopkThreads / 64;
constexpr int kTopkWaveSlots = 128; // sampled-threshold candidates one wave may hold
static_assert(kTopkThreads == SPINN_HIP_TOPK_MAX_K, "the sort holds one candidate per thread");
constexpr int kTopkBins = 257; // per-wave histograms, padded so equal bins of two waves sit in different banks

// Radix-select state shared by the workgroup.
struct TopkSel {
    uint32_t whist[kTopkWaves * kTopkBins];
    uint32_t hist[256];
    uint32_t prefix, mask, need, gt, eq_base;
    uint32_t wave_eq[kTopkWaves];
};

// Count this lane's element (when `match`) into its wave's histogram `wh`. When
// every matching lane of the wave falls in one bin (the usual case for the
// leading digit of scores in a narrow range) the wave adds its lane count with
// one atomic instead of 64 serialised ones. The lead lane's bin is read with
// readlane (the lane index is wave-uniform): no LDS round trip per element.
__device__ __forceinline__ void topk_count(bool match, uint32_t bin, int lane, uint32_t *wh) {
    const uint64_t act = __ballot(match);
    if (act) {
        const int lead = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)act) - 1);
        const uint32_t lead_bin = (uint32_t)__builtin_amdgcn_readlane((int)bin, lead);
        const uint64_t same = __ballot(match && bin == lead_bin);
        if (same == act) {
            if (lane == lead) atomicAdd(&wh[lead_bin], (uint32_t)__popcll(act));
        } else if (match) {
            atomicAdd(&wh[bin], 1u);
        }
    }
}

// After every element of the pass at `shift` is counted (a barrier behind the
// counting): sum the wave histograms and fix the digit of the need-th largest
// key. With above(b) the count of elements whose digit exceeds b, it is the one
// digit b where above(b) < need <= above(b) + hist[b]; thread t < 256 holds bin
// 255 - t, so above() is an exclusive prefix sum over t. Ends with a barrier.
__device__ __forceinline__ void topk_pick_digit(TopkSel &sh, int shift, uint32_t prefix, uint32_t mask, int tid,
                                                int lane, int wave) {
    for (int b = tid; b < 256; b += kTopkThreads) {
        uint32_t t = 0u;
#pragma unroll
        for (int w = 0; w < kTopkWaves; ++w) t += sh.whist[w * kTopkBins + b];
        sh.hist[b] = t;
    }
    __syncthreads();
    const uint32_t need = sh.need;
    const int b = 255 - tid;
    uint32_t v = 0u, incl = 0u;
    if (tid < 256) {
        v = sh.hist[b];
        incl = v;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t o = (uint32_t)__shfl_up((int)incl, off);
            if (lane >= off) incl += o;
        }
        if (lane == 63) sh.wave_eq[wave] = incl;
    }
    __syncthreads();
    if (tid < 256) {
        for (int w = 0; w < wave; ++w) incl += sh.wave_eq[w];
        const uint32_t above = incl - v;
        if (above < need && above + v >= need) {
            sh.need = need - above;
            sh.prefix = prefix | ((uint32_t)b << shift);
            sh.mask = mask | (255u << shift);
        }
    }
    __syncthreads();
}

// Bitonic network over P2 elements, descending, thread t holding element t in
// registers: a compare-exchange stage of stride < 64 pairs lanes of one wave
// (a shuffle), one of stride >= 64 goes through LDS (10 of the 55 stages for
// 1024), alternating between the two 1024-entry buffers xa and xb so that each
// needs one barrier (a buffer is rewritten only after the barrier of the next
// exchange, which every thread reaches after its read). Fully unrolled: no loop
// or branch between stages. Callers may still read xa / xb until the first
// exchange's leading barrier.
template <int P2>
__device__ __forceinline__ uint64_t bitonic_regs(uint64_t x, uint64_t *xa, uint64_t *xb, int tid) {
    int ex = 0; // LDS exchanges so far
#pragma unroll
    for (int size = 2; size <= P2; size <<= 1) {
        const bool desc = (tid & size) == 0;
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            uint64_t y;
            if (stride >= 64) {
                uint64_t *buf = (ex & 1) ? xb : xa;
                if (ex == 0) __syncthreads(); // the callers' reads of xa / xb are done
                buf[tid] = x;
                __syncthreads();
                y = buf[tid ^ stride];
                ++ex;
            } else {
                y = __shfl_xor(x, stride, 64);
            }
            const bool hi = ((tid & stride) == 0) == desc; // keep the larger one
            x = hi ? (x > y ? x : y) : (x < y ? x : y);
        }
    }
    return x;
}

// Sort count (<= 1024) elements descending, pads (0) last, then write the first
// k in that order as the row's values and indices. `x` is this thread's element
// (0 past count); xa and xb are the exchange buffers. The value is rebuilt from the
// order key except for zeros (whose sign the key drops) and NaNs, which are read
// back from the row.
__device__ __forceinline__ void topk_sort_store(uint64_t *xa, uint64_t *xb, uint64_t x, int count, int k, int tid,
                                                const float *xr, float *values, int64_t *indices) {
    if (count <= 64) x = bitonic_regs<64>(x, xa, xb, tid); // uniform branches
    else if (count <= 128) x = bitonic_regs<128>(x, xa, xb, tid);
    else if (count <= 256) x = bitonic_regs<256>(x, xa, xb, tid);
    else if (count <= 512) x = bitonic_regs<512>(x, xa, xb, tid);
    else x = bitonic_regs<1024>(x, xa, xb, tid);
    if (tid < k) {
        const uint32_t key = (uint32_t)(x >> 32);
        const uint32_t i = 0xffffffffu - (uint32_t)x;
        const uint32_t u = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
        const float v = (key == 0x80000000u || key == 0u) ? xr[i] : __uint_as_float(u);
        values[(int64_t)blockIdx.x * k + tid] = v;
        indices[(int64_t)blockIdx.x * k + tid] = (int64_t)i;
    }
}

// Rows of at most R * 1024 elements: each thread loads its R keys (element
// u * 1024 + tid) once, all loads in flight together, and every pass runs from
// registers. The threshold-equal elements are ranked in index order from
// per-(chunk, wave) counts with three barriers, instead of one block-wide count
// per chunk. Same keys, threshold and sort as topk_rows_kernel: identical output.
//
// Rows of at least 4096 elements with k <= 512 first try a sampled threshold:
// the q-th largest of 1024 keys spread over the row's full chunks (thread t
// samples element (t mod chunks) * 1024 + t), with q = e + 3 sqrt(e) + 2 for
// e = k * 1024 / n the sample's expected count above the k-th largest key, is
// bounded from below by the same radix select over one key per thread, three
// digits deep (T: that key with its low 8 bits cleared). When between k and
// 1024 keys of the row are >= T, they hold the row's top k (every key above
// the k-th largest one is >= T, and at least k keys are), so they alone are
// sorted: one pass of compares over the row writes each wave's candidates to
// its own 128 slots in index order, instead of four histogram passes and the
// threshold ranking. Otherwise (ties around T, or a sample that misjudged the
// row, or more than 128 candidates in one wave) the full selection below runs.
// Either way the output is the unique top k by (key desc, index asc).
template <int R>
__global__ __launch_bounds__(kTopkThreads) void topk_rows_reg_kernel(const float *__restrict__ x, int n, int k,
                                                                     float *__restrict__ values,
                                                                     int64_t *__restrict__ indices) {
    __shared__ TopkSel sh;
    __shared__ uint32_t ceq[R][kTopkWaves]; // threshold-equal elements per (chunk, wave)
    __shared__ uint32_t cbase[R];           // ... in the chunks before this one
    __shared__ uint64_t cand[SPINN_HIP_TOPK_MAX_K];
    __shared__ uint64_t wcand[kTopkWaves * kTopkWaveSlots]; // sampled-threshold candidates, per wave
    __shared__ uint32_t wcount[kTopkWaves];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const float *xr = x + (int64_t)blockIdx.x * n;
    uint32_t key[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int i = u * kTopkThreads + tid;
        key[u] = i < n ? order_key(xr[i]) : 0u;
    }
    if (n >= 4 * kTopkThreads && k <= 512) { // uniform
        const int chunks = n / kTopkThreads;
        const uint32_t skey = order_key(xr[(tid % chunks) * kTopkThreads + tid]);
        const float e = (float)k * (float)kTopkThreads / (float)n;
        const uint32_t q = min((uint32_t)kTopkThreads, (uint32_t)ceilf(e + 3.f * sqrtf(e)) + 2u);
        if (tid == 0) {
            sh.prefix = 0u;
            sh.mask = 0u;
            sh.need = q;
            sh.gt = 0u;
        }
        for (int shift = 24; shift >= 8; shift -= 8) {
            for (int b = tid; b < kTopkWaves * kTopkBins; b += kTopkThreads) sh.whist[b] = 0u;
            __syncthreads();
            const uint32_t prefix = sh.prefix, mask = sh.mask;
            topk_count((skey & mask) == prefix, (skey >> shift) & 255u, lane, sh.whist + wave * kTopkBins);
            __syncthreads();
            topk_pick_digit(sh, shift, prefix, mask, tid, lane, wave);
        }
        const uint32_t T = sh.prefix; // the q-th largest sample key with its low 8 bits cleared
        // this wave's keys >= T into its own slots, in index order
        uint64_t *const wc = wcand + wave * kTopkWaveSlots;
        uint32_t c = 0u;
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int i = u * kTopkThreads + tid;
            const bool take = i < n && key[u] >= T;
            const uint64_t tb = __ballot(take);
            const uint32_t pos = c + (uint32_t)__popcll(tb & ((1ull << lane) - 1ull));
            if (take && pos < (uint32_t)kTopkWaveSlots)
                wc[pos] = ((uint64_t)key[u] << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
            c += (uint32_t)__popcll(tb);
        }
        if (lane == 0) wcount[wave] = c;
        __syncthreads();
        // element tid of the waves' slots concatenated in wave order
        uint32_t total = 0u;
        int src = -1;
        bool fits = true;
#pragma unroll
        for (int w = 0; w < kTopkWaves; ++w) {
            const uint32_t cw = wcount[w];
            if ((uint32_t)tid >= total && (uint32_t)tid < total + cw) src = w * kTopkWaveSlots + (tid - (int)total);
            total += cw;
            fits = fits && cw <= (uint32_t)kTopkWaveSlots;
        }
        if (fits && total >= (uint32_t)k && total <= (uint32_t)SPINN_HIP_TOPK_MAX_K) { // uniform
            topk_sort_store(cand, wcand, src >= 0 ? wcand[src] : 0ull, (int)total, k, tid, xr, values, indices);
            return;
        }
        __syncthreads(); // every thread has read wcount before the full selection reuses the state
    }
    if (tid == 0) {
        sh.prefix = 0u;
        sh.mask = 0u;
        sh.need = (uint32_t)k;
        sh.gt = 0u;
    }
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int b = tid; b < kTopkWaves * kTopkBins; b += kTopkThreads) sh.whist[b] = 0u;
        __syncthreads();
        const uint32_t prefix = sh.prefix, mask = sh.mask;
        uint32_t *wh = sh.whist + wave * kTopkBins;
#pragma unroll
        for (int u = 0; u < R; ++u)
            if (u * kTopkThreads < n) // wave-uniform
                topk_count(u * kTopkThreads + tid < n && (key[u] & mask) == prefix, (key[u] >> shift) & 255u, lane,
                           wh);
        __syncthreads();
        topk_pick_digit(sh, shift, prefix, mask, tid, lane, wave);
    }
    const uint32_t thr = sh.prefix;   // key of the k-th largest element
    const uint32_t take_eq = sh.need; // how many elements equal to it are kept: the lowest-index ones
    const uint32_t n_gt = (uint32_t)k - take_eq;
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int i = u * kTopkThreads + tid;
        const bool valid = i < n;
        if (valid && key[u] > thr) {
            const uint32_t slot = atomicAdd(&sh.gt, 1u); // < n_gt by construction of thr
            if (slot < n_gt) cand[slot] = ((uint64_t)key[u] << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
        }
        const uint64_t eqb = __ballot(valid && key[u] == thr);
        if (lane == 0) ceq[u][wave] = (uint32_t)__popcll(eqb);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t t = 0u;
        for (int u = 0; u < R; ++u) {
            cbase[u] = t;
            for (int w = 0; w < kTopkWaves; ++w) t += ceq[u][w];
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int i = u * kTopkThreads + tid;
        const bool eq = i < n && key[u] == thr;
        const uint64_t eqb = __ballot(eq);
        if (eq) {
            uint32_t rank = cbase[u] + (uint32_t)__popcll(eqb & ((1ull << lane) - 1ull));
            for (int w = 0; w < wave; ++w) rank += ceq[u][w];
            if (rank < take_eq) cand[n_gt + rank] = ((uint64_t)key[u] << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
        }
    }
    __syncthreads();
    topk_sort_store(cand, wcand, tid < k ? cand[tid] : 0ull, k, k, tid, xr, values, indices);
}

__global__ __launch_bounds__(kTopkThreads) void topk_rows_kernel(const float *__restrict__ x, int64_t n, int k,
                                                                 float *__restrict__ values,
                                                                 int64_t *__restrict__ indices) {
    __shared__ TopkSel sh;
    __shared__ uint64_t cand[SPINN_HIP_TOPK_MAX_K];
    __shared__ uint64_t xb[SPINN_HIP_TOPK_MAX_K]; // the sort's second exchange buffer
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const float *xr = x + (int64_t)blockIdx.x * n;
    const int64_t nchunks = (n + kTopkThreads - 1) / kTopkThreads;

    // key of element c * 1024 + tid (chunk c), and whether it exists
    auto key_at = [&](int64_t c, bool &valid) -> uint32_t {
        const int64_t i = c * kTopkThreads + tid;
        valid = i < n;
        return valid ? order_key(xr[i]) : 0u;
    };

    if (tid == 0) {
        sh.prefix = 0u;
        sh.mask = 0u;
        sh.need = (uint32_t)k;
    }
    // 1. radix select, most significant digit first, each wave counting into
    // its own histogram.
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int b = tid; b < kTopkWaves * kTopkBins; b += kTopkThreads) sh.whist[b] = 0u;
        __syncthreads();
        const uint32_t prefix = sh.prefix, mask = sh.mask;
        uint32_t *wh = sh.whist + wave * kTopkBins;
        for (int64_t c0 = 0; c0 < nchunks; c0 += 4) {
            // four chunks' loads in flight before any is counted
            uint32_t kk[4];
            bool vv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) kk[u] = key_at(c0 + u, vv[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u) topk_count(vv[u] && (kk[u] & mask) == prefix, (kk[u] >> shift) & 255u, lane, wh);
        }
        __syncthreads();
        topk_pick_digit(sh, shift, prefix, mask, tid, lane, wave);
    }
    const uint32_t thr = sh.prefix;   // key of the k-th largest element
    const uint32_t take_eq = sh.need; // how many elements equal to it are kept
    const uint32_t n_gt = (uint32_t)k - take_eq;
    if (tid == 0) sh.gt = 0u;

    // 2. compaction. Slots only need to be distinct (step 3 orders by key and
    // index), so winners take slots with LDS atomics; what must follow index
    // order is which elements equal to the threshold are kept: the first
    // take_eq. A block-wide count per chunk of 1024 elements tells whether a
    // chunk's equal elements are all in, all out, or (one chunk) split, and
    // only that chunk ranks its equal elements exactly.
    if (tid == 0) sh.eq_base = 0u;
    __syncthreads();
    uint32_t cum = 0u; // equal elements in the chunks before this one (block-uniform)
    bool vnext;
    uint32_t knext = key_at(0, vnext);
    for (int64_t c = 0; c < nchunks; ++c) {
        const bool valid = vnext;
        const uint32_t key = knext;
        knext = key_at(c + 1, vnext); // next chunk's load in flight across this one's barriers
        const int64_t i = c * kTopkThreads + tid;
        const bool gt = valid && key > thr;
        const bool eq = valid && key == thr;
        const uint64_t packed = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
        const uint32_t cnt = (uint32_t)__syncthreads_count(eq);
        if (gt) {
            const uint32_t slot = atomicAdd(&sh.gt, 1u); // < n_gt by construction of thr
            if (slot < n_gt) cand[slot] = packed;
        }
        if (cum < take_eq) {
            if (cum + cnt <= take_eq) {
                if (eq) cand[n_gt + atomicAdd(&sh.eq_base, 1u)] = packed;
            } else {
                const uint64_t ball = __ballot(eq);
                if (lane == 0) sh.wave_eq[wave] = (uint32_t)__popcll(ball);
                __syncthreads();
                uint32_t rank = cum + (uint32_t)__popcll(ball & ((1ull << lane) - 1ull));
                for (int w = 0; w < wave; ++w) rank += sh.wave_eq[w];
                if (eq && rank < take_eq) cand[n_gt + rank] = packed;
            }
        }
        cum += cnt;
    }
    __syncthreads();

    // 3. bitonic sort, descending, and the output
    topk_sort_store(cand, xb, tid < k ? cand[tid] : 0ull, k, k, tid, xr, values, indices);
}

// ---------------------------------------------------------------------------
// GatherElements (SPINN/run_time/ops/tensor/gather_elements.c:36-73), one thread
// per output element.
// ---------------------------------------------------------------------------
struct GatherGeom {
    int ndim, axis;
    int64_t out_dims[8];
    int64_t in_strides[8];
    int64_t axis_dim;
};

template <typename IT>
__global__ __launch_bounds__(256) void gather_elements_kernel(const float *__restrict__ data,
                                                              const IT *__restrict__ idx, float *__restrict__ y,
                                                              int64_t total, GatherGeom g) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        int64_t gi = (int64_t)idx[e];
        if (gi < 0) gi += g.axis_dim;
        if (gi < 0 || gi >= g.axis_dim) gi = 0;
        int64_t rem = e, off = 0;
        for (int d = g.ndim - 1; d >= 0; --d) {
            const int64_t c = rem % g.out_dims[d];
            rem /= g.out_dims[d];
            off += (d == g.axis ? gi : c) * g.in_strides[d];
        }
        y[e] = data[off];
    }
}

// ---------------------------------------------------------------------------
// Tile (SPINN/run_time/ops/tensor/tile.c:45-62), one thread per output element.
// ---------------------------------------------------------------------------
struct TileGeom {
    int ndim;
    int64_t in_dims[8];
    int64_t out_dims[8];
    int64_t in_strides[8];
};

template <typename T>
__global__ __launch_bounds__(256) void tile_kernel(const T *__restrict__ x, T *__restrict__ y, int64_t total,
                                                   TileGeom g) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        int64_t rem = e, off = 0;
        for (int d = g.ndim - 1; d >= 0; --d) {
            const int64_t c = rem % g.out_dims[d];
            rem /= g.out_dims[d];
            off += (c % g.in_dims[d]) * g.in_strides[d];
        }
        y[e] = x[off];
    }
}

// ---------------------------------------------------------------------------
// Cast (SPINN/run_time/ops/tensor/cast.c:31-66) and integer Div / Mod
// (SPINN/run_time/ops/math/div.c:33-48, mod.c:18-45).
// ---------------------------------------------------------------------------
template <typename S, typename D>
__global__ __launch_bounds__(256) void cast_kernel(const S *__restrict__ x, D *__restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = (D)x[i];
}

template <typename T, int OP>
__global__ __launch_bounds__(256) void binary_int_kernel(const T *__restrict__ a, int64_t na, const T *__restrict__ b,
                                                         int64_t nb, T *__restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const T va = a[i % na], vb = b[i % nb];
        y[i] = vb != 0 ? (OP == SPINN_BINARY_DIV ? (T)(va / vb) : (T)(va % vb)) : (T)0;
    }
}

__global__ __launch_bounds__(256) void fmod_kernel(const float *__restrict__ a, int64_t na,
                                                   const float *__restrict__ b, int64_t nb, float *__restrict__ y,
                                                   int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = fmodf(a[i % na], b[i % nb]);
}

int grid_for(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 65536)); }

} // namespace

int reduce_max_rows(int64_t rows, int64_t block, const float *x, float *y, hipStream_t st) {
    if (block <= 256 && block % 16 == 0 && ((uintptr_t)x & 15u) == 0 && rows <= INT64_MAX / 4) {
        const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>((rows * 4 + 255) / 256, 65536)));
        hipLaunchKernelGGL(reduce_max_short4_kernel, grid, dim3(256), 0, st, x, y, rows, (int)block);
        return check_launch();
    }
    if (block <= 256) {
        const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>((rows + 255) / 256, 65536)));
        if (block % 4 == 0 && ((uintptr_t)x & 15u) == 0)
            hipLaunchKernelGGL(reduce_max_short_kernel<true>, grid, dim3(256), 0, st, x, y, rows, (int)block);
        else
            hipLaunchKernelGGL(reduce_max_short_kernel<false>, grid, dim3(256), 0, st, x, y, rows, (int)block);
        return check_launch();
    }
    hipLaunchKernelGGL(reduce_max_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, y, rows, block);
    return check_launch();
}

int topk_rows(int64_t rows, int64_t n, int k, const float *x, float *values, int64_t *indices, hipStream_t st) {
    const dim3 grid((unsigned)rows), block(kTopkThreads);
    if (n <= 8 * kTopkThreads)
        hipLaunchKernelGGL(topk_rows_reg_kernel<8>, grid, block, 0, st, x, (int)n, k, values, indices);
    else if (n <= 16 * kTopkThreads)
        hipLaunchKernelGGL(topk_rows_reg_kernel<16>, grid, block, 0, st, x, (int)n, k, values, indices);
    else if (n <= 32 * kTopkThreads)
        hipLaunchKernelGGL(topk_rows_reg_kernel<32>, grid, block, 0, st, x, (int)n, k, values, indices);
    else
        hipLaunchKernelGGL(topk_rows_kernel, dim3((unsigned)rows), dim3(kTopkThreads), 0, st, x, n, k, values, indices);
    return check_launch();
}

int gather_elements(const SpinnHipGatherDesc *d, const float *data, const void *indices, float *y, hipStream_t st) {
    GatherGeom g{};
    g.ndim = d->ndim;
    g.axis = d->axis;
    g.axis_dim = d->in_dims[d->axis];
    int64_t total = 1, stride = 1;
    for (int i = d->ndim - 1; i >= 0; --i) {
        g.out_dims[i] = d->out_dims[i];
        g.in_strides[i] = stride;
        stride *= d->in_dims[i];
        total *= d->out_dims[i];
    }
    if (d->index_dtype == ENNF_TYPE_INT64)
        hipLaunchKernelGGL(gather_elements_kernel<int64_t>, dim3(grid_for(total)), dim3(256), 0, st, data,
                           (const int64_t *)indices, y, total, g);
    else
        hipLaunchKernelGGL(gather_elements_kernel<int32_t>, dim3(grid_for(total)), dim3(256), 0, st, data,
                           (const int32_t *)indices, y, total, g);
    return check_launch();
}

int tile(int ndim, const int64_t *in_dims, const int64_t *out_dims, int elem_bytes, const void *x, void *y,
         hipStream_t st) {
    TileGeom g{};
    g.ndim = ndim;
    int64_t total = 1, stride = 1;
    for (int i = ndim - 1; i >= 0; --i) {
        g.in_dims[i] = in_dims[i];
        g.out_dims[i] = out_dims[i];
        g.in_strides[i] = stride;
        stride *= in_dims[i];
        total *= out_dims[i];
    }
    const dim3 grid(grid_for(total)), blk(256);
    switch (elem_bytes) {
    case 1: hipLaunchKernelGGL(tile_kernel<uint8_t>, grid, blk, 0, st, (const uint8_t *)x, (uint8_t *)y, total, g); break;
    case 2: hipLaunchKernelGGL(tile_kernel<uint16_t>, grid, blk, 0, st, (const uint16_t *)x, (uint16_t *)y, total, g); break;
    case 4: hipLaunchKernelGGL(tile_kernel<uint32_t>, grid, blk, 0, st, (const uint32_t *)x, (uint32_t *)y, total, g); break;
    default: hipLaunchKernelGGL(tile_kernel<uint64_t>, grid, blk, 0, st, (const uint64_t *)x, (uint64_t *)y, total, g); break;
    }
    return check_launch();
}

int cast(int src, int dst, int64_t n, const void *x, void *y, hipStream_t st) {
    const dim3 grid(grid_for(n)), blk(256);
    const int F = ENNF_TYPE_FLOAT32, I32 = ENNF_TYPE_INT32, I64 = ENNF_TYPE_INT64;
    if (src == dst) {
        const size_t bytes = (size_t)n * (src == I64 ? 8 : 4);
        return x == y ? 0 : hip_code(hipMemcpyAsync(y, x, bytes, hipMemcpyDeviceToDevice, st));
    }
    if (src == I64 && dst == F) hipLaunchKernelGGL((cast_kernel<int64_t, float>), grid, blk, 0, st, (const int64_t *)x, (float *)y, n);
    else if (src == I32 && dst == F) hipLaunchKernelGGL((cast_kernel<int32_t, float>), grid, blk, 0, st, (const int32_t *)x, (float *)y, n);
    else if (src == F && dst == I64) hipLaunchKernelGGL((cast_kernel<float, int64_t>), grid, blk, 0, st, (const float *)x, (int64_t *)y, n);
    else if (src == F && dst == I32) hipLaunchKernelGGL((cast_kernel<float, int32_t>), grid, blk, 0, st, (const float *)x, (int32_t *)y, n);
    else if (src == I64 && dst == I32) hipLaunchKernelGGL((cast_kernel<int64_t, int32_t>), grid, blk, 0, st, (const int64_t *)x, (int32_t *)y, n);
    else if (src == I32 && dst == I64) hipLaunchKernelGGL((cast_kernel<int32_t, int64_t>), grid, blk, 0, st, (const int32_t *)x, (int64_t *)y, n);
    else return SPINN_HIP_EUNSUPPORTED;
    return check_launch();
}

int binary_typed(int op, int dtype, const void *a, int64_t na, const void *b, int64_t nb, void *y, int64_t n,
                 hipStream_t st) {
    const dim3 grid(grid_for(n)), blk(256);
    if (dtype == ENNF_TYPE_FLOAT32) {
        if (op == SPINN_BINARY_MOD) {
            hipLaunchKernelGGL(fmod_kernel, grid, blk, 0, st, (const float *)a, na, (const float *)b, nb, (float *)y, n);
            return check_launch();
        }
        return binary_op(op, (const float *)a, na, (const float *)b, nb, (float *)y, n, st);
    }
    if (op != SPINN_BINARY_DIV && op != SPINN_BINARY_MOD) return SPINN_HIP_EUNSUPPORTED;
    if (dtype == ENNF_TYPE_INT64) {
        if (op == SPINN_BINARY_DIV)
            hipLaunchKernelGGL((binary_int_kernel<int64_t, SPINN_BINARY_DIV>), grid, blk, 0, st, (const int64_t *)a, na, (const int64_t *)b, nb, (int64_t *)y, n);
        else
            hipLaunchKernelGGL((binary_int_kernel<int64_t, SPINN_BINARY_MOD>), grid, blk, 0, st, (const int64_t *)a, na, (const int64_t *)b, nb, (int64_t *)y, n);
    } else if (dtype == ENNF_TYPE_INT32) {
        if (op == SPINN_BINARY_DIV)
            hipLaunchKernelGGL((binary_int_kernel<int32_t, SPINN_BINARY_DIV>), grid, blk, 0, st, (const int32_t *)a, na, (const int32_t *)b, nb, (int32_t *)y, n);
        else
            hipLaunchKernelGGL((binary_int_kernel<int32_t, SPINN_BINARY_MOD>), grid, blk, 0, st, (const int32_t *)a, na, (const int32_t *)b, nb, (int32_t *)y, n);
    } else {
        return SPINN_HIP_EUNSUPPORTED;
    }
    return check_launch();
}

} // namespace spinn
