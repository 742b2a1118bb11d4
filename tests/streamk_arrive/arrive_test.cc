// Host unit test of the stream-K arrival protocol (spinn_amd/csrc/sk_arrive.h),
// the same template the conv kernel instantiates over system-scope HIP atomics,
// here over std::atomic. Prints one line per case and exits non-zero on the
// first failure.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>

#define SK_HOST_DEVICE
#include "sk_arrive.h"

using spinn::sk_arrive_count;
using spinn::sk_arrive_outcome;

namespace {

struct AtomicOps {
    std::atomic<uint64_t> *p;
    uint64_t load() { return p->load(std::memory_order_relaxed); }
    uint64_t fetch_add(uint64_t d) { return p->fetch_add(d, std::memory_order_relaxed); }
    bool cas(uint64_t &e, uint64_t d) { return p->compare_exchange_strong(e, d, std::memory_order_relaxed); }
};

// One part's arrival as the kernel makes it: count, outcome, reset by the last.
int arrive(std::atomic<uint64_t> &c, uint64_t epoch, int nparts, int tries = 4) {
    AtomicOps ops{&c};
    const int o = sk_arrive_outcome(sk_arrive_count(ops, epoch, tries), nparts);
    if (o == 1) c.store(epoch << 16, std::memory_order_relaxed);
    return o;
}

int g_fail = 0;
void check(bool ok, const char *what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
    if (!ok) g_fail = 1;
}

// Sequential arrivals of n parts on a counter starting at `start`.
bool sequential(uint64_t start, uint64_t epoch, int n) {
    std::atomic<uint64_t> c{start};
    for (int i = 0; i < n; ++i) {
        const int o = arrive(c, epoch, n);
        if (o != (i == n - 1 ? 1 : 0)) return false;
    }
    return c.load() == (epoch << 16);
}

// A counter another part changes between this part's load and its exchange:
// the first exchange fails and the second round must add.
struct RacedOps {
    std::atomic<uint64_t> *p;
    uint64_t epoch;
    bool raced = false;
    uint64_t load() { return p->load(); }
    uint64_t fetch_add(uint64_t d) { return p->fetch_add(d); }
    bool cas(uint64_t &e, uint64_t d) {
        if (!raced) { // the other part installs the epoch first
            raced = true;
            uint64_t g = p->load();
            p->compare_exchange_strong(g, (epoch << 16) | 1ull);
        }
        return p->compare_exchange_strong(e, d);
    }
};

// A counter something else rewrites with a foreign epoch on every access.
struct HostileOps {
    uint64_t state = 0x123456789abcdefull;
    uint64_t next() { return state = state * 6364136223846793005ull + 1442695040888963407ull; }
    uint64_t load() { return next(); }
    uint64_t fetch_add(uint64_t) { return next(); }
    bool cas(uint64_t &e, uint64_t) { e = next(); return false; }
};

} // namespace

int main() {
    const uint64_t epoch = 0xBEEF12345678ull;
    check(sequential(0, epoch, 1), "one part on a zero counter is the last");
    check(sequential(0xDEADBEEFCAFEF00Dull, epoch, 3), "3 parts on a garbage counter: 0, 0, last; reset to zero count");
    check(sequential(((epoch - 1) << 16) | 7, epoch, 8), "8 parts on an earlier launch's counter");
    check(sequential(epoch << 16, epoch, 5), "graph replay: same epoch, zero count");
    {
        std::atomic<uint64_t> c{(epoch << 16) | 2};
        const int o = arrive(c, epoch, 2);
        check(o == -1, "same epoch with a stale count past the parts: reported (-1)");
    }
    {
        std::atomic<uint64_t> c{0};
        check(arrive(c, epoch, 2, 0) == -1, "no rounds allowed (test hook): reported (-1)");
    }
    {
        std::atomic<uint64_t> c{0x42};
        RacedOps ops{&c, epoch};
        const int count = sk_arrive_count(ops, epoch, 2);
        check(count == 2, "exchange lost to another part's install: second round adds (count 2)");
    }
    {
        HostileOps ops;
        check(sk_arrive_count(ops, epoch, 4) == -1, "counter rewritten on every access: gives up after 4 rounds");
    }
    {
        // concurrent parts on fresh garbage each round: exactly one last part,
        // counts 1..n each once, nobody reports a failure
        std::mt19937_64 rng(7);
        bool ok = true;
        for (int round = 0; round < 300 && ok; ++round) {
            const int n = 2 + round % 7;
            const uint64_t ep = (epoch + 1 + round) & ((1ull << 48) - 1);
            std::atomic<uint64_t> c{rng()};
            std::atomic<int> go{0};
            std::vector<int> counts(n, 0);
            std::vector<std::thread> th;
            for (int t = 0; t < n; ++t)
                th.emplace_back([&, t]() {
                    while (!go.load()) {
                    }
                    AtomicOps ops{&c};
                    counts[t] = sk_arrive_count(ops, ep, 4);
                });
            go.store(1);
            for (auto &x : th) x.join();
            std::vector<int> seen(n + 1, 0);
            int lasts = 0;
            for (int v : counts) {
                if (v < 1 || v > n || seen[v]++) ok = false;
                if (sk_arrive_outcome(v, n) == 1) ++lasts;
                if (sk_arrive_outcome(v, n) < 0) ok = false;
            }
            ok = ok && lasts == 1;
        }
        check(ok, "300 rounds of 2-8 concurrent parts on garbage counters");
    }
    return g_fail;
}
