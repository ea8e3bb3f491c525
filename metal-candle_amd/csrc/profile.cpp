#include "profile.hpp"

#include <atomic>
#include <mutex>
#include <vector>

namespace mc {
namespace prof {
namespace {

struct Entry {
    hipEvent_t begin = nullptr, end = nullptr;
    int kind = 0;
    double flops = 0, bytes = 0;
    bool pending = false;
};

struct Totals {
    double ms = 0, flops = 0, bytes = 0;
    long long launches = 0;
};

std::atomic<bool> g_on{false};
std::mutex g_mu;
std::vector<Entry> g_entries;   // event pairs, reused across collect() calls
size_t g_used = 0;              // entries recorded since the last collect()
Totals g_tot[kNumKinds];

constexpr size_t kMaxEntries = 1 << 16;

}  // namespace

bool enabled() { return g_on.load(std::memory_order_relaxed); }
void set_enabled(bool on) { g_on.store(on, std::memory_order_relaxed); }

Scope::Scope(Kind kind, hipStream_t stream, double flops, double bytes) : stream_(stream) {
    if (!enabled()) return;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_used >= kMaxEntries) return;  // record nothing past the cap
    if (g_used == g_entries.size()) {
        Entry e;
        // Timing-only events: no system-scope fence when they are recorded.
        // The default fence writes back and invalidates the caches at every
        // event, which slows the kernel that follows and adds a few
        // microseconds to every short scope.
        constexpr unsigned kFlags = hipEventDisableSystemFence;
        if (hipEventCreateWithFlags(&e.begin, kFlags) != hipSuccess ||
            hipEventCreateWithFlags(&e.end, kFlags) != hipSuccess)
            return;
        g_entries.push_back(e);
    }
    Entry& e = g_entries[g_used];
    if (hipEventRecord(e.begin, stream) != hipSuccess) return;
    e.kind = kind;
    e.flops = flops;
    e.bytes = bytes;
    e.pending = true;
    slot_ = (int)g_used++;
}

Scope::~Scope() {
    if (slot_ < 0) return;
    std::lock_guard<std::mutex> lk(g_mu);
    if (hipEventRecord(g_entries[slot_].end, stream_) != hipSuccess) g_entries[slot_].pending = false;
}

hipError_t collect() {
    std::lock_guard<std::mutex> lk(g_mu);
    hipError_t err = hipSuccess;
    for (size_t i = 0; i < g_used; ++i) {
        Entry& e = g_entries[i];
        if (!e.pending) continue;
        e.pending = false;
        hipError_t s = hipEventSynchronize(e.end);
        float ms = 0.f;
        if (s == hipSuccess) s = hipEventElapsedTime(&ms, e.begin, e.end);
        if (s != hipSuccess) {
            err = s;
            continue;
        }
        Totals& t = g_tot[e.kind];
        t.ms += ms;
        t.flops += e.flops;
        t.bytes += e.bytes;
        t.launches += 1;
    }
    g_used = 0;
    return err;
}

void read(int kind, double* ms, long long* launches, double* flops, double* bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    const Totals& t = g_tot[kind];
    if (ms) *ms = t.ms;
    if (launches) *launches = t.launches;
    if (flops) *flops = t.flops;
    if (bytes) *bytes = t.bytes;
}

void reset() {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& t : g_tot) t = Totals{};
    for (size_t i = 0; i < g_used; ++i) g_entries[i].pending = false;
    g_used = 0;
}

}  // namespace prof
}  // namespace mc
