// Launch timer: HIP event pairs stamped by the kernel dispatches themselves
// (hipExtLaunchKernelGGL), for benchmark harnesses that need one kernel's
// device time out of a multi-kernel call.
#include <atomic>
#include <mutex>
#include <vector>

#include "prime_kernels.h"

namespace prime {
namespace {

struct Pair {
    hipEvent_t start = nullptr, stop = nullptr;
    int kernel = -1;
};

std::atomic<unsigned> g_mask{0};
std::mutex g_mu;
std::vector<Pair> g_pairs;   // recorded since the last reset, in launch order
std::vector<Pair> g_spare;   // created events kept for reuse

}  // namespace

TimerEvents timer_events(int kernel) {
    TimerEvents t;
    if (!(g_mask.load(std::memory_order_relaxed) & (1u << kernel))) return t;
    std::lock_guard<std::mutex> lk(g_mu);
    Pair p;
    if (!g_spare.empty()) {
        p = g_spare.back();
        g_spare.pop_back();
    } else {
        if (hipEventCreate(&p.start) != hipSuccess) return t;  // untimed launch
        if (hipEventCreate(&p.stop) != hipSuccess) {
            (void)hipEventDestroy(p.start);
            return t;
        }
    }
    p.kernel = kernel;
    g_pairs.push_back(p);
    t.start = p.start;
    t.stop = p.stop;
    return t;
}

void timer_drop(const TimerEvents &t) {
    if (!t.start) return;
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto &p : g_pairs)
        if (p.start == t.start) p.kernel = -1;  // never recorded: left out of every reading
}

}  // namespace prime

extern "C" {

int prime_timer_enable(unsigned mask) {
    prime::g_mask.store(mask);
    return PRIME_OK;
}

int prime_timer_reset(void) {
    std::lock_guard<std::mutex> lk(prime::g_mu);
    for (auto &p : prime::g_pairs) {
        if (p.kernel >= 0 && hipEventSynchronize(p.stop) != hipSuccess) return PRIME_ERR_HIP;
        p.kernel = -1;
        prime::g_spare.push_back(p);
    }
    prime::g_pairs.clear();
    return PRIME_OK;
}

int prime_timer_read(int kernel, double *total_ms, int64_t *launches) {
    if (!total_ms || !launches || kernel < 0 || kernel >= PRIME_KERNEL_COUNT) return PRIME_ERR_INVALID_ARG;
    std::lock_guard<std::mutex> lk(prime::g_mu);
    double sum = 0.0;
    int64_t n = 0;
    for (const auto &p : prime::g_pairs) {
        if (p.kernel != kernel) continue;
        float ms = 0.f;
        if (hipEventSynchronize(p.stop) != hipSuccess || hipEventElapsedTime(&ms, p.start, p.stop) != hipSuccess)
            return PRIME_ERR_HIP;
        sum += ms;
        ++n;
    }
    *total_ms = sum;
    *launches = n;
    return PRIME_OK;
}

}  // extern "C"
