// Launch timer: HIP event pairs around kernel launches, for benchmark harnesses
// that need one kernel's device time out of a multi-kernel call.
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
thread_local int t_open = -1;  // index into g_pairs of the pair begun by this thread

}  // namespace

void timer_begin(int kernel, hipStream_t stream) {
    if (!(g_mask.load(std::memory_order_relaxed) & (1u << kernel))) return;
    std::lock_guard<std::mutex> lk(g_mu);
    Pair p;
    if (!g_spare.empty()) {
        p = g_spare.back();
        g_spare.pop_back();
    } else if (hipEventCreate(&p.start) != hipSuccess || hipEventCreate(&p.stop) != hipSuccess) {
        t_open = -1;
        return;
    }
    if (hipEventRecord(p.start, stream) != hipSuccess) {
        g_spare.push_back(p);
        t_open = -1;
        return;
    }
    p.kernel = kernel;
    g_pairs.push_back(p);
    t_open = static_cast<int>(g_pairs.size()) - 1;
}

void timer_end(int kernel, hipStream_t stream) {
    if (t_open < 0) return;
    std::lock_guard<std::mutex> lk(g_mu);
    if (t_open < static_cast<int>(g_pairs.size()) && g_pairs[t_open].kernel == kernel &&
        hipEventRecord(g_pairs[t_open].stop, stream) != hipSuccess)
        g_pairs[t_open].kernel = -1;  // unusable pair: left out of every reading
    t_open = -1;
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
        if (hipEventSynchronize(p.stop) != hipSuccess) return PRIME_ERR_HIP;
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
