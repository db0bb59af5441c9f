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

// Bandwidth probe: dst[i] = src[i] over n 16-byte words (read + write), or a
// read-only pass that folds every word into one XOR per workgroup (written to
// dst[blockIdx.x], so the loads cannot be dropped).  Nontemporal 16-byte loads
// and stores, a grid-stride loop with every wave's loads of one trip issued
// before its stores.
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t stream_word;

template <bool COPY>
__global__ __launch_bounds__(256) void hbm_stream_kernel(const stream_word *__restrict__ src,
                                                        stream_word *__restrict__ dst, int64_t n) {
    constexpr int U = 4;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    stream_word acc = {0u, 0u, 0u, 0u};
    for (; i + (U - 1) * stride < n; i += U * stride) {
        stream_word v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (COPY) __builtin_nontemporal_store(v[u], dst + i + u * stride);
            else acc ^= v[u];
        }
    }
    for (; i < n; i += stride) {
        const stream_word v = __builtin_nontemporal_load(src + i);
        if constexpr (COPY) __builtin_nontemporal_store(v, dst + i);
        else acc ^= v;
    }
    if constexpr (!COPY) {
        __shared__ stream_word red[256];
        red[threadIdx.x] = acc;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int t = 1; t < 256; ++t) acc ^= red[t];
            dst[blockIdx.x] = acc;
        }
    }
}

}  // namespace prime

extern "C" {

int prime_hbm_stream(const void *src, void *dst, size_t bytes, int copy, int blocks, void *stream) {
    if (!src || !dst || bytes == 0 || bytes % 16 || blocks <= 0 || (reinterpret_cast<uintptr_t>(src) & 15) ||
        (reinterpret_cast<uintptr_t>(dst) & 15))
        return PRIME_ERR_INVALID_ARG;
    const int64_t n = static_cast<int64_t>(bytes / 16);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (copy)
        hipLaunchKernelGGL((prime::hbm_stream_kernel<true>), dim3(blocks), dim3(256), 0, s,
                           static_cast<const prime::stream_word *>(src), static_cast<prime::stream_word *>(dst), n);
    else
        hipLaunchKernelGGL((prime::hbm_stream_kernel<false>), dim3(blocks), dim3(256), 0, s,
                           static_cast<const prime::stream_word *>(src), static_cast<prime::stream_word *>(dst), n);
    return hipGetLastError() == hipSuccess ? PRIME_OK : PRIME_ERR_HIP;
}

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
