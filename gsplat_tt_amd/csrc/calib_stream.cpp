// calib_stream.cpp - streaming-rate calibration of one GPU (a measurement aid,
// not linked into the library): how fast plain kernels move HBM when nothing
// but streaming is asked of them, next to the device-to-device copy of the HIP
// runtime. Each kernel moves 1 GiB (copy: 1 GiB read + 1 GiB written) in
// 16-byte lanes, each workgroup taking U consecutive 4 KiB blocks; the best and
// the median of 10 timed launches (after 2 warm-ups) are printed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <vector>

#define CHECK(x)                                                                    \
    do {                                                                            \
        hipError_t e_ = (x);                                                        \
        if (e_ != hipSuccess) {                                                     \
            std::printf("%s failed: %s\n", #x, hipGetErrorString(e_));             \
            return 1;                                                               \
        }                                                                           \
    } while (0)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;

// Copy, plain or with non-temporal loads and stores (NT).
template <int U, bool NT>
__global__ __launch_bounds__(kThreads) void k_copy(const u32x4* __restrict__ a,
                                                   u32x4* __restrict__ b, size_t n) {
    const size_t i0 = (size_t)blockIdx.x * kThreads * U + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = i0 + (size_t)u * kThreads;
        if (i < n) v[u] = NT ? __builtin_nontemporal_load(a + i) : a[i];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = i0 + (size_t)u * kThreads;
        if (i >= n) continue;
        if (NT)
            __builtin_nontemporal_store(v[u], b + i);
        else
            b[i] = v[u];
    }
}

// Read only: the words are folded into one value that is stored only if it
// matches a sentinel (so the loads are not optimised away).
template <int U>
__global__ __launch_bounds__(kThreads) void k_read(const u32x4* __restrict__ a, uint32_t* out,
                                                   size_t n) {
    const size_t i0 = (size_t)blockIdx.x * kThreads * U + threadIdx.x;
    uint32_t x = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = i0 + (size_t)u * kThreads;
        if (i < n) {
            const u32x4 v = a[i];
            x ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
    if (x == 0x9E3779B9u) out[0] = x;
}

// Write only.
template <int U>
__global__ __launch_bounds__(kThreads) void k_write(u32x4* __restrict__ b, size_t n) {
    const size_t i0 = (size_t)blockIdx.x * kThreads * U + threadIdx.x;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = i0 + (size_t)u * kThreads;
        if (i < n) b[i] = u32x4{(uint32_t)i, (uint32_t)u, 1u, 2u};
    }
}

int main() {
    const size_t bytes = (size_t)1 << 30, n = bytes / 16;
    u32x4 *a = nullptr, *b = nullptr;
    uint32_t* sink = nullptr;
    CHECK(hipMalloc(&a, bytes));
    CHECK(hipMalloc(&b, bytes));
    CHECK(hipMalloc(&sink, 64));
    CHECK(hipMemset(a, 1, bytes));
    CHECK(hipMemset(b, 0, bytes));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    auto grid = [&](int u) { return (unsigned)((n + (size_t)kThreads * u - 1) / ((size_t)kThreads * u)); };
    auto run = [&](const char* name, double moved, auto launch) -> int {
        std::vector<float> ms;
        for (int r = 0; r < 12; ++r) {
            CHECK(hipEventRecord(e0));
            launch();
            CHECK(hipGetLastError());
            CHECK(hipEventRecord(e1));
            CHECK(hipEventSynchronize(e1));
            float t = 0.0f;
            CHECK(hipEventElapsedTime(&t, e0, e1));
            if (r >= 2) ms.push_back(t);
        }
        std::sort(ms.begin(), ms.end());
        const float best = ms.front(), med = ms[ms.size() / 2];
        std::printf("%-28s best %7.1f us  median %7.1f us  -> %5.0f GB/s (median %5.0f)\n", name,
                    best * 1e3, med * 1e3, moved / best / 1e6, moved / med / 1e6);
        std::fflush(stdout);
        return 0;
    };
    const double two = 2.0 * (double)bytes, one = (double)bytes;
    if (run("copy, 2 blocks/wg", two, [&] { k_copy<2, false><<<grid(2), kThreads>>>(a, b, n); })) return 1;
    if (run("copy, 4 blocks/wg", two, [&] { k_copy<4, false><<<grid(4), kThreads>>>(a, b, n); })) return 1;
    if (run("copy nontemporal, 2 blocks", two, [&] { k_copy<2, true><<<grid(2), kThreads>>>(a, b, n); })) return 1;
    if (run("copy nontemporal, 4 blocks", two, [&] { k_copy<4, true><<<grid(4), kThreads>>>(a, b, n); })) return 1;
    if (run("read, 4 blocks/wg", one, [&] { k_read<4><<<grid(4), kThreads>>>(a, sink, n); })) return 1;
    if (run("write, 4 blocks/wg", one, [&] { k_write<4><<<grid(4), kThreads>>>(b, n); })) return 1;
    if (run("hipMemcpyAsync device-device", two,
            [&] { (void)hipMemcpyAsync(b, a, bytes, hipMemcpyDeviceToDevice, 0); }))
        return 1;
    CHECK(hipDeviceSynchronize());
    CHECK(hipFree(a));
    CHECK(hipFree(b));
    CHECK(hipFree(sink));
    return 0;
}
