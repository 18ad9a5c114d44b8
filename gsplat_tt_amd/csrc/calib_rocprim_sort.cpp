// calib_rocprim_sort.cpp - measurement aid, not part of the library: times
// rocPRIM's own radix_sort_pairs on the standalone sort workload (50M 64-bit
// keys, hi32 = Zipf(1.1) tile id over 5000 tiles, lo32 = fp32 bits of a
// log-uniform depth in [0.2, 100], payload = index; 45 key bits) so that the
// onesweep kernels in sort.hip can be compared with AMD's tuned library on the
// same machine. Prints one line per repetition and checks the result is a
// stable sort. Built by `make -C gsplat_tt_amd/csrc calib`.
#include <cstring>
#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#define CK(x)                                                                       \
    do {                                                                            \
        hipError_t e_ = (x);                                                        \
        if (e_ != hipSuccess) {                                                     \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            return 1;                                                               \
        }                                                                           \
    } while (0)

int main() {
    const size_t n = 50000000;
    const int tiles = 5000, end_bit = 45, reps = 6;
    std::vector<uint64_t> keys(n);
    std::vector<uint32_t> vals(n);
    std::mt19937_64 rng(4);
    std::vector<double> cdf(tiles);
    double s = 0.0;
    for (int i = 0; i < tiles; ++i) cdf[i] = (s += 1.0 / std::pow(i + 1.0, 1.1));
    for (auto& c : cdf) c /= s;
    std::uniform_real_distribution<double> U(0.0, 1.0);
    const double l0 = std::log(0.2), l1 = std::log(100.0);
    for (size_t i = 0; i < n; ++i) {
        uint64_t t = (uint64_t)(std::lower_bound(cdf.begin(), cdf.end(), U(rng)) - cdf.begin());
        t = std::min<uint64_t>(t, tiles - 1);
        const float d = (float)std::exp(l0 + U(rng) * (l1 - l0));
        uint32_t db;
        std::memcpy(&db, &d, 4);
        keys[i] = (t << 32) | db;
        vals[i] = (uint32_t)i;
    }
    uint64_t *k0, *k1;
    uint32_t *v0, *v1;
    CK(hipMalloc(&k0, n * 8));
    CK(hipMalloc(&k1, n * 8));
    CK(hipMalloc(&v0, n * 4));
    CK(hipMalloc(&v1, n * 4));
    CK(hipMemcpy(k0, keys.data(), n * 8, hipMemcpyHostToDevice));
    CK(hipMemcpy(v0, vals.data(), n * 4, hipMemcpyHostToDevice));
    size_t tmp_bytes = 0;
    CK(rocprim::radix_sort_pairs(nullptr, tmp_bytes, k0, k1, v0, v1, n, 0, end_bit));
    void* tmp;
    CK(hipMalloc(&tmp, tmp_bytes));
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    const double bytes = (double)n * (24 * 6 + 8);  // six 8-bit passes + one histogram read
    float best = 1e30f;
    for (int rep = 0; rep < reps; ++rep) {
        CK(hipEventRecord(a));
        CK(rocprim::radix_sort_pairs(tmp, tmp_bytes, k0, k1, v0, v1, n, 0, end_bit));
        CK(hipEventRecord(b));
        CK(hipEventSynchronize(b));
        float ms;
        CK(hipEventElapsedTime(&ms, a, b));
        if (rep > 0) best = std::min(best, ms);
        std::printf("rocprim::radix_sort_pairs 50M u64/u32, %d key bits: %.3f ms  %.2f Gkeys/s  "
                    "%.1f GB/s at N*(24*6+8) B = %.1f%% of 8 TB/s%s\n",
                    end_bit, ms, n / ms / 1e6, bytes / ms / 1e6, bytes / ms / 1e6 / 80.0,
                    rep == 0 ? "  (first call, excluded)" : "");
    }
    std::vector<uint64_t> out(n);
    std::vector<uint32_t> ov(n);
    CK(hipMemcpy(out.data(), k1, n * 8, hipMemcpyDeviceToHost));
    CK(hipMemcpy(ov.data(), v1, n * 4, hipMemcpyDeviceToHost));
    size_t unstable = 0;
    for (size_t i = 1; i < n; ++i)
        if (out[i] == out[i - 1] && ov[i] < ov[i - 1]) ++unstable;
    const bool sorted = std::is_sorted(out.begin(), out.end());
    std::printf("best %.3f ms (%.2f Gkeys/s, %.1f%% of 8 TB/s); sorted %d, stability violations %zu\n",
                best, n / best / 1e6, bytes / best / 1e6 / 80.0, (int)sorted, unstable);
    return (sorted && unstable == 0) ? 0 : 2;
}
