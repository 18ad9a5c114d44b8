// noalloc.hip - the standalone tile/depth sort with its per-tile ranges, with no
// device or host allocation: for callers that cannot allocate (tight serving
// loops, harnesses that forbid hipMalloc). It is not capturable into a HIP
// graph: it reads the error word back and waits for the stream, and its host
// bookkeeping of the look-back halves advances per call. A call on a stream
// that is capturing is refused (GS_E_INVALID) before anything is enqueued.
//
// Every scratch buffer of gs_sort_tile_depth_dev (the ping-pong key and value
// arrays, the look-back descriptors, the digit histograms and tickets, the
// control words) lives in one file-scope device array, `scratch`, sized for
// kNoallocMaxKeys keys. Each GPU the library runs on holds its own copy of it
// until the process ends; its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// used from the host. Calls on one GPU share the array, so calls that overlap
// on one GPU race; each call clears the parts that must start at zero.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "../../include/gsplat_hip.h"
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int64_t kNoallocMaxKeys = int64_t(1) << 20;
constexpr size_t kAlign = 256;
constexpr size_t align_up(size_t b) { return (b + kAlign - 1) / kAlign * kAlign; }

// Scratch layout for kNoallocMaxKeys keys: keys_alt (8 B/key), vals_alt
// (4 B/key), look-back descriptors (sort_partitions(n) x 256 x 8 B: 128 rows
// of 8192-key partitions), digit histograms + tickets (8 x 256 + 8 words),
// control words (2).
constexpr size_t kOffKeys = 0;
constexpr size_t kOffVals = align_up(kOffKeys + kNoallocMaxKeys * 8);
constexpr size_t kStateParts = (kNoallocMaxKeys + 8191) / 8192;
constexpr size_t kOffState = align_up(kOffVals + kNoallocMaxKeys * 4);
constexpr size_t kOffHist = align_up(kOffState + kStateParts * 256 * 8);
constexpr size_t kHistWords = 8 * 256 + 8;
constexpr size_t kOffCtl = align_up(kOffHist + kHistWords * 4);
constexpr size_t kScratchBytes = align_up(kOffCtl + 2 * 4);  // 12.5 MiB

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
struct DeviceScratch {
    unsigned char* ptr = nullptr;  // device address of `scratch` on this GPU
    SortTemp tmp;                  // host bookkeeping of its look-back halves
};
DeviceScratch g_dev[kMaxDevices];
std::once_flag g_once[kMaxDevices];
hipError_t g_init_err[kMaxDevices] = {};

int tile_bits_of(int64_t num_tiles) {
    int b = 0;
    while ((int64_t(1) << b) < num_tiles) ++b;
    return std::max(b, 1);
}

// First call on a device (that device current): the array's address, and the
// look-back descriptors cleared (they must start at zero; later passes keep
// them so, see SortTemp).
void init_device(int dev, hipStream_t st) {
    DeviceScratch& d = g_dev[dev];
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess)
        e = launch_fill_u32(reinterpret_cast<uint32_t*>(static_cast<unsigned char*>(p) + kOffState),
                            0u, kStateParts * 256 * 2, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess) {
        d.ptr = static_cast<unsigned char*>(p);
        d.tmp.keys_alt = d.ptr + kOffKeys;
        d.tmp.vals_alt = reinterpret_cast<uint32_t*>(d.ptr + kOffVals);
        d.tmp.state = reinterpret_cast<uint64_t*>(d.ptr + kOffState);
        d.tmp.hist = reinterpret_cast<uint32_t*>(d.ptr + kOffHist);
        d.tmp.state_parts = kStateParts;
        d.tmp.ctl = reinterpret_cast<uint32_t*>(d.ptr + kOffCtl);
    }
    g_init_err[dev] = e;
}

int fail(int code, const std::string& msg) {
    set_last_error(msg.c_str());
    return code;
}

}  // namespace
}  // namespace gs

extern "C" int gs_sort_tile_depth_noalloc(gs_ctx* ctx, uint64_t* keys, uint32_t* vals, int64_t n,
                                          int64_t num_tiles, uint32_t* tile_ranges,
                                          int* passes_out) {
    using namespace gs;
    if (ctx == nullptr || keys == nullptr || vals == nullptr || tile_ranges == nullptr)
        return fail(GS_E_INVALID, "sort_tile_depth_noalloc: null argument");
    if (n < 0 || n > kNoallocMaxKeys)
        return fail(GS_E_CAPACITY, "sort_tile_depth_noalloc: n = " + std::to_string(n) +
                                       " is beyond the scratch array's " +
                                       std::to_string(kNoallocMaxKeys) + " keys");
    if (num_tiles < 1 || num_tiles > (int64_t(1) << 31))
        return fail(GS_E_INVALID, "sort_tile_depth_noalloc: num_tiles out of range");
    const CtxInfo ci = ctx_info(ctx);
    if (ci.device < 0 || ci.device >= kMaxDevices)
        return fail(GS_E_INVALID, "sort_tile_depth_noalloc: device index out of range");
    hipError_t e = hipSetDevice(ci.device);
    if (e != hipSuccess) return fail(GS_E_DEVICE, std::string("hipSetDevice: ") + hipGetErrorString(e));
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(ci.stream, &cap);
    if (e != hipSuccess)
        return fail(GS_E_DEVICE, std::string("hipStreamIsCapturing: ") + hipGetErrorString(e));
    if (cap != hipStreamCaptureStatusNone)
        return fail(GS_E_INVALID, "sort_tile_depth_noalloc: the context's stream is capturing a "
                                  "graph; this call waits for the stream and cannot be captured");
    std::call_once(g_once[ci.device], init_device, ci.device, ci.stream);
    if (g_init_err[ci.device] != hipSuccess)
        return fail(GS_E_DEVICE, std::string("sort_tile_depth_noalloc: scratch set-up: ") +
                                     hipGetErrorString(g_init_err[ci.device]));
    DeviceScratch& d = g_dev[ci.device];
    SortTemp& tmp = d.tmp;
    hipStream_t st = ci.stream;
    const int end_bit = 32 + tile_bits_of(num_tiles);
    const int npass = (end_bit + 7) / 8;
    uint32_t* tickets = tmp.hist + (size_t)8 * 256;
    // histograms, tickets and control words start at zero
    e = launch_fill_u32(tmp.hist, 0u, kHistWords, st);
    if (e == hipSuccess) e = launch_fill_u32(tmp.ctl, 0u, 2, st);
    void* kf = keys;
    uint32_t* vf = vals;
    if (e == hipSuccess && n > 0)
        e = radix_sort_pairs_dev_chain(keys, vals, n, 0, end_bit, tmp.hist, tickets, tmp, st,
                                       &kf, &vf);
    if (e == hipSuccess && kf != keys) {
        e = hipMemcpyAsync(keys, kf, (size_t)n * 8, hipMemcpyDeviceToDevice, st);
        if (e == hipSuccess)
            e = hipMemcpyAsync(vals, vf, (size_t)n * 4, hipMemcpyDeviceToDevice, st);
    }
    if (e == hipSuccess)
        e = launch_tile_bounds64(keys, (uint32_t)n, tile_ranges, num_tiles, tmp.ctl, st);
    uint32_t flags = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&flags, tmp.ctl, 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return fail(GS_E_DEVICE, std::string("sort_tile_depth_noalloc: ") + hipGetErrorString(e));
    if (flags & kErrKeyRange)
        return fail(GS_E_INVALID, "sort_tile_depth_noalloc: a key's tile id is >= num_tiles");
    if (flags != 0u)
        return fail(GS_E_DEVICE, "sort_tile_depth_noalloc: a bounded look-back wait gave up "
                                 "(outputs discarded)");
    if (passes_out) *passes_out = n > 0 ? npass : 0;
    return GS_OK;
}
