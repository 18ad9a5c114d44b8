// gs_common.h - device helpers shared by the gfx950 kernels: wave64 scans,
// decoupled look-back, coherent (agent-scope) loads/stores, launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gs_internal.h"

#define GS_WAVE 64

namespace gs {

// Agent-scope relaxed accesses: visible across the eight XCD L2s of one GPU.
template <typename T>
__device__ __forceinline__ T ld_agent(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_agent(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t lanemask_lt() {
    const int l = lane_id();
    return (l == 0) ? 0ull : (~0ull >> (64 - l));
}

// Inclusive wave-wide prefix sum of a 32-bit value (Hillis-Steele over shfl_up).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    const int l = lane_id();
#pragma unroll
    for (int o = 1; o < GS_WAVE; o <<= 1) {
        const uint32_t u = __shfl_up(v, o, GS_WAVE);
        if (l >= o) v += u;
    }
    return v;
}

__device__ __forceinline__ uint64_t wave_incl_scan64(uint64_t v) {
    const int l = lane_id();
#pragma unroll
    for (int o = 1; o < GS_WAVE; o <<= 1) {
        const uint64_t u = __shfl_up(v, o, GS_WAVE);
        if (l >= o) v += u;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, GS_WAVE);
    return v;
}

// LDS histogram increment of `bin` for the lanes with `on` set: the lanes whose
// bin equals lane 0's add as one atomic (a skewed digit would otherwise
// serialise up to 64 lanes on one LDS address). Call from uniform control flow.
__device__ __forceinline__ void hist_add_wave(uint32_t* hist, uint32_t bin, bool on) {
    const uint32_t b0 = __builtin_amdgcn_readfirstlane(bin);
    const uint64_t same = __ballot(on && bin == b0);
    if (on && bin != b0) atomicAdd(&hist[bin], 1u);
    if (lane_id() == 0 && same != 0ull) atomicAdd(&hist[b0], (uint32_t)__popcll(same));
}

// ---------------------------------------------------------------------------
// Tile rectangle of a projected Gaussian (src/gsplat_cpu/tile_assign.cpp:60-102):
// (centre -+ radius) / tile_size as a float division, truncated toward zero,
// clamped to the tile grid. For a power-of-two tile size the quotient is an
// exact scaling by 2^-k, which the product with the (exact) reciprocal
// reproduces bit for bit, denormals included; other sizes divide.
// ---------------------------------------------------------------------------
struct TsDiv {
    float ts, inv;
    bool pow2;
};
__device__ __forceinline__ TsDiv ts_div(int tile_size) {
    TsDiv d;
    d.ts = (float)tile_size;
    d.pow2 = tile_size > 0 && (tile_size & (tile_size - 1)) == 0;
    d.inv = d.pow2 ? 1.0f / d.ts : 0.0f;
    return d;
}
__device__ __forceinline__ float div_ts(float x, const TsDiv& d) {
    if (d.pow2) return x * d.inv;
    return x / d.ts;
}

struct Rect {
    int x0, x1, y0, y1;
};
// r = (px, py, rx, ry)
__device__ __forceinline__ Rect tile_rect(float4 r, int tiles_x, int tiles_y, const TsDiv& d) {
    Rect o;
    o.x0 = max(0, min((int)div_ts(r.x - r.z, d), tiles_x - 1));
    o.x1 = max(0, min((int)div_ts(r.x + r.z, d), tiles_x - 1));
    o.y0 = max(0, min((int)div_ts(r.y - r.w, d), tiles_y - 1));
    o.y1 = max(0, min((int)div_ts(r.y + r.w, d), tiles_y - 1));
    return o;
}

// Depth-sort values of the frame: compact index in the low idx_bits bits, the
// Gaussian's tile count above them, saturated at the field's largest value
// (which, like a zero field, means "not held: read the rectangle").
// idx_bits 0: plain compact indices.
__device__ __forceinline__ uint32_t dval_index(uint32_t v, int idx_bits) {
    return idx_bits ? (v & ((1u << idx_bits) - 1u)) : v;
}
__device__ __forceinline__ uint32_t dval_count(uint32_t v, int idx_bits) {
    if (idx_bits == 0) return 0u;
    const uint32_t c = v >> idx_bits;
    return c == (0xFFFFFFFFu >> idx_bits) ? 0u : c;
}
__device__ __forceinline__ uint32_t dval_pack(uint32_t m, uint32_t count, int idx_bits) {
    const uint32_t sat = 0xFFFFFFFFu >> idx_bits;
    return m | ((count < sat ? count : sat) << idx_bits);
}

// ---------------------------------------------------------------------------
// Control words of a launch (ctl, may be null): ctl[0] collects error flags
// (kErrLookback: a bounded look-back wait gave up, so a prefix may be wrong),
// ctl[1] is the wait's spin limit (0: kLbMaxSpins). The host clears ctl[0]
// before the launches and turns a nonzero value into an error status.
// ---------------------------------------------------------------------------
constexpr uint32_t kLbMaxSpins = 1u << 20;  // about 0.45 s of polls (kLbSleep below)
// Back-off between polls of an unpublished predecessor (s_sleep units of 64
// clocks). With frames in flight the waiting waves share their SIMDs with
// other frames' kernels; polling every ~0.4 us instead of every ~27 ns gives
// those kernels the issue slots (orbit 997 -> 1007 frames/s; 4: 1006, 64: 993).
constexpr int kLbSleep = 16;

// Read only when a wait happens, with a plain load (the host wrote it before
// the launch): an atomic load of one address by every wave would serialise.
__device__ __forceinline__ uint32_t spin_limit(const uint32_t* ctl) {
    const uint32_t v = ctl != nullptr ? ctl[1] : 0u;
    return v != 0u ? v : kLbMaxSpins;
}
__device__ __forceinline__ void report_error(uint32_t* ctl, uint32_t bits) {
    if (ctl != nullptr) __hip_atomic_fetch_or(ctl, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// True once a launch earlier in the sequence raised an error flag. Kernels
// whose indices come from a look-back result (compaction slots, scan offsets,
// sorted ids) return at once then, before taking a ticket: their inputs may
// be wrong, so they write nothing and read nothing through them, and the host
// reports the error.
// A plain load: a flag that matters here was raised by an earlier launch, and
// launch boundaries make it visible (an agent-scope atomic load of the one
// address by every workgroup would serialise on it).
// fp32 -> bf16 bits, round to nearest even (a NaN stays a quiet NaN), as
// torch's float -> bfloat16 conversion rounds.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}

__device__ __forceinline__ bool upstream_failed(const uint32_t* ctl) {
    return ctl != nullptr && *ctl != 0u;
}

// ---------------------------------------------------------------------------
// Decoupled look-back over a chain of 64-bit partition descriptors.
// Descriptor = flag (2 bits, 62..63) | value (62 bits). flag 0 = not yet
// published, 1 = aggregate of this partition only, 2 = inclusive prefix.
// The caller is one full wave (all 64 lanes) of the partition with virtual id
// `vid` (taken from an atomic ticket, so every predecessor is already
// resident and never waits on us). Returns the exclusive prefix. The wait for
// an unpublished predecessor is bounded: after spin_limit(ctl) rounds the wave
// goes on with what it has and flags kErrLookback in ctl[0].
// ---------------------------------------------------------------------------
constexpr uint64_t kLbAgg = 1ull << 62;
constexpr uint64_t kLbInc = 2ull << 62;
constexpr uint64_t kLbVal = (1ull << 62) - 1;

// The first half of lookback_exclusive: publishes the partition's aggregate
// (partition 0: its inclusive prefix), so that successors can walk past it
// while this partition does other work before its own walk.
__device__ __forceinline__ void lookback_publish(uint64_t* state, uint32_t vid,
                                                 uint64_t aggregate) {
    if (lane_id() == 0) st_agent(&state[vid], (vid == 0 ? kLbInc : kLbAgg) | aggregate);
}

// The second half: the walk over the predecessors, then the inclusive prefix.
__device__ __forceinline__ uint64_t lookback_walk(uint64_t* state, uint32_t vid,
                                                  uint64_t aggregate, uint32_t* ctl) {
    const int l = lane_id();
    if (vid == 0) return 0;
    uint32_t limit = 0;  // read at the first wait
    uint64_t excl = 0;
    int64_t base = (int64_t)vid - 1;
    uint32_t spins = 0;
    bool gave_up = false;
    while (true) {
        const int64_t idx = base - l;
        uint64_t s = (idx >= 0) ? ld_agent(&state[idx]) : (kLbInc | 0ull);
        const uint64_t flag = s >> 62;
        const uint64_t inc_mask = __ballot(flag == 2);
        const uint64_t rdy_mask = __ballot(flag != 0);
        // lanes [0, first_inc] are needed (all 64 when no inclusive seen)
        uint64_t need;
        if (inc_mask) {
            const int first = __ffsll((unsigned long long)inc_mask) - 1;
            need = (first == 63) ? ~0ull : ((2ull << first) - 1);
        } else {
            need = ~0ull;
        }
        if ((rdy_mask & need) != need) {
            // predecessors are resident (ticket order), so this only trips on
            // a broken chain or a host-set tiny limit: report, never hang
            if (limit == 0) limit = spin_limit(ctl);
            if (++spins < limit) {
                __builtin_amdgcn_s_sleep(kLbSleep);
                continue;
            }
            gave_up = true;
        }
        uint64_t v = ((need >> l) & 1ull) ? (s & kLbVal) : 0ull;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, GS_WAVE);
        excl += v;
        if (inc_mask) break;
        base -= GS_WAVE;
    }
    if (l == 0) {
        if (gave_up) report_error(ctl, kErrLookback);
        st_agent(&state[vid], kLbInc | (excl + aggregate));
    }
    return excl;
}

__device__ __forceinline__ uint64_t lookback_exclusive(uint64_t* state, uint32_t vid,
                                                      uint64_t aggregate, uint32_t* ctl) {
    lookback_publish(state, vid, aggregate);
    return lookback_walk(state, vid, aggregate, ctl);
}

}  // namespace gs

// Host-side launch check: every launcher returns hipError_t.
#define GS_LAUNCH_CHECK() hipGetLastError()
