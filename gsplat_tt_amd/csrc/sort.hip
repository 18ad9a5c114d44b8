// sort.hip - stable onesweep LSD radix sort of (key, u32 value) pairs on gfx950.
//
// One upsweep pass builds the digit histograms of every pass at once; each
// digit pass is then a single kernel (Adinets & Merrill, "Onesweep", 2022):
//   * an 8192-key partition per 1024-thread workgroup (64-bit keys staged in
//     LDS without their values), partitions taken in order from an atomic
//     ticket so look-back only waits on resident predecessors;
//   * wave64 stable ranking with 8 ballots per key (peer mask of equal digits)
//     plus per-wave digit counters in LDS;
//   * per-digit decoupled look-back, walked after the partition has published
//     its counts and re-ordered its keys in LDS (32-bit descriptors in two
//     alternating halves, each pass clearing the next one's; epoch-tagged
//     64-bit descriptors above 2^30 keys);
//   * keys re-ordered by digit in LDS and written out in digit runs, so global
//     stores are contiguous per digit.
// Stability across passes makes the whole sort stable, which is what the
// reference's per-tile depth sort requires (src/gsplat_cpu/sort.cpp:24-85,
// ties keep input order).
#include <algorithm>
#include <utility>

#include "gs_common.h"
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kWaves = 4;  // waves of the 256-thread histogram / scan blocks
constexpr int kHistThreads = 256;
constexpr int kMaxPasses = 8;
constexpr int kLbBatch = 4;  // predecessors read per look-back round trip

// descriptor: [63:34] epoch, [33:32] flag (1 aggregate, 2 inclusive), [31:0] value
__device__ __forceinline__ uint64_t make_desc(uint32_t epoch, uint32_t flag, uint32_t v) {
    return ((uint64_t)epoch << 34) | ((uint64_t)flag << 32) | v;
}

// Look-back descriptors. 32-bit: [31:30] flag, [29:0] count, the array cleared
// before every pass (key counts below 2^30). 64-bit: the epoch tag above, never
// cleared.
template <bool D32> struct Desc;
template <> struct Desc<true> {
    using T = uint32_t;
    __device__ static T make(uint32_t, uint32_t flag, uint32_t v) { return (flag << 30) | v; }
    __device__ static uint32_t flag(T s, uint32_t) { return s >> 30; }
    __device__ static uint32_t val(T s) { return s & 0x3FFFFFFFu; }
};
template <> struct Desc<false> {
    using T = uint64_t;
    __device__ static T make(uint32_t e, uint32_t flag, uint32_t v) { return make_desc(e, flag, v); }
    __device__ static uint32_t flag(T s, uint32_t e) {
        return (uint32_t)(s >> 34) == e ? (uint32_t)(s >> 32) & 3u : 0u;
    }
    __device__ static uint32_t val(T s) { return (uint32_t)s; }
};

template <typename K>
__device__ __forceinline__ uint32_t digit_of(K k, int shift, uint32_t mask) {
    return (uint32_t)(k >> shift) & mask;
}

// Exclusive scan of one value per thread over a 256-thread block.
__device__ __forceinline__ uint32_t block_excl_scan256(uint32_t v, uint32_t* s_tmp) {
    const int w = threadIdx.x / GS_WAVE;
    const int lane = lane_id();
    const uint32_t incl = wave_incl_scan(v);
    if (lane == GS_WAVE - 1) s_tmp[w] = incl;
    __syncthreads();
    uint32_t pre = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i)
        if (i < w) pre += s_tmp[i];
    __syncthreads();
    return pre + incl - v;
}

// Digit histograms of up to NP passes in one read of the keys. Eight keys per
// thread per step keep enough loads in flight (four: 90.6 us for 50M 64-bit
// keys, eight: 81.3, sixteen: 79.9); per wave and pass, the lanes
// whose digit equals lane 0's add as one (skewed digits, e.g. the high bits of
// Zipf tile ids, would otherwise serialise up to 64 lanes on one LDS bin).
// The bins take NP x 4 KB of LDS: one pass's fit eight workgroups per CU, so
// the whole grid is resident at once.
constexpr int kHistItems = 8;
template <typename K, int NP = kMaxPasses>
__global__ __launch_bounds__(kHistThreads) void k_hist(const K* __restrict__ keys, int64_t n,
                                                       int begin_bit, int end_bit, int npass,
                                                       int dw, uint32_t* __restrict__ g_hist) {
    __shared__ uint32_t h[kWaves][NP][256];
    const int w = threadIdx.x / GS_WAVE;
    const int lane = lane_id();
    for (int i = threadIdx.x; i < kWaves * NP * 256; i += kHistThreads)
        (&h[0][0][0])[i] = 0;
    __syncthreads();
    constexpr int64_t kStep = (int64_t)kHistThreads * kHistItems;
    const int64_t stride = (int64_t)gridDim.x * kStep;
    // the loop bound is uniform over the workgroup, so every lane takes part in
    // the ballots; lanes past n carry ok = false
    for (int64_t base = (int64_t)blockIdx.x * kStep; base < n; base += stride) {
        K k[kHistItems];
        bool ok[kHistItems];
#pragma unroll
        for (int it = 0; it < kHistItems; ++it) {
            const int64_t i = base + it * kHistThreads + threadIdx.x;
            ok[it] = i < n;
            k[it] = ok[it] ? keys[i] : K(0);
        }
        // passes outside, items inside: the items' digit tests of one pass are
        // independent and interleave
        for (int p = 0; p < min(npass, NP); ++p) {
            const int shift = begin_bit + dw * p;
            const uint32_t mask = (1u << min(dw, end_bit - shift)) - 1u;
            uint32_t d[kHistItems], d0[kHistItems];
            uint64_t same[kHistItems];
#pragma unroll
            for (int it = 0; it < kHistItems; ++it) {
                d[it] = digit_of(k[it], shift, mask);
                d0[it] = __builtin_amdgcn_readfirstlane(d[it]);
                same[it] = __ballot(ok[it] && d[it] == d0[it]);
            }
#pragma unroll
            for (int it = 0; it < kHistItems; ++it) {
                if (ok[it] && d[it] != d0[it]) atomicAdd(&h[w][p][d[it]], 1u);
                if (lane == 0 && same[it] != 0ull)
                    atomicAdd(&h[w][p][d0[it]], (uint32_t)__popcll(same[it]));
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < min(npass, NP) * 256; i += kHistThreads) {
        const int p = i / 256, d = i % 256;
        uint32_t s = 0;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) s += h[ww][p][d];
        if (s) atomicAdd(&g_hist[p * 256 + d], s);
    }
}

// Per-digit decoupled look-back of partition vid (one thread per digit), in two
// steps so that the partition's local work runs between them:
// digit_publish makes the partition's count `agg` for the digit visible
// (already inclusive for the first partition); digit_walk then walks back
// kLbBatch predecessors per round trip (independent loads: one memory latency
// covers the batch) until an inclusive prefix, publishes its own inclusive
// prefix and returns the exclusive one.
template <typename D, typename DT>
__device__ __forceinline__ void digit_publish(DT* state, uint32_t vid, int digit, uint32_t agg,
                                              uint32_t epoch) {
    st_agent(&state[(size_t)vid * 256 + digit], D::make(epoch, vid == 0 ? 2u : 1u, agg));
}

template <typename D, typename DT>
__device__ __forceinline__ uint32_t digit_walk(DT* state, uint32_t vid, int digit, uint32_t agg,
                                               uint32_t epoch, uint32_t* ctl) {
    if (vid == 0) return 0u;
    uint32_t limit = 0;  // read at the first wait
    uint32_t excl = 0;
    int64_t j = (int64_t)vid - 1;
    uint32_t spins = 0;
    bool done = false;
    while (!done) {
        DT sv[kLbBatch];
#pragma unroll
        for (int q = 0; q < kLbBatch; ++q)
            sv[q] = (j - q >= 0) ? ld_agent(&state[(size_t)(j - q) * 256 + digit])
                                 : D::make(epoch, 2u, 0u);
        int used = 0;
#pragma unroll
        for (int q = 0; q < kLbBatch; ++q) {
            if (done || used < q) continue;  // stop at the first gap
            const uint32_t flag = D::flag(sv[q], epoch);
            if (flag == 0u) continue;
            excl += D::val(sv[q]);
            ++used;
            if (flag == 2u) done = true;
        }
        j -= used;
        if (!done && used < kLbBatch) {
            // bounded wait (see lookback_exclusive): never hang the GPU; a
            // give-up is reported to the host through ctl
            if (limit == 0) limit = spin_limit(ctl);
            if (++spins < limit) {
                __builtin_amdgcn_s_sleep(kLbSleep);
            } else {
                report_error(ctl, kErrLookback);
                done = true;
            }
        }
    }
    st_agent(&state[(size_t)vid * 256 + digit], D::make(epoch, 2u, excl + agg));
    return excl;
}

// DROP: keys equal to kPairDrop are left out (not ranked, not written): the
// pass stably compacts the kept keys while it sorts them.
// SPLIT: the keys are re-ordered in LDS and written out first, then the values
// in the same LDS space, so a partition holds only its keys in LDS (larger
// partitions, fewer look-back links).
// RUNS (the last pass of a sort whose keys' high bits index run_cnt): the
// sorted keys are not written; instead every run of equal key >> run_shift in
// the partition (the last pass leaves a partition sorted by all the key bits
// in LDS) adds its length to run_cnt[key >> run_shift], with at most two
// atomics per run.
// part_offs (optional, 2^bits words per partition): partition vid's keys of
// digit d start at part_offs[vid << bits | d] of the output (the digit's base
// plus the kept keys of that digit in all earlier partitions, counted by the
// keys' producer): the partition neither publishes nor walks back.
// NARROW (64-bit keys, split partitions): each key and its value leave as one
// 64-bit word, (key >> out_shift) << val_bits | value (the key bits the later
// passes still read, above the value; vout is not written). The words are
// staged in LDS instead of the keys, so an element's digit, gone from its
// word, is found from the partition's digit offsets (a start digit per 32
// elements, then a short forward scan). A key bit lost off the word's top
// flags kErrKeyRange, a value >= val_limit (when not 0) kErrValRange, in
// *key_err (val_limit <= 2^val_bits).
// KONLY (64-bit keys, split partitions): the keys carry their values (the
// words NARROW writes); vin is not read and, unless RUNS, vout not written.
// A RUNS run at or past run_limit flags kErrKeyRange in *key_err instead of
// counting; with KONLY the low val_bits bits of each sorted key go to vout.
// key_err (nullable) is not the control word:
// partitions of the same pass that start after the flag still sort and
// publish (every access stays in bounds whatever the keys), so no look-back
// wait is left to run into its limit.
template <typename K, bool IOTA, int THREADS, int ITEMS, bool D32, bool DROP, bool SPLIT,
          bool RUNS, bool NARROW = false, bool KONLY = false>
__global__ __launch_bounds__(THREADS) void k_onesweep(
    const K* __restrict__ kin, const uint32_t* __restrict__ vin, K* __restrict__ kout,
    uint32_t* __restrict__ vout, int64_t n_cap, const uint32_t* __restrict__ n_dev, int shift,
    int bits, const uint32_t* __restrict__ g_hist_pass, void* __restrict__ state_raw,
    uint32_t* __restrict__ ticket, uint32_t epoch, uint32_t* __restrict__ clear_next,
    uint32_t* ctl, uint32_t* __restrict__ next_hist, int next_shift, int next_bits,
    uint32_t* __restrict__ run_cnt, const uint32_t* __restrict__ part_offs, int out_shift,
    int run_shift, uint32_t run_limit, uint32_t* key_err, int val_bits, uint32_t val_limit) {
    static_assert(!NARROW || (sizeof(K) == 8 && SPLIT && !RUNS && !KONLY),
                  "narrowing: 64-bit split passes");
    static_assert(!KONLY || (sizeof(K) == 8 && SPLIT && !IOTA && !DROP),
                  "keys with their values: 64-bit split passes");
    using D = Desc<D32>;
    using DT = typename D::T;
    DT* state = static_cast<DT*>(state_raw);
    constexpr int WAVES = THREADS / GS_WAVE;
    constexpr int PART = THREADS * ITEMS;
    static_assert(THREADS >= 256, "one thread per digit");
    __shared__ uint32_t s_vid, s_count;
    // per-wave digit counts and their prefixes are below PART <= 65535: 16-bit
    // counters halve this table, which leaves room for 8192 u32 keys per
    // partition at two workgroups per CU
    static_assert(PART <= 65535, "16-bit wave counters");
    using WC = uint16_t;
    __shared__ WC s_wcnt[WAVES][256];
    __shared__ uint32_t s_loff[256];
    __shared__ uint32_t s_gpos[256];
    __shared__ uint32_t s_tmp[2][4];
    __shared__ uint32_t s_nh[256];  // next pass's digit counts (next_hist given)
    __shared__ uint8_t s_blk[NARROW ? PART / 32 : 1];  // NARROW: digit of element 32 b
    __shared__ K s_keys[PART];
    __shared__ uint32_t s_vals_own[SPLIT ? 1 : PART];
    uint32_t* const s_vals = SPLIT ? reinterpret_cast<uint32_t*>(s_keys) : s_vals_own;

    const int tid = threadIdx.x;
    const int w = tid / GS_WAVE;
    const int lane = lane_id();
    const uint32_t mask = (1u << bits) - 1u;

    if (tid == 0) s_vid = atomicAdd(ticket, 1u);
    // this workgroup's row of the descriptors that the next pass uses
    if (clear_next != nullptr && tid < 256) clear_next[(size_t)blockIdx.x * 256 + tid] = 0u;
    for (int i = tid; i < WAVES * 256; i += THREADS) (&s_wcnt[0][0])[i] = 0;
    if (next_hist != nullptr && tid < 256) s_nh[tid] = 0u;
    // A pass whose digit is the same for all n keys (one histogram bin holds
    // them all, e.g. the exponent byte of depths within one binade) leaves the
    // order as it is, the sort being stable: every partition then copies its
    // keys in place, with no ranking and no look-back (all partitions see the
    // same histogram, so none waits on another). The first four waves vote,
    // one ballot each.
    constexpr bool kIdentityOk = !DROP && !RUNS && !NARROW && !KONLY;
    __shared__ uint32_t s_vote[kIdentityOk ? 4 : 1];
    if constexpr (kIdentityOk) {
        if (tid < 256) {
            const int64_t nn = n_dev ? min(n_cap, (int64_t)*n_dev) : n_cap;
            const bool v = next_hist == nullptr && part_offs == nullptr &&
                           (int64_t)g_hist_pass[tid] == nn;
            const uint64_t b = __ballot(v);
            if (lane == 0) s_vote[w] = b != 0ull ? 1u : 0u;
        }
    }
    __syncthreads();
    bool identity = false;
    if constexpr (kIdentityOk) identity = (s_vote[0] | s_vote[1] | s_vote[2] | s_vote[3]) != 0u;
    const uint32_t vid = s_vid;
    // after an earlier give-up or a capacity overflow the keys may be partial:
    // sort nothing (this workgroup's row of the next pass's descriptors is
    // cleared above all the same)
    if (__builtin_amdgcn_readfirstlane(upstream_failed(ctl) ? 1 : 0)) return;
    const int64_t part_base = (int64_t)vid * PART;
    // grid sized for a capacity; the key count may be known only on the device
    const int64_t n = n_dev ? min(n_cap, (int64_t)*n_dev) : n_cap;
    if (part_base >= n) return;  // tickets are in order: no later partition has keys
    const int64_t wave_base = part_base + (int64_t)w * (ITEMS * GS_WAVE);
    if (identity) {
#pragma unroll
        for (int it = 0; it < ITEMS; ++it) {
            const int64_t idx = wave_base + it * GS_WAVE + lane;
            if (idx < n) {
                if (kout != nullptr) kout[idx] = kin[idx];
                vout[idx] = IOTA ? (uint32_t)idx : vin[idx];
            }
        }
        return;
    }

    K key[ITEMS];
    uint32_t val[ITEMS];
    uint32_t rank[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t idx = wave_base + it * GS_WAVE + lane;
        if (idx < n) {
            key[it] = kin[idx];
            val[it] = KONLY ? 0u : IOTA ? (uint32_t)idx : vin[idx];
        } else {
            key[it] = 0;
            val[it] = 0;
        }
    }

    // Stable wave ranking: peers = lanes with the same digit (8 ballots);
    // rank = earlier items of this wave with that digit + lower peer lanes.
    const uint64_t lt = lanemask_lt();
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t idx = wave_base + it * GS_WAVE + lane;
        rank[it] = 0;
        if (idx < n && !(DROP && key[it] == (K)kPairDrop)) {
            const uint32_t d = digit_of(key[it], shift, mask);
            // all 8 bit planes, unrolled: a narrower last digit has zeros
            // above its width in every lane, whose planes change nothing.
            // x = the lane's bit b as 0 / all-ones; the lanes whose bit b
            // differs from this lane's are ballot ^ x, collected in `diff` by
            // one three-input op per half (diff | (ballot ^ x): truth table
            // 0xF6 over the inputs' 0xF0 / 0xCC / 0xAA planes).
            uint32_t diff_lo = 0u, diff_hi = 0u;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const uint32_t x = (uint32_t)__builtin_amdgcn_sbfe((int32_t)d, b, 1);
                const uint64_t bb = __ballot(x != 0u);
                diff_lo = __builtin_amdgcn_bitop3_b32(diff_lo, (uint32_t)bb, x, 0xF6);
                diff_hi = __builtin_amdgcn_bitop3_b32(diff_hi, (uint32_t)(bb >> 32), x, 0xF6);
            }
            const uint64_t peers =
                __ballot(1) & ~(((uint64_t)diff_hi << 32) | (uint64_t)diff_lo);
            const uint32_t before = s_wcnt[w][d];
            rank[it] = before + (uint32_t)__popcll(peers & lt);
            // every peer stores the same new count (no leader election)
            s_wcnt[w][d] = (WC)(before + (uint32_t)__popcll(peers));
        }
    }
    __syncthreads();

    // Threads 0..255 own one digit each: per-wave exclusive offsets and the
    // digit total of this partition, published at once for later partitions.
    // A digit absent from the whole pass publishes nothing and looks back at
    // nothing (all partitions agree: the histogram is global).
    uint32_t tot = 0;
    const bool has_digit = part_offs == nullptr && tid < 256 && g_hist_pass[tid] != 0u;
    if (tid < 256) {
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) {
            const uint32_t c = s_wcnt[ww][tid];
            s_wcnt[ww][tid] = (WC)tot;
            tot += c;
        }
        if (has_digit) digit_publish<D, DT>(state, vid, tid, tot, epoch);
    }
    // Exclusive scans over the 256 digits: partition-local offsets (tot) and
    // global digit bases (histogram of this pass).
    const uint32_t v1 = (tid < 256) ? tot : 0u;
    const uint32_t v2 = (tid < 256) ? g_hist_pass[tid] : 0u;
    const uint32_t i1 = wave_incl_scan(v1);
    const uint32_t i2 = wave_incl_scan(v2);
    if (lane == GS_WAVE - 1 && w < 4) {
        s_tmp[0][w] = i1;
        s_tmp[1][w] = i2;
    }
    __syncthreads();
    uint32_t loff = 0, gbase = 0;
    if (tid < 256) {
        uint32_t p1 = 0, p2 = 0;
        for (int ww = 0; ww < w; ++ww) {
            p1 += s_tmp[0][ww];
            p2 += s_tmp[1][ww];
        }
        loff = p1 + i1 - v1;
        gbase = p2 + i2 - v2;
        s_loff[tid] = loff;
        if (tid == 255) s_count = p1 + i1;  // keys of this partition (kept ones)
    }
    __syncthreads();

    // keys re-ordered by digit in LDS while predecessors publish their prefixes
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int64_t idx = wave_base + it * GS_WAVE + lane;
        if (idx < n && !(DROP && key[it] == (K)kPairDrop)) {
            const uint32_t d = digit_of(key[it], shift, mask);
            const uint32_t lp = s_loff[d] + s_wcnt[w][d] + rank[it];
            if (lp < (uint32_t)PART) {
                if constexpr (NARROW) {
                    const uint64_t kk = (uint64_t)key[it] >> out_shift;
                    if ((kk >> (64 - val_bits)) != 0u) report_error(key_err, kErrKeyRange);
                    if (val_limit != 0u && val[it] >= val_limit) report_error(key_err, kErrValRange);
                    s_keys[lp] = (K)((kk << val_bits) | val[it]);
                } else {
                    s_keys[lp] = key[it];
                }
                if (!SPLIT) s_vals[lp] = val[it];
            }
        }
    }
    if (NARROW && tid < 256) {
        // digit tid's elements are [s_loff[tid], next digit's offset): it owns
        // the 32-element blocks that start inside that range
        const uint32_t lo = s_loff[tid], hi = tid == 255 ? s_count : s_loff[tid + 1];
        for (uint32_t b = (lo + 31u) >> 5; (b << 5) < hi; ++b) s_blk[b] = (uint8_t)tid;
    }
    if (tid < 256) {
        if (part_offs != nullptr) {
            s_gpos[tid] = tid <= (int)mask ? part_offs[((size_t)vid << bits) | tid] - loff : 0u;
        } else {
            const uint32_t excl =
                has_digit ? digit_walk<D, DT>(state, vid, tid, tot, epoch, ctl) : 0u;
            s_gpos[tid] = gbase + excl - loff;
        }
    }
    if (next_hist != nullptr) {
        // the next pass's digit histogram from the keys in registers: the
        // waves that do not walk count while the first four walk
        const uint32_t nmask = (1u << next_bits) - 1u;
#pragma unroll
        for (int it = 0; it < ITEMS; ++it) {
            const int64_t idx = wave_base + it * GS_WAVE + lane;
            const bool on = idx < n && !(DROP && key[it] == (K)kPairDrop);
            hist_add_wave(s_nh, digit_of(key[it], next_shift, nmask), on);
        }
    }
    __syncthreads();
    if (next_hist != nullptr && tid < 256 && s_nh[tid] != 0u) atomicAdd(&next_hist[tid], s_nh[tid]);
    const int64_t cnt64 = n - part_base;
    const int count = DROP ? (int)min(s_count, (uint32_t)PART) : (cnt64 < PART ? (int)cnt64 : PART);
    if constexpr (!SPLIT) {
        for (int j = tid; j < count; j += THREADS) {
            const K k = s_keys[j];
            const uint32_t d = digit_of(k, shift, mask);
            const uint32_t g = s_gpos[d] + (uint32_t)j;
            if ((int64_t)g < n) {
                if (!RUNS && kout != nullptr) kout[g] = k;
                vout[g] = s_vals[j];
            }
            if (RUNS) {
                // run [a, b) of key k: + b at its last key, - a at its first
                // (modulo 2^32; a run of one adds 1)
                const K r = k >> run_shift;
                const bool first = j == 0 || (s_keys[j - 1] >> run_shift) != r;
                const bool last = j == count - 1 || (s_keys[j + 1] >> run_shift) != r;
                const uint32_t delta = (last ? (uint32_t)j + 1u : 0u) - (first ? (uint32_t)j : 0u);
                if (first || last) {
                    if (r < (K)run_limit) atomicAdd(&run_cnt[(uint32_t)r], delta);
                    else report_error(key_err, kErrKeyRange);
                }
            }
        }
    } else {
        constexpr int OUT = (PART + THREADS - 1) / THREADS;
        uint32_t gq[OUT];
#pragma unroll
        for (int q = 0; q < OUT; ++q) {
            const int j = tid + q * THREADS;
            gq[q] = 0xFFFFFFFFu;
            if (j < count) {
                const K k = s_keys[j];
                uint32_t d;
                if constexpr (NARROW) {
                    d = s_blk[j >> 5];
                    while (d < 255u && s_loff[d + 1] <= (uint32_t)j) ++d;
                } else {
                    d = digit_of(k, shift, mask);
                }
                const uint32_t g = s_gpos[d] + (uint32_t)j;
                gq[q] = g;
                if (!RUNS && kout != nullptr && (int64_t)g < n) kout[g] = k;
                if (KONLY && RUNS && (int64_t)g < n)
                    vout[g] = (uint32_t)k & (uint32_t)(0xFFFFFFFFull >> (32 - val_bits));
                if (RUNS) {
                    // run [a, b) of key k: + b at its last key, - a at its first
                    const K r = k >> run_shift;
                    const bool first = j == 0 || (s_keys[j - 1] >> run_shift) != r;
                    const bool last = j == count - 1 || (s_keys[j + 1] >> run_shift) != r;
                    const uint32_t delta =
                        (last ? (uint32_t)j + 1u : 0u) - (first ? (uint32_t)j : 0u);
                    if (first || last) {
                        if (r < (K)run_limit) atomicAdd(&run_cnt[(uint32_t)r], delta);
                        else report_error(key_err, kErrKeyRange);
                    }
                }
            }
        }
        if constexpr (KONLY || NARROW) return;  // the values left with the keys
        __syncthreads();  // the keys are out: their LDS space takes the values
#pragma unroll
        for (int it = 0; it < ITEMS; ++it) {
            const int64_t idx = wave_base + it * GS_WAVE + lane;
            if (idx < n && !(DROP && key[it] == (K)kPairDrop)) {
                const uint32_t d = digit_of(key[it], shift, mask);
                const uint32_t lp = s_loff[d] + s_wcnt[w][d] + rank[it];
                if (lp < (uint32_t)PART) s_vals[lp] = val[it];
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < OUT; ++q) {
            const int j = tid + q * THREADS;
            if (j < count && (int64_t)gq[q] < n) vout[gq[q]] = s_vals[j];
        }
    }
}

// Partition shapes (LDS: the staged keys (+ values unless split) and the 16
// per-wave digit counters must leave room for two workgroups per CU, and at
// most 64 VGPRs keep eight waves per SIMD). 64-bit keys: 8192 per partition,
// split (5120 unsplit: 2.37 -> 2.04 ms of passes on 50M keys). 32-bit keys:
// 8192, not split; 10240 split made the frame's tile sort 5 % faster alone
// but the orbit with frames in flight 2 % slower.
struct Sweep64 { static constexpr int T = 1024, I = 8; static constexpr bool SPLIT = true; };
struct Sweep32 { static constexpr int T = 1024, I = 8; static constexpr bool SPLIT = false; };
constexpr int kMinPart = Sweep32::T * Sweep32::I;  // the smallest partition of all shapes
static_assert(kMinPart == (int)kSortPartition32, "first-pass offsets index these partitions");
static_assert(kMinPart <= Sweep64::T * Sweep64::I, "kMinPart sizes the look-back state");

// Up to kFillRanges fills in one launch: range r is n[r] words at p[r] set to
// v[r] (one thread per word of the concatenated ranges).
constexpr int kFillRanges = 6;
struct FillRanges {
    uint32_t* p[kFillRanges];
    uint32_t v[kFillRanges];
    uint32_t n[kFillRanges];
};
__global__ void k_fill_ranges(FillRanges f) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
#pragma unroll
    for (int r = 0; r < kFillRanges; ++r) {
        if (i < f.n[r]) {
            f.p[r][i] = f.v[r];
            return;
        }
        i -= f.n[r];
    }
}

__global__ void k_fill_u32(uint32_t* p, uint32_t v, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_iota_u32(uint32_t* p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = (uint32_t)i;
}

// How a pass writes its keys: narrow (64-bit keys and values in, one 64-bit
// word (key >> out_shift) << 32 | value out), konly (those words in and out)
// and, for a RUNS pass, the runs' shift and tile limit.
struct PassOut {
    bool narrow = false;
    bool konly = false;
    int out_shift = 0;
    int run_shift = 0;
    uint32_t run_limit = 0xFFFFFFFFu;
    uint32_t* key_err = nullptr;  // kErrKeyRange of narrowing and run counting
    int val_bits = 32;            // the value field of the joined words
    uint32_t val_limit = 0u;      // values must be below it (0: any)
};

// A digit pass with partition shape CFG.
template <typename K, typename CFG>
hipError_t launch_cfg(bool iota, const K* kin, const uint32_t* vin, K* kout, uint32_t* vout,
                      int64_t n_cap, const uint32_t* n_dev, int shift, int bits,
                      const uint32_t* hist_pass, SortTemp& tmp, uint32_t* ticket, hipStream_t st,
                      bool drop, uint32_t* next_hist, int next_shift, int next_bits,
                      uint32_t* run_cnt, const uint32_t* part_offs, const PassOut& po) {
    constexpr int T = CFG::T, I = CFG::I;
    constexpr bool SP = CFG::SPLIT;
    const unsigned grid = (unsigned)((n_cap + T * I - 1) / (T * I));
    const bool d32 = n_cap < ((int64_t)1 << 30);
    uint32_t* state = reinterpret_cast<uint32_t*>(tmp.state);
    uint32_t* clear_next = nullptr;
    if (d32 && tmp.state_parts >= grid) {
        const int h = tmp.half;
        const size_t half_words = tmp.state_parts * 256;
        uint32_t* cur = state + (size_t)h * half_words;
        clear_next = state + (size_t)(h ^ 1) * half_words;
        // the rows this pass uses that may hold descriptors
        const uint32_t lo = tmp.clean[h], hi = std::min<uint32_t>(tmp.dirty[h], grid);
        if (hi > lo) {
            const size_t words = (size_t)(hi - lo) * 256;
            k_fill_u32<<<(unsigned)((words + 255) / 256), 256, 0, st>>>(cur + (size_t)lo * 256,
                                                                         0u, words);
        }
        // this pass fills rows [0, grid) of its half (rows past them keep what
        // they held) and clears them in the other
        tmp.dirty[h] = std::max<uint32_t>(tmp.dirty[h], grid);
        tmp.clean[h] = 0u;
        tmp.clean[h ^ 1] = std::max<uint32_t>(tmp.clean[h ^ 1], grid);
        if (tmp.clean[h ^ 1] >= tmp.dirty[h ^ 1]) tmp.clean[h ^ 1] = tmp.dirty[h ^ 1] = 0u;
        tmp.half ^= 1;
        state = cur;
    } else {
        const size_t words = (size_t)grid * 256 * (d32 ? 1 : 2);
        k_fill_u32<<<(unsigned)((words + 255) / 256), 256, 0, st>>>(state, 0u, words);
        tmp.dirty[0] = tmp.dirty[1] = (uint32_t)std::min<size_t>(tmp.state_parts, 0xFFFFFFFFu);
        tmp.clean[0] = tmp.clean[1] = 0u;
    }
    const uint32_t epoch = ++tmp.epoch;
#define GS_OSN(IO, DD, DR, RU, NA, KO)                                                          \
    k_onesweep<K, IO, T, I, DD, DR, SP, RU, NA, KO><<<grid, T, 0, st>>>(                        \
        kin, vin, kout, vout, n_cap, n_dev, shift, bits, hist_pass, state, ticket, epoch,       \
        clear_next, tmp.ctl, next_hist, next_shift, next_bits, run_cnt, part_offs, po.out_shift,\
        po.run_shift, po.run_limit, po.key_err, po.val_bits, po.val_limit)
#define GS_OS(IO, DD, DR, RU) GS_OSN(IO, DD, DR, RU, false, false)
    if (po.narrow || po.konly) {
        if constexpr (sizeof(K) == 8 && SP) {
            if (iota || drop || (po.narrow && (po.konly || run_cnt != nullptr)))
                return hipErrorInvalidValue;
            if (po.narrow) {
                if (d32) GS_OSN(false, true, false, false, true, false);
                else GS_OSN(false, false, false, false, true, false);
            } else if (run_cnt != nullptr) {
                if (d32) GS_OSN(false, true, false, true, false, true);
                else GS_OSN(false, false, false, true, false, true);
            } else {
                if (d32) GS_OSN(false, true, false, false, false, true);
                else GS_OSN(false, false, false, false, false, true);
            }
        } else {
            return hipErrorInvalidValue;
        }
    } else if (run_cnt != nullptr) {
        if (iota || sizeof(K) != 4) return hipErrorInvalidValue;
        if (drop) {  // a one-pass sort: it drops and counts
            if (d32) GS_OS(false, true, true, true); else GS_OS(false, false, true, true);
        } else {
            if (d32) GS_OS(false, true, false, true); else GS_OS(false, false, false, true);
        }
    } else if (drop) {
        if (iota || sizeof(K) != 4) return hipErrorInvalidValue;
        if (d32) GS_OS(false, true, true, false); else GS_OS(false, false, true, false);
    } else if (iota) {
        if (d32) GS_OS(true, true, false, false); else GS_OS(true, false, false, false);
    } else {
        if (d32) GS_OS(false, true, false, false); else GS_OS(false, false, false, false);
    }
#undef GS_OS
#undef GS_OSN
    return hipGetLastError();
}

// One digit pass: clears the look-back descriptors of its partitions (32-bit
// ones below 2^30 keys, else 64-bit), then runs the onesweep kernel.
// next_hist (optional): the pass also adds the digit histogram of bits
// [next_shift, next_shift + next_bits) of its keys there (for the next pass).
template <typename K>
hipError_t launch_pass(bool iota, const K* kin, const uint32_t* vin, K* kout, uint32_t* vout,
                       int64_t n_cap, const uint32_t* n_dev, int shift, int bits,
                       const uint32_t* hist_pass, SortTemp& tmp, uint32_t* ticket,
                       hipStream_t st, bool drop = false, uint32_t* next_hist = nullptr,
                       int next_shift = 0, int next_bits = 0, uint32_t* run_cnt = nullptr,
                       const uint32_t* part_offs = nullptr, const PassOut& po = PassOut()) {
    if constexpr (sizeof(K) == 8)
        return launch_cfg<K, Sweep64>(iota, kin, vin, kout, vout, n_cap, n_dev, shift, bits,
                                      hist_pass, tmp, ticket, st, drop, next_hist, next_shift,
                                      next_bits, run_cnt, part_offs, po);
    return launch_cfg<K, Sweep32>(iota, kin, vin, kout, vout, n_cap, n_dev, shift, bits,
                                  hist_pass, tmp, ticket, st, drop, next_hist, next_shift,
                                  next_bits, run_cnt, part_offs, po);
}

template <typename K>
hipError_t sort_impl(K* keys, uint32_t* vals, int64_t n, int begin_bit, int end_bit,
                     SortTemp& tmp, uint32_t* host_hist, hipStream_t st, int* passes_run,
                     bool vals_iota, K** keys_final, uint32_t** vals_final) {
    *passes_run = 0;
    *keys_final = keys;
    *vals_final = vals;
    if (n <= 0) return hipSuccess;
    if (n >= (int64_t)1 << 32) return hipErrorInvalidValue;
    const int npass = (end_bit - begin_bit + 7) / 8;
    if (npass <= 0 || npass > kMaxPasses) return hipErrorInvalidValue;
    hipError_t e;
    // clear histograms and tickets in one small launch
    {
        const size_t words = (size_t)kMaxPasses * 256 + kMaxPasses;
        k_fill_u32<<<(unsigned)((words + 255) / 256), 256, 0, st>>>(tmp.hist, 0u, words);
    }
    const unsigned hgrid =
        (unsigned)std::min<int64_t>((n + kHistThreads * kHistItems - 1) / (kHistThreads * kHistItems), 2048);
    k_hist<K><<<hgrid, kHistThreads, 0, st>>>(keys, n, begin_bit, end_bit, npass, 8, tmp.hist);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = hipMemcpyAsync(host_hist, tmp.hist, (size_t)npass * 256 * 4,
                            hipMemcpyDeviceToHost, st)) != hipSuccess)
        return e;
    if ((e = hipStreamSynchronize(st)) != hipSuccess) return e;

    K* kin = keys;
    uint32_t* vin = vals;
    K* kalt = static_cast<K*>(tmp.keys_alt);
    uint32_t* valt = tmp.vals_alt;
    bool iota_pending = vals_iota;
    uint32_t* tickets = tmp.hist + (size_t)kMaxPasses * 256;
    for (int p = 0; p < npass; ++p) {
        bool trivial = false;
        for (int d = 0; d < 256; ++d)
            if (host_hist[p * 256 + d] == (uint32_t)n) trivial = true;
        if (trivial) continue;
        const int shift = begin_bit + 8 * p;
        const int bits = std::min(8, end_bit - shift);
        const bool timed = tmp.pass_events != nullptr && *passes_run < tmp.max_timed_passes;
        if (timed) (void)hipEventRecord(tmp.pass_events[2 * *passes_run], st);
        e = launch_pass<K>(iota_pending, kin, vin, kalt, valt, n, nullptr, shift, bits,
                           tmp.hist + p * 256, tmp, tickets + p, st);
        iota_pending = false;
        if (e != hipSuccess) return e;
        if (timed) (void)hipEventRecord(tmp.pass_events[2 * *passes_run + 1], st);
        std::swap(kin, kalt);
        std::swap(vin, valt);
        ++*passes_run;
    }
    if (iota_pending) {
        k_iota_u32<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(vin, (size_t)n);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    *keys_final = kin;
    *vals_final = vin;
    return hipSuccess;
}

// Every pass runs (no trivial-pass skipping: the host does not see the
// histogram); n is min(n_cap, *n_dev), read on the device. The key bits are
// spread evenly over the passes (sort_digit_width), and `hist` holds 256 words
// per pass for digits of that width.
// chain_hist (optional, the same buffer as hist): only the first pass's
// histogram is given; each pass adds the next one's. pass_events: record the
// SortTemp's per-pass events (when it has them).
template <typename K>
hipError_t sort_dev_impl(K* keys, uint32_t* vals, int64_t n_cap, const uint32_t* n_dev,
                         int begin_bit, int end_bit, const uint32_t* hist, uint32_t* tickets,
                         SortTemp& tmp, hipStream_t st, bool vals_iota, K** keys_final,
                         uint32_t** vals_final, const uint32_t* n_kept_dev,
                         uint32_t* chain_hist = nullptr, bool pass_events = false,
                         uint32_t* run_cnt = nullptr, const uint32_t* first_offs = nullptr,
                         uint32_t run_limit = 0xFFFFFFFFu, bool keys_out = true) {
    *keys_final = keys;
    *vals_final = vals;
    if (n_cap <= 0) return hipSuccess;
    if (n_cap >= (int64_t)1 << 32) return hipErrorInvalidValue;
    const int npass = (end_bit - begin_bit + 7) / 8;
    if (npass <= 0 || npass > kMaxPasses) return hipErrorInvalidValue;
    K* kin = keys;
    uint32_t* vin = vals;
    K* kalt = static_cast<K*>(tmp.keys_alt);
    uint32_t* valt = tmp.vals_alt;
    const int dw = sort_digit_width(end_bit - begin_bit);
    PassOut po;
    po.run_limit = run_limit;
    for (int p = 0; p < npass; ++p) {
        const int shift = begin_bit + dw * p;
        const int bits = std::min(dw, end_bit - shift);
        const bool drop = p == 0 && n_kept_dev != nullptr;
        const uint32_t* cnt = (p > 0 && n_kept_dev != nullptr) ? n_kept_dev : n_dev;
        const bool chain = chain_hist != nullptr && p + 1 < npass;
        const int nshift = shift + dw;
        const bool timed = pass_events && tmp.pass_events != nullptr && p < tmp.max_timed_passes;
        if (timed) (void)hipEventRecord(tmp.pass_events[2 * p], st);
        K* kdst = (p + 1 == npass && !keys_out) ? nullptr : kalt;
        hipError_t e = launch_pass<K>(p == 0 && vals_iota, kin, vin, kdst, valt, n_cap, cnt,
                                      shift, bits, hist + p * 256, tmp, tickets + p, st, drop,
                                      chain ? chain_hist + (p + 1) * 256 : nullptr, nshift,
                                      chain ? std::min(dw, end_bit - nshift) : 0,
                                      p + 1 == npass ? run_cnt : nullptr,
                                      p == 0 ? first_offs : nullptr, po);
        if (timed) (void)hipEventRecord(tmp.pass_events[2 * p + 1], st);
        if (e != hipSuccess) return e;
        std::swap(kin, kalt);
        std::swap(vin, valt);
    }
    *keys_final = keys_out ? kin : nullptr;
    *vals_final = vin;
    return hipSuccess;
}

}  // namespace

hipError_t radix_sort_pairs_dev(void* keys, uint32_t* vals, int64_t n_cap, const uint32_t* n_dev,
                                int key_bytes, int begin_bit, int end_bit, const uint32_t* hist,
                                uint32_t* tickets, SortTemp& tmp, hipStream_t st, bool vals_iota,
                                void** keys_final, uint32_t** vals_final,
                                const uint32_t* n_kept_dev, uint32_t* run_cnt,
                                const uint32_t* first_offs, uint32_t run_limit, bool keys_out) {
    if (key_bytes == 4) {
        uint32_t* kf = nullptr;
        hipError_t e = sort_dev_impl<uint32_t>(static_cast<uint32_t*>(keys), vals, n_cap, n_dev,
                                               begin_bit, end_bit, hist, tickets, tmp, st,
                                               vals_iota, &kf, vals_final, n_kept_dev, nullptr,
                                               false, run_cnt, first_offs, run_limit, keys_out);
        *keys_final = run_cnt != nullptr ? nullptr : kf;
        return e;
    }
    if (key_bytes == 8) {
        if (n_kept_dev != nullptr || run_cnt != nullptr || first_offs != nullptr)
            return hipErrorInvalidValue;
        uint64_t* kf = nullptr;
        hipError_t e = sort_dev_impl<uint64_t>(static_cast<uint64_t*>(keys), vals, n_cap, n_dev,
                                               begin_bit, end_bit, hist, tickets, tmp, st,
                                               vals_iota, &kf, vals_final, nullptr);
        *keys_final = kf;
        return e;
    }
    return hipErrorInvalidValue;
}

hipError_t radix_sort_pairs_dev_chain(uint64_t* keys, uint32_t* vals, int64_t n, int begin_bit,
                                      int end_bit, uint32_t* hist, uint32_t* tickets,
                                      SortTemp& tmp, hipStream_t st, void** keys_final,
                                      uint32_t** vals_final) {
    *keys_final = keys;
    *vals_final = vals;
    if (n <= 0) return hipSuccess;
    if (n >= (int64_t)1 << 32) return hipErrorInvalidValue;
    const int npass = (end_bit - begin_bit + 7) / 8;
    if (npass <= 0 || npass > kMaxPasses) return hipErrorInvalidValue;
    const int dw = sort_digit_width(end_bit - begin_bit);
    // the first pass's histogram only; the passes chain the others
    const unsigned grid = (unsigned)std::min<int64_t>(
        (n + kHistThreads * kHistItems - 1) / (kHistThreads * kHistItems), 2048);
    k_hist<uint64_t, 1><<<grid, kHistThreads, 0, st>>>(keys, n, begin_bit,
                                                       std::min(end_bit, begin_bit + dw), 1, dw,
                                                       hist);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    uint64_t* kf = nullptr;
    e = sort_dev_impl<uint64_t>(keys, vals, n, nullptr, begin_bit, end_bit, hist, tickets, tmp,
                                st, false, &kf, vals_final, nullptr, hist, true);
    *keys_final = kf;
    return e;
}

hipError_t radix_sort_ids_dev_chain(uint64_t* keys, uint32_t* vals, int64_t n, int tile_bits,
                                    uint64_t val_limit, uint32_t num_tiles, uint32_t* run_cnt,
                                    uint32_t* key_err, uint32_t* hist, uint32_t* tickets,
                                    SortTemp& tmp, hipStream_t st, int* passes_out) {
    *passes_out = 0;
    const int end_bit = 32 + tile_bits;
    const int npass = (end_bit + 7) / 8;
    if (tile_bits < 1 || npass > kMaxPasses || val_limit > ((uint64_t)1 << 32))
        return hipErrorInvalidValue;
    // the value field: the bits of val_limit - 1 (all 32 for no limit)
    int val_bits = 32;
    if (val_limit != 0) {
        val_bits = 1;
        while (val_bits < 32 && ((uint64_t)1 << val_bits) < val_limit) ++val_bits;
    }
    const int dw = sort_digit_width(end_bit);
    // q passes over 64-bit keys with separate values, the last of them
    // joining each key's bits [q*dw, end_bit) and its value into one word
    // (the fewest passes after which they fit): key bit b >= q*dw sits at bit
    // val_bits + b - q*dw of the word
    int q = 1;
    while (q < npass && end_bit - q * dw + val_bits > 64) ++q;
    if (q >= npass) return hipErrorNotSupported;
    if (n <= 0) return hipSuccess;
    if (n >= (int64_t)1 << 32) return hipErrorInvalidValue;
    const int nshift = q * dw;
    const unsigned grid = (unsigned)std::min<int64_t>(
        (n + kHistThreads * kHistItems - 1) / (kHistThreads * kHistItems), 2048);
    k_hist<uint64_t, 1><<<grid, kHistThreads, 0, st>>>(keys, n, 0, dw, 1, dw, hist);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // keys (and then the joined words) ping-pong between keys and keys_alt,
    // values between vals and vals_alt until they are joined; the last pass
    // writes the sorted values into vals
    uint64_t* k64[2] = {keys, static_cast<uint64_t*>(tmp.keys_alt)};
    uint32_t* vb[2] = {vals, tmp.vals_alt};
    int ki = 0, vi = 0;
    for (int p = 0; p < npass; ++p) {
        const bool wide = p < q;
        const int at = wide ? 0 : val_bits - nshift;  // key bit b of this pass's input: at b + at
        const int shift = dw * p + at;
        const int bits = std::min(dw, end_bit - dw * p);
        const bool last = p + 1 == npass;
        // the next pass's digits, counted from this pass's input keys
        const int next_shift = dw * (p + 1) + at;
        const int next_bits = last ? 0 : std::min(dw, end_bit - dw * (p + 1));
        uint32_t* nh = last ? nullptr : hist + (p + 1) * 256;
        PassOut po;
        po.key_err = key_err;
        po.val_bits = val_bits;
        po.val_limit = val_limit == ((uint64_t)1 << 32) ? 0u : (uint32_t)val_limit;
        const bool timed = tmp.pass_events != nullptr && p < tmp.max_timed_passes;
        if (timed) (void)hipEventRecord(tmp.pass_events[2 * p], st);
        if (wide) {
            po.narrow = p + 1 == q;
            po.out_shift = nshift;
            e = launch_pass<uint64_t>(false, k64[ki], vb[vi], k64[ki ^ 1], vb[vi ^ 1], n, nullptr,
                                      shift, bits, hist + p * 256, tmp, tickets + p, st, false,
                                      nh, next_shift, next_bits, nullptr, nullptr, po);
            vi ^= 1;
        } else {
            po.konly = true;
            po.run_shift = 32 + at;  // the tile field of the joined word
            po.run_limit = num_tiles;
            e = launch_pass<uint64_t>(false, k64[ki], nullptr, k64[ki ^ 1],
                                      last ? vals : nullptr, n, nullptr, shift, bits,
                                      hist + p * 256, tmp, tickets + p, st, false, nh,
                                      next_shift, next_bits, last ? run_cnt : nullptr, nullptr,
                                      po);
        }
        if (timed) (void)hipEventRecord(tmp.pass_events[2 * p + 1], st);
        if (e != hipSuccess) return e;
        ki ^= 1;
        ++*passes_out;
    }
    return hipSuccess;
}

size_t sort_partitions(int64_t n) { return (size_t)((n + kMinPart - 1) / kMinPart); }


hipError_t launch_digit_hist_u64(const uint64_t* keys, int64_t n, int begin_bit, int end_bit,
                                 uint32_t* hist, hipStream_t st) {
    const int npass = (end_bit - begin_bit + 7) / 8;
    if (n <= 0) return hipSuccess;
    if (npass <= 0 || npass > kMaxPasses) return hipErrorInvalidValue;
    const int dw = sort_digit_width(end_bit - begin_bit);
    const unsigned grid = (unsigned)std::min<int64_t>(
        (n + kHistThreads * kHistItems - 1) / (kHistThreads * kHistItems), 2048);
    k_hist<uint64_t><<<grid, kHistThreads, 0, st>>>(keys, n, begin_bit, end_bit, npass, dw, hist);
    return hipGetLastError();
}
size_t sort_state_bytes(int64_t n) { return sort_partitions(n) * 256 * sizeof(uint64_t); }
size_t sort_hist_words() { return (size_t)kMaxPasses * 256 + kMaxPasses; }

hipError_t radix_sort_pairs(void* keys, uint32_t* vals, int64_t n, int key_bytes, int begin_bit,
                            int end_bit, SortTemp& tmp, uint32_t* host_hist, hipStream_t st,
                            int* passes_run, bool vals_iota, void** keys_final,
                            uint32_t** vals_final) {
    if (key_bytes == 4) {
        uint32_t* kf = nullptr;
        hipError_t e = sort_impl<uint32_t>(static_cast<uint32_t*>(keys), vals, n, begin_bit,
                                           end_bit, tmp, host_hist, st, passes_run, vals_iota,
                                           &kf, vals_final);
        *keys_final = kf;
        return e;
    }
    if (key_bytes == 8) {
        uint64_t* kf = nullptr;
        hipError_t e = sort_impl<uint64_t>(static_cast<uint64_t*>(keys), vals, n, begin_bit,
                                           end_bit, tmp, host_hist, st, passes_run, vals_iota,
                                           &kf, vals_final);
        *keys_final = kf;
        return e;
    }
    return hipErrorInvalidValue;
}

hipError_t launch_fill_ranges(uint32_t* const* p, const uint32_t* v, const uint32_t* n, int count,
                              hipStream_t st) {
    if (count < 0 || count > kFillRanges) return hipErrorInvalidValue;
    FillRanges f{};
    uint64_t total = 0;
    for (int r = 0; r < count; ++r) {
        f.p[r] = p[r];
        f.v[r] = v[r];
        f.n[r] = n[r];
        total += n[r];
    }
    if (total == 0) return hipSuccess;
    if (total > 0xFFFFFFFFull) return hipErrorInvalidValue;
    k_fill_ranges<<<(unsigned)((total + 255) / 256), 256, 0, st>>>(f);
    return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    k_fill_u32<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(p, v, n);
    return hipGetLastError();
}

}  // namespace gs
