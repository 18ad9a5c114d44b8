// tiles.hip - tile assignment: per-Gaussian tile rectangle, exclusive scan of
// rectangle areas (decoupled look-back), pair-centric emission with the
// per-pair Mahalanobis cull and a stable compaction of the kept pairs, and
// tile-range extraction from the tile-sorted pair list.
//
// Reference: src/gsplat_cpu/tile_assign.cpp:60-102 (rectangle: float divide,
// truncate toward zero, clamp), :121-149 (row-major pairs per Gaussian),
// :151-290 (constrained minimum of the Mahalanobis distance over the tile
// rectangle, keep iff num <= det * m2thr), :298-349 (stable compaction);
// src/gsplat_cpu/sort.cpp:146-165 (tile_ranges, (0,0) for empty tiles).
// Compiled with -ffp-contract=off: every comparison sees the reference's
// fp32 values.
#include <algorithm>

#include "gs_common.h"
#include "gs_internal.h"

namespace gs {
namespace {

// The count scan's partitions are chained by a decoupled look-back: 2048 ranks
// per 512-thread workgroup halve the chain of 1024-rank ones (measured: the
// tile-assign stage 0.41 -> 0.38 ms; 4096 per workgroup is slower again).
constexpr int kCountThreads = 512;
constexpr int kCountWaves = kCountThreads / GS_WAVE;
constexpr int kCountItems = 4;
constexpr int kCountPart = kCountThreads * kCountItems;  // ranks per scan partition
constexpr int kEmitThreads = 512;                    // workgroup of the pair emission
constexpr int kEmitWaves = kEmitThreads / GS_WAVE;
constexpr int kEmitPart = 2048;                      // candidates per emit partition
constexpr int kEmitItems = kEmitPart / kEmitThreads;
constexpr int kRankCache = 384;
static_assert(kEmitPart == (int)kEmitPartition, "emit partition size is part of the interface");
static_assert(kEmitPart + 1 <= 65535, "a partition's ranks are held as 16-bit indices");

__device__ __forceinline__ float fmin_std(float a, float b) { return (b < a) ? b : a; }
__device__ __forceinline__ float fmax_std(float a, float b) { return (a < b) ? b : a; }

// q = j / w, r = j % w for j < 2^24 and a quotient below 2^16 (a tile row of a
// Gaussian's rectangle): float reciprocal estimate, then one exact correction.
__device__ __forceinline__ void divmod_small(uint32_t j, uint32_t w, uint32_t& q, uint32_t& r) {
    const int qi = (int)((float)j * __builtin_amdgcn_rcpf((float)w));
    const int ri = (int)j - qi * (int)w;
    const int fix = (ri < 0) ? -1 : ((ri >= (int)w) ? 1 : 0);
    q = (uint32_t)(qi + fix);
    r = (uint32_t)(ri - fix * (int)w);
}

// tile_assign.cpp:151-290, one (Gaussian, tile) pair. Both edge distances are
// always evaluated and the unused one is selected away, so the test has no
// branches and the evaluations of several candidates can be interleaved; the
// values compared are the same expressions as in the reference's test.
__device__ __forceinline__ bool pair_keep(float px, float py, float4 cv, int tile_x, int tile_y,
                                          const TileParams& tp) {
    const float m2thr = cv.w;
    const float a = cv.x, b = cv.y, c = cv.z;
    const float det = fmax_std(a * c - b * b, 1e-6f);
    const float ts = (float)tp.tile_size;
    const float tx_tile = (float)tile_x * ts;
    const float ty_tile = (float)tile_y * ts;
    const float u_lo = tx_tile - px;
    const float u_hi = u_lo + ts;
    const float v_lo = ty_tile - py;
    const float v_hi = v_lo + ts;
    const bool x_in = (u_lo <= 0.0f) & (0.0f <= u_hi);
    const bool y_in = (v_lo <= 0.0f) & (0.0f <= v_hi);
    const float scaled = det * m2thr;
    // nearest point on the vertical edge facing the centre (used when !x_in)
    const float uf = (u_lo > 0.0f) ? u_lo : u_hi;
    const float a_safe = fmax_std(a, 1e-12f);
    float vs = (b * uf) / a_safe;
    vs = fmax_std(v_lo, fmin_std(vs, v_hi));
    const float m2_v = x_in ? __builtin_inff() : c * uf * uf - 2.0f * b * uf * vs + a * vs * vs;
    // nearest point on the horizontal edge facing the centre (used when !y_in)
    const float vf = (v_lo > 0.0f) ? v_lo : v_hi;
    const float c_safe = fmax_std(c, 1e-12f);
    float us = (b * vf) / c_safe;
    us = fmax_std(u_lo, fmin_std(us, u_hi));
    const float m2_h = y_in ? __builtin_inff() : c * us * us - 2.0f * b * us * vf + a * vf * vf;
    // opacity <= floor (m2thr < 0 or NaN) never keeps
    // bitwise operators: no short-circuit branches around the divisions
    return (m2thr >= 0.0f) & ((x_in & y_in) | (fmin_std(m2_v, m2_h) <= scaled));
}

// Rectangle area per rank, exclusive scan -> offs[r]; the total candidate
// count goes to *total_out (saturated to 0xFFFFFFFF on overflow). Also
// records, for every emit partition b (candidates [b*kEmitPart, ...)), the
// rank that owns its first candidate: bstart[b].
//   kScanLookback: one kernel, partitions chained by a decoupled look-back.
//   kScanReduce / kScanFinal: reduce-then-scan without waits, for a frame with
//     other frames in flight (a look-back chain advances only as fast as its
//     slowest partition, and other frames' kernels slow its partitions): the
//     reduce kernel writes each partition's sum to part[vid], a one-workgroup
//     kernel turns them into exclusive bases (k_scan_part_sums), and the final
//     kernel re-reads the counts and writes the offsets from its base.
constexpr int kScanLookback = 0, kScanReduce = 1, kScanFinal = 2;
template <int PHASE>
__global__ __launch_bounds__(kCountThreads) void k_rect_count_scan(const float4* __restrict__ rect,
                                                              int stride,
                                                              const uint32_t* __restrict__ order,
                                                              int64_t m_cap,
                                                              const uint32_t* __restrict__ m_dev,
                                                              TileParams tp,
                                                              uint32_t* __restrict__ offs,
                                                              uint32_t* __restrict__ bstart,
                                                              uint32_t bstart_cap,
                                                              uint64_t* lb_state,
                                                              uint32_t* ticket,
                                                              uint32_t* total_out,
                                                              uint32_t cap) {
    __shared__ uint32_t s_vid;
    __shared__ uint32_t s_wsum[kCountItems][kCountWaves];
    __shared__ uint64_t s_excl;
    const int tid = threadIdx.x, w = tid / GS_WAVE, lane = lane_id();
    if (tid == 0) {
        const bool failed = upstream_failed(tp.ctl);
        s_vid = failed ? 0xFFFFFFFFu : (PHASE == kScanLookback ? atomicAdd(ticket, 1u) : blockIdx.x);
    }
    __syncthreads();
    const uint32_t vid = s_vid;
    if (vid == 0xFFFFFFFFu) return;  // the depth order may be wrong: touch nothing
    // the grid may be sized for a capacity; the real count can live on the device
    const int64_t m = m_dev ? min(m_cap, (int64_t)*m_dev) : m_cap;
    const uint32_t nparts = (uint32_t)((m + kCountPart - 1) / kCountPart);
    if (vid >= nparts) return;  // no later partition has work either
    const int64_t base = (int64_t)vid * kCountPart;
    // loads in stages (all ranks' ids, then all rectangles) so that the four
    // gathers of a thread are in flight together
    const TsDiv tsd = ts_div(tp.tile_size);
    // (indices past m are clamped to m - 1: unconditional loads, no branches
    // whose joins would wait for each load in turn)
    // A packed rank order carries each Gaussian's tile count (the projection
    // computed it): only ranks whose count field is saturated read their
    // rectangle, a 16-byte gather in depth order.
    uint32_t gid[kCountItems], held[kCountItems];
    float4 rr[kCountItems];
#pragma unroll
    for (int it = 0; it < kCountItems; ++it)
        gid[it] = (uint32_t)min(base + it * kCountThreads + tid, m - 1);
    if (order != nullptr) {
#pragma unroll
        for (int it = 0; it < kCountItems; ++it) gid[it] = order[gid[it]];
    }
#pragma unroll
    for (int it = 0; it < kCountItems; ++it) {
        held[it] = dval_count(gid[it], tp.idx_bits);
        gid[it] = dval_index(gid[it], tp.idx_bits);
    }
#pragma unroll
    for (int it = 0; it < kCountItems; ++it)
        if (held[it] == 0u) rr[it] = rect[(int64_t)gid[it] * stride];
    uint32_t incl[kCountItems], cnt[kCountItems];
#pragma unroll
    for (int it = 0; it < kCountItems; ++it) {
        const int64_t r = base + it * kCountThreads + tid;
        uint32_t c = 0;
        if (r < m) {
            if (held[it] != 0u) {
                c = held[it];
            } else {
                const Rect q = tile_rect(rr[it], tp.tiles_x, tp.tiles_y, tsd);
                c = (uint32_t)((q.x1 - q.x0 + 1) * (q.y1 - q.y0 + 1));
            }
        }
        cnt[it] = c;
        incl[it] = wave_incl_scan(c);
        if (lane == GS_WAVE - 1) s_wsum[it][w] = incl[it];
    }
    __syncthreads();
    uint64_t total = 0;
    uint64_t my_off[kCountItems];
#pragma unroll
    for (int it = 0; it < kCountItems; ++it)
#pragma unroll
        for (int ww = 0; ww < kCountWaves; ++ww) {
            if (ww == w) my_off[it] = total;
            total += s_wsum[it][ww];
        }
    if (PHASE == kScanReduce) {
        // lb_state[vid]: this partition's sum, for k_scan_part_sums
        if (tid == 0) lb_state[vid] = total;
        return;
    }
    if (PHASE == kScanFinal) {
        if (tid == 0) s_excl = lb_state[vid];  // the exclusive base
    } else if (w == 0) {
        const uint64_t ex = lookback_exclusive(lb_state, vid, total, tp.ctl);
        if (lane == 0) {
            s_excl = ex;
            if (vid == nparts - 1) {
                const uint64_t t = ex + total;
                *total_out = t > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)t;
                // the frame is run again with room for them: the kernels after
                // this one skip their work
                if (cap != 0u && t > cap) report_error(tp.ctl, kErrCapacity);
            }
        }
    }
    __syncthreads();
    const uint64_t ex = s_excl;
#pragma unroll
    for (int it = 0; it < kCountItems; ++it) {
        const int64_t r = base + it * kCountThreads + tid;
        if (r < m) {
            const uint64_t o = ex + my_off[it] + incl[it] - cnt[it];
            offs[r] = (uint32_t)o;
            // emit partitions whose first candidate lies in [o, o + cnt)
            uint64_t b = (o + kEmitPart - 1) / kEmitPart;
            for (; b * kEmitPart < o + cnt[it] && b < bstart_cap; ++b) bstart[b] = (uint32_t)r;
        }
    }
}

// Exclusive scan of the count scan's partition sums in place (one workgroup:
// each thread a run of consecutive partitions), the total candidate count to
// *total_out (saturated to 0xFFFFFFFF) and kErrCapacity when it exceeds cap.
constexpr int kSumThreads = 1024;
__global__ __launch_bounds__(kSumThreads) void k_scan_part_sums(uint64_t* __restrict__ part,
                                                               int64_t m_cap,
                                                               const uint32_t* __restrict__ m_dev,
                                                               uint32_t* total_out, uint32_t cap,
                                                               uint32_t* ctl) {
    __shared__ uint64_t s_w[kSumThreads / GS_WAVE];
    if (upstream_failed(ctl)) return;  // uniform over the workgroup
    const int tid = threadIdx.x, w = tid / GS_WAVE, lane = lane_id();
    const int64_t m = m_dev ? min(m_cap, (int64_t)*m_dev) : m_cap;
    const uint32_t nparts = (uint32_t)((m + kCountPart - 1) / kCountPart);
    const uint32_t per = (nparts + kSumThreads - 1) / kSumThreads;
    const uint32_t p0 = min(nparts, (uint32_t)tid * per), p1 = min(nparts, p0 + per);
    uint64_t sum = 0;
    for (uint32_t q = p0; q < p1; ++q) sum += part[q];
    const uint64_t inc = wave_incl_scan64(sum);
    if (lane == GS_WAVE - 1) s_w[w] = inc;
    __syncthreads();
    uint64_t run = inc - sum;
    for (int i = 0; i < w; ++i) run += s_w[i];
    for (uint32_t q = p0; q < p1; ++q) {
        const uint64_t v = part[q];
        part[q] = run;
        run += v;
    }
    if (tid == kSumThreads - 1) {
        *total_out = run > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)run;
        // the frame is run again with room for them: the kernels after this
        // one skip their work
        if (cap != 0u && run > cap) report_error(ctl, kErrCapacity);
    }
}

// Pair-centric emission: candidate c -> (rank r, j-th tile of r's rectangle),
// cull, stable compaction of kept pairs in candidate order. The ranks of a
// partition are [bstart[vid], bstart[vid+1]]; each candidate finds its rank by
// an inclusive max-scan over rank heads in LDS. A rank's rectangle and conic
// are read once per partition, from its record in compact order (by_order:
// the lines the count scan fetched just before, not a rank-ordered copy).
// COMPACT: kept pairs are compacted (ticket-ordered partitions, look-back).
// Otherwise every candidate slot c < cap is written, the tile id of a kept
// pair or kPairDrop for a culled one (the pair id only for kept ones), and the
// kept count is added to *total_out: the tile sort's first pass drops the
// culled slots, so no partition waits on another here.
// NDIG: tile-id digit histograms made (2, or 3 above 16 tile bits).
template <bool COMPACT, int NDIG>
__global__ __launch_bounds__(kEmitThreads) void k_pair_emit(
    const float4* __restrict__ rect, const float4* __restrict__ cov, int stride,
    bool by_order, const uint32_t* __restrict__ order, const uint32_t* __restrict__ offs,
    const uint32_t* __restrict__ bstart, int64_t m_cap, const uint32_t* __restrict__ m_dev,
    uint32_t p_pre_cap, const uint32_t* __restrict__ p_pre_dev, TileParams tp,
    uint32_t* __restrict__ pair_tile, uint32_t* __restrict__ pair_id, uint32_t cap,
    uint64_t* lb_state, uint32_t* ticket, uint32_t* total_out,
    uint32_t* __restrict__ part_hist, int dig_bits) {
    __shared__ uint32_t s_vid;
    __shared__ uint32_t s_off[kEmitPart + 1];
    __shared__ uint32_t s_xy[kEmitPart + 1];
    __shared__ uint32_t s_w[kEmitPart + 1];
    __shared__ uint16_t s_own[kEmitPart];  // rank heads, then each slot's rank (nr <= 2049)
    // centre and conic of the first kRankCache ranks (the usual partition has
    // ~10x fewer ranks than candidates; larger ones read them from memory)
    __shared__ float2 s_pc[kRankCache];
    __shared__ float4 s_cv[kRankCache];
    __shared__ uint32_t s_wmax[kEmitWaves];
    __shared__ uint32_t s_cnt[kEmitItems][kEmitWaves];
    __shared__ uint32_t s_th[NDIG][256];
    __shared__ uint64_t s_excl;
    const int tid = threadIdx.x, w = tid / GS_WAVE, lane = lane_id();
    // The counts and this partition's rank bounds, loaded together (every
    // caller's bstart holds a word past the grid's last partition, so vid + 1 is
    // in bounds; a partition past the candidates ignores what it read). Without
    // compaction the partition is the workgroup's, and they load alongside the
    // error word below.
    const int64_t m = m_dev ? min(m_cap, (int64_t)*m_dev) : m_cap;
    const uint32_t p_pre = p_pre_dev ? min(p_pre_cap, *p_pre_dev) : p_pre_cap;
    uint32_t b_lo = 0, b_hi = 0;
    if constexpr (!COMPACT) {
        b_lo = bstart[blockIdx.x];
        b_hi = bstart[blockIdx.x + 1];
    }
    // one thread decides for the workgroup: after an earlier give-up the scan's
    // offsets and owner table may be wrong, so touch nothing
    if (tid == 0) {
        const bool failed = upstream_failed(tp.ctl);
        s_vid = failed ? 0xFFFFFFFFu : (COMPACT ? atomicAdd(ticket, 1u) : blockIdx.x);
    }
    for (int i = tid; i < kEmitPart; i += kEmitThreads) s_own[i] = 0;
    if (part_hist != nullptr)
        for (int i = tid; i < NDIG * 256; i += kEmitThreads) (&s_th[0][0])[i] = 0;
    __syncthreads();
    const uint32_t vid = s_vid;
    if (vid == 0xFFFFFFFFu) return;
    if constexpr (COMPACT) {
        b_lo = bstart[vid];
        b_hi = bstart[vid + 1];
    }
    const uint32_t nparts = (uint32_t)(((uint64_t)p_pre + kEmitPart - 1) / kEmitPart);
    if (vid >= nparts) return;  // no later partition has work either
    const uint64_t c0 = (uint64_t)vid * kEmitPart;
    const uint64_t c1 = min((uint64_t)p_pre, c0 + kEmitPart);
    const int64_t rlo = b_lo;
    const int64_t rend = (c1 < (uint64_t)p_pre) ? (int64_t)b_hi + 1 : m;
    // every rank owns >= 1 candidate, so nr <= kEmitPart + 1; clamp defensively
    const int64_t nr = min(rend - rlo, (int64_t)kEmitPart + 1);
    const TsDiv tsd = ts_div(tp.tile_size);
    for (int64_t k = tid; k < nr; k += kEmitThreads) {
        const int64_t r = rlo + k;
        const int64_t e = by_order ? (int64_t)dval_index(order[r], tp.idx_bits) : r;  // its record
        const float4 rr = rect[e * stride];
        const Rect q = tile_rect(rr, tp.tiles_x, tp.tiles_y, tsd);
        const uint32_t o = offs[r];
        if (k < kRankCache) {
            s_pc[k] = make_float2(rr.x, rr.y);
            if (tp.cull) s_cv[k] = cov[e * stride];
        }
        s_off[k] = o;
        s_xy[k] = (uint32_t)q.x0 | ((uint32_t)q.y0 << 16);
        s_w[k] = (uint32_t)(q.x1 - q.x0 + 1);
        if (o > c0 && o < c1) s_own[o - c0] = (uint16_t)k;  // rank head
    }
    __syncthreads();
    // inclusive max-scan of the heads: kEmitItems consecutive slots per thread
    {
        uint32_t v[kEmitItems];
        uint32_t run = 0;
#pragma unroll
        for (int i = 0; i < kEmitItems; ++i) {
            run = max(run, (uint32_t)s_own[tid * kEmitItems + i]);
            v[i] = run;
        }
        uint32_t inc = run;
#pragma unroll
        for (int o = 1; o < GS_WAVE; o <<= 1) {
            const uint32_t u = __shfl_up(inc, o, GS_WAVE);
            if (lane >= o) inc = max(inc, u);
        }
        if (lane == GS_WAVE - 1) s_wmax[w] = inc;
        uint32_t pre = __shfl_up(inc, 1, GS_WAVE);
        if (lane == 0) pre = 0;
        __syncthreads();
        for (int ww = 0; ww < w; ++ww) pre = max(pre, s_wmax[ww]);
#pragma unroll
        for (int i = 0; i < kEmitItems; ++i) s_own[tid * kEmitItems + i] = (uint16_t)max(pre, v[i]);
    }
    __syncthreads();

    // Every slot of s_own holds a rank in [0, nr), also past c1, so all LDS
    // reads below are issued unconditionally, item by item in stages, and the
    // evaluations overlap instead of waiting on each other.
    bool keep[kEmitItems];
    uint32_t tile[kEmitItems], gid[kEmitItems];
    uint64_t bal[kEmitItems];
    uint32_t lo[kEmitItems], off[kEmitItems], wdt[kEmitItems], xy[kEmitItems];
    int tx[kEmitItems], ty[kEmitItems];
#pragma unroll
    for (int it = 0; it < kEmitItems; ++it) lo[it] = s_own[it * kEmitThreads + tid];
    // The Gaussian id from the rank order itself (an L2-resident read; a table
    // of it in LDS would cost a quarter of the workgroup's LDS). The raw words
    // are loaded here and decoded only where the pairs are written, so the four
    // loads stay in flight through the evaluation.
    if (order != nullptr) {
#pragma unroll
        for (int it = 0; it < kEmitItems; ++it) gid[it] = order[rlo + lo[it]];
    }
#pragma unroll
    for (int it = 0; it < kEmitItems; ++it) {
        off[it] = s_off[lo[it]];
        wdt[it] = s_w[lo[it]];
        xy[it] = s_xy[lo[it]];
    }
#pragma unroll
    for (int it = 0; it < kEmitItems; ++it) {
        const uint64_t c = c0 + it * kEmitThreads + tid;
        uint32_t row, col;
        divmod_small((uint32_t)c - off[it], wdt[it], row, col);
        ty[it] = (int)((xy[it] >> 16) + row);
        tx[it] = (int)((xy[it] & 0xFFFFu) + col);
        tile[it] = (uint32_t)(ty[it] * tp.tiles_x + tx[it]);
        // without compaction a slot past the capacity is not written, so it
        // must not be counted either (the frame is re-run with more room)
        keep[it] = c < c1 && (COMPACT || c < cap);
    }
    if (tp.cull) {
        if (nr <= kRankCache) {
            float2 pc[kEmitItems];
            float4 cv[kEmitItems];
#pragma unroll
            for (int it = 0; it < kEmitItems; ++it) {
                pc[it] = s_pc[lo[it]];
                cv[it] = s_cv[lo[it]];
            }
#pragma unroll
            for (int it = 0; it < kEmitItems; ++it)
                keep[it] = keep[it] & pair_keep(pc[it].x, pc[it].y, cv[it], tx[it], ty[it], tp);
        } else {
            // records through the order words already loaded
            float4 rr[kEmitItems], cv[kEmitItems];
#pragma unroll
            for (int it = 0; it < kEmitItems; ++it) {
                const int64_t e = by_order ? (int64_t)dval_index(gid[it], tp.idx_bits)
                                           : rlo + lo[it];
                rr[it] = rect[e * stride];
                cv[it] = cov[e * stride];
            }
#pragma unroll
            for (int it = 0; it < kEmitItems; ++it)
                keep[it] = keep[it] & pair_keep(rr[it].x, rr[it].y, cv[it], tx[it], ty[it], tp);
        }
    }
    // bookkeeping after all candidates are evaluated, so the evaluations of the
    // candidates of one thread can overlap
#pragma unroll
    for (int it = 0; it < kEmitItems; ++it) {
        bal[it] = __ballot(keep[it]);
        if (lane == 0) s_cnt[it][w] = (uint32_t)__popcll(bal[it]);
        if (part_hist != nullptr && keep[it]) {
            // digit histograms of the tile keys, for the tile sort's passes: a
            // partition's kept tiles spread over the digits, so one LDS atomic
            // per lane (no aggregation of equal digits)
            const uint32_t dm = (1u << dig_bits) - 1u;
#pragma unroll
            for (int q = 0; q < NDIG; ++q) atomicAdd(&s_th[q][(tile[it] >> (q * dig_bits)) & dm], 1u);
        }
    }
#pragma unroll
    for (int it = 0; it < kEmitItems; ++it)
        gid[it] = order != nullptr ? dval_index(gid[it], tp.idx_bits) : (uint32_t)(rlo + lo[it]);
    __syncthreads();
    if (part_hist != nullptr) {
        // the row holds digit q's 2^dig_bits counts at [q << dig_bits], then zeros
        // up to tile_hist_cols(tile bits) words
        const int cols = (NDIG == 2 ? 2 : 4) << dig_bits;
        const uint32_t dm = (1u << dig_bits) - 1u;
        for (int i = tid; i < cols; i += kEmitThreads)
            part_hist[(size_t)vid * cols + i] = (i >> dig_bits) < NDIG ? s_th[i >> dig_bits][i & dm] : 0u;
    }
    if (!COMPACT) {
#pragma unroll
        for (int it = 0; it < kEmitItems; ++it) {
            const uint64_t c = c0 + it * kEmitThreads + tid;
            if (c < c1 && c < cap) {
                pair_tile[c] = keep[it] ? tile[it] : kPairDrop;
                if (keep[it]) pair_id[c] = gid[it];
            }
        }
        if (tid == 0) {
            uint32_t kept = 0;
#pragma unroll
            for (int it = 0; it < kEmitItems; ++it)
#pragma unroll
                for (int ww = 0; ww < kEmitWaves; ++ww) kept += s_cnt[it][ww];
            if (kept) atomicAdd(total_out, kept);
        }
        return;
    }
    uint32_t total = 0, my_off[kEmitItems];
#pragma unroll
    for (int it = 0; it < kEmitItems; ++it)
#pragma unroll
        for (int ww = 0; ww < kEmitWaves; ++ww) {
            if (ww == w) my_off[it] = total;
            total += s_cnt[it][ww];
        }
    if (w == 0) {
        const uint64_t ex = lookback_exclusive(lb_state, vid, total, tp.ctl);
        if (lane == 0) {
            s_excl = ex;
            if (vid == nparts - 1) {
                const uint64_t t = ex + total;
                *total_out = t > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)t;
            }
        }
    }
    __syncthreads();
    const uint64_t ex = s_excl;
    const uint64_t ltm = lanemask_lt();
#pragma unroll
    for (int it = 0; it < kEmitItems; ++it) {
        if (!keep[it]) continue;
        const uint64_t pos = ex + my_off[it] + (uint64_t)__popcll(bal[it] & ltm);
        if (pos < cap) {
            pair_tile[pos] = tile[it];
            pair_id[pos] = gid[it];
        }
    }
}

__global__ void k_tile_ranges(const uint32_t* __restrict__ st, uint32_t p_cap,
                              const uint32_t* __restrict__ p_dev, uint32_t* __restrict__ ranges) {
    const uint32_t p = p_dev ? min(p_cap, *p_dev) : p_cap;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < p;
         i += gridDim.x * blockDim.x) {
        const uint32_t t = st[i];
        if (i == 0 || st[i - 1] != t) ranges[2 * (size_t)t] = i;
        if (i == p - 1 || st[i + 1] != t) ranges[2 * (size_t)t + 1] = i + 1;
    }
}

// Tile id of a sorted key: the key itself (u32 tile keys) or its high word
// ((tile << 32) | depth bits).
__device__ __forceinline__ uint32_t tile_of(uint32_t k) { return k; }
__device__ __forceinline__ uint32_t tile_of(uint64_t k) { return (uint32_t)(k >> 32); }

// First index in [0, p) whose tile is >= t, by a wave-wide 64-ary search
// (about log64(p) dependent loads). Keys are sorted ascending.
template <typename K>
__device__ __forceinline__ uint32_t wave_lower_bound(const K* __restrict__ keys, uint32_t p,
                                                     uint32_t t, int lane) {
    uint32_t lo = 0, hi = p;  // answer in [lo, hi]
    while (hi - lo > (uint32_t)GS_WAVE) {
        const uint32_t step = (hi - lo + GS_WAVE - 1) / GS_WAVE;
        const uint64_t q = (uint64_t)lo + (uint64_t)(lane + 1) * step - 1;
        const bool pred = q < hi && tile_of(keys[q]) < t;
        const uint32_t c = (uint32_t)__popcll(__ballot(pred));
        const uint64_t nhi = (uint64_t)lo + (uint64_t)(c + 1) * step - 1;
        lo += c * step;
        hi = (uint32_t)min((uint64_t)hi, nhi);
    }
    const uint32_t q = lo + (uint32_t)lane;
    const bool pred = q < hi && tile_of(keys[q]) < t;
    return lo + (uint32_t)__popcll(__ballot(pred));
}

// ranges[t] = [first, end) of tile t in the tile-sorted keys, (0, 0) when
// empty (sort.cpp:146-165); one wave per tile, no clearing pass needed. A key
// whose tile is >= num_tiles (only the last key can show it) is flagged
// kErrKeyRange in ctl; no range is written for it.
template <typename K>
__global__ __launch_bounds__(256) void k_tile_bounds(const K* __restrict__ st, uint32_t p_cap,
                                                     const uint32_t* __restrict__ p_dev,
                                                     uint32_t* __restrict__ ranges,
                                                     uint32_t num_tiles, uint32_t* ctl) {
    const uint32_t p = p_dev ? min(p_cap, *p_dev) : p_cap;
    const uint32_t t = blockIdx.x * (256 / GS_WAVE) + threadIdx.x / GS_WAVE;
    const int lane = lane_id();
    if (t >= num_tiles) return;
    if (t == 0 && lane == 0 && p > 0 && tile_of(st[p - 1]) >= num_tiles)
        report_error(ctl, kErrKeyRange);
    const uint32_t a = wave_lower_bound(st, p, t, lane);
    const uint32_t b = wave_lower_bound(st, p, t + 1, lane);
    if (lane == 0) {
        ranges[2 * (size_t)t] = a < b ? a : 0u;
        ranges[2 * (size_t)t + 1] = a < b ? b : 0u;
    }
}

// Rows of part that hold counts: ceil(min(*count_dev, count_cap) / per_row)
// when count_dev is given, else all rows_cap.
__device__ __forceinline__ uint32_t rows_in_use(uint32_t rows_cap, const uint32_t* count_dev,
                                                uint32_t count_cap, uint32_t per_row) {
    if (count_dev == nullptr) return rows_cap;
    const uint32_t c = min(*count_dev, count_cap);
    return min(rows_cap, (uint32_t)(((uint64_t)c + per_row - 1) / per_row));
}

// out[c] += column sums of part (rows x cols, cols / 4 dividing 1024), rows
// bounded by rows_in_use. A 1024-thread workgroup takes `span` rows: cols / 4
// column quads x (4096 / cols) row lanes, 16-byte loads with 8 rows in flight
// per lane; the row lanes are summed in LDS and each workgroup adds its column
// sums with one atomic per column (few workgroups, so little contention on the
// atomics). chunk_out (optional): workgroup b also stores its column sums at
// chunk_out[b * cols + c], zeros included (workgroups past the rows in use
// store nothing). After an upstream failure (ctl) nothing is read or written:
// the rows may not have been written by this frame.
constexpr int kRedThreads = 1024;
constexpr uint32_t kRedBlocks = 96;  // workgroups for the largest row count
__global__ __launch_bounds__(kRedThreads) void k_reduce_rows(
    const uint32_t* __restrict__ part, int cols, uint32_t rows_cap, uint32_t span,
    const uint32_t* __restrict__ count_dev, uint32_t count_cap, uint32_t per_row, int dig_w,
    uint32_t* __restrict__ out, uint32_t* __restrict__ chunk_out, const uint32_t* ctl) {
    __shared__ uint4 s_acc[kRedThreads];
    if (upstream_failed(ctl)) return;  // uniform over the workgroup
    const uint32_t rows = rows_in_use(rows_cap, count_dev, count_cap, per_row);
    const uint32_t r0 = blockIdx.x * span;
    if (r0 >= rows) return;  // uniform over the workgroup
    const int quads = cols / 4;
    const int lanes = kRedThreads / quads;  // row lanes
    const int q = threadIdx.x % quads, rl = threadIdx.x / quads;
    const uint32_t r1 = min(rows, r0 + span);
    const uint4* p = reinterpret_cast<const uint4*>(part) + (size_t)r0 * quads + q;
    uint4 acc = make_uint4(0, 0, 0, 0);
#pragma unroll 8
    for (uint32_t r = r0 + rl; r < r1; r += lanes) {
        const uint4 v = p[(size_t)(r - r0) * quads];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    }
    s_acc[threadIdx.x] = acc;
    __syncthreads();
    if (rl == 0) {
        for (int l = 1; l < lanes; ++l) {
            const uint4 v = s_acc[l * quads + q];
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
        if (chunk_out != nullptr)
            reinterpret_cast<uint4*>(chunk_out + (size_t)blockIdx.x * cols)[q] = acc;
        // column c -> out[c], or with digit rows of 2^dig_w words -> the digit's
        // row of 256 words
        const uint32_t a[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t c = (uint32_t)(q * 4 + j);
            const uint32_t o = dig_w ? ((c >> dig_w) << 8) | (c & ((1u << dig_w) - 1u)) : c;
            if (a[j]) atomicAdd(out + o, a[j]);
        }
    }
}

// Output positions of a sort pass per partition of rows_per_part rows of
// `part` (the per-partition digit counts of the keys' producer, the pass's
// digit in the first 2^dig_w columns of each row) and per digit:
// offs[s << dig_w | d] = base[d] + sum over rows e < s * rows_per_part of
// part[e][d], base[d] = sum of hist[d'] over d' < d (the pass's histogram).
// Workgroup b covers the rows of k_reduce_rows's workgroup b (span rows, a
// multiple of rows_per_part) and starts from the column sums of the chunks
// before it. Thread (d, g): digit d, g-th contiguous run of the chunk's
// partitions; the runs' sums are scanned in LDS, then each thread writes its
// partitions' offsets. No look-back: every workgroup reads only sums that the
// reduce finished before this kernel started. Nothing is done after an
// upstream failure (ctl).
constexpr int kOffsThreads = 1024;
__global__ __launch_bounds__(kOffsThreads) void k_part_offsets(
    const uint32_t* __restrict__ part, int cols, uint32_t rows_cap, uint32_t span,
    const uint32_t* __restrict__ count_dev, uint32_t count_cap, uint32_t per_row,
    int rows_per_part, int dig_w, const uint32_t* __restrict__ chunks,
    const uint32_t* __restrict__ hist, uint32_t* __restrict__ offs, const uint32_t* ctl) {
    __shared__ uint32_t s_base[256];
    __shared__ uint32_t s_run[kOffsThreads];
    if (upstream_failed(ctl)) return;  // uniform over the workgroup
    const uint32_t rows = rows_in_use(rows_cap, count_dev, count_cap, per_row);
    const uint32_t r0 = blockIdx.x * span;
    if (r0 >= rows) return;  // uniform over the workgroup
    const int nd = 1 << dig_w, G = kOffsThreads / nd;
    const int tid = threadIdx.x, d = tid % nd, g = tid / nd;
    // digit bases: exclusive scan of the pass's histogram (one wave, four
    // digits per lane)
    if (tid < GS_WAVE) {
        uint32_t h[4], sum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int dd = tid * 4 + i;
            h[i] = dd < nd ? hist[dd] : 0u;
            sum += h[i];
        }
        uint32_t ex = wave_incl_scan(sum) - sum;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (tid * 4 + i < nd) s_base[tid * 4 + i] = ex;
            ex += h[i];
        }
    }
    // counts of the chunks before this one
    uint32_t pre = 0;
#pragma unroll 4
    for (uint32_t b = (uint32_t)g; b < blockIdx.x; b += (uint32_t)G)
        pre += chunks[(size_t)b * cols + d];
    // this thread's run of partitions inside the chunk
    const uint32_t r1 = min(rows, r0 + span);
    const uint32_t p0 = r0 / rows_per_part;
    const uint32_t nparts = (r1 - r0 + rows_per_part - 1) / rows_per_part;
    const uint32_t per = (nparts + G - 1) / G;
    const uint32_t q0 = min(nparts, (uint32_t)g * per), q1 = min(nparts, q0 + per);
    uint32_t run = 0;
    const uint32_t ea = r0 + q0 * rows_per_part, eb = min(r1, r0 + q1 * rows_per_part);
#pragma unroll 8
    for (uint32_t e = ea; e < eb; ++e) run += part[(size_t)e * cols + d];
    s_run[tid] = pre;
    __syncthreads();
    uint32_t carry = s_base[d];
    for (int gg = 0; gg < G; ++gg) carry += s_run[gg * nd + d];  // chunks before
    __syncthreads();
    s_run[tid] = run;
    __syncthreads();
    for (int gg = 0; gg < g; ++gg) carry += s_run[gg * nd + d];  // earlier runs
    for (uint32_t q = q0; q < q1; ++q) {
        offs[((size_t)(p0 + q) << dig_w) | (uint32_t)d] = carry;
        const uint32_t e0 = r0 + q * rows_per_part;
        const uint32_t e1 = min(r1, e0 + rows_per_part);
#pragma unroll 4
        for (uint32_t e = e0; e < e1; ++e) carry += part[(size_t)e * cols + d];
    }
}

// Tile ranges from per-tile pair counts in one workgroup: each thread sums a
// block of consecutive tiles, the block sums are scanned, and each thread
// writes its tiles' [start, end) (sort.cpp:146-165: (0, 0) for an empty tile).
constexpr int kRangeThreads = 1024;
__global__ __launch_bounds__(kRangeThreads) void k_ranges_from_counts(
    const uint32_t* __restrict__ counts, uint32_t ntiles, uint32_t* __restrict__ ranges) {
    __shared__ uint32_t s_w[kRangeThreads / GS_WAVE];
    const int tid = threadIdx.x, w = tid / GS_WAVE, lane = lane_id();
    const uint32_t per = (ntiles + kRangeThreads - 1) / kRangeThreads;
    const uint32_t t0 = min(ntiles, (uint32_t)tid * per), t1 = min(ntiles, t0 + per);
    uint32_t sum = 0;
    for (uint32_t t = t0; t < t1; ++t) sum += counts[t];
    const uint32_t inc = wave_incl_scan(sum);
    if (lane == GS_WAVE - 1) s_w[w] = inc;
    __syncthreads();
    uint32_t pre = 0;
    for (int i = 0; i < w; ++i) pre += s_w[i];
    uint32_t start = pre + inc - sum;
    for (uint32_t t = t0; t < t1; ++t) {
        const uint32_t c = counts[t];
        ranges[2 * (size_t)t] = c ? start : 0u;
        ranges[2 * (size_t)t + 1] = c ? start + c : 0u;
        start += c;
    }
}

// key = (tile << 32) | fp32 depth bits of the pair's Gaussian (sort.cpp:180-205).
__global__ void k_make_keys64(const uint32_t* __restrict__ gid, const uint32_t* __restrict__ tid,
                              const float* __restrict__ depths, uint32_t p,
                              uint64_t* __restrict__ keys) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= p) return;
    keys[i] = ((uint64_t)tid[i] << 32) | (uint64_t)__float_as_uint(depths[gid[i]]);
}

__global__ void k_tile_ranges64(const uint64_t* __restrict__ keys, uint32_t p,
                                uint32_t* __restrict__ ranges) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= p) return;
    const uint32_t t = (uint32_t)(keys[i] >> 32);
    if (i == 0 || (uint32_t)(keys[i - 1] >> 32) != t) ranges[2 * (size_t)t] = i;
    if (i == p - 1 || (uint32_t)(keys[i + 1] >> 32) != t) ranges[2 * (size_t)t + 1] = i + 1;
}

}  // namespace

hipError_t launch_make_keys64(const uint32_t* gid, const uint32_t* tid, const float* depths,
                              uint32_t p, uint64_t* keys, hipStream_t st) {
    if (p == 0) return hipSuccess;
    k_make_keys64<<<(p + 255) / 256, 256, 0, st>>>(gid, tid, depths, p, keys);
    return hipGetLastError();
}

hipError_t launch_tile_ranges64(const uint64_t* keys, uint32_t p, uint32_t* ranges,
                                int64_t num_tiles, hipStream_t st) {
    hipError_t e = launch_fill_u32(ranges, 0u, (size_t)num_tiles * 2, st);
    if (e != hipSuccess || p == 0) return e;
    k_tile_ranges64<<<(p + 255) / 256, 256, 0, st>>>(keys, p, ranges);
    return hipGetLastError();
}

size_t rect_scan_partitions(int64_t m) { return (size_t)((m + kCountPart - 1) / kCountPart); }
size_t emit_partitions(uint64_t p_pre) { return (size_t)((p_pre + kEmitPart - 1) / kEmitPart); }

hipError_t launch_rect_count_scan(const float4* rect, int stride, const uint32_t* order,
                                  int64_t m, const uint32_t* m_dev, TileParams tp, uint32_t* offs,
                                  uint32_t* bstart, uint32_t bstart_cap, uint64_t* lb_state,
                                  uint32_t* ticket, uint32_t* total_out, uint32_t cap,
                                  bool reduce_scan, hipStream_t st) {
    if (m <= 0) return hipSuccess;
    if (stride < 1) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)rect_scan_partitions(m);
    if (!reduce_scan) {
        k_rect_count_scan<kScanLookback><<<grid, kCountThreads, 0, st>>>(
            rect, stride, order, m, m_dev, tp, offs, bstart, bstart_cap, lb_state, ticket,
            total_out, cap);
        return hipGetLastError();
    }
    k_rect_count_scan<kScanReduce><<<grid, kCountThreads, 0, st>>>(
        rect, stride, order, m, m_dev, tp, offs, bstart, bstart_cap, lb_state, ticket, total_out,
        cap);
    k_scan_part_sums<<<1, kSumThreads, 0, st>>>(lb_state, m, m_dev, total_out, cap, tp.ctl);
    k_rect_count_scan<kScanFinal><<<grid, kCountThreads, 0, st>>>(
        rect, stride, order, m, m_dev, tp, offs, bstart, bstart_cap, lb_state, ticket, total_out,
        cap);
    return hipGetLastError();
}

hipError_t launch_pair_emit(const float4* rect, const float4* cov, int stride, bool by_order,
                            const uint32_t* order,
                            const uint32_t* offs, const uint32_t* bstart, int64_t m,
                            const uint32_t* m_dev, uint32_t p_pre, const uint32_t* p_pre_dev,
                            TileParams tp, uint32_t* pair_tile, uint32_t* pair_id, uint32_t cap,
                            uint64_t* lb_state, uint32_t* ticket, uint32_t* total_out,
                            uint32_t* part_hist, int tile_bits, bool compact, hipStream_t st) {
    if (p_pre == 0 || m <= 0) return hipSuccess;
    if (stride < 1 || (by_order && order == nullptr)) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)emit_partitions(p_pre);
    // at most three digits of at most 8 bits (tile ids below 2^24)
    if (tile_bits < 1 || tile_bits > 24) return hipErrorInvalidValue;
    // a rectangle's corner is held in two 16-bit fields
    if (tp.tiles_x < 1 || tp.tiles_x > 65535 || tp.tiles_y < 1 || tp.tiles_y > 65535)
        return hipErrorInvalidValue;
    const int dbits = sort_digit_width(tile_bits);
    const bool three = tile_bits > 16;
#define GS_EMIT(CP, ND)                                                                    \
    k_pair_emit<CP, ND><<<grid, kEmitThreads, 0, st>>>(                                    \
        rect, cov, stride, by_order, order, offs, bstart, m, m_dev, p_pre, p_pre_dev, tp,    \
        pair_tile, pair_id,                                                                \
        cap, lb_state, ticket, total_out, part_hist, dbits)
    if (compact) {
        if (three) GS_EMIT(true, 3); else GS_EMIT(true, 2);
    } else {
        if (three) GS_EMIT(false, 3); else GS_EMIT(false, 2);
    }
#undef GS_EMIT
    return hipGetLastError();
}

hipError_t launch_tile_ranges(const uint32_t* sorted_tile, uint32_t p, const uint32_t* p_dev,
                              uint32_t* ranges, int64_t num_tiles, hipStream_t st) {
    hipError_t e = launch_fill_u32(ranges, 0u, (size_t)num_tiles * 2, st);
    if (e != hipSuccess || p == 0) return e;
    const unsigned grid = std::min<unsigned>((p + 255) / 256, 4096u);
    k_tile_ranges<<<grid, 256, 0, st>>>(sorted_tile, p, p_dev, ranges);
    return hipGetLastError();
}

hipError_t launch_ranges_from_counts(const uint32_t* counts, int64_t num_tiles, uint32_t* ranges,
                                     hipStream_t st) {
    if (num_tiles <= 0) return hipSuccess;
    if (num_tiles > ((int64_t)1 << 24)) return hipErrorInvalidValue;
    k_ranges_from_counts<<<1, kRangeThreads, 0, st>>>(counts, (uint32_t)num_tiles, ranges);
    return hipGetLastError();
}

hipError_t launch_tile_bounds(const uint32_t* sorted_tile, uint32_t p_cap, const uint32_t* p_dev,
                              uint32_t* ranges, int64_t num_tiles, hipStream_t st) {
    if (num_tiles <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((num_tiles + 3) / 4);
    k_tile_bounds<uint32_t><<<grid, 256, 0, st>>>(sorted_tile, p_cap, p_dev, ranges,
                                                  (uint32_t)num_tiles, nullptr);
    return hipGetLastError();
}

hipError_t launch_tile_bounds64(const uint64_t* sorted_keys, uint32_t p, uint32_t* ranges,
                                int64_t num_tiles, uint32_t* ctl, hipStream_t st) {
    if (num_tiles <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((num_tiles + 3) / 4);
    k_tile_bounds<uint64_t><<<grid, 256, 0, st>>>(sorted_keys, p, nullptr, ranges,
                                                  (uint32_t)num_tiles, ctl);
    return hipGetLastError();
}

uint32_t reduce_span(uint32_t rows_cap) {
    const uint32_t span = std::max<uint32_t>(32, (rows_cap + kRedBlocks - 1) / kRedBlocks);
    return (span + 3u) & ~3u;
}

size_t reduce_chunks(uint32_t rows_cap) {
    const uint32_t span = reduce_span(rows_cap);
    return (rows_cap + span - 1) / span;
}

hipError_t launch_reduce_rows(const uint32_t* part, int cols, uint32_t rows_cap,
                              const uint32_t* count_dev, uint32_t count_cap, uint32_t per_row,
                              int dig_w, uint32_t* out, hipStream_t st, uint32_t* chunk_out,
                              const uint32_t* ctl) {
    if (rows_cap == 0) return hipSuccess;
    if (cols <= 0 || cols % 4 != 0 || kRedThreads % (cols / 4) != 0) return hipErrorInvalidValue;
    const uint32_t span = reduce_span(rows_cap);
    const unsigned grid = (rows_cap + span - 1) / span;
    if (dig_w < 0 || dig_w > 8) return hipErrorInvalidValue;
    k_reduce_rows<<<grid, kRedThreads, 0, st>>>(part, cols, rows_cap, span, count_dev,
                                                count_cap, per_row, dig_w, out, chunk_out, ctl);
    return hipGetLastError();
}

hipError_t launch_part_offsets(const uint32_t* part, int cols, uint32_t rows_cap,
                               const uint32_t* count_dev, uint32_t count_cap, uint32_t per_row,
                               int rows_per_part, int dig_w, const uint32_t* chunks,
                               const uint32_t* hist, uint32_t* offs, hipStream_t st,
                               const uint32_t* ctl) {
    if (rows_cap == 0) return hipSuccess;
    const uint32_t span = reduce_span(rows_cap);
    if (dig_w < 0 || dig_w > 8 || (1 << dig_w) > cols || rows_per_part <= 0 ||
        span % (uint32_t)rows_per_part != 0)
        return hipErrorInvalidValue;
    const unsigned grid = (rows_cap + span - 1) / span;
    k_part_offsets<<<grid, kOffsThreads, 0, st>>>(part, cols, rows_cap, span, count_dev,
                                                  count_cap, per_row, rows_per_part, dig_w,
                                                  chunks, hist, offs, ctl);
    return hipGetLastError();
}

}  // namespace gs
