// blend.hip - per-tile microblock cull + front-to-back alpha blend on gfx950.
//
// The reference blends each tile as 8x4-pixel microblocks, each with its own
// depth-ordered kept list (src/gsplat_cpu/cull_and_blend.cpp:384-504) and its
// own early-out (:578-616). Here one wave64 owns a 16x4 pixel band of a tile,
// i.e. two horizontally adjacent microblocks: lanes 0-31 are microblock A,
// lanes 32-63 microblock B, lane = row*8 + column inside the microblock.
//
// Per batch of 32 depth-ordered tile entries the wave
//   1. loads the 48-byte records (lane q and lane q+32 hold entry q),
//   2. evaluates the constrained-minimum microblock cull for (entry, own
//      microblock) -> a 64-bit ballot = both halves' kept masks,
//   3. stages the entries in LDS and walks the union of the two kept masks in
//      depth order; transmittance and colour stay in VGPRs.
// Bands whose two microblocks are fully inside the image (all but the image
// edge) follow the reference's AVX2 arithmetic exactly (degree-4 exp, power
// clamp [-30,0], T -= alpha*T, early-out test every 4 kept entries): per entry,
// the terms that depend on the pixel row or column only are staged once and
// every lane evaluates the entry, its half's opacity being 0 where that half
// drops it. Edge bands follow the scalar rule for edge microblocks (exp,
// T *= 1-alpha, test after every entry) (cull_and_blend.cpp:506-670,
// simd_exp_avx2.h:12-32), a lane evaluating only what its half keeps. The wave
// exits when both microblocks are done.
#include <algorithm>

#include "gs_common.h"
#include "gs_internal.h"

namespace gs {
namespace {

__device__ __forceinline__ float fmin_std(float a, float b) { return (b < a) ? b : a; }
__device__ __forceinline__ float fmax_std(float a, float b) { return (a < b) ? b : a; }
__device__ __forceinline__ float fclamp_std(float v, float lo, float hi) {
    return (v < lo) ? lo : ((hi < v) ? hi : v);
}

// Degree-4 Maclaurin exp with 2^n reconstruction, simd_exp_avx2.h:12-32.
__device__ __forceinline__ float exp4(float x) {
    const float LOG2E = 1.44269504088896f;
    const float LN2 = 0.69314718055994530942f;
    const float y = x * LOG2E;
    const float fn = __builtin_rintf(y);
    const int n = (int)fn;
    const float r = __builtin_fmaf(-fn, LN2, x);
    const float r2 = r * r;
    const float p0 = __builtin_fmaf(r, 1.0f, 1.0f);
    float p1 = __builtin_fmaf(r, 0.166666666667f, 0.5f);
    p1 = __builtin_fmaf(r2, 0.041666666667f, p1);
    const float p = __builtin_fmaf(r2, p1, p0);
    // p * 2^n with 2^n a normal float (n >= -44 here): exact scaling.
    return __builtin_amdgcn_ldexpf(p, n);
}


// u8 of a bf16 colour, uint8(float32(clip(float32(b), 0, 1)) * 255) with
// truncation, in integer form: a bf16 in [0, 1) is (128 + m) 2^(e - 134), so
// the product with 255 is exact and truncates to ((128 + m) 255) >> (134 - e)
// (render/kernels/dataflow/img_pack_u8.h:9-14,31-41, the u8 that the
// reference's render_view returns).
__device__ __forceinline__ uint8_t bf16_to_u8(uint32_t b) {
    const uint32_t e = (b >> 7) & 0xFFu;
    if ((b & 0x8000u) != 0u || e < 119u) return 0u;
    if (e >= 127u) return 255u;
    const uint32_t sig = 128u + (b & 0x7Fu);
    return (uint8_t)(((sig << 8) - sig) >> (134u - e));
}

// Per-wave geometry of one 16x4 band (two microblocks).
struct Band {
    int tile, tile_x, tile_y, mbx, mby;
    int px_start, py0;
    float tx_tile, ty_tile, pxs, offx, pxc, pyc, mb_ox, mb_oy;
    float ext_x0, ext_x1, ext_y0, ext_y1;  // the microblock's extent-test bounds
    float pxsA, pyr0;  // band: microblock A's first column, first row centre (+0.5)
    bool emptyA, emptyB, fullA, fullB, full, pix_valid;
};

template <int TS>
__device__ __forceinline__ Band make_band(const BlendParams& bp, int lane) {
    constexpr int BX = TS / 16;  // 16-pixel band columns per tile
    constexpr int BY = TS / 4;   // 4-row bands per tile
    Band g;
    const int band = blockIdx.x % (BX * BY);
    g.tile = blockIdx.x / (BX * BY);
    const int bx = band % BX, by = band / BX;
    g.tile_x = g.tile % bp.tiles_x;
    g.tile_y = g.tile / bp.tiles_x;
    const int h = lane >> 5, q = lane & 31, pi = q >> 3, pj = q & 7;
    g.mbx = bx * 2 + h;
    g.mby = by;
    const int px_tile = g.tile_x * TS, py_tile = g.tile_y * TS;
    const int px_end_tile = min(px_tile + TS, bp.width);
    const int py_end_tile = min(py_tile + TS, bp.height);
    // microblock extents of both halves (wave-uniform)
    const int pxA = px_tile + (bx * 2) * 8, pxB = pxA + 8;
    g.py0 = py_tile + g.mby * 4;
    const int pyE = min(g.py0 + 4, py_end_tile);
    const int pxEA = min(pxA + 8, px_end_tile), pxEB = min(pxB + 8, px_end_tile);
    g.emptyA = (g.py0 >= pyE) || (pxA >= pxEA);
    g.emptyB = (g.py0 >= pyE) || (pxB >= pxEB);
    g.fullA = !g.emptyA && (pxEA - pxA == 8) && (pyE - g.py0 == 4);
    g.fullB = !g.emptyB && (pxEB - pxB == 8) && (pyE - g.py0 == 4);
    g.px_start = h ? pxB : pxA;
    const int px_end = h ? pxEB : pxEA;
    g.full = h ? g.fullB : g.fullA;
    g.pix_valid = !(h ? g.emptyB : g.emptyA) && (g.px_start + pj < px_end) && (g.py0 + pi < pyE);
    g.tx_tile = (float)(g.tile_x * TS);
    g.ty_tile = (float)(g.tile_y * TS);
    g.pxs = (float)g.px_start;                  // full path: px_base = pxs - mx
    g.offx = (float)pj + 0.5f;
    g.pxc = (float)(g.px_start + pj) + 0.5f;    // scalar path pixel centre
    g.pyc = (float)(g.py0 + pi) + 0.5f;
    g.pxsA = (float)pxA;
    g.pyr0 = (float)g.py0 + 0.5f;
    // microblock cull rectangle (cull_and_blend.cpp:447-498)
    g.mb_oy = g.ty_tile + (float)(g.mby * 4);
    g.mb_ox = g.tx_tile + (float)(g.mbx * 8);
    g.ext_x0 = (float)(8 * g.mbx);
    g.ext_x1 = (float)(8 * g.mbx + 8);
    g.ext_y0 = (float)(4 * g.mby);
    g.ext_y1 = (float)(4 * g.mby + 4);
    return g;
}

// Constrained-minimum cull of one entry against the lane's microblock
// (cull_and_blend.cpp:447-498).
__device__ __forceinline__ bool mb_keep(const Band& g, float4 r0, float4 r1, int cull_disabled) {
    const float lt = r1.w;
    const float mx = r0.x, my = r0.y;
    // The reference's microblock range of the extent, mx_lo = max(0, floor(ax / 8)),
    // mx_hi = min(3, floor(bx / 8)) (and 4-row ones in y), tested against this
    // microblock's column mbx without the integer round trip: mbx >= 0 and
    // mbx <= 3, the divisions by 8 and 4 are exact, and floor(t) <= k <=> t < k + 1,
    // k <= floor(t) <=> k <= t for an integer k, so
    // mx_lo <= mbx <=> ax < 8 mbx + 8 and mbx <= mx_hi <=> 8 mbx <= bx.
    // (The extents of a projected record are finite and far inside the int range.)
    const float ax = (mx - r0.z) - g.tx_tile, bx = (mx + r0.z) - g.tx_tile;
    const float ay = (my - r0.w) - g.ty_tile, by = (my + r0.w) - g.ty_tile;
    // (one test with the floor check, lt < 0, so the record is read whole first)
    if (!((lt < 0.0f) & (ax < g.ext_x1) & (g.ext_x0 <= bx) & (ay < g.ext_y1) & (g.ext_y0 <= by)))
        return false;
    const float ci_a = r1.x, ci_b = r1.y, ci_c = r1.z;
    const float v_lo = g.mb_oy - my;
    const float v_hi = v_lo + 4.0f;
    const bool y_in = (v_lo <= 0.0f) && (0.0f <= v_hi);
    const float v_fix = (v_lo > 0.0f) ? v_lo : v_hi;
    const float u_lo = g.mb_ox - mx;
    const float u_hi = u_lo + 8.0f;
    const bool x_in = (u_lo <= 0.0f) && (0.0f <= u_hi);
    float m2_min;
    if (cull_disabled || (x_in && y_in)) {
        m2_min = 0.0f;
    } else {
        float m2_v = __builtin_inff(), m2_h = __builtin_inff();
        if (!x_in) {
            const float uf = (u_lo > 0.0f) ? u_lo : u_hi;
            float vs = -ci_b * uf / fmax_std(ci_c, 1e-12f);
            // clamp to [v_lo, v_hi] (v_lo < v_hi; vs is not NaN for a projected record)
            vs = __builtin_amdgcn_fmed3f(vs, v_lo, v_hi);
            m2_v = ci_a * uf * uf + 2.0f * ci_b * uf * vs + ci_c * vs * vs;
        }
        if (!y_in) {
            float us = -ci_b * v_fix / fmax_std(ci_a, 1e-12f);
            us = __builtin_amdgcn_fmed3f(us, u_lo, u_hi);
            m2_h = ci_a * us * us + 2.0f * ci_b * us * v_fix + ci_c * v_fix * v_fix;
        }
        m2_min = fmin_std(m2_v, m2_h);
    }
    return m2_min <= -2.0f * lt;
}

// Entry parameters of an image-edge band's batch, staged in LDS (mx, my, op |
// -ci_a/2, -ci_b, -ci_c/2 | r, g, b) and read back with wave-uniform addresses
// (a broadcast, on the LDS pipe).
struct BatchRec {
    float4 p0, p1, p2;
};

// LDS staging of an interior band's batch: per entry, the terms of the AVX2
// power that depend on the pixel row (y_term = C dy dy, xy_coef = B dy for the
// band's 4 rows) and on the pixel column (dx = (px0 - mx) + (c + 0.5) for the
// 16 columns of the two microblocks), the quadratic coefficient with each
// half's opacity (zero where that half's microblock drops the entry), and the
// colour: each computed once per entry instead of once per pixel. 4 KiB, so
// eight one-wave workgroups per SIMD still fit in the CU's LDS.
struct BandStage {
    float4 rows[32][2];   // rows 2k, 2k+1: (y_term, xy_coef, y_term, xy_coef)
    float4 dx[32][4];     // columns 4k .. 4k+3
    float2 aop[32][2];    // (-ci_a/2, op or 0) per half
    float4 rgb[32];       // the record's (r, g, b, opacity)
};
union BlendLds {
    BatchRec rec[32];     // image-edge bands
    BandStage band;       // interior bands
};

// The batch loop of an interior band (both microblocks fully inside the
// image: AVX2 rule, every pixel valid). Costs are per (entry, wave), and a
// scalar instruction costs about two vector ones (one scalar unit serves the
// CU's four SIMDs), so the bookkeeping is vector and per lane, uniform within
// each half: `mine` = the half's kept entries of the batch, `cnt` = entries
// the half has blended. The entries where a half tests for its early-out
// (its count reaches a multiple of 4, cull_and_blend.cpp:578-616) are found
// once per batch, lane-parallel (lane q marks entry q). The 32 entries of a
// batch are then walked in a loop unrolled at compile time: each entry is
// evaluated for every lane (about 92 % of the batch's entries are kept by one
// half or the other, so no scalar walk of the union pays off), staged terms
// are read at immediate LDS offsets, and a lane whose half drops the entry
// sees opacity 0: alpha 0 leaves T and the colour exactly as they are
// (fma(0, c, x) = x, x - 0 = x), so no per-entry select. A half that retires
// inside a batch keeps evaluating that batch's entries it had kept, so its
// colour is saved at the retirement and restored at the end.
__device__ __forceinline__ void blend_band_interior(const Band& g, const float4* __restrict__ brec,
                                                    const uint32_t* __restrict__ sid,
                                                    uint32_t start, uint32_t end,
                                                    const BlendParams& bp, int lane,
                                                    BandStage* st, float& cr, float& cg,
                                                    float& cb, uint32_t& cnt,
                                                    uint32_t& n_batch, uint32_t& n_iter,
                                                    uint32_t& n_kept) {
    const int h = lane >> 5, q = lane & 31;
    const int pi = q >> 3, col = h * 8 + (q & 7);  // the lane's pixel in the band
    const int half = (int)(blockDim.x >> 1);  // 32 lanes per microblock
    const uint32_t below = (1u << q) - 1u;    // lanes of the half before this one
    const float thr = bp.thr;
    float T = 1.0f;
    float sr = 0.0f, sg = 0.0f, sb = 0.0f;  // colour at the half's retirement
    bool alive = true;  // this lane's half has not retired
    for (uint32_t base = start; base < end; base += 32) {
        const uint32_t idx = base + q;
        const bool has = idx < end;
        // lanes past the tile's end load its last entry (never walked: not kept)
        const uint32_t gi = sid[has ? idx : end - 1];
        const float4 r0 = brec[3 * (size_t)gi + 0];
        const float4 r1 = brec[3 * (size_t)gi + 1];
        const float4 r2 = brec[3 * (size_t)gi + 2];
        const bool keep = has && alive && mb_keep(g, r0, r1, bp.cull_disabled);
        const uint64_t mask = __ballot(keep);
        ++n_batch;
        uint32_t mlo = (uint32_t)mask, mhi = (uint32_t)(mask >> half);
        n_kept += (uint32_t)(__builtin_popcount(mlo) + __builtin_popcount(mhi));
        const uint32_t mine = h ? mhi : mlo;
        uint32_t uni = mlo | mhi;  // uniform: entries either half keeps
        n_iter += (uint32_t)__builtin_popcount(uni);
        // early-out test points of this batch: lane q marks entry q
        const bool pt = ((mine >> q) & 1u) &&
                        ((cnt + (uint32_t)__builtin_popcount(mine & below) + 1u) & 3u) == 0u;
        const uint64_t pts = __ballot(pt);
        uint32_t plo = (uint32_t)pts, phi = (uint32_t)(pts >> half);
        uint32_t pany = plo | phi;  // uniform: entries after which a half tests
        cnt += (uint32_t)__builtin_popcount(mine);
        // stage entry q (both halves hold its record): half h its rows 2h, 2h+1,
        // its columns 8h .. 8h+7 and its own opacity, both the colour (the
        // AVX2 rule's operations, cull_and_blend.cpp:194-279: px_base = px0 - mx,
        // dx = px_base + (c + 0.5), dy = py + 0.5 - my, y_term = C dy dy,
        // xy_coef = B dy)
        {
            const float Bq = -r1.y, Cq = -0.5f * r1.z;
            const float dy0 = g.pyr0 + (float)(2 * h) - r0.y;
            const float dy1 = g.pyr0 + (float)(2 * h + 1) - r0.y;
            st->rows[q][h] = make_float4(Cq * dy0 * dy0, Bq * dy0, Cq * dy1 * dy1, Bq * dy1);
            const float pb = g.pxs - r0.x;
            st->dx[q][2 * h] = make_float4(pb + 0.5f, pb + 1.5f, pb + 2.5f, pb + 3.5f);
            st->dx[q][2 * h + 1] = make_float4(pb + 4.5f, pb + 5.5f, pb + 6.5f, pb + 7.5f);
            st->aop[q][h] = make_float2(-0.5f * r1.x, keep ? r2.w : 0.0f);
            st->rgb[q] = r2;  // both halves hold entry q's record: the same words
        }
        __syncthreads();  // one wave per workgroup: orders the LDS writes and reads
        const float* rowp = &st->rows[0][pi >> 1].x + 2 * (pi & 1);
        const float* dxp = &st->dx[0][0].x + col;
        bool retired = false;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            if (((uni >> j) & 1u) == 0u) continue;  // neither half keeps entry j
            // AVX2 rule for the lane's pixel: power clamp [-30, 0], degree-4
            // exp, alpha <= 0.99 (the staged terms are the same fp32 values)
            const float2 rt = *reinterpret_cast<const float2*>(rowp + 8 * j);
            const float dx = dxp[16 * j];
            const float2 ao = st->aop[j][h];
            float pwr = __builtin_fmaf(rt.y, dx, rt.x);
            pwr = __builtin_fmaf(ao.x, dx * dx, pwr);
            pwr = __builtin_amdgcn_fmed3f(pwr, -30.0f, 0.0f);
            float al = ao.y * exp4(pwr);
            al = (al < 0.99f) ? al : 0.99f;
            const float4 e2 = st->rgb[j];
            const float at = al * T;
            cr = __builtin_fmaf(at, e2.x, cr);
            cg = __builtin_fmaf(at, e2.y, cg);
            cb = __builtin_fmaf(at, e2.z, cb);
            T = T - at;
            if ((pany >> j) & 1u) {
                // max over the microblock's pixels < thr <=> no pixel has T >= thr
                const uint64_t live = __ballot(!(T < thr));
                const bool deadA = ((plo >> j) & 1u) && (uint32_t)live == 0u;
                const bool deadB = ((phi >> j) & 1u) && (uint32_t)(live >> half) == 0u;
                if (deadA || deadB) {
                    // a retired half blends nothing more: its later kept entries
                    // are dropped (from its count too, which the statistics
                    // report) and it has no later test points
                    const bool me = h ? deadB : deadA;
                    if (me) {
                        cnt -= (uint32_t)__builtin_popcount((mine >> j) >> 1);
                        alive = false;
                        sr = cr;
                        sg = cg;
                        sb = cb;
                    }
                    if (deadA) mlo = plo = 0u;
                    if (deadB) mhi = phi = 0u;
                    const uint32_t later = uni & ~(mlo | mhi);
                    n_iter -= (uint32_t)__builtin_popcount((later >> j) >> 1);
                    uni = mlo | mhi;
                    pany = plo | phi;
                    if (__ballot(alive) == 0ull) {
                        retired = true;
                        break;
                    }
                }
            }
        }
        if (retired) break;
        __syncthreads();  // the next batch overwrites the staged records
    }
    if (!alive) {
        cr = sr;
        cg = sg;
        cb = sb;
    }
}

// The batch loop of a band that the image edge cuts: per-half state in VGPRs
// (uniform within the half: `mine` = the half's kept entries of the batch,
// cleared once the half is done; `cnt` = entries the half has blended), the
// scalar unit walks the union of both halves' masks, and a lane evaluates an
// entry only when its half keeps it and its pixel is inside the image.
__device__ __forceinline__ void blend_band_edge(const Band& g, const float4* __restrict__ brec,
                                           const uint32_t* __restrict__ sid, uint32_t start,
                                           uint32_t end, const BlendParams& bp, int lane,
                                           BatchRec* s_rec, float& T, float& cr, float& cg,
                                           float& cb, uint32_t& cnt, uint32_t& n_batch,
                                           uint32_t& n_iter, uint32_t& n_kept) {
    const int h = lane >> 5, q = lane & 31;
    bool doneA = g.emptyA, doneB = g.emptyB;
    for (uint32_t base = start; base < end && !(doneA && doneB); base += 32) {
        const uint32_t idx = base + q;
        const bool has = idx < end;
        float4 r0 = make_float4(0, 0, 0, 0), r1 = r0, r2 = r0;
        if (has) {
            const uint32_t gi = sid[idx];
            r0 = brec[3 * (size_t)gi + 0];
            r1 = brec[3 * (size_t)gi + 1];
            r2 = brec[3 * (size_t)gi + 2];
        }
        const bool my_done = h ? doneB : doneA;
        const bool keep = has && !my_done && mb_keep(g, r0, r1, bp.cull_disabled);
        const uint64_t mask = __ballot(keep);
        ++n_batch;
        n_kept += (uint32_t)__popcll(mask);
        const uint32_t mA = (uint32_t)mask, mB = (uint32_t)(mask >> 32);
        uint32_t mine = h ? mB : mA;
        // power coefficients of the AVX2 path (cull_and_blend.cpp:198-200): exact
        // scalings of the conic, so the image-edge rule recovers it exactly
        if (h == 0) {
            s_rec[q].p0 = make_float4(r0.x, r0.y, r2.w, 0.0f);
            s_rec[q].p1 = make_float4(-0.5f * r1.x, -r1.y, -0.5f * r1.z, 0.0f);
            s_rec[q].p2 = r2;
        }
        __syncthreads();  // one wave per workgroup: orders the LDS writes and reads
        uint32_t uni = mA | mB;
        while (uni) {
            const int j = __builtin_ctz(uni);
            uni &= uni - 1;
            ++n_iter;
            const float4 e0 = s_rec[j].p0, e1 = s_rec[j].p1, e2 = s_rec[j].p2;
            const float mx = e0.x, my = e0.y, op = e0.z;
            const float A = e1.x, B = e1.y, C = e1.z;
            const bool run = (mine >> j) & 1u;
            if (run) {
                if (g.full) {
                    const float px_base = g.pxs - mx;
                    const float dx = px_base + g.offx;
                    const float dx_sq = dx * dx;
                    const float dy = g.pyc - my;
                    const float y_term = C * dy * dy;
                    const float xy_coef = B * dy;
                    float pwr = __builtin_fmaf(xy_coef, dx, y_term);
                    pwr = __builtin_fmaf(A, dx_sq, pwr);
                    pwr = (pwr < 0.0f) ? pwr : 0.0f;
                    pwr = (pwr > -30.0f) ? pwr : -30.0f;
                    const float gw = exp4(pwr);
                    float al = op * gw;
                    al = (al < 0.99f) ? al : 0.99f;
                    const float at = al * T;
                    cr = __builtin_fmaf(at, e2.x, cr);
                    cg = __builtin_fmaf(at, e2.y, cg);
                    cb = __builtin_fmaf(at, e2.z, cb);
                    T = T - at;
                } else if (g.pix_valid) {
                    const float ci_a = -2.0f * A, ci_b = -B, ci_c = -2.0f * C;
                    const float dx = g.pxc - mx;
                    const float dy = g.pyc - my;
                    const float power =
                        -0.5f * (ci_a * dx * dx + 2.0f * ci_b * dx * dy + ci_c * dy * dy);
                    const float gw = expf(fmin_std(power, 0.0f));
                    const float al = fmin_std(op * gw, 0.99f);
                    const float at = al * T;
                    cr += at * e2.x;
                    cg += at * e2.y;
                    cb += at * e2.z;
                    T = T * (1.0f - al);
                }
                ++cnt;
            }
            // early-out test: every 4 kept entries of a full microblock, after
            // every entry of an image-edge one (cull_and_blend.cpp:578-616)
            const bool chk = run && (!g.full || (cnt & 3u) == 0u);
            const uint64_t chkm = __ballot(chk);
            if (chkm != 0) {
                // max over the microblock's pixels < thr  <=>  no pixel has T >= thr
                // (T is never NaN; edge pixels outside the image do not vote)
                const uint64_t live = __ballot(g.pix_valid && !(T < bp.thr));
                const bool deadA = (uint32_t)chkm != 0u && (uint32_t)live == 0u;
                const bool deadB = (uint32_t)(chkm >> 32) != 0u && (uint32_t)(live >> 32) == 0u;
                if (deadA) doneA = true;
                if (deadB) doneB = true;
                const uint32_t keepA = doneA ? 0u : mA, keepB = doneB ? 0u : mB;
                uni &= keepA | keepB;
                mine = h ? keepB : keepA;
                if (doneA && doneB) return;
            }
        }
        __syncthreads();  // the next batch overwrites the staged records
    }
}

template <int TS, int OUT>
__global__ __launch_bounds__(GS_WAVE) void k_blend(const float4* __restrict__ brec,
                                                   const uint32_t* __restrict__ sid,
                                                   const uint32_t* __restrict__ ranges,
                                                   BlendParams bp, void* __restrict__ out) {
    const int lane = threadIdx.x;
    // after an earlier give-up the sorted ids may be wrong: read nothing
    if (__builtin_amdgcn_readfirstlane(upstream_failed(bp.ctl) ? 1 : 0)) return;
    const Band g = make_band<TS>(bp, lane);
    float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
    uint32_t cnt = 0, n_batch = 0, n_iter = 0, n_kept = 0;
    const uint32_t start = ranges[2 * g.tile], end = ranges[2 * g.tile + 1];
    __shared__ BlendLds lds;
    if (g.fullA && g.fullB)
        blend_band_interior(g, brec, sid, start, end, bp, lane, &lds.band, cr, cg, cb, cnt,
                            n_batch, n_iter, n_kept);
    else
        blend_band_edge(g, brec, sid, start, end, bp, lane, lds.rec, T, cr, cg, cb, cnt,
                        n_batch, n_iter, n_kept);

    if (bp.evals != nullptr) {
        // pixel-Gaussian evaluations = sum over valid pixels of entries blended
        uint32_t ev = g.pix_valid ? cnt : 0u;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ev += __shfl_xor(ev, o, GS_WAVE);
        if (lane == 0) {
            // 64 slot groups of 8 counters: spreads the per-wave atomics
            unsigned long long* slot = bp.evals + (size_t)(blockIdx.x & 63u) * 8;
            atomicAdd(slot + 0, (unsigned long long)ev);
            atomicAdd(slot + 1, (unsigned long long)n_batch);
            atomicAdd(slot + 2, (unsigned long long)n_iter);
            atomicAdd(slot + 3, (unsigned long long)n_kept);
            atomicMax(slot + 4, (unsigned long long)n_iter);
        }
    }
    if (!g.pix_valid) return;
    const int q = lane & 31, pi = q >> 3, pj = q & 7;
    const size_t o = ((size_t)(g.py0 + pi) * bp.width + (size_t)(g.px_start + pj)) * 3;
    if (OUT == 2) {
        float* img = static_cast<float*>(out);
        img[o + 0] = cr;
        img[o + 1] = cg;
        img[o + 2] = cb;
    } else if (OUT == 1) {
        uint16_t* img = static_cast<uint16_t*>(out);
        img[o + 0] = f32_to_bf16_rne(cr);
        img[o + 1] = f32_to_bf16_rne(cg);
        img[o + 2] = f32_to_bf16_rne(cb);
    } else {
        // the bf16 image packed to u8, as the reference's render_view does
        uint8_t* img = static_cast<uint8_t*>(out);
        img[o + 0] = bf16_to_u8(f32_to_bf16_rne(cr));
        img[o + 1] = bf16_to_u8(f32_to_bf16_rne(cg));
        img[o + 2] = bf16_to_u8(f32_to_bf16_rne(cb));
    }
}

// Statistics of the reference's per-microblock cull (cull_and_blend.cpp:
// 384-504, 835-836) over the tile-sorted pairs: pairs that no microblock keeps
// (out[0]) and kept (pair, microblock) pairs (out[1]). The reference walks the
// 4x8 grid of 8x4-pixel microblocks at the tile origin whatever the tile size
// (with 16-pixel tiles that grid reaches past the tile), and so does this
// count; the blend itself evaluates the microblocks inside the tile only.
constexpr int kStatThreads = 256;
__global__ __launch_bounds__(kStatThreads) void k_mb_stats(
    const float4* __restrict__ brec, const uint32_t* __restrict__ sid,
    const uint32_t* __restrict__ stile, uint32_t p_cap, const uint32_t* __restrict__ p_dev,
    int tiles_x, int tile_size, int cull_disabled, unsigned long long* __restrict__ out,
    const uint32_t* ctl) {
    if (__builtin_amdgcn_readfirstlane(upstream_failed(ctl) ? 1 : 0)) return;
    const uint32_t p = p_dev ? min(p_cap, *p_dev) : p_cap;
    uint32_t dropped = 0, kept = 0;
    for (uint32_t i = blockIdx.x * kStatThreads + threadIdx.x; i < p;
         i += gridDim.x * kStatThreads) {
        const uint32_t t = stile[i], gi = sid[i];
        const float4 r0 = brec[3 * (size_t)gi + 0], r1 = brec[3 * (size_t)gi + 1];
        const float lt = r1.w;
        if (lt >= 0.0f) {
            ++dropped;
            continue;
        }
        const float tx_tile = (float)((int)(t % (uint32_t)tiles_x) * tile_size);
        const float ty_tile = (float)((int)(t / (uint32_t)tiles_x) * tile_size);
        const float mx = r0.x, my = r0.y;
        const int mx_lo = max(0, (int)floorf(((mx - r0.z) - tx_tile) / 8.0f));
        const int mx_hi = min(3, (int)floorf(((mx + r0.z) - tx_tile) / 8.0f));
        const int my_lo = max(0, (int)floorf(((my - r0.w) - ty_tile) / 4.0f));
        const int my_hi = min(7, (int)floorf(((my + r0.w) - ty_tile) / 4.0f));
        if (mx_lo > mx_hi || my_lo > my_hi) {
            ++dropped;
            continue;
        }
        const float ci_a = r1.x, ci_b = r1.y, ci_c = r1.z;
        const float thresh_m2 = -2.0f * lt;
        const float ci_a_safe = fmax_std(ci_a, 1e-12f), ci_c_safe = fmax_std(ci_c, 1e-12f);
        uint32_t k = 0;
        for (int by = my_lo; by <= my_hi; ++by) {
            const float v_lo = (ty_tile + (float)(by * 4)) - my;
            const float v_hi = v_lo + 4.0f;
            const bool y_in = (v_lo <= 0.0f) && (0.0f <= v_hi);
            const float v_fix = (v_lo > 0.0f) ? v_lo : v_hi;
            for (int bx = mx_lo; bx <= mx_hi; ++bx) {
                const float u_lo = (tx_tile + (float)(bx * 8)) - mx;
                const float u_hi = u_lo + 8.0f;
                const bool x_in = (u_lo <= 0.0f) && (0.0f <= u_hi);
                float m2_min = 0.0f;
                if (!cull_disabled && !(x_in && y_in)) {
                    float m2_v = __builtin_inff(), m2_h = __builtin_inff();
                    if (!x_in) {
                        const float uf = (u_lo > 0.0f) ? u_lo : u_hi;
                        const float vs = fclamp_std(-ci_b * uf / ci_c_safe, v_lo, v_hi);
                        m2_v = ci_a * uf * uf + 2.0f * ci_b * uf * vs + ci_c * vs * vs;
                    }
                    if (!y_in) {
                        const float us = fclamp_std(-ci_b * v_fix / ci_a_safe, u_lo, u_hi);
                        m2_h = ci_a * us * us + 2.0f * ci_b * us * v_fix + ci_c * v_fix * v_fix;
                    }
                    m2_min = fmin_std(m2_v, m2_h);
                }
                k += (m2_min <= thresh_m2) ? 1u : 0u;
            }
        }
        kept += k;
        dropped += (k == 0u) ? 1u : 0u;
    }
    unsigned long long d = dropped, kk = kept;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        d += __shfl_xor(d, o, GS_WAVE);
        kk += __shfl_xor(kk, o, GS_WAVE);
    }
    if (lane_id() == 0) {
        if (d) atomicAdd(out + 0, d);
        if (kk) atomicAdd(out + 1, kk);
    }
}

template <int TS>
hipError_t launch_ts(const float4* brec, const uint32_t* sid, const uint32_t* ranges,
                     BlendParams bp, void* out, hipStream_t st) {
    const unsigned grid = (unsigned)(bp.tiles_x * bp.tiles_y * (TS / 16) * (TS / 4));
    switch (bp.out_format) {
        case 0: k_blend<TS, 0><<<grid, GS_WAVE, 0, st>>>(brec, sid, ranges, bp, out); break;
        case 1: k_blend<TS, 1><<<grid, GS_WAVE, 0, st>>>(brec, sid, ranges, bp, out); break;
        case 2: k_blend<TS, 2><<<grid, GS_WAVE, 0, st>>>(brec, sid, ranges, bp, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_mb_stats(const float4* brec, const uint32_t* sid, const uint32_t* stile,
                           uint32_t p_cap, const uint32_t* p_dev, int tiles_x, int tile_size,
                           int cull_disabled, unsigned long long* out, const uint32_t* ctl,
                           hipStream_t st) {
    if (p_cap == 0 || tiles_x <= 0) return hipSuccess;
    const unsigned grid = std::min<unsigned>((p_cap + kStatThreads - 1) / kStatThreads, 4096u);
    k_mb_stats<<<grid, kStatThreads, 0, st>>>(brec, sid, stile, p_cap, p_dev, tiles_x, tile_size,
                                              cull_disabled, out, ctl);
    return hipGetLastError();
}

hipError_t launch_blend(const float4* brec, const uint32_t* sid, const uint32_t* ranges,
                        BlendParams bp, void* out, hipStream_t st) {
    if (bp.tiles_x <= 0 || bp.tiles_y <= 0) return hipSuccess;
    if (bp.tile_size == 16) return launch_ts<16>(brec, sid, ranges, bp, out, st);
    if (bp.tile_size == 32) return launch_ts<32>(brec, sid, ranges, bp, out, st);
    return hipErrorInvalidValue;
}

}  // namespace gs
