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
//   3. walks the union of the two kept masks in depth order: the entry's
//      parameters are read into SGPRs (v_readlane), the halves that keep it
//      blend it, transmittance and colour stay in VGPRs.
// Full microblocks follow the reference's AVX2 arithmetic exactly (degree-4
// exp, power clamp [-30,0], T -= alpha*T, early-out test every 4 kept entries);
// image-edge microblocks follow its scalar rule (exp, T *= 1-alpha, test after
// every entry) (cull_and_blend.cpp:506-670, simd_exp_avx2.h:12-32). A half
// whose microblock is done stops issuing; the wave exits when both are done.
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

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <int TS, int OUT>
__global__ __launch_bounds__(GS_WAVE) void k_blend(const float4* __restrict__ brec,
                                                   const uint32_t* __restrict__ sid,
                                                   const uint32_t* __restrict__ ranges,
                                                   BlendParams bp, void* __restrict__ out) {
    constexpr int BX = TS / 16;  // 16-pixel band columns per tile
    constexpr int BY = TS / 4;   // 4-row bands per tile

    const int band = blockIdx.x % (BX * BY);
    const int tile = blockIdx.x / (BX * BY);
    const int bx = band % BX, by = band / BX;
    const int tile_x = tile % bp.tiles_x, tile_y = tile / bp.tiles_x;
    const int lane = threadIdx.x;
    const int h = lane >> 5, q = lane & 31, pi = q >> 3, pj = q & 7;
    const int mbx = bx * 2 + h, mby = by;

    const int px_tile = tile_x * TS, py_tile = tile_y * TS;
    const int px_end_tile = min(px_tile + TS, bp.width);
    const int py_end_tile = min(py_tile + TS, bp.height);
    // Microblock extents of both halves (wave-uniform).
    const int pxA = px_tile + (bx * 2) * 8, pxB = pxA + 8;
    const int py0 = py_tile + mby * 4;
    const int pyE = min(py0 + 4, py_end_tile);
    const int pxEA = min(pxA + 8, px_end_tile), pxEB = min(pxB + 8, px_end_tile);
    const bool emptyA = (py0 >= pyE) || (pxA >= pxEA);
    const bool emptyB = (py0 >= pyE) || (pxB >= pxEB);
    const bool fullA = !emptyA && (pxEA - pxA == 8) && (pyE - py0 == 4);
    const bool fullB = !emptyB && (pxEB - pxB == 8) && (pyE - py0 == 4);
    const int px_start = h ? pxB : pxA;
    const int px_end = h ? pxEB : pxEA;
    const bool full = h ? fullB : fullA;
    const bool pix_valid = !(h ? emptyB : emptyA) && (px_start + pj < px_end) && (py0 + pi < pyE);

    const float tx_tile = (float)(tile_x * TS);
    const float ty_tile = (float)(tile_y * TS);
    const float pxs = (float)px_start;                 // full path: px_base = pxs - mx
    const float offx = (float)pj + 0.5f;
    const float pxc = (float)(px_start + pj) + 0.5f;   // scalar path pixel centre
    const float pyc = (float)(py0 + pi) + 0.5f;
    // Microblock cull rectangle (cull_and_blend.cpp:447-498).
    const float mb_oy = ty_tile + (float)(mby * 4);
    const float mb_ox = tx_tile + (float)(mbx * 8);

    float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
    bool doneA = emptyA, doneB = emptyB;
    const uint32_t npixA = emptyA ? 0u : (uint32_t)((pxEA - pxA) * (pyE - py0));
    const uint32_t npixB = emptyB ? 0u : (uint32_t)((pxEB - pxB) * (pyE - py0));
    uint64_t evals = 0, n_batch = 0, n_iter = 0, n_kept = 0;
    uint32_t cntA = 0, cntB = 0;

    const uint32_t start = ranges[2 * tile], end = ranges[2 * tile + 1];
    for (uint32_t base = start; base < end && !(doneA && doneB); base += 32) {
        const uint32_t idx = base + q;
        const bool has = idx < end;
        float4 r0 = make_float4(0, 0, 0, 0), r1 = r0, r2 = r0;
        if (has) {
            const uint32_t g = sid[idx];
            r0 = brec[3 * (size_t)g + 0];
            r1 = brec[3 * (size_t)g + 1];
            r2 = brec[3 * (size_t)g + 2];
        }
        bool keep = false;
        const bool my_done = h ? doneB : doneA;
        if (has && !my_done) {
            const float lt = r1.w;
            if (lt < 0.0f) {
                const float mx = r0.x, my = r0.y;
                const int mx_lo = max(0, (int)floorf(((mx - r0.z) - tx_tile) / 8.0f));
                const int mx_hi = min(3, (int)floorf(((mx + r0.z) - tx_tile) / 8.0f));
                const int my_lo = max(0, (int)floorf(((my - r0.w) - ty_tile) / 4.0f));
                const int my_hi = min(7, (int)floorf(((my + r0.w) - ty_tile) / 4.0f));
                if (mx_lo <= mbx && mbx <= mx_hi && my_lo <= mby && mby <= my_hi) {
                    const float ci_a = r1.x, ci_b = r1.y, ci_c = r1.z;
                    const float v_lo = mb_oy - my;
                    const float v_hi = v_lo + 4.0f;
                    const bool y_in = (v_lo <= 0.0f) && (0.0f <= v_hi);
                    const float v_fix = (v_lo > 0.0f) ? v_lo : v_hi;
                    const float u_lo = mb_ox - mx;
                    const float u_hi = u_lo + 8.0f;
                    const bool x_in = (u_lo <= 0.0f) && (0.0f <= u_hi);
                    float m2_min;
                    if (bp.cull_disabled || (x_in && y_in)) {
                        m2_min = 0.0f;
                    } else {
                        float m2_v = __builtin_inff(), m2_h = __builtin_inff();
                        if (!x_in) {
                            const float uf = (u_lo > 0.0f) ? u_lo : u_hi;
                            float vs = -ci_b * uf / fmax_std(ci_c, 1e-12f);
                            vs = fclamp_std(vs, v_lo, v_hi);
                            m2_v = ci_a * uf * uf + 2.0f * ci_b * uf * vs + ci_c * vs * vs;
                        }
                        if (!y_in) {
                            float us = -ci_b * v_fix / fmax_std(ci_a, 1e-12f);
                            us = fclamp_std(us, u_lo, u_hi);
                            m2_h = ci_a * us * us + 2.0f * ci_b * us * v_fix +
                                   ci_c * v_fix * v_fix;
                        }
                        m2_min = fmin_std(m2_v, m2_h);
                    }
                    keep = (m2_min <= -2.0f * lt);
                }
            }
        }
        const uint64_t mask = __ballot(keep);
        ++n_batch;
        n_kept += (uint64_t)__popcll(mask);
        // Power coefficients of the AVX2 path (cull_and_blend.cpp:198-200),
        // computed once per entry in its own lane.
        const float qA = -0.5f * r1.x, qB = -r1.y, qC = -0.5f * r1.z;
        // Walk the union of both halves' kept entries in depth order; the
        // entry's parameters are wave-uniform (SGPRs), a half that does not
        // keep the entry (or is done) is masked off.
        uint32_t mA = __builtin_amdgcn_readfirstlane((uint32_t)mask);
        uint32_t mB = __builtin_amdgcn_readfirstlane((uint32_t)(mask >> 32));
        uint32_t uni = mA | mB;
        while (uni) {
            const int j = __builtin_ctz(uni);
            uni &= uni - 1;
            const bool inA = (mA >> j) & 1u, inB = (mB >> j) & 1u;
            const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r0.x), j));
            const float my = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r0.y), j));
            const float op = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r2.x), j));
            const float col_r = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r2.y), j));
            const float col_g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r2.z), j));
            const float col_b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r2.w), j));
            // v_readlane reads lane j whatever EXEC is, so every read happens
            // here, in wave-uniform control flow, before the per-half branch.
            const float A = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qA), j));
            const float B = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qB), j));
            const float C = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qC), j));
            float ci_a = 0.0f, ci_b = 0.0f, ci_c = 0.0f;
            if (!(fullA && fullB)) {  // image-edge band: scalar-rule parameters
                ci_a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r1.x), j));
                ci_b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r1.y), j));
                ci_c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r1.z), j));
            }
            const bool runA = inA && !doneA, runB = inB && !doneB;
            if (h ? runB : runA) {
                if (full) {
                    const float px_base = pxs - mx;
                    const float dx = px_base + offx;
                    const float dx_sq = dx * dx;
                    const float dy = pyc - my;
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
                    cr = __builtin_fmaf(at, col_r, cr);
                    cg = __builtin_fmaf(at, col_g, cg);
                    cb = __builtin_fmaf(at, col_b, cb);
                    T = T - at;
                } else if (pix_valid) {
                    const float dx = pxc - mx;
                    const float dy = pyc - my;
                    const float power =
                        -0.5f * (ci_a * dx * dx + 2.0f * ci_b * dx * dy + ci_c * dy * dy);
                    const float gw = expf(fmin_std(power, 0.0f));
                    const float al = fmin_std(op * gw, 0.99f);
                    const float at = al * T;
                    cr += at * col_r;
                    cg += at * col_g;
                    cb += at * col_b;
                    T = T * (1.0f - al);
                }
            }
            evals += (runA ? npixA : 0u) + (runB ? npixB : 0u);
            ++n_iter;
            bool chkA = false, chkB = false;
            if (runA) {
                ++cntA;
                chkA = fullA ? ((cntA & 3u) == 0u) : true;
            }
            if (runB) {
                ++cntB;
                chkB = fullB ? ((cntB & 3u) == 0u) : true;
            }
            if (chkA || chkB) {
                // max over the microblock's pixels < thr  <=>  no pixel has T >= thr
                // (T is never NaN; edge pixels outside the image do not vote).
                const uint64_t live = __ballot(pix_valid && !(T < bp.thr));
                if (chkA && (uint32_t)live == 0u) doneA = true;
                if (chkB && (uint32_t)(live >> 32) == 0u) doneB = true;
                if (doneA && doneB) break;
            }
        }
    }

    if (bp.evals != nullptr && lane == 0) {
        // 64 slot groups of 8 counters: spreads the per-wave atomics
        unsigned long long* slot = bp.evals + (size_t)(blockIdx.x & 63u) * 8;
        atomicAdd(slot + 0, (unsigned long long)evals);
        atomicAdd(slot + 1, (unsigned long long)n_batch);
        atomicAdd(slot + 2, (unsigned long long)n_iter);
        atomicAdd(slot + 3, (unsigned long long)n_kept);
        atomicMax(slot + 4, (unsigned long long)n_iter);
    }
    if (!pix_valid) return;
    const size_t o = ((size_t)(py0 + pi) * bp.width + (size_t)(px_start + pj)) * 3;
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
        uint8_t* img = static_cast<uint8_t*>(out);
        img[o + 0] = (uint8_t)(fminf(fmaxf(cr, 0.0f), 1.0f) * 255.0f);
        img[o + 1] = (uint8_t)(fminf(fmaxf(cg, 0.0f), 1.0f) * 255.0f);
        img[o + 2] = (uint8_t)(fminf(fmaxf(cb, 0.0f), 1.0f) * 255.0f);
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

hipError_t launch_blend(const float4* brec, const uint32_t* sid, const uint32_t* ranges,
                        BlendParams bp, void* out, hipStream_t st) {
    if (bp.tiles_x <= 0 || bp.tiles_y <= 0) return hipSuccess;
    if (bp.tile_size == 16) return launch_ts<16>(brec, sid, ranges, bp, out, st);
    if (bp.tile_size == 32) return launch_ts<32>(brec, sid, ranges, bp, out, st);
    return hipErrorInvalidValue;
}

}  // namespace gs
