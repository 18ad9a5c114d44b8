// project.hip - fused per-Gaussian projection + SH colour + stable visibility
// compaction, one pass over the scene.
//
// Per Gaussian (reference src/gsplat_cpu/project.cpp:558-685): camera-space
// mean (R*m first, then +t), near-plane / opacity reject, pixel mean, EWA
// Jacobian, cov_cam from the 6 unique cov3d entries, cov2d + 0.3 low-pass,
// opacity-aware radius and the image-overlap validity test. Visible
// Gaussians are written in source order (project.cpp:710-797) with a
// decoupled look-back over 2048-Gaussian partitions, so compact index m equals
// the reference's.
//
// All float expressions keep the reference's operation order and the unit is
// compiled with -ffp-contract=off, so every output is bit-identical to the
// reference's fp32 results.
#include "gs_common.h"
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kProjThreads = 512;
constexpr int kProjItems = 4;
constexpr int kProjPart = kProjThreads * kProjItems;
static_assert(kProjPart == (int)kProjPartition, "project partition size is part of the interface");

__device__ __forceinline__ float fmin_std(float a, float b) { return (b < a) ? b : a; }
__device__ __forceinline__ float fmax_std(float a, float b) { return (a < b) ? b : a; }

// 3DGS real SH basis (gsplat/train_oracle.py:46-52, 99-122), fp32,
// left-to-right. `rec` is one Gaussian's record of (DEG+1)^2 coefficients x 3
// channels, coefficient k channel c at rec[k*3 + c] (the scene's own layout).
// Only visible Gaussians are evaluated, so a per-Gaussian record touches just
// the cache lines of the Gaussians on screen, where planes would touch nearly
// every line of every plane.
template <int DEG>
__device__ __forceinline__ void sh_eval(const float* __restrict__ rec, float x, float y, float z,
                                        int clamp_hi, float* rgb) {
    constexpr int K = (DEG + 1) * (DEG + 1);
    float v[3 * K];
    if constexpr ((3 * K) % 4 == 0) {
        // records of degree 1 and 3 are 16-byte aligned: whole-vector loads
#pragma unroll
        for (int q = 0; q < 3 * K / 4; ++q) {
            const float4 t = reinterpret_cast<const float4*>(rec)[q];
            v[4 * q + 0] = t.x;
            v[4 * q + 1] = t.y;
            v[4 * q + 2] = t.z;
            v[4 * q + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < 3 * K; ++q) v[q] = rec[q];
    }
    constexpr float C0 = 0.28209479177387814f;
    constexpr float C1 = 0.4886025119029199f;
    constexpr float C20 = 1.0925484305920792f, C21 = -1.0925484305920792f,
                    C22 = 0.31539156525252005f, C23 = -1.0925484305920792f,
                    C24 = 0.5462742152960396f;
    constexpr float C30 = -0.5900435899266435f, C31 = 2.890611442640554f,
                    C32 = -0.4570457994644658f, C33 = 0.3731763325901154f,
                    C34 = -0.4570457994644658f, C35 = 1.445305721320277f,
                    C36 = -0.5900435899266435f;
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, yz = y * z, xz = x * z;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        auto S = [&](int k) { return v[k * 3 + c]; };
        float o = C0 * S(0);
        if (DEG >= 1) {
            o = o - C1 * y * S(1) + C1 * z * S(2) - C1 * x * S(3);
        }
        if (DEG >= 2) {
            o = o + C20 * xy * S(4) + C21 * yz * S(5) + C22 * (2.0f * zz - xx - yy) * S(6) +
                C23 * xz * S(7) + C24 * (xx - yy) * S(8);
        }
        if (DEG >= 3) {
            o = o + C30 * y * (3.0f * xx - yy) * S(9) + C31 * xy * z * S(10) +
                C32 * y * (4.0f * zz - xx - yy) * S(11) +
                C33 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy) * S(12) +
                C34 * x * (4.0f * zz - xx - yy) * S(13) + C35 * z * (xx - yy) * S(14) +
                C36 * x * (xx - 3.0f * yy) * S(15);
        }
        o = o + 0.5f;
        o = (o < 0.0f) ? 0.0f : o;
        if (clamp_hi) o = (o > 1.0f) ? 1.0f : o;
        rgb[c] = o;
    }
}

template <int DEG>
__global__ __launch_bounds__(kProjThreads) void k_project(SceneDev s, ProjParams p, Compact out,
                                                          uint8_t* __restrict__ valid_mask,
                                                          uint64_t* lb_state, uint32_t* ticket,
                                                          uint32_t* count_out,
                                                          uint32_t* __restrict__ part_hist) {
    __shared__ uint32_t s_vid;
    __shared__ uint32_t s_cnt[kProjItems][kProjThreads / GS_WAVE];
    __shared__ uint32_t s_hist[4][256];
    __shared__ uint64_t s_excl;
    // each item's projected values, held here over the colour evaluation (in
    // registers they would leave one workgroup per CU instead of two)
    __shared__ float4 s_iv[2][kProjItems][kProjThreads];
    const int tid = threadIdx.x;
    const int w = tid / GS_WAVE;
    const int lane = lane_id();
    if (tid == 0) s_vid = atomicAdd(ticket, 1u);
    if (part_hist != nullptr)
        for (int i = tid; i < 4 * 256; i += kProjThreads) (&s_hist[0][0])[i] = 0;
    __syncthreads();
    const uint32_t vid = s_vid;
    const int64_t base = (int64_t)vid * kProjPart;
    const int64_t n = s.n;
    // a partition the view's frustum test rules out reads nothing: its Gaussians
    // are all invalid (it still publishes its zero count to the compaction)
    const bool skipped = p.skip != nullptr && p.skip[vid] != 0;

    float vmx[kProjItems], vmy[kProjItems], vtz[kProjItems];
    float va[kProjItems], vb[kProjItems], vc[kProjItems], vrx[kProjItems], vry[kProjItems];
    bool valid[kProjItems];
    uint64_t bal[kProjItems];

    // loads in two stages over all items: the means and opacities, then the
    // covariance words of the items that pass the depth and opacity tests
    float ltx[kProjItems], lty[kProjItems], ltz[kProjItems];
    bool lok[kProjItems];
    {
        float lmx[kProjItems], lmy[kProjItems], lmz[kProjItems], lop[kProjItems];
#pragma unroll
        for (int it = 0; it < kProjItems; ++it) {
            const int64_t i = base + it * kProjThreads + tid;
            const bool in = i < n && !skipped;
            lmx[it] = in ? s.mean[0][i] : 0.0f;
            lmy[it] = in ? s.mean[1][i] : 0.0f;
            lmz[it] = in ? s.mean[2][i] : 0.0f;
            lop[it] = (in && p.has_opac) ? s.opac[i] : 1.0f;
        }
#pragma unroll
        for (int it = 0; it < kProjItems; ++it) {
            const int64_t i = base + it * kProjThreads + tid;
            const float mx = lmx[it], my = lmy[it], mz = lmz[it];
            const float rmx = mx * p.r[0] + my * p.r[1] + mz * p.r[2];
            const float rmy = mx * p.r[3] + my * p.r[4] + mz * p.r[5];
            const float rmz = mx * p.r[6] + my * p.r[7] + mz * p.r[8];
            ltx[it] = rmx + p.t[0];
            lty[it] = rmy + p.t[1];
            ltz[it] = rmz + p.t[2];
            bool ok = i < n && !skipped && !(ltz[it] <= 0.2f);
            if (p.has_opac) ok = ok && !(lop[it] < p.min_opacity);
            lok[it] = ok;
        }
    }
    float lc[6][kProjItems], lk[kProjItems];
#pragma unroll
    for (int it = 0; it < kProjItems; ++it) {
        const int64_t i = base + it * kProjThreads + tid;
#pragma unroll
        for (int q = 0; q < 6; ++q) lc[q][it] = lok[it] ? s.cov[q][i] : 0.0f;
        lk[it] = lok[it] ? s.kfac[i] : 0.0f;
    }

#pragma unroll
    for (int it = 0; it < kProjItems; ++it) {
        const int64_t i = base + it * kProjThreads + tid;
        valid[it] = false;
        vmx[it] = vmy[it] = vtz[it] = va[it] = vb[it] = vc[it] = vrx[it] = vry[it] = 0.0f;
        {
            const float tx = ltx[it], ty = lty[it], tz = ltz[it];
            if (lok[it]) {
                const float inv_tz = 1.0f / tz;
                const float mean_x = p.fx * tx * inv_tz + p.cx;
                const float mean_y = p.fy * ty * inv_tz + p.cy;
                const float tz2 = tz * tz;
                const float j00 = p.fx / tz, j02 = -p.fx * tx / tz2;
                const float j11 = p.fy / tz, j12 = -p.fy * ty / tz2;
                const float c00 = lc[0][it], c01 = lc[1][it], c02 = lc[2][it];
                const float c11 = lc[3][it], c12 = lc[4][it], c22 = lc[5][it];
                const float r00 = p.r[0], r01 = p.r[1], r02 = p.r[2];
                const float r10 = p.r[3], r11 = p.r[4], r12 = p.r[5];
                const float r20 = p.r[6], r21 = p.r[7], r22 = p.r[8];
                const float v0_0 = c00 * r00 + c01 * r01 + c02 * r02;
                const float v0_1 = c01 * r00 + c11 * r01 + c12 * r02;
                const float v0_2 = c02 * r00 + c12 * r01 + c22 * r02;
                const float v1_0 = c00 * r10 + c01 * r11 + c02 * r12;
                const float v1_1 = c01 * r10 + c11 * r11 + c12 * r12;
                const float v1_2 = c02 * r10 + c12 * r11 + c22 * r12;
                const float v2_0 = c00 * r20 + c01 * r21 + c02 * r22;
                const float v2_1 = c01 * r20 + c11 * r21 + c12 * r22;
                const float v2_2 = c02 * r20 + c12 * r21 + c22 * r22;
                const float cc00 = r00 * v0_0 + r01 * v0_1 + r02 * v0_2;
                const float cc01 = r00 * v1_0 + r01 * v1_1 + r02 * v1_2;
                const float cc02 = r00 * v2_0 + r01 * v2_1 + r02 * v2_2;
                const float cc11 = r10 * v1_0 + r11 * v1_1 + r12 * v1_2;
                const float cc12 = r10 * v2_0 + r11 * v2_1 + r12 * v2_2;
                const float cc22 = r20 * v2_0 + r21 * v2_1 + r22 * v2_2;
                const float m00 = j00 * cc00 + j02 * cc02;
                const float m01 = j00 * cc01 + j02 * cc12;
                const float m02 = j00 * cc02 + j02 * cc22;
                const float m11 = j11 * cc11 + j12 * cc12;
                const float m12 = j11 * cc12 + j12 * cc22;
                const float a = m00 * j00 + m02 * j02 + 0.3f;
                const float b = m01 * j11 + m02 * j12;
                const float c = m11 * j11 + m12 * j12 + 0.3f;
                const float k = lk[it];
                float rx, ry;
                if (p.use_iso) {
                    const float trace = a + c;
                    const float disc =
                        sqrtf(fmax_std(trace * trace - 4.0f * (a * c - b * b), 0.0f));
                    const float l1 = 0.5f * (trace + disc);
                    const float l2 = 0.5f * (trace - disc);
                    const float theta = 0.5f * atan2f(2.0f * b, a - c);
                    const float ct = cosf(theta), st = sinf(theta);
                    const float cos2 = ct * ct, sin2 = st * st;
                    rx = ceilf(k * sqrtf(fmax_std(l1 * cos2 + l2 * sin2, 0.0f)));
                    ry = ceilf(k * sqrtf(fmax_std(l1 * sin2 + l2 * cos2, 0.0f)));
                } else {
                    rx = ceilf(k * sqrtf(fmax_std(a, 0.0f)));
                    ry = ceilf(k * sqrtf(fmax_std(c, 0.0f)));
                }
                const bool v = (mean_x + rx > 0.0f) && (mean_x - rx < (float)p.width) &&
                               (mean_y + ry > 0.0f) && (mean_y - ry < (float)p.height) &&
                               (rx > 0.0f) && (ry > 0.0f) && (rx <= p.max_radius) &&
                               (ry <= p.max_radius);
                valid[it] = v;
                vmx[it] = mean_x;
                vmy[it] = mean_y;
                vtz[it] = tz;
                va[it] = a;
                vb[it] = b;
                vc[it] = c;
                vrx[it] = rx;
                vry[it] = ry;
            }
        }
        if (i < n && valid_mask != nullptr) valid_mask[i] = valid[it] ? 1 : 0;
        s_iv[0][it][tid] = make_float4(vmx[it], vmy[it], vrx[it], vry[it]);
        s_iv[1][it][tid] = make_float4(va[it], vb[it], vc[it], vtz[it]);
        bal[it] = __ballot(valid[it]);
        if (lane == 0) s_cnt[it][w] = (uint32_t)__popcll(bal[it]);
        if (part_hist != nullptr) {
            // digit histograms of the depth keys, for the depth sort's passes
            const uint32_t k = __float_as_uint(vtz[it]);
            hist_add_wave(s_hist[0], k & 255u, valid[it]);
            hist_add_wave(s_hist[1], (k >> 8) & 255u, valid[it]);
            hist_add_wave(s_hist[2], (k >> 16) & 255u, valid[it]);
            hist_add_wave(s_hist[3], k >> 24, valid[it]);
        }
    }
    __syncthreads();
    if (part_hist != nullptr)
        for (int i = tid; i < 4 * 256; i += kProjThreads)
            part_hist[(size_t)vid * 1024 + i] = (&s_hist[0][0])[i];

    uint32_t total = 0;
    uint32_t my_off[kProjItems];
#pragma unroll
    for (int it = 0; it < kProjItems; ++it) {
#pragma unroll
        for (int ww = 0; ww < kProjThreads / GS_WAVE; ++ww) {
            if (ww == w) my_off[it] = total;
            total += s_cnt[it][ww];
        }
    }
    // The partition's count goes out first; the colours of the valid items
    // (the SH records, the kernel's largest reads) are evaluated before the
    // walk over the predecessors, so that the walk finds them mostly done.
    if (w == 0) lookback_publish(lb_state, vid, total);
    float vr[kProjItems], vg[kProjItems], vbl[kProjItems];
#pragma unroll
    for (int it = 0; it < kProjItems; ++it) {
        vr[it] = vg[it] = vbl[it] = 0.0f;
        if (!valid[it]) continue;
        const int64_t i = base + it * kProjThreads + tid;
        float rgb[3];
        if (DEG < 0) {
            rgb[0] = s.sh[i * 3 + 0];
            rgb[1] = s.sh[i * 3 + 1];
            rgb[2] = s.sh[i * 3 + 2];
        } else {
            const float dx = s.mean[0][i] - p.ccx;
            const float dy = s.mean[1][i] - p.ccy;
            const float dz = s.mean[2][i] - p.ccz;
            const float nrm = sqrtf(dx * dx + dy * dy + dz * dz);
            constexpr int D = DEG < 0 ? 0 : DEG;
            sh_eval<D>(s.sh + i * (3 * (D + 1) * (D + 1)), dx / nrm, dy / nrm, dz / nrm,
                       p.sh_clamp_hi, rgb);
        }
        vr[it] = rgb[0];
        vg[it] = rgb[1];
        vbl[it] = rgb[2];
    }
    if (w == 0) {
        const uint64_t excl = lookback_walk(lb_state, vid, total, p.ctl);
        if (lane == 0) {
            s_excl = excl;
            if (vid == gridDim.x - 1) *count_out = (uint32_t)(excl + total);
        }
    }
    __syncthreads();
    const uint64_t excl = s_excl;
    const uint64_t lt_mask = lanemask_lt();

#pragma unroll
    for (int it = 0; it < kProjItems; ++it) {
        if (!valid[it]) continue;
        const int64_t i = base + it * kProjThreads + tid;
        const uint64_t m = excl + my_off[it] + (uint64_t)__popcll(bal[it] & lt_mask);
        const float4 q0 = s_iv[0][it][tid], q1 = s_iv[1][it][tid];
        vmx[it] = q0.x;
        vmy[it] = q0.y;
        vrx[it] = q0.z;
        vry[it] = q0.w;
        va[it] = q1.x;
        vb[it] = q1.y;
        vc[it] = q1.z;
        vtz[it] = q1.w;
        const float a = va[it], b = vb[it], c = vc[it];
        out.rc[2 * m + 0] = make_float4(vmx[it], vmy[it], vrx[it], vry[it]);
        out.rc[2 * m + 1] = make_float4(a, b, c, s.m2thr[i]);
        out.dkey[m] = __float_as_uint(vtz[it]);
        if (p.dvals != nullptr) {
            // the tile count that the candidate scan would read the rectangle for
            const Rect q = tile_rect(make_float4(vmx[it], vmy[it], vrx[it], vry[it]), p.tiles_x,
                                     p.tiles_y, ts_div(p.tile_size));
            const uint32_t cnt = (uint32_t)(q.x1 - q.x0 + 1) * (uint32_t)(q.y1 - q.y0 + 1);
            p.dvals[m] = dval_pack((uint32_t)m, cnt, p.idx_bits);
        }
        // Microblock cull / blend record (cull_and_blend.cpp:723-777).
        const float det = fmax_std(a * c - b * b, 1e-6f);
        const float ci_a = c / det;
        const float ci_b = -b / det;
        const float ci_c = a / det;
        const float lt = s.lthr[i];
        float xh = 0.0f, yh = 0.0f;
        if (lt < 0.0f) {
            const float rd = sqrtf(-2.0f * lt);
            xh = rd * sqrtf(fmax_std(a, 0.0f));
            yh = rd * sqrtf(fmax_std(c, 0.0f));
        }
        const float op = p.has_opac ? s.opac[i] : 1.0f;
        out.brec[m * 3 + 0] = make_float4(vmx[it], vmy[it], xh, yh);
        out.brec[m * 3 + 1] = make_float4(ci_a, ci_b, ci_c, lt);
        out.brec[m * 3 + 2] = make_float4(vr[it], vg[it], vbl[it], op);
        if (out.src != nullptr) out.src[m] = (uint32_t)i;
    }
}

// ---- chunk frustum skip ------------------------------------------------------
// render/host/chunk_cull.h:26-58 (per scene) and :62-99 (per view), over this
// kernel's partitions of kProjPart Gaussians; double precision throughout.

// One workgroup per partition: min/max of mean -+ k rho over its Gaussians.
__global__ __launch_bounds__(kProjThreads) void k_chunk_boxes(SceneDev s, double k,
                                                              double* __restrict__ box) {
    constexpr int W = kProjThreads / GS_WAVE;
    __shared__ double s_v[7][W];
    __shared__ int s_bad[W];
    const int tid = threadIdx.x, w = tid / GS_WAVE, lane = lane_id();
    const int64_t base = (int64_t)blockIdx.x * kProjPart;
    double lo[3] = {1e300, 1e300, 1e300}, hi[3] = {-1e300, -1e300, -1e300}, rmax = 0.0;
    bool bad = false;
#pragma unroll
    for (int it = 0; it < kProjItems; ++it) {
        const int64_t i = base + it * kProjThreads + tid;
        if (i >= s.n) continue;
        const double tr = (double)s.cov[0][i] + (double)s.cov[3][i] + (double)s.cov[5][i];
        if (!isfinite(tr)) bad = true;
        const double rho = 3.0 * sqrt(tr > 0.0 ? tr : 0.0);
        rmax = rho > rmax ? rho : rmax;
#pragma unroll
        for (int d = 0; d < 3; ++d) {
            const double m = (double)s.mean[d][i];
            if (!isfinite(m)) bad = true;
            const double l = m - k * rho, h = m + k * rho;
            lo[d] = l < lo[d] ? l : lo[d];
            hi[d] = h > hi[d] ? h : hi[d];
        }
    }
    for (int o = 1; o < GS_WAVE; o <<= 1) {
#pragma unroll
        for (int d = 0; d < 3; ++d) {
            lo[d] = fmin(lo[d], __shfl_xor(lo[d], o, GS_WAVE));
            hi[d] = fmax(hi[d], __shfl_xor(hi[d], o, GS_WAVE));
        }
        rmax = fmax(rmax, __shfl_xor(rmax, o, GS_WAVE));
    }
    const bool any_bad = __ballot(bad) != 0ull;
    if (lane == 0) {
        for (int d = 0; d < 3; ++d) {
            s_v[d][w] = lo[d];
            s_v[3 + d][w] = hi[d];
        }
        s_v[6][w] = rmax;
        s_bad[w] = any_bad ? 1 : 0;
    }
    __syncthreads();
    if (tid == 0) {
        double* b = box + 8 * (size_t)blockIdx.x;
        int nb = 0;
        for (int q = 0; q < 7; ++q) {
            double v = s_v[q][0];
            for (int ww = 1; ww < W; ++ww)
                v = (q < 3) ? fmin(v, s_v[q][ww]) : fmax(v, s_v[q][ww]);
            b[q] = v;
        }
        for (int ww = 0; ww < W; ++ww) nb |= s_bad[ww];
        b[7] = nb ? 1.0 : 0.0;
    }
}

// One thread per partition. Skipped when the box is behind z = near, or when
// every corner lies beyond one side plane x = U0 z of the image widened by 5 px
// and the largest rho, seen from the nearest depth, subtends less than that
// plane's margin for k: no Gaussian's footprint can then reach the image.
__global__ void k_chunk_cull(const double* __restrict__ box, int64_t nchunks, ProjParams p,
                             double k, uint8_t* __restrict__ skip, uint32_t* __restrict__ n_skipped) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= nchunks) return;
    const double* b = box + 8 * (size_t)c;
    bool cull = false;
    if (b[7] == 0.0) {
        constexpr double kNear = 0.2, kPad = 5.0;
        double pc[8][3];
        double zmin = 1e300, zmax = -1e300;
        for (int q = 0; q < 8; ++q) {
            const double x = b[(q & 1) ? 3 : 0], y = b[(q & 2) ? 4 : 1], z = b[(q & 4) ? 5 : 2];
            for (int a = 0; a < 3; ++a)
                pc[q][a] = (double)p.r[3 * a] * x + (double)p.r[3 * a + 1] * y +
                           (double)p.r[3 * a + 2] * z + (double)p.t[a];
            zmin = fmin(zmin, pc[q][2]);
            zmax = fmax(zmax, pc[q][2]);
        }
        cull = zmax <= kNear;
        const double ang = b[6] / fmax(zmin, kNear);
        const double W = (double)p.width, H = (double)p.height;
        const double u0[4] = {(W - p.cx + kPad) / p.fx, (p.cx + kPad) / p.fx,
                              (H - p.cy + kPad) / p.fy, (p.cy + kPad) / p.fy};
        for (int sd = 0; sd < 4 && !cull; ++sd) {
            const int axis = sd >> 1;
            const double sgn = (sd & 1) ? -1.0 : 1.0, U0 = u0[sd];
            const double uk = sqrt(fmax(0.0, k * k * (1.0 + U0 * U0) - 1.0));
            const double margin = (uk - U0) / sqrt(1.0 + uk * uk);
            if (ang > margin) continue;
            bool all = true;
            for (int q = 0; q < 8 && all; ++q) all = sgn * pc[q][axis] - U0 * pc[q][2] > 0.0;
            cull = all;
        }
    }
    skip[c] = cull ? 1 : 0;
    if (cull && n_skipped != nullptr) atomicAdd(n_skipped, 1u);
}

struct ColMap {
    int c[64];
};

// AoS (n x cols) -> SoA planes; plane j takes column map.c[j].
__global__ void k_soa_transpose(const float* __restrict__ aos, int64_t n, int cols, ColMap map,
                                int planes, float* __restrict__ soa) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    for (int j = 0; j < planes; ++j) soa[(int64_t)j * n + i] = aos[i * cols + map.c[j]];
}

__global__ void k_brec_from_arrays(const float* __restrict__ means2d,
                                   const float* __restrict__ covs2d,
                                   const float* __restrict__ colors,
                                   const float* __restrict__ opac,
                                   const float* __restrict__ lthr, int64_t m,
                                   float4* __restrict__ brec) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m) return;
    const float a = covs2d[i * 4 + 0], b = covs2d[i * 4 + 1], c = covs2d[i * 4 + 3];
    const float det = fmax_std(a * c - b * b, 1e-6f);
    const float lt = lthr[i];
    float xh = 0.0f, yh = 0.0f;
    if (lt < 0.0f) {
        const float rd = sqrtf(-2.0f * lt);
        xh = rd * sqrtf(fmax_std(a, 0.0f));
        yh = rd * sqrtf(fmax_std(c, 0.0f));
    }
    brec[i * 3 + 0] = make_float4(means2d[i * 2 + 0], means2d[i * 2 + 1], xh, yh);
    brec[i * 3 + 1] = make_float4(c / det, -b / det, a / det, lt);
    brec[i * 3 + 2] = make_float4(colors[i * 3 + 0], colors[i * 3 + 1], colors[i * 3 + 2],
                                  opac[i]);
}

}  // namespace

hipError_t launch_project(const SceneDev& s, const ProjParams& p, Compact out,
                          uint8_t* valid_mask, uint64_t* lb_state, uint32_t* ticket,
                          uint32_t* count_out, uint32_t* part_hist, hipStream_t st) {
    if (s.n <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((s.n + kProjPart - 1) / kProjPart);
    switch (s.sh_degree) {
        case -1: k_project<-1><<<grid, kProjThreads, 0, st>>>(s, p, out, valid_mask, lb_state, ticket, count_out, part_hist); break;
        case 0: k_project<0><<<grid, kProjThreads, 0, st>>>(s, p, out, valid_mask, lb_state, ticket, count_out, part_hist); break;
        case 1: k_project<1><<<grid, kProjThreads, 0, st>>>(s, p, out, valid_mask, lb_state, ticket, count_out, part_hist); break;
        case 2: k_project<2><<<grid, kProjThreads, 0, st>>>(s, p, out, valid_mask, lb_state, ticket, count_out, part_hist); break;
        case 3: k_project<3><<<grid, kProjThreads, 0, st>>>(s, p, out, valid_mask, lb_state, ticket, count_out, part_hist); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

size_t project_partitions(int64_t n) { return (size_t)((n + kProjPart - 1) / kProjPart); }

const void* project_kernel(int sh_degree) {
    switch (sh_degree) {
        case -1: return reinterpret_cast<const void*>(&k_project<-1>);
        case 0: return reinterpret_cast<const void*>(&k_project<0>);
        case 1: return reinterpret_cast<const void*>(&k_project<1>);
        case 2: return reinterpret_cast<const void*>(&k_project<2>);
        case 3: return reinterpret_cast<const void*>(&k_project<3>);
        default: return nullptr;
    }
}

bool graph_project_args_are(hipGraphNode_t node, const SceneDev& s, const ProjParams& p) {
    hipKernelNodeParams kp;
    if (hipGraphKernelNodeGetParams(node, &kp) != hipSuccess || kp.kernelParams == nullptr)
        return false;
    const SceneDev& a = *static_cast<const SceneDev*>(kp.kernelParams[0]);
    const ProjParams& b = *static_cast<const ProjParams*>(kp.kernelParams[1]);
    bool same = a.n == s.n && a.sh_degree == s.sh_degree && a.sh == s.sh && a.opac == s.opac &&
                a.mean[0] == s.mean[0] && a.cov[5] == s.cov[5] && a.lthr == s.lthr &&
                b.ctl == p.ctl && b.dvals == p.dvals && b.skip == p.skip && b.fx == p.fx &&
                b.fy == p.fy && b.width == p.width && b.height == p.height;
    for (int j = 0; j < 9; ++j) same = same && b.r[j] == p.r[j];
    for (int j = 0; j < 3; ++j) same = same && b.t[j] == p.t[j];
    return same;
}

hipError_t graph_set_project_params(hipGraphExec_t exec, hipGraphNode_t node, const ProjParams& p) {
    hipKernelNodeParams kp;
    hipError_t e = hipGraphKernelNodeGetParams(node, &kp);
    if (e != hipSuccess) return e;
    if (kp.kernelParams == nullptr) return hipErrorInvalidValue;
    // the node's arguments as launch_project passed them, the view's replaced
    SceneDev a0 = *static_cast<const SceneDev*>(kp.kernelParams[0]);
    ProjParams a1 = p;
    Compact a2 = *static_cast<const Compact*>(kp.kernelParams[2]);
    uint8_t* a3 = *static_cast<uint8_t* const*>(kp.kernelParams[3]);
    uint64_t* a4 = *static_cast<uint64_t* const*>(kp.kernelParams[4]);
    uint32_t* a5 = *static_cast<uint32_t* const*>(kp.kernelParams[5]);
    uint32_t* a6 = *static_cast<uint32_t* const*>(kp.kernelParams[6]);
    uint32_t* a7 = *static_cast<uint32_t* const*>(kp.kernelParams[7]);
    void* args[8] = {&a0, &a1, &a2, &a3, &a4, &a5, &a6, &a7};
    kp.kernelParams = args;
    kp.extra = nullptr;
    return hipGraphExecKernelNodeSetParams(exec, node, &kp);
}

size_t chunk_box_doubles(int64_t n) { return project_partitions(n) * 8; }

hipError_t launch_chunk_boxes(const SceneDev& s, double k, double* box, hipStream_t st) {
    if (s.n <= 0) return hipSuccess;
    const unsigned grid = (unsigned)project_partitions(s.n);
    k_chunk_boxes<<<grid, kProjThreads, 0, st>>>(s, k, box);
    return hipGetLastError();
}

hipError_t launch_chunk_cull(const double* box, int64_t n, const ProjParams& p, double k,
                             uint8_t* skip, uint32_t* n_skipped, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int64_t nc = (int64_t)project_partitions(n);
    k_chunk_cull<<<(unsigned)((nc + 255) / 256), 256, 0, st>>>(box, nc, p, k, skip, n_skipped);
    return hipGetLastError();
}

hipError_t launch_soa_transpose(const float* aos, int64_t n, int cols, const int* col_map,
                                int planes, float* soa, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (planes > 64 || planes <= 0) return hipErrorInvalidValue;
    ColMap map{};
    for (int j = 0; j < planes; ++j) {
        if (col_map[j] < 0 || col_map[j] >= cols) return hipErrorInvalidValue;
        map.c[j] = col_map[j];
    }
    const unsigned grid = (unsigned)((n + 255) / 256);
    k_soa_transpose<<<grid, 256, 0, st>>>(aos, n, cols, map, planes, soa);
    return hipGetLastError();
}

hipError_t launch_brec_from_arrays(const float* means2d, const float* covs2d,
                                   const float* colors, const float* opac, const float* lthr,
                                   int64_t m, float4* brec, hipStream_t st) {
    if (m <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((m + 255) / 256);
    k_brec_from_arrays<<<grid, 256, 0, st>>>(means2d, covs2d, colors, opac, lthr, m, brec);
    return hipGetLastError();
}

}  // namespace gs
