// train.hip - one training step of the splat rasterizer on gfx950: projection of
// the optimizer-space parameters, per-tile forward with the 3DGS blend rules and
// the L1 gradient, per-tile blend backward with per-Gaussian reduction, the
// analytic projection backward, and sparse Adam over the visible rows.
//
// Follows the reference's training oracle gsplat/train_oracle.py:
//   projection + colour + 3-sigma visibility  :125-181
//   blend (skip alpha < alpha_min, stop without blending when
//   T (1 - alpha) < t_min, alpha clamp)         :183-233
//   sparse Adam                                  :434-470
// and the L1 gradient of gsplat/train_loss.py:166-171. Every Gaussian that can
// reach alpha_min somewhere is kept: its footprint uses the opacity-aware
// radius k = sqrt(2 ln(op / alpha_min)) (uncapped) and the per-pair tile cull at
// the same floor, so the tiled forward blends exactly the pairs the per-pixel
// oracle blends.
#include "gs_common.h"
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kTThreads = 512;
constexpr int kTItems = 4;
constexpr int kTPart = kTThreads * kTItems;
static_assert(kTPart == (int)kProjPartition, "projection partition size");

constexpr float kC0 = 0.28209479177387814f;
constexpr float kC1 = 0.4886025119029199f;
__constant__ float kC2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f,
                             -1.0925484305920792f, 0.5462742152960396f};
__constant__ float kC3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f,
                             0.3731763325901154f, -0.4570457994644658f, 1.445305721320277f,
                             -0.5900435899266435f};

// Real SH basis (3DGS order) of direction (x, y, z) up to DEG, and optionally its
// gradient with respect to (x, y, z) taken as a polynomial.
template <int DEG, bool GRAD>
__device__ __forceinline__ void sh_basis(float x, float y, float z, float* b, float (*g)[3]) {
    b[0] = kC0;
    if (GRAD) g[0][0] = g[0][1] = g[0][2] = 0.0f;
    if (DEG >= 1) {
        b[1] = -kC1 * y;
        b[2] = kC1 * z;
        b[3] = -kC1 * x;
        if (GRAD) {
            g[1][0] = 0.0f; g[1][1] = -kC1; g[1][2] = 0.0f;
            g[2][0] = 0.0f; g[2][1] = 0.0f; g[2][2] = kC1;
            g[3][0] = -kC1; g[3][1] = 0.0f; g[3][2] = 0.0f;
        }
    }
    if (DEG >= 2) {
        const float xx = x * x, yy = y * y, zz = z * z;
        b[4] = kC2[0] * x * y;
        b[5] = kC2[1] * y * z;
        b[6] = kC2[2] * (2.0f * zz - xx - yy);
        b[7] = kC2[3] * x * z;
        b[8] = kC2[4] * (xx - yy);
        if (GRAD) {
            g[4][0] = kC2[0] * y; g[4][1] = kC2[0] * x; g[4][2] = 0.0f;
            g[5][0] = 0.0f; g[5][1] = kC2[1] * z; g[5][2] = kC2[1] * y;
            g[6][0] = -2.0f * kC2[2] * x; g[6][1] = -2.0f * kC2[2] * y; g[6][2] = 4.0f * kC2[2] * z;
            g[7][0] = kC2[3] * z; g[7][1] = 0.0f; g[7][2] = kC2[3] * x;
            g[8][0] = 2.0f * kC2[4] * x; g[8][1] = -2.0f * kC2[4] * y; g[8][2] = 0.0f;
        }
        if (DEG >= 3) {
            b[9] = kC3[0] * y * (3.0f * xx - yy);
            b[10] = kC3[1] * x * y * z;
            b[11] = kC3[2] * y * (4.0f * zz - xx - yy);
            b[12] = kC3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
            b[13] = kC3[4] * x * (4.0f * zz - xx - yy);
            b[14] = kC3[5] * z * (xx - yy);
            b[15] = kC3[6] * x * (xx - 3.0f * yy);
            if (GRAD) {
                g[9][0] = 6.0f * kC3[0] * x * y; g[9][1] = kC3[0] * (3.0f * xx - 3.0f * yy);
                g[9][2] = 0.0f;
                g[10][0] = kC3[1] * y * z; g[10][1] = kC3[1] * x * z; g[10][2] = kC3[1] * x * y;
                g[11][0] = -2.0f * kC3[2] * x * y;
                g[11][1] = kC3[2] * (4.0f * zz - xx - 3.0f * yy);
                g[11][2] = 8.0f * kC3[2] * y * z;
                g[12][0] = -6.0f * kC3[3] * x * z; g[12][1] = -6.0f * kC3[3] * y * z;
                g[12][2] = kC3[3] * (6.0f * zz - 3.0f * xx - 3.0f * yy);
                g[13][0] = kC3[4] * (4.0f * zz - 3.0f * xx - yy);
                g[13][1] = -2.0f * kC3[4] * x * y; g[13][2] = 8.0f * kC3[4] * x * z;
                g[14][0] = 2.0f * kC3[5] * x * z; g[14][1] = -2.0f * kC3[5] * y * z;
                g[14][2] = kC3[5] * (xx - yy);
                g[15][0] = kC3[6] * (3.0f * xx - 3.0f * yy); g[15][1] = -6.0f * kC3[6] * x * y;
                g[15][2] = 0.0f;
            }
        }
    }
}

// Per-Gaussian projection values (train_oracle.py:125-181), fp32.
struct Geo {
    float x, y, z, iz;
    bool valid;
    float u, v;
    float qn[4], qinv;
    float Rq[9];
    float s[3];
    float S[6];       // cov3d: s00 s01 s02 s11 s12 s22
    float T0[3], T1[3];
    float a, b, c;    // low-passed 2D covariance
    float A, B, C;    // conic
};

__device__ __forceinline__ float s3(const float* S, int i, int k) {
    const int lo = i < k ? i : k, hi = i < k ? k : i;
    return lo == 0 ? S[hi] : (lo == 1 ? S[2 + hi] : S[5]);
}

__device__ __forceinline__ void geometry(const TrainParamsDev& P, int64_t i, const TrainCam& cam,
                                         Geo& g) {
    const float mx = P.mean[0][i], my = P.mean[1][i], mz = P.mean[2][i];
    const float* R = cam.r;
    g.x = R[0] * mx + R[1] * my + R[2] * mz + cam.t[0];
    g.y = R[3] * mx + R[4] * my + R[5] * mz + cam.t[1];
    g.z = R[6] * mx + R[7] * my + R[8] * mz + cam.t[2];
    g.valid = g.z > cam.near;
    const float zs = g.valid ? g.z : 1.0f;
    g.iz = 1.0f / zs;
    g.u = cam.fx * g.x * g.iz + cam.cx;
    g.v = cam.fy * g.y * g.iz + cam.cy;
    const float q0 = P.quat[0][i], q1 = P.quat[1][i], q2 = P.quat[2][i], q3 = P.quat[3][i];
    g.qinv = 1.0f / sqrtf(q0 * q0 + q1 * q1 + q2 * q2 + q3 * q3);
    const float w = q0 * g.qinv, x = q1 * g.qinv, y = q2 * g.qinv, z = q3 * g.qinv;
    g.qn[0] = w; g.qn[1] = x; g.qn[2] = y; g.qn[3] = z;
    float* Q = g.Rq;
    Q[0] = 1.0f - 2.0f * (y * y + z * z); Q[1] = 2.0f * (x * y - w * z); Q[2] = 2.0f * (x * z + w * y);
    Q[3] = 2.0f * (x * y + w * z); Q[4] = 1.0f - 2.0f * (x * x + z * z); Q[5] = 2.0f * (y * z - w * x);
    Q[6] = 2.0f * (x * z - w * y); Q[7] = 2.0f * (y * z + w * x); Q[8] = 1.0f - 2.0f * (x * x + y * y);
    g.s[0] = expf(P.ls[0][i]);
    g.s[1] = expf(P.ls[1][i]);
    g.s[2] = expf(P.ls[2][i]);
    float M[9];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) M[3 * r + k] = Q[3 * r + k] * g.s[k];
    int idx = 0;
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = r; k < 3; ++k)
            g.S[idx++] = M[3 * r] * M[3 * k] + M[3 * r + 1] * M[3 * k + 1] + M[3 * r + 2] * M[3 * k + 2];
    const float j00 = cam.fx * g.iz, j02 = -cam.fx * g.x * g.iz * g.iz;
    const float j11 = cam.fy * g.iz, j12 = -cam.fy * g.y * g.iz * g.iz;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        g.T0[k] = j00 * R[k] + j02 * R[6 + k];
        g.T1[k] = j11 * R[3 + k] + j12 * R[6 + k];
    }
    float CT0[3], CT1[3];
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        CT0[r] = s3(g.S, r, 0) * g.T0[0] + s3(g.S, r, 1) * g.T0[1] + s3(g.S, r, 2) * g.T0[2];
        CT1[r] = s3(g.S, r, 0) * g.T1[0] + s3(g.S, r, 1) * g.T1[1] + s3(g.S, r, 2) * g.T1[2];
    }
    g.a = g.T0[0] * CT0[0] + g.T0[1] * CT0[1] + g.T0[2] * CT0[2] + cam.lowpass;
    g.b = g.T1[0] * CT0[0] + g.T1[1] * CT0[1] + g.T1[2] * CT0[2];
    g.c = g.T1[0] * CT1[0] + g.T1[1] * CT1[1] + g.T1[2] * CT1[2] + cam.lowpass;
    const float det = g.a * g.c - g.b * g.b;
    g.A = g.c / det;
    g.B = -g.b / det;
    g.C = g.a / det;
}

template <int DEG>
__device__ __forceinline__ void colour(const TrainParamsDev& P, int64_t i, const TrainCam& cam,
                                       float* raw, float* dir, float& dnorm) {
    constexpr int K = (DEG + 1) * (DEG + 1);
    const float dx = P.mean[0][i] - cam.ccx, dy = P.mean[1][i] - cam.ccy,
                dz = P.mean[2][i] - cam.ccz;
    dnorm = sqrtf(dx * dx + dy * dy + dz * dz);
    dir[0] = dx / dnorm; dir[1] = dy / dnorm; dir[2] = dz / dnorm;
    float b[16];
    sh_basis<DEG, false>(dir[0], dir[1], dir[2], b, nullptr);
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) acc += b[k] * P.sh[(size_t)(3 * k + ch) * P.n + i];
        raw[ch] = acc + 0.5f;
    }
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

// Projection of the optimizer-space parameters; stable compaction of the
// Gaussians that can reach alpha_min somewhere in the image.
template <int DEG>
__global__ __launch_bounds__(kTThreads) void k_train_project(
    TrainParamsDev P, TrainCam cam, Compact out, float4* __restrict__ trec,
    uint32_t* __restrict__ cidx, uint8_t* __restrict__ visible, uint64_t* lb_state,
    uint32_t* ticket, uint32_t* count_out, uint32_t* __restrict__ part_hist, TrainDebug dbg) {
    __shared__ uint32_t s_vid;
    __shared__ uint32_t s_cnt[kTItems][kTThreads / GS_WAVE];
    __shared__ uint32_t s_hist[4][256];
    __shared__ uint64_t s_excl;
    const int tid = threadIdx.x, w = tid / GS_WAVE, lane = lane_id();
    if (tid == 0) s_vid = atomicAdd(ticket, 1u);
    for (int k = tid; k < 1024; k += kTThreads) (&s_hist[0][0])[k] = 0;
    __syncthreads();
    const uint32_t vid = s_vid;
    const int64_t base = (int64_t)vid * kTPart;
    const int64_t n = P.n;
    bool keep[kTItems];
    float4 rect[kTItems], cov[kTItems], r0[kTItems], r1[kTItems], r2[kTItems];
    float depth[kTItems];
    uint64_t bal[kTItems];
#pragma unroll
    for (int it = 0; it < kTItems; ++it) {
        const int64_t i = base + it * kTThreads + tid;
        keep[it] = false;
        depth[it] = 0.0f;
        if (i < n) {
            Geo g;
            geometry(P, i, cam, g);
            const float op = sigmoidf(P.ol[i]);
            float raw[3], dir[3], dn;
            colour<DEG>(P, i, cam, raw, dir, dn);
            // sparse-Adam rows: 3-sigma box overlaps the image (train_oracle.py:175-181)
            const float rx3 = ceilf(3.0f * sqrtf(fmaxf(g.a, 0.0f)));
            const float ry3 = ceilf(3.0f * sqrtf(fmaxf(g.c, 0.0f)));
            const bool vis = g.valid && (g.u + rx3 > 0.0f) && (g.u - rx3 < (float)cam.W) &&
                             (g.v + ry3 > 0.0f) && (g.v - ry3 < (float)cam.H);
            visible[i] = vis ? 1 : 0;
            // blendable: alpha = op exp(power) >= alpha_min somewhere in the image
            bool k = g.valid && op >= cam.alpha_min && g.a * g.c - g.b * g.b > 0.0f;
            float m2thr = 0.0f, rx = 0.0f, ry = 0.0f;
            if (k) {
                m2thr = 2.0f * logf(op / cam.alpha_min);
                const float kk = sqrtf(m2thr);
                rx = ceilf(kk * sqrtf(fmaxf(g.a, 0.0f)));
                ry = ceilf(kk * sqrtf(fmaxf(g.c, 0.0f)));
                k = rx > 0.0f && ry > 0.0f && (g.u + rx > 0.0f) && (g.u - rx < (float)cam.W) &&
                    (g.v + ry > 0.0f) && (g.v - ry < (float)cam.H);
            }
            keep[it] = k;
            const float col[3] = {raw[0] < 0.0f ? 0.0f : raw[0], raw[1] < 0.0f ? 0.0f : raw[1],
                                  raw[2] < 0.0f ? 0.0f : raw[2]};
            rect[it] = make_float4(g.u, g.v, rx, ry);
            cov[it] = make_float4(g.a, g.b, g.c, m2thr);
            r0[it] = make_float4(g.u, g.v, op, 0.0f);
            r1[it] = make_float4(g.A, g.B, g.C, 0.0f);
            r2[it] = make_float4(col[0], col[1], col[2], 0.0f);
            depth[it] = g.z;
            if (dbg.means2d != nullptr) {
                dbg.means2d[2 * i] = g.u;
                dbg.means2d[2 * i + 1] = g.v;
                dbg.conic[3 * i] = g.A;
                dbg.conic[3 * i + 1] = g.B;
                dbg.conic[3 * i + 2] = g.C;
                dbg.opacity[i] = op;
                dbg.colors[3 * i] = col[0];
                dbg.colors[3 * i + 1] = col[1];
                dbg.colors[3 * i + 2] = col[2];
                dbg.depth[i] = g.z;
                dbg.valid[i] = g.valid ? 1 : 0;
            }
            if (!k) cidx[i] = 0xFFFFFFFFu;
        }
        {
            const uint32_t key = __float_as_uint(depth[it]);
            hist_add_wave(s_hist[0], key & 255u, keep[it]);
            hist_add_wave(s_hist[1], (key >> 8) & 255u, keep[it]);
            hist_add_wave(s_hist[2], (key >> 16) & 255u, keep[it]);
            hist_add_wave(s_hist[3], key >> 24, keep[it]);
        }
        bal[it] = __ballot(keep[it]);
        if (lane == 0) s_cnt[it][w] = (uint32_t)__popcll(bal[it]);
    }
    __syncthreads();
    for (int k = tid; k < 1024; k += kTThreads)
        part_hist[(size_t)vid * 1024 + k] = (&s_hist[0][0])[k];
    uint32_t total = 0, my_off[kTItems];
#pragma unroll
    for (int it = 0; it < kTItems; ++it)
#pragma unroll
        for (int ww = 0; ww < kTThreads / GS_WAVE; ++ww) {
            if (ww == w) my_off[it] = total;
            total += s_cnt[it][ww];
        }
    if (w == 0) {
        const uint64_t excl = lookback_exclusive(lb_state, vid, total, cam.ctl);
        if (lane == 0) {
            s_excl = excl;
            if (vid == gridDim.x - 1) *count_out = (uint32_t)(excl + total);
        }
    }
    __syncthreads();
    const uint64_t excl = s_excl;
    const uint64_t ltm = lanemask_lt();
#pragma unroll
    for (int it = 0; it < kTItems; ++it) {
        if (!keep[it]) continue;
        const int64_t i = base + it * kTThreads + tid;
        const uint64_t m = excl + my_off[it] + (uint64_t)__popcll(bal[it] & ltm);
        out.rc[2 * m + 0] = rect[it];
        out.rc[2 * m + 1] = cov[it];
        out.dkey[m] = __float_as_uint(depth[it]);
        trec[3 * m + 0] = r0[it];
        trec[3 * m + 1] = r1[it];
        trec[3 * m + 2] = r2[it];
        out.src[m] = (uint32_t)i;
        cidx[i] = (uint32_t)m;
    }
}

// Forward of one 16x16 tile, one pixel per thread, entries staged in LDS in
// batches of 256 (3DGS rules, train_oracle.py:196-229). Writes the image, the
// final transmittance, the entry index where the pixel stopped, and - with a
// target - the L1 gradient and the loss.
__global__ __launch_bounds__(256) void k_train_fwd(const float4* __restrict__ trec,
                                                   const uint32_t* __restrict__ sid,
                                                   const uint32_t* __restrict__ ranges,
                                                   TrainFwdParams fp) {
    __shared__ float4 s0[256], s1[256], s2[256];
    __shared__ double s_loss[4];
    __shared__ unsigned long long s_pairs[2][4];
    // after an earlier give-up the sorted ids may be wrong: read nothing (the
    // flag was raised by an earlier launch, so every thread sees the same value)
    if (upstream_failed(fp.ctl)) return;
    const int tid = threadIdx.x;
    const int tile = blockIdx.x;
    const int tx = tile % fp.tiles_x, ty = tile / fp.tiles_x;
    const int px = tx * 16 + (tid & 15), py = ty * 16 + (tid >> 4);
    const bool inside = px < fp.width && py < fp.height;
    const float pxc = (float)px + 0.5f, pyc = (float)py + 0.5f;
    const uint32_t start = ranges[2 * tile], end = ranges[2 * tile + 1];
    float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
    bool done = !inside;
    uint32_t stop = end - start;
    uint32_t blended = 0;
    for (uint32_t base = start; base < end; base += 256) {
        const uint32_t nb = min(256u, end - base);
        if ((uint32_t)tid < nb) {
            const uint32_t gi = sid[base + tid];
            s0[tid] = trec[3 * (size_t)gi + 0];
            s1[tid] = trec[3 * (size_t)gi + 1];
            s2[tid] = trec[3 * (size_t)gi + 2];
        }
        __syncthreads();
        if (!done) {
            for (uint32_t j = 0; j < nb; ++j) {
                const float4 r0 = s0[j], r1 = s1[j];
                const float dx = pxc - r0.x, dy = pyc - r0.y;
                const float power = -0.5f * (r1.x * dx * dx + 2.0f * r1.y * dx * dy + r1.z * dy * dy);
                const float raw = r0.z * __expf(power < 0.0f ? power : 0.0f);
                const float alpha = raw > fp.alpha_max ? fp.alpha_max : raw;
                if (alpha < fp.alpha_min) continue;
                const float tn = T * (1.0f - alpha);
                if (tn < fp.t_min) {
                    done = true;
                    stop = base - start + j;
                    break;
                }
                const float4 c = s2[j];
                const float at = alpha * T;
                cr += at * c.x;
                cg += at * c.y;
                cb += at * c.z;
                T = tn;
                ++blended;
            }
        }
        if (__syncthreads_count(!done) == 0) break;
    }
    double lsum = 0.0;
    if (inside) {
        const size_t p = (size_t)py * fp.width + px;
        const float o[3] = {cr + T * fp.bg[0], cg + T * fp.bg[1], cb + T * fp.bg[2]};
        fp.image[3 * p + 0] = o[0];
        fp.image[3 * p + 1] = o[1];
        fp.image[3 * p + 2] = o[2];
        fp.final_T[p] = T;
        fp.stop[p] = stop;
        if (fp.target != nullptr) {
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) {
                const float d = o[ch] - fp.target[3 * p + ch];
                const float sg = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
                fp.dimage[3 * p + ch] = sg * fp.grad_scale;
                lsum += (double)fabsf(d);
            }
        }
    }
    if (fp.target != nullptr) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o, GS_WAVE);
        if (lane_id() == 0) s_loss[tid / GS_WAVE] = lsum;
    }
    if (fp.pairs != nullptr) {
        unsigned long long pc = inside ? stop : 0u, pb = inside ? blended : 0u;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            pc += __shfl_xor(pc, o, GS_WAVE);
            pb += __shfl_xor(pb, o, GS_WAVE);
        }
        if (lane_id() == 0) {
            s_pairs[0][tid / GS_WAVE] = pc;
            s_pairs[1][tid / GS_WAVE] = pb;
        }
    }
    __syncthreads();
    if (tid == 0) {
        if (fp.target != nullptr)
            atomicAdd(fp.loss, s_loss[0] + s_loss[1] + s_loss[2] + s_loss[3]);
        if (fp.pairs != nullptr) {
            atomicAdd(&fp.pairs[0], s_pairs[0][0] + s_pairs[0][1] + s_pairs[0][2] + s_pairs[0][3]);
            atomicAdd(&fp.pairs[1], s_pairs[1][0] + s_pairs[1][1] + s_pairs[1][2] + s_pairs[1][3]);
        }
    }
}

// ---------------------------------------------------------------------------
// Full 3DGS loss (train_oracle.py:253-279): SSIM with an 11-tap Gaussian window
// (sigma 1.5), zero padding, S = A B / (C D); the image gradient in the
// fused-SSIM form of train_loss.py:5-19. One workgroup per 16x16 tile and
// channel loop; a 26x26 halo in LDS, row pass then column pass.
// ---------------------------------------------------------------------------
constexpr int kSsimT = 16, kSsimR = 5, kSsimE = kSsimT + 2 * kSsimR;

// Forward: mu_x, mu_y, E_xx, E_yy, E_xy -> S and the three per-pixel terms
// w dS/dmu_x, w dS/dE_xx, w dS/dE_xy (zero outside the image), sum of S.
__global__ __launch_bounds__(256) void k_ssim_fwd(SsimParams sp) {
    __shared__ float s_x[kSsimE][kSsimE + 1], s_y[kSsimE][kSsimE + 1];
    __shared__ float s_h[5][kSsimE][kSsimT + 1];
    __shared__ double s_sum[4];
    const int tid = threadIdx.x;
    const int tiles_x = (sp.width + kSsimT - 1) / kSsimT;
    const int tx = blockIdx.x % tiles_x, ty = blockIdx.x / tiles_x;
    const int x0 = tx * kSsimT - kSsimR, y0 = ty * kSsimT - kSsimR;
    const int lx = tid & 15, ly = tid >> 4;
    const int px = tx * kSsimT + lx, py = ty * kSsimT + ly;
    const bool inside = px < sp.width && py < sp.height;
    const size_t npx = (size_t)sp.width * sp.height;
    double ssum = 0.0;
    for (int ch = 0; ch < 3; ++ch) {
        for (int i = tid; i < kSsimE * kSsimE; i += 256) {
            const int r = i / kSsimE, c = i % kSsimE;
            const int gx = x0 + c, gy = y0 + r;
            float xv = 0.0f, yv = 0.0f;
            if (gx >= 0 && gx < sp.width && gy >= 0 && gy < sp.height) {
                const size_t q = ((size_t)gy * sp.width + gx) * 3 + ch;
                xv = sp.image[q];
                yv = sp.target[q];
            }
            s_x[r][c] = xv;
            s_y[r][c] = yv;
        }
        __syncthreads();
        // row pass over all 26 halo rows, 16 output columns
        for (int i = tid; i < kSsimE * kSsimT; i += 256) {
            const int r = i / kSsimT, c = i % kSsimT;
            float hx = 0.0f, hy = 0.0f, hxx = 0.0f, hyy = 0.0f, hxy = 0.0f;
#pragma unroll
            for (int k = 0; k < 11; ++k) {
                const float xv = s_x[r][c + k], yv = s_y[r][c + k], g = sp.g[k];
                hx += g * xv;
                hy += g * yv;
                hxx += g * (xv * xv);
                hyy += g * (yv * yv);
                hxy += g * (xv * yv);
            }
            s_h[0][r][c] = hx;
            s_h[1][r][c] = hy;
            s_h[2][r][c] = hxx;
            s_h[3][r][c] = hyy;
            s_h[4][r][c] = hxy;
        }
        __syncthreads();
        float mu_x = 0.0f, mu_y = 0.0f, e_xx = 0.0f, e_yy = 0.0f, e_xy = 0.0f;
#pragma unroll
        for (int k = 0; k < 11; ++k) {
            const float g = sp.g[k];
            mu_x += g * s_h[0][ly + k][lx];
            mu_y += g * s_h[1][ly + k][lx];
            e_xx += g * s_h[2][ly + k][lx];
            e_yy += g * s_h[3][ly + k][lx];
            e_xy += g * s_h[4][ly + k][lx];
        }
        if (inside) {
            const float c1 = 0.01f * 0.01f, c2 = 0.03f * 0.03f;
            const float mxy = mu_x * mu_y;
            const float A = 2.0f * mxy + c1;
            const float B = 2.0f * (e_xy - mxy) + c2;
            const float C = mu_x * mu_x + mu_y * mu_y + c1;
            const float D = (e_xx - mu_x * mu_x) + (e_yy - mu_y * mu_y) + c2;
            const float S = (A * B) / (C * D);
            const float Sw = S * sp.w;
            const float d_mu = Sw * (2.0f * mu_y / A - 2.0f * mu_y / B - 2.0f * mu_x / C +
                                     2.0f * mu_x / D);
            const size_t q = ((size_t)py * sp.width + px) * 3 + ch;
            sp.maps[q] = d_mu;
            sp.maps[3 * npx + q] = -Sw / D;
            sp.maps[6 * npx + q] = 2.0f * Sw / B;
            ssum += (double)S;
        }
        __syncthreads();  // the next channel overwrites the LDS planes
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ssum += __shfl_xor(ssum, o, GS_WAVE);
    if (lane_id() == 0) s_sum[tid / GS_WAVE] = ssum;
    __syncthreads();
    if (tid == 0) atomicAdd(sp.ssim_sum, (s_sum[0] + s_sum[1]) + (s_sum[2] + s_sum[3]));
}

// Backward: dimage += G*(w dS/dmu_x) + 2 x G*(w dS/dE_xx) + y G*(w dS/dE_xy)
// (G symmetric, so its adjoint is the same zero-padded filter).
__global__ __launch_bounds__(256) void k_ssim_bwd(SsimParams sp) {
    __shared__ float s_m[3][kSsimE][kSsimE + 1];
    __shared__ float s_h[3][kSsimE][kSsimT + 1];
    const int tid = threadIdx.x;
    const int tiles_x = (sp.width + kSsimT - 1) / kSsimT;
    const int tx = blockIdx.x % tiles_x, ty = blockIdx.x / tiles_x;
    const int x0 = tx * kSsimT - kSsimR, y0 = ty * kSsimT - kSsimR;
    const int lx = tid & 15, ly = tid >> 4;
    const int px = tx * kSsimT + lx, py = ty * kSsimT + ly;
    const bool inside = px < sp.width && py < sp.height;
    const size_t npx = (size_t)sp.width * sp.height;
    for (int ch = 0; ch < 3; ++ch) {
        for (int i = tid; i < kSsimE * kSsimE; i += 256) {
            const int r = i / kSsimE, c = i % kSsimE;
            const int gx = x0 + c, gy = y0 + r;
            float a = 0.0f, b = 0.0f, d = 0.0f;
            if (gx >= 0 && gx < sp.width && gy >= 0 && gy < sp.height) {
                const size_t q = ((size_t)gy * sp.width + gx) * 3 + ch;
                a = sp.maps[q];
                b = sp.maps[3 * npx + q];
                d = sp.maps[6 * npx + q];
            }
            s_m[0][r][c] = a;
            s_m[1][r][c] = b;
            s_m[2][r][c] = d;
        }
        __syncthreads();
        for (int i = tid; i < kSsimE * kSsimT; i += 256) {
            const int r = i / kSsimT, c = i % kSsimT;
            float h0 = 0.0f, h1 = 0.0f, h2 = 0.0f;
#pragma unroll
            for (int k = 0; k < 11; ++k) {
                const float g = sp.g[k];
                h0 += g * s_m[0][r][c + k];
                h1 += g * s_m[1][r][c + k];
                h2 += g * s_m[2][r][c + k];
            }
            s_h[0][r][c] = h0;
            s_h[1][r][c] = h1;
            s_h[2][r][c] = h2;
        }
        __syncthreads();
        if (inside) {
            float P = 0.0f, Q = 0.0f, R = 0.0f;
#pragma unroll
            for (int k = 0; k < 11; ++k) {
                const float g = sp.g[k];
                P += g * s_h[0][ly + k][lx];
                Q += g * s_h[1][ly + k][lx];
                R += g * s_h[2][ly + k][lx];
            }
            const size_t q = ((size_t)py * sp.width + px) * 3 + ch;
            sp.dimage[q] += P + 2.0f * sp.image[q] * Q + sp.target[q] * R;
        }
        __syncthreads();
    }
}

// dimage = scale * sign(image - target), sum |image - target| (stage path).
__global__ __launch_bounds__(256) void k_l1(const float* __restrict__ image,
                                            const float* __restrict__ target, int64_t count,
                                            float scale, float* __restrict__ dimage,
                                            double* l1_sum) {
    __shared__ double s_sum[4];
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    double a = 0.0;
    if (i < count) {
        const float d = image[i] - target[i];
        dimage[i] = (d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f)) * scale;
        a = (double)fabsf(d);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o, GS_WAVE);
    if (lane_id() == 0) s_sum[threadIdx.x / GS_WAVE] = a;
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(l1_sum, (s_sum[0] + s_sum[1]) + (s_sum[2] + s_sum[3]));
}

// v plus the value a DPP move brings into the lane (all lanes active).
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_add(float v) {
    const int x = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false);
    return v + __int_as_float(x);
}

// Lanes whose per-pair terms are summed together before one of them adds the
// sums into LDS: fewer LDS atomics against more DPP steps. Measured on the 1M
// training step (backward ms): 8 lanes 0.99, 16 lanes 0.63, 32 lanes 0.57,
// 64 lanes 0.58 (LDS float atomics cost more per lane than the DPP adds).
constexpr int kBwdGroup = 32;
constexpr int kBwdCopies = GS_WAVE / kBwdGroup;  // LDS accumulator copies, one per group
constexpr int kBwdBatch = 128;

// Sum over each group of kBwdGroup lanes, complete in the group's last lane
// (quad swaps, half-row and row mirrors, then row broadcasts across rows).
__device__ __forceinline__ float group_fsum(float v) {
    v = dpp_add<0xB1, 0xF>(v);   // quad_perm 1,0,3,2
    v = dpp_add<0x4E, 0xF>(v);   // quad_perm 2,3,0,1
    v = dpp_add<0x141, 0xF>(v);  // row_half_mirror
    if constexpr (kBwdGroup >= 16) v = dpp_add<0x140, 0xF>(v);  // row_mirror
    // Across rows: v += lane 15 of the row before (rows 1, 3), then v += lane 31
    // (rows 2, 3). One DPP add each, the rows outside the row mask keeping v; the
    // s_nop gives the two wait states a DPP read needs after a VALU write.
    if constexpr (kBwdGroup >= 32)
        asm volatile("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf"
                     : "+v"(v));
    if constexpr (kBwdGroup >= 64)
        asm volatile("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf"
                     : "+v"(v));
    return v;
}

// Backward of one 16x16 tile: entries from the last one any pixel considered
// down to the first; per pixel the reverse recursion T_i = T_{i+1}/(1 - alpha_i),
// behind_i = alpha_{i+1} c_{i+1} + (1 - alpha_{i+1}) behind_{i+1},
// dL/dalpha_i = T_i (c_i - behind_i) . g - T_final bg . g / (1 - alpha_i).
// Per (wave, entry): the entry's alpha for every lane, a ballot of the lanes
// that blend it, and only when one does, the nine per-pair terms (dmx dmy dA
// dB dC dop dr dg db) for every lane with the lanes that do not blend it
// contributing exact zeros (selects, no divergent branches). The terms are
// summed over each group of kBwdGroup lanes with DPP moves and the group's last
// lane adds them into its own LDS accumulator copy (copies interleaved, so the
// lanes hit distinct banks); the copies' sum goes to the Gaussian's accumulator
// with one global atomic per term. 1/(1 - alpha) is one reciprocal estimate,
// exp the hardware exponential (the forward uses the same one, so both see the
// same alpha).
__global__ __launch_bounds__(256) void k_train_bwd(const float4* __restrict__ trec,
                                                   const uint32_t* __restrict__ sid,
                                                   const uint32_t* __restrict__ ranges,
                                                   TrainBwdParams bp) {
    __shared__ float4 s0[kBwdBatch], s1[kBwdBatch], s2[kBwdBatch];
    __shared__ __align__(16) float s_acc[kBwdBatch][9][kBwdCopies];
    __shared__ uint32_t s_has[4][kBwdBatch];
    __shared__ uint32_t s_nmax;
    const int tid = threadIdx.x, w = tid / GS_WAVE, lane = lane_id();
    const int tile = blockIdx.x;
    const int tx = tile % bp.tiles_x, ty = tile / bp.tiles_x;
    const int px = tx * 16 + (tid & 15), py = ty * 16 + (tid >> 4);
    const bool inside = px < bp.width && py < bp.height;
    const float pxc = (float)px + 0.5f, pyc = (float)py + 0.5f;
    const uint32_t start = ranges[2 * tile], end = ranges[2 * tile + 1];
    if (tid == 0) s_nmax = 0;
    float T = 1.0f, g0 = 0.0f, g1 = 0.0f, g2 = 0.0f, tbg = 0.0f;
    uint32_t stop = 0;
    if (inside) {
        const size_t p = (size_t)py * bp.width + px;
        T = bp.final_T[p];
        stop = bp.stop[p];
        g0 = bp.dimage[3 * p + 0];
        g1 = bp.dimage[3 * p + 1];
        g2 = bp.dimage[3 * p + 2];
        tbg = T * (bp.bg[0] * g0 + bp.bg[1] * g1 + bp.bg[2] * g2);
    }
    __syncthreads();
    if (stop > 0) atomicMax(&s_nmax, stop);
    __syncthreads();
    const uint32_t nmax = min(s_nmax, end - start);
    // the wave's own last considered entry: entries past it are skipped
    uint32_t wstop = stop;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) wstop = max(wstop, (uint32_t)__shfl_xor((int)wstop, o, GS_WAVE));
    float* const acc_lane = &s_acc[0][0][lane / kBwdGroup];  // this lane's copy (group leaders)
    const bool leader = (lane % kBwdGroup) == kBwdGroup - 1;
    float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f;  // colour behind (normalised)
    for (int32_t hi = (int32_t)nmax; hi > 0; hi -= kBwdBatch) {
        const int32_t lo = max(0, hi - kBwdBatch);
        const int32_t nb = hi - lo;
        if (tid < nb) {
            const uint32_t gi = sid[start + lo + tid];
            s0[tid] = trec[3 * (size_t)gi + 0];
            s1[tid] = trec[3 * (size_t)gi + 1];
            s2[tid] = trec[3 * (size_t)gi + 2];
        }
        for (int i = tid; i < kBwdBatch * 9 * kBwdCopies / 4; i += 256)
            reinterpret_cast<float4*>(&s_acc[0][0][0])[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int i = lane; i < nb; i += GS_WAVE) s_has[w][i] = 0u;
        __syncthreads();
        const int32_t jtop = min(nb, (int32_t)wstop - lo) - 1;
        for (int32_t j = jtop; j >= 0; --j) {
            const uint32_t e = (uint32_t)(lo + j);
            const float4 r0 = s0[j], r1 = s1[j];
            const float dx = pxc - r0.x, dy = pyc - r0.y;
            const float power = -0.5f * (r1.x * dx * dx + 2.0f * r1.y * dx * dy + r1.z * dy * dy);
            const float wgt = __expf(power < 0.0f ? power : 0.0f);
            const float raw = r0.z * wgt;
            const bool clamp = raw > bp.alpha_max;
            const float alpha = fminf(raw, bp.alpha_max);  // raw is finite: = clamp ? max : raw
            const bool live = e < stop && alpha >= bp.alpha_min;
            const uint64_t any = __ballot(live);
            if (any) {
                const float4 c = s2[j];
                const float om = 1.0f - alpha;
                const float rom = __builtin_amdgcn_rcpf(om);
                const float Tn = T * rom;
                const float dalpha =
                    Tn * ((c.x - b0) * g0 + (c.y - b1) * g1 + (c.z - b2) * g2) - tbg * rom;
                // a lane that does not blend the entry contributes exact zeros
                const float at = live ? alpha * Tn : 0.0f;
                const float d5 = (live && !clamp) ? dalpha : 0.0f;  // no gradient through the clamp
                const float dp = (power <= 0.0f ? d5 : 0.0f) * raw;
                float v[9];
                v[0] = dp * (r1.x * dx + r1.y * dy);
                v[1] = dp * (r1.y * dx + r1.z * dy);
                v[2] = -0.5f * dp * dx * dx;
                v[3] = -dp * dx * dy;
                v[4] = -0.5f * dp * dy * dy;
                v[5] = d5 * wgt;
                v[6] = at * g0;
                v[7] = at * g1;
                v[8] = at * g2;
                const float nb0 = alpha * c.x + om * b0;
                const float nb1 = alpha * c.y + om * b1;
                const float nb2 = alpha * c.z + om * b2;
                T = live ? Tn : T;
                b0 = live ? nb0 : b0;
                b1 = live ? nb1 : b1;
                b2 = live ? nb2 : b2;
#pragma unroll
                for (int k = 0; k < 9; ++k) {
                    v[k] = group_fsum(v[k]);
                    // keep the last step in every lane (one DPP add) rather than
                    // a DPP move for every lane plus an add in the leaders' branch
                    asm volatile("" : : "v"(v[k]));
                }
                if (leader) {
#pragma unroll
                    for (int k = 0; k < 9; ++k) atomicAdd(acc_lane + (j * 9 + k) * kBwdCopies, v[k]);
                }
            }
            if (lane == 0) s_has[w][j] = any ? 1u : 0u;
        }
        __syncthreads();
        if (tid < nb) {
            const bool has = (s_has[0][tid] | s_has[1][tid] | s_has[2][tid] | s_has[3][tid]) != 0u;
            if (has) {
                float acc[9];
#pragma unroll
                for (int k = 0; k < 9; ++k) {
                    float a = 0.0f;
#pragma unroll
                    for (int c = 0; c < kBwdCopies; ++c) a += s_acc[tid][k][c];
                    acc[k] = a;
                }
                const uint32_t gi = sid[start + lo + tid];
                float* dst = bp.grad2d + 9 * (size_t)gi;
#pragma unroll
                for (int k = 0; k < 9; ++k)
                    if (acc[k] != 0.0f) atomicAdd(dst + k, acc[k]);
            }
        }
        __syncthreads();
    }
}

// Optimizer-space gradients of every Gaussian from its accumulated 2D
// gradients (zero for Gaussians that blended nowhere).
template <int DEG>
__global__ __launch_bounds__(256) void k_train_param_grads(TrainParamsDev P, TrainCam cam,
                                                           const uint32_t* __restrict__ cidx,
                                                           const float* __restrict__ grad2d,
                                                           TrainParamsDev G) {
    constexpr int K = (DEG + 1) * (DEG + 1);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= P.n) return;
    const uint32_t ci = cidx[i];
    float gg[9];
    if (ci != 0xFFFFFFFFu) {
#pragma unroll
        for (int k = 0; k < 9; ++k) gg[k] = grad2d[9 * (size_t)ci + k];
    } else {
#pragma unroll
        for (int k = 0; k < 9; ++k) gg[k] = 0.0f;
    }
    bool any = false;
#pragma unroll
    for (int k = 0; k < 9; ++k) any |= gg[k] != 0.0f;
    if (!any) {
        for (int c = 0; c < 3; ++c) G.mean[c][i] = 0.0f;
        for (int c = 0; c < 3; ++c) G.ls[c][i] = 0.0f;
        for (int c = 0; c < 4; ++c) G.quat[c][i] = 0.0f;
        G.ol[i] = 0.0f;
        for (int c = 0; c < 3 * K; ++c) G.sh[(size_t)c * P.n + i] = 0.0f;
        return;
    }
    Geo g;
    geometry(P, i, cam, g);
    const float gu = gg[0], gv = gg[1], gA = gg[2], gB = gg[3], gC = gg[4], gop = gg[5];
    // conic = inv(S2): dL/dS2 = -Q Gq Q, Gq = [[gA, gB/2], [gB/2, gC]]
    const float hB = 0.5f * gB;
    const float P00 = g.A * gA + g.B * hB, P01 = g.A * hB + g.B * gC;
    const float P10 = g.B * gA + g.C * hB, P11 = g.B * hB + g.C * gC;
    const float G00 = -(P00 * g.A + P01 * g.B);
    const float G01 = -(P00 * g.B + P01 * g.C);
    const float G11 = -(P10 * g.B + P11 * g.C);
    // dL/dcov3 = T^T G2 T ; dL/dT = 2 G2 T cov3
    float G3[9];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k)
            G3[3 * r + k] = G00 * g.T0[r] * g.T0[k] + G01 * (g.T0[r] * g.T1[k] + g.T1[r] * g.T0[k]) +
                            G11 * g.T1[r] * g.T1[k];
    float TC0[3], TC1[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        TC0[k] = g.T0[0] * s3(g.S, 0, k) + g.T0[1] * s3(g.S, 1, k) + g.T0[2] * s3(g.S, 2, k);
        TC1[k] = g.T1[0] * s3(g.S, 0, k) + g.T1[1] * s3(g.S, 1, k) + g.T1[2] * s3(g.S, 2, k);
    }
    float dT0[3], dT1[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        dT0[k] = 2.0f * (G00 * TC0[k] + G01 * TC1[k]);
        dT1[k] = 2.0f * (G01 * TC0[k] + G11 * TC1[k]);
    }
    const float* R = cam.r;
    const float dj00 = dT0[0] * R[0] + dT0[1] * R[1] + dT0[2] * R[2];
    const float dj02 = dT0[0] * R[6] + dT0[1] * R[7] + dT0[2] * R[8];
    const float dj11 = dT1[0] * R[3] + dT1[1] * R[4] + dT1[2] * R[5];
    const float dj12 = dT1[0] * R[6] + dT1[1] * R[7] + dT1[2] * R[8];
    const float iz = g.iz, iz2 = iz * iz, fx = cam.fx, fy = cam.fy;
    float gx = gu * fx * iz - dj02 * fx * iz2;
    float gy = gv * fy * iz - dj12 * fy * iz2;
    float gz = -(gu * fx * g.x + gv * fy * g.y + dj00 * fx + dj11 * fy) * iz2 +
               2.0f * (dj02 * fx * g.x + dj12 * fy * g.y) * iz2 * iz;
    if (!g.valid) gx = gy = gz = 0.0f;
    float gm[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) gm[k] = R[k] * gx + R[3 + k] * gy + R[6 + k] * gz;
    // cov3 = M M^T, M = Rq diag(s): dM = 2 G3 M
    float M[9];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) M[3 * r + k] = g.Rq[3 * r + k] * g.s[k];
    float gR[9], gls[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) gls[k] = 0.0f;
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const float dM = 2.0f * (G3[3 * r] * M[k] + G3[3 * r + 1] * M[3 + k] +
                                     G3[3 * r + 2] * M[6 + k]);
            gls[k] += dM * g.Rq[3 * r + k];
            gR[3 * r + k] = dM * g.s[k];
        }
    float gq[4];
    {
        const float w = g.qn[0], x = g.qn[1], y = g.qn[2], z = g.qn[3];
        const float gw = 2.0f * (-z * gR[1] + y * gR[2] + z * gR[3] - x * gR[5] - y * gR[6] + x * gR[7]);
        const float gxq = 2.0f * (y * gR[1] + z * gR[2] + y * gR[3] - 2.0f * x * gR[4] - w * gR[5] +
                                  z * gR[6] + w * gR[7] - 2.0f * x * gR[8]);
        const float gyq = 2.0f * (-2.0f * y * gR[0] + x * gR[1] + w * gR[2] + x * gR[3] + z * gR[5] -
                                  w * gR[6] + z * gR[7] - 2.0f * y * gR[8]);
        const float gzq = 2.0f * (-2.0f * z * gR[0] - w * gR[1] + x * gR[2] + w * gR[3] -
                                  2.0f * z * gR[4] + y * gR[5] + x * gR[6] + y * gR[7]);
        const float dot = w * gw + x * gxq + y * gyq + z * gzq;
        gq[0] = (gw - w * dot) * g.qinv;
        gq[1] = (gxq - x * dot) * g.qinv;
        gq[2] = (gyq - y * dot) * g.qinv;
        gq[3] = (gzq - z * dot) * g.qinv;
    }
    if (!g.valid) {
        gq[0] = gq[1] = gq[2] = gq[3] = 0.0f;
        gls[0] = gls[1] = gls[2] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) gls[k] *= g.s[k];
    const float op = sigmoidf(P.ol[i]);
    const float gol = gop * op * (1.0f - op);
    // colour = max(SH(d) + 0.5, 0)
    float raw[3], dir[3], dn;
    colour<DEG>(P, i, cam, raw, dir, dn);
    float gcol[3];
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) gcol[ch] = raw[ch] >= 0.0f ? gg[6 + ch] : 0.0f;
    float b[16], db[16][3];
    sh_basis<DEG, true>(dir[0], dir[1], dir[2], b, db);
    float gd[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < K; ++k) {
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
            G.sh[(size_t)(3 * k + ch) * P.n + i] = b[k] * gcol[ch];
            if (K > 1) {
                const float c = P.sh[(size_t)(3 * k + ch) * P.n + i] * gcol[ch];
                gd[0] += c * db[k][0];
                gd[1] += c * db[k][1];
                gd[2] += c * db[k][2];
            }
        }
    }
    if (K > 1) {
        const float dd = dir[0] * gd[0] + dir[1] * gd[1] + dir[2] * gd[2];
#pragma unroll
        for (int k = 0; k < 3; ++k) gm[k] += (gd[k] - dir[k] * dd) / dn;
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        G.mean[k][i] = gm[k];
        G.ls[k][i] = gls[k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) G.quat[k][i] = gq[k];
    G.ol[i] = gol;
}

// Sparse Adam (train_oracle.py:434-470): rows with visible[i] set; every plane
// of the parameter block, fp32 arithmetic, bias correction folded into the
// per-plane step sizes and sqrt(1 - beta2^t) computed by the host. Moments
// stored as MOM: float, or bf16 bits (uint16_t) read exactly into fp32, updated
// in fp32, the update taken from the fp32 values, stored rounded to nearest
// even (train_oracle.py:445-470 with moment_dtype bfloat16,
// t2_param_backward.py:195-224): half the moments' bytes.
template <typename MOM>
__device__ __forceinline__ float mom_load(const MOM* a, size_t k);
template <>
__device__ __forceinline__ float mom_load<float>(const float* a, size_t k) { return a[k]; }
template <>
__device__ __forceinline__ float mom_load<uint16_t>(const uint16_t* a, size_t k) {
    return bf16_to_f32(a[k]);
}
__device__ __forceinline__ void mom_store(float* a, size_t k, float x) { a[k] = x; }
__device__ __forceinline__ void mom_store(uint16_t* a, size_t k, float x) {
    a[k] = f32_to_bf16_rne(x);
}

template <typename MOM>
__global__ __launch_bounds__(256) void k_sparse_adam(float* __restrict__ p, MOM* __restrict__ m,
                                                     MOM* __restrict__ v,
                                                     const float* __restrict__ g,
                                                     const uint8_t* __restrict__ visible,
                                                     int64_t n, int planes, AdamParams ap) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n || !visible[i]) return;
    for (int j = 0; j < planes; ++j) {
        const size_t k = (size_t)j * n + i;
        const float gj = g[k];
        const float m1 = ap.beta1 * mom_load(m, k) + ap.one_minus_beta1 * gj;
        const float v1 = ap.beta2 * mom_load(v, k) + ap.one_minus_beta2 * gj * gj;
        const float den = sqrtf(v1) / ap.sqrt_bc2 + ap.eps;
        p[k] = p[k] - ap.step[j] * (m1 / den);
        mom_store(m, k, m1);
        mom_store(v, k, v1);
    }
}

}  // namespace

hipError_t launch_train_project(const TrainParamsDev& P, const TrainCam& cam, Compact out,
                                float4* trec, uint32_t* cidx, uint8_t* visible,
                                uint64_t* lb_state, uint32_t* ticket, uint32_t* count_out,
                                uint32_t* part_hist, const TrainDebug& dbg, hipStream_t st) {
    if (P.n <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((P.n + kTPart - 1) / kTPart);
#define GS_TP(D)                                                                            \
    k_train_project<D><<<grid, kTThreads, 0, st>>>(P, cam, out, trec, cidx, visible, lb_state, \
                                                   ticket, count_out, part_hist, dbg)
    switch (P.sh_degree) {
        case 0: GS_TP(0); break;
        case 1: GS_TP(1); break;
        case 2: GS_TP(2); break;
        case 3: GS_TP(3); break;
        default: return hipErrorInvalidValue;
    }
#undef GS_TP
    return hipGetLastError();
}

hipError_t launch_train_fwd(const float4* trec, const uint32_t* sid, const uint32_t* ranges,
                            const TrainFwdParams& fp, hipStream_t st) {
    const int tiles = fp.tiles_x * fp.tiles_y;
    if (tiles <= 0) return hipSuccess;
    k_train_fwd<<<tiles, 256, 0, st>>>(trec, sid, ranges, fp);
    return hipGetLastError();
}

hipError_t launch_ssim(const SsimParams& sp, hipStream_t st) {
    if (sp.width <= 0 || sp.height <= 0) return hipSuccess;
    const unsigned tiles = (unsigned)(((sp.width + kSsimT - 1) / kSsimT) *
                                      ((sp.height + kSsimT - 1) / kSsimT));
    k_ssim_fwd<<<tiles, 256, 0, st>>>(sp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_ssim_bwd<<<tiles, 256, 0, st>>>(sp);
    return hipGetLastError();
}

hipError_t launch_l1(const float* image, const float* target, int64_t count, float scale,
                     float* dimage, double* l1_sum, hipStream_t st) {
    if (count <= 0) return hipSuccess;
    k_l1<<<(unsigned)((count + 255) / 256), 256, 0, st>>>(image, target, count, scale, dimage,
                                                          l1_sum);
    return hipGetLastError();
}

hipError_t launch_train_bwd(const float4* trec, const uint32_t* sid, const uint32_t* ranges,
                            const TrainBwdParams& bp, hipStream_t st) {
    const int tiles = bp.tiles_x * bp.tiles_y;
    if (tiles <= 0) return hipSuccess;
    k_train_bwd<<<tiles, 256, 0, st>>>(trec, sid, ranges, bp);
    return hipGetLastError();
}

hipError_t launch_train_param_grads(const TrainParamsDev& P, const TrainCam& cam,
                                    const uint32_t* cidx, const float* grad2d,
                                    const TrainParamsDev& G, hipStream_t st) {
    if (P.n <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((P.n + 255) / 256);
    switch (P.sh_degree) {
        case 0: k_train_param_grads<0><<<grid, 256, 0, st>>>(P, cam, cidx, grad2d, G); break;
        case 1: k_train_param_grads<1><<<grid, 256, 0, st>>>(P, cam, cidx, grad2d, G); break;
        case 2: k_train_param_grads<2><<<grid, 256, 0, st>>>(P, cam, cidx, grad2d, G); break;
        case 3: k_train_param_grads<3><<<grid, 256, 0, st>>>(P, cam, cidx, grad2d, G); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_sparse_adam(float* p, void* m, void* v, const float* g,
                              const uint8_t* visible, int64_t n, int planes, const AdamParams& ap,
                              bool bf16_moments, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (planes > kMaxTrainPlanes) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (bf16_moments)
        k_sparse_adam<uint16_t><<<grid, 256, 0, st>>>(p, static_cast<uint16_t*>(m),
                                                      static_cast<uint16_t*>(v), g, visible, n,
                                                      planes, ap);
    else
        k_sparse_adam<float><<<grid, 256, 0, st>>>(p, static_cast<float*>(m),
                                                   static_cast<float*>(v), g, visible, n, planes,
                                                   ap);
    return hipGetLastError();
}

}  // namespace gs
