/*
 * gs_oracle.c - CPU oracle of the Gaussian-splat forward pipeline.
 *
 * TEST INFRASTRUCTURE ONLY (see gs_oracle.h). Single-threaded plain C,
 * compiled with -ffp-contract=off. Each function names the reference lines it
 * restates; operation order inside every float expression follows the
 * reference so that results agree bit for bit.
 */
#include "gs_oracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* std::min / std::max / std::clamp semantics (first-operand tie rules). */
static inline float smin(float a, float b) { return (b < a) ? b : a; }
static inline float smax(float a, float b) { return (a < b) ? b : a; }
static inline int imin(int a, int b) { return (b < a) ? b : a; }
static inline int imax(int a, int b) { return (a < b) ? b : a; }
static inline float sclamp(float v, float lo, float hi) {
    return (v < lo) ? lo : ((hi < v) ? hi : v);
}

/* ---------------------------------------------------------------- cov3d --
 * src/gsplat_cpu/types.h:68-97 (quat_to_rotation_matrix, build_covariance_3d)
 * and project.cpp:190-202 (compute_cov3d_batch). Quaternion wxyz, used as
 * given (not normalised). */
void orc_cov3d(const float* scales, const float* quats, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        const float q0 = quats[i * 4 + 0], q1 = quats[i * 4 + 1];
        const float q2 = quats[i * 4 + 2], q3 = quats[i * 4 + 3];
        float r[9];
        r[0] = 1.0f - 2.0f * (q2 * q2 + q3 * q3);
        r[1] = 2.0f * (q1 * q2 - q0 * q3);
        r[2] = 2.0f * (q1 * q3 + q0 * q2);
        r[3] = 2.0f * (q1 * q2 + q0 * q3);
        r[4] = 1.0f - 2.0f * (q1 * q1 + q3 * q3);
        r[5] = 2.0f * (q2 * q3 - q0 * q1);
        r[6] = 2.0f * (q1 * q3 - q0 * q2);
        r[7] = 2.0f * (q2 * q3 + q0 * q1);
        r[8] = 1.0f - 2.0f * (q1 * q1 + q2 * q2);
        for (int col = 0; col < 3; ++col) {
            const float s = scales[i * 3 + col];
            for (int row = 0; row < 3; ++row) r[row * 3 + col] *= s;
        }
        /* (RS)(RS)^T via the reference's generic mat3_mul (types.h:50-58). */
        for (int a = 0; a < 3; ++a)
            for (int b = 0; b < 3; ++b)
                out[i * 9 + a * 3 + b] = r[a * 3 + 0] * r[b * 3 + 0] +
                                         r[a * 3 + 1] * r[b * 3 + 1] +
                                         r[a * 3 + 2] * r[b * 3 + 2];
    }
}

/* ------------------------------------------------------------------- SH --
 * 3DGS real SH basis, gsplat/train_oracle.py:46-52 (constants), :99-122
 * (sh_eval) and :163-173 (dir = normalize(mean - cam_centre),
 * cam_centre = -R^T t, rgb = SH + 0.5, clamp). fp32, left-to-right. */
#define SH_C0 0.28209479177387814f
#define SH_C1 0.4886025119029199f
static const float SH_C2[5] = {1.0925484305920792f, -1.0925484305920792f,
                               0.31539156525252005f, -1.0925484305920792f,
                               0.5462742152960396f};
static const float SH_C3[7] = {-0.5900435899266435f, 2.890611442640554f,
                               -0.4570457994644658f, 0.3731763325901154f,
                               -0.4570457994644658f, 1.445305721320277f,
                               -0.5900435899266435f};

void orc_sh_rgb(const float* means, const float* sh, int64_t n, int degree,
                const float* w2c, int clamp_hi, float* rgb) {
    const int K = (degree + 1) * (degree + 1);
    const float t0 = w2c[3], t1 = w2c[7], t2 = w2c[11];
    const float ccx = -(w2c[0] * t0 + w2c[4] * t1 + w2c[8] * t2);
    const float ccy = -(w2c[1] * t0 + w2c[5] * t1 + w2c[9] * t2);
    const float ccz = -(w2c[2] * t0 + w2c[6] * t1 + w2c[10] * t2);
    for (int64_t i = 0; i < n; ++i) {
        const float dx = means[i * 3 + 0] - ccx;
        const float dy = means[i * 3 + 1] - ccy;
        const float dz = means[i * 3 + 2] - ccz;
        const float nrm = sqrtf(dx * dx + dy * dy + dz * dz);
        const float x = dx / nrm, y = dy / nrm, z = dz / nrm;
        const float xx = x * x, yy = y * y, zz = z * z;
        const float xy = x * y, yz = y * z, xz = x * z;
        const float* s = sh + i * K * 3;
        for (int c = 0; c < 3; ++c) {
            float o = SH_C0 * s[0 * 3 + c];
            if (degree >= 1) {
                o = o - SH_C1 * y * s[1 * 3 + c] + SH_C1 * z * s[2 * 3 + c] -
                    SH_C1 * x * s[3 * 3 + c];
            }
            if (degree >= 2) {
                o = o + SH_C2[0] * xy * s[4 * 3 + c] + SH_C2[1] * yz * s[5 * 3 + c] +
                    SH_C2[2] * (2.0f * zz - xx - yy) * s[6 * 3 + c] +
                    SH_C2[3] * xz * s[7 * 3 + c] + SH_C2[4] * (xx - yy) * s[8 * 3 + c];
            }
            if (degree >= 3) {
                o = o + SH_C3[0] * y * (3.0f * xx - yy) * s[9 * 3 + c] +
                    SH_C3[1] * xy * z * s[10 * 3 + c] +
                    SH_C3[2] * y * (4.0f * zz - xx - yy) * s[11 * 3 + c] +
                    SH_C3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy) * s[12 * 3 + c] +
                    SH_C3[4] * x * (4.0f * zz - xx - yy) * s[13 * 3 + c] +
                    SH_C3[5] * z * (xx - yy) * s[14 * 3 + c] +
                    SH_C3[6] * x * (xx - 3.0f * yy) * s[15 * 3 + c];
            }
            o = o + 0.5f;
            o = (o < 0.0f) ? 0.0f : o;
            if (clamp_hi) o = (o > 1.0f) ? 1.0f : o;
            rgb[i * 3 + c] = o;
        }
    }
}

/* -------------------------------------------------------------- project --
 * src/gsplat_cpu/project.cpp:484-798 (project_full_fused) with
 * types.h:141-176 (opacity_aware_k, isoellipse_aabb_half_extents,
 * apply_k_cap). Per-Gaussian body, then a stable source-order compaction
 * of the valid Gaussians (project.cpp:710-797). Returns M. */
int64_t orc_project(const float* means, const float* cov3d, const float* e,
                    const float* intr, const float* colors, const float* opac,
                    float min_opacity, int64_t n, int height, int width,
                    int max_radius_param, float contrib_floor, float k_cap,
                    int use_isoellipse,
                    uint8_t* valid_mask, float* means2d, float* covs2d,
                    float* depths, float* radii, float* colors_out,
                    float* opac_out) {
    const float r00 = e[0], r01 = e[1], r02 = e[2];
    const float r10 = e[4], r11 = e[5], r12 = e[6];
    const float r20 = e[8], r21 = e[9], r22 = e[10];
    const float t0 = e[3], t1 = e[7], t2 = e[11];
    const float fx = intr[0], fy = intr[4], cx = intr[2], cy = intr[5];
    const float k_near = 0.2f;
    const int max_radius = (max_radius_param < 0) ? INT_MAX
                           : (max_radius_param > 0 ? max_radius_param
                                                   : imin(height, width) / 2);
    int64_t m = 0;
    for (int64_t i = 0; i < n; ++i) {
        const float mx = means[i * 3 + 0], my = means[i * 3 + 1], mz = means[i * 3 + 2];
        /* R @ mean first, then + t (project.cpp:539-545, 559-561). */
        const float rmx = mx * r00 + my * r01 + mz * r02;
        const float rmy = mx * r10 + my * r11 + mz * r12;
        const float rmz = mx * r20 + my * r21 + mz * r22;
        const float tx = rmx + t0, ty = rmy + t1, tz = rmz + t2;
        valid_mask[i] = 0;
        if (tz <= k_near || (opac != NULL && opac[i] < min_opacity)) continue;

        const float inv_tz = 1.0f / tz;
        const float mean_x = fx * tx * inv_tz + cx;
        const float mean_y = fy * ty * inv_tz + cy;
        const float tz2 = tz * tz;
        const float j00 = fx / tz, j02 = -fx * tx / tz2;
        const float j11 = fy / tz, j12 = -fy * ty / tz2;

        const float c00 = cov3d[i * 9 + 0], c01 = cov3d[i * 9 + 1], c02 = cov3d[i * 9 + 2];
        const float c11 = cov3d[i * 9 + 4], c12 = cov3d[i * 9 + 5], c22 = cov3d[i * 9 + 8];
        /* v_j = cov3d @ R(j,:)^T, cov_cam(i,j) = R(i,:) . v_j (project.cpp:618-640) */
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
        /* cov2d = J cov_cam J^T + 0.3 I (project.cpp:645-657) */
        const float m00 = j00 * cc00 + j02 * cc02;
        const float m01 = j00 * cc01 + j02 * cc12;
        const float m02 = j00 * cc02 + j02 * cc22;
        const float m11 = j11 * cc11 + j12 * cc12;
        const float m12 = j11 * cc12 + j12 * cc22;
        const float a = m00 * j00 + m02 * j02 + 0.3f;
        const float b = m01 * j11 + m02 * j12;
        const float c = m11 * j11 + m12 * j12 + 0.3f;

        float k = 3.0f;
        if (opac != NULL) {
            const float arg = smax(opac[i] / contrib_floor, 1.0f);
            k = sqrtf(2.0f * logf(arg));
        }
        if (k_cap > 0.0f) k = smin(k, k_cap);
        float rx, ry;
        if (use_isoellipse) {
            const float trace = a + c;
            const float disc = sqrtf(smax(trace * trace - 4.0f * (a * c - b * b), 0.0f));
            const float l1 = 0.5f * (trace + disc);
            const float l2 = 0.5f * (trace - disc);
            const float theta = 0.5f * atan2f(2.0f * b, a - c);
            const float ct = cosf(theta), st = sinf(theta);
            const float cos2 = ct * ct, sin2 = st * st;
            rx = ceilf(k * sqrtf(smax(l1 * cos2 + l2 * sin2, 0.0f)));
            ry = ceilf(k * sqrtf(smax(l1 * sin2 + l2 * cos2, 0.0f)));
        } else {
            rx = ceilf(k * sqrtf(smax(a, 0.0f)));
            ry = ceilf(k * sqrtf(smax(c, 0.0f)));
        }
        const int valid = (mean_x + rx > 0.0f) && (mean_x - rx < (float)width) &&
                          (mean_y + ry > 0.0f) && (mean_y - ry < (float)height) &&
                          (rx > 0.0f) && (ry > 0.0f) &&
                          (rx <= (float)max_radius) && (ry <= (float)max_radius);
        if (!valid) continue;
        valid_mask[i] = 1;
        means2d[m * 2 + 0] = mean_x;
        means2d[m * 2 + 1] = mean_y;
        covs2d[m * 4 + 0] = a;
        covs2d[m * 4 + 1] = b;
        covs2d[m * 4 + 2] = b;
        covs2d[m * 4 + 3] = c;
        depths[m] = tz;
        radii[m * 2 + 0] = rx;
        radii[m * 2 + 1] = ry;
        if (colors_out != NULL && colors != NULL) {
            colors_out[m * 3 + 0] = colors[i * 3 + 0];
            colors_out[m * 3 + 1] = colors[i * 3 + 1];
            colors_out[m * 3 + 2] = colors[i * 3 + 2];
        }
        if (opac_out != NULL && opac != NULL) opac_out[m] = opac[i];
        ++m;
    }
    return m;
}

/* ---------------------------------------------------------- tile_assign --
 * src/gsplat_cpu/tile_assign.cpp:60-102 (rect: float divide, truncate toward
 * zero, clamp), :107-149 (Gaussian-major, row-major pair order), :151-290
 * (per-pair constrained-minimum Mahalanobis cull), :298-349 (stable
 * compaction). */
static void tile_rect(const float* means2d, const float* radii, int64_t g,
                      int tiles_x, int tiles_y, int tile_size, int* r4) {
    const float px = means2d[g * 2 + 0], py = means2d[g * 2 + 1];
    const float rx = radii[g * 2 + 0], ry = radii[g * 2 + 1];
    const float ts = (float)tile_size;
    r4[0] = imax(0, imin((int)((px - rx) / ts), tiles_x - 1));
    r4[1] = imax(0, imin((int)((px + rx) / ts), tiles_x - 1));
    r4[2] = imax(0, imin((int)((py - ry) / ts), tiles_y - 1));
    r4[3] = imax(0, imin((int)((py + ry) / ts), tiles_y - 1));
}

int64_t orc_tile_count(const float* means2d, const float* radii, int64_t m,
                       int height, int width, int tile_size) {
    const int tiles_x = (width + tile_size - 1) / tile_size;
    const int tiles_y = (height + tile_size - 1) / tile_size;
    int64_t total = 0;
    for (int64_t g = 0; g < m; ++g) {
        int r[4];
        tile_rect(means2d, radii, g, tiles_x, tiles_y, tile_size, r);
        total += (int64_t)(r[1] - r[0] + 1) * (int64_t)(r[3] - r[2] + 1);
    }
    return total;
}

int64_t orc_tile_assign(const float* means2d, const float* radii, int64_t m,
                        int height, int width, int tile_size,
                        const float* covs2d, const float* opac, float floor_,
                        int64_t* gids, int64_t* tids) {
    const int tiles_x = (width + tile_size - 1) / tile_size;
    const int tiles_y = (height + tile_size - 1) / tile_size;
    const int cull = (covs2d != NULL && opac != NULL);
    int64_t out = 0;
    for (int64_t g = 0; g < m; ++g) {
        int r[4];
        tile_rect(means2d, radii, g, tiles_x, tiles_y, tile_size, r);
        int above = 1;
        float m2thr = 0.0f, a = 0, b = 0, c = 0, det = 0, px = 0, py = 0;
        if (cull) {
            const float op = opac[g];
            if (op > floor_) {
                m2thr = -2.0f * logf(floor_ / op);
            } else {
                above = 0;
            }
            a = covs2d[g * 4 + 0];
            b = covs2d[g * 4 + 1];
            c = covs2d[g * 4 + 3];
            det = smax(a * c - b * b, 1e-6f);
            px = means2d[g * 2 + 0];
            py = means2d[g * 2 + 1];
        }
        for (int ty = r[2]; ty <= r[3]; ++ty) {
            for (int tx = r[0]; tx <= r[1]; ++tx) {
                const int64_t tile_id = (int64_t)ty * tiles_x + tx;
                int keep = 1;
                if (cull) {
                    if (!above) {
                        keep = 0;
                    } else {
                        const float tx_tile = (float)(tile_id % tiles_x) * (float)tile_size;
                        const float ty_tile = (float)(tile_id / tiles_x) * (float)tile_size;
                        const float u_lo = tx_tile - px;
                        const float u_hi = u_lo + (float)tile_size;
                        const float v_lo = ty_tile - py;
                        const float v_hi = v_lo + (float)tile_size;
                        const int x_in = (u_lo <= 0.0f) && (0.0f <= u_hi);
                        const int y_in = (v_lo <= 0.0f) && (0.0f <= v_hi);
                        const float scaled = det * m2thr;
                        if (!(x_in && y_in)) {
                            float m2_v = INFINITY, m2_h = INFINITY;
                            if (!x_in) {
                                const float uf = (u_lo > 0.0f) ? u_lo : u_hi;
                                const float a_safe = smax(a, 1e-12f);
                                float vs = (b * uf) / a_safe;
                                vs = smax(v_lo, smin(vs, v_hi));
                                m2_v = c * uf * uf - 2.0f * b * uf * vs + a * vs * vs;
                            }
                            if (!y_in) {
                                const float vf = (v_lo > 0.0f) ? v_lo : v_hi;
                                const float c_safe = smax(c, 1e-12f);
                                float us = (b * vf) / c_safe;
                                us = smax(u_lo, smin(us, u_hi));
                                m2_h = c * us * us - 2.0f * b * us * vf + a * vf * vf;
                            }
                            const float num = smin(m2_v, m2_h);
                            keep = (num <= scaled);
                        }
                    }
                }
                if (keep) {
                    gids[out] = g;
                    tids[out] = tile_id;
                    ++out;
                }
            }
        }
    }
    return out;
}

/* ---------------------------------------------------------- sort_and_bin --
 * src/gsplat_cpu/sort.cpp:89-263: stable bucket by tile (input order kept),
 * tile_ranges [start,end) with (0,0) for empty tiles, then a stable LSD
 * radix on the fp32 depth bits inside each tile (sort.cpp:24-85). */
void orc_sort_and_bin(const int64_t* gids, const int64_t* tids, const float* depths,
                      int64_t p, int tiles_x, int tiles_y,
                      int64_t* sorted_ids, int64_t* tile_ranges) {
    const int64_t T = (int64_t)tiles_x * tiles_y;
    memset(tile_ranges, 0, (size_t)T * 2 * sizeof(int64_t));
    if (p == 0) return;
    int64_t* start = (int64_t*)calloc((size_t)T + 1, sizeof(int64_t));
    for (int64_t i = 0; i < p; ++i) start[tids[i] + 1]++;
    for (int64_t t = 0; t < T; ++t) {
        const int64_t cnt = start[t + 1];
        start[t + 1] = start[t] + cnt;
        if (cnt > 0) {
            tile_ranges[t * 2 + 0] = start[t];
            tile_ranges[t * 2 + 1] = start[t + 1];
        }
    }
    uint32_t* keys = (uint32_t*)malloc((size_t)p * sizeof(uint32_t));
    uint32_t* tk = (uint32_t*)malloc((size_t)p * sizeof(uint32_t));
    int64_t* tv = (int64_t*)malloc((size_t)p * sizeof(int64_t));
    int64_t* cur = (int64_t*)malloc((size_t)T * sizeof(int64_t));
    memcpy(cur, start, (size_t)T * sizeof(int64_t));
    for (int64_t i = 0; i < p; ++i) {
        const int64_t pos = cur[tids[i]]++;
        uint32_t db;
        memcpy(&db, &depths[gids[i]], 4);
        keys[pos] = db;
        sorted_ids[pos] = gids[i];
    }
    for (int64_t t = 0; t < T; ++t) {
        const int64_t lo = start[t], n = start[t + 1] - lo;
        if (n <= 1) continue;
        uint32_t* ik = keys + lo;
        int64_t* iv = sorted_ids + lo;
        uint32_t* ok = tk;
        int64_t* ov = tv;
        for (int shift = 0; shift < 32; shift += 8) {
            int64_t cnt[257] = {0};
            for (int64_t i = 0; i < n; ++i) cnt[((ik[i] >> shift) & 0xFFu) + 1]++;
            for (int d = 0; d < 256; ++d) cnt[d + 1] += cnt[d];
            for (int64_t i = 0; i < n; ++i) {
                const int64_t pos = cnt[(ik[i] >> shift) & 0xFFu]++;
                ok[pos] = ik[i];
                ov[pos] = iv[i];
            }
            uint32_t* sk = ik; ik = ok; ok = sk;
            int64_t* sv = iv; iv = ov; ov = sv;
        }
        /* four passes: data is back in keys/sorted_ids */
    }
    free(keys); free(tk); free(tv); free(cur); free(start);
}

/* ------------------------------------------------------ cull_and_blend --
 * src/gsplat_cpu/cull_and_blend.cpp:316-838 built with the AVX2 blend
 * (GSPLAT_SIMD_AVX2, simd_config.h:11-23): full 8x4 microblocks use the
 * degree-4 exp of simd_exp_avx2.h:12-32, power clamped to [-30, 0],
 * T -= alpha*T and an early-out test every 4 kept Gaussians
 * (cull_and_blend.cpp:578-616); partial (image-edge) microblocks use the
 * scalar rule (:620-669). */
float orc_exp4(float x) {
    const float LOG2E = 1.44269504088896f;
    const float LN2 = 0.69314718055994530942f;
    const float y = x * LOG2E;
    const float fn = nearbyintf(y); /* round-half-even, default mode */
    const int n = (int)fn;
    const float r = fmaf(-fn, LN2, x);
    const float r2 = r * r;
    const float p0 = fmaf(r, 1.0f, 1.0f);
    float p1 = fmaf(r, 0.166666666667f, 0.5f);
    p1 = fmaf(r2, 0.041666666667f, p1);
    const float p = fmaf(r2, p1, p0);
    const uint32_t bits = (uint32_t)(n + 127) << 23;
    float two_n;
    memcpy(&two_n, &bits, 4);
    return two_n * p;
}

typedef struct {
    float mx, my, ci_a, ci_b, ci_c, log_thresh, x_half, y_half, opacity, cr, cg, cb;
} CullRec;

void orc_cull_and_blend(const float* means2d, const float* covs2d,
                        const float* colors, const float* opac,
                        const int64_t* sorted_ids, const int64_t* tile_ranges,
                        int64_t m, int64_t p, int tiles_x, int tiles_y,
                        int tile_size, int height, int width,
                        float mbf, int cull_disabled, float thr, float* image,
                        int64_t* stats3) {
    memset(image, 0, (size_t)height * (size_t)width * 3 * sizeof(float));
    CullRec* rec = (CullRec*)malloc((size_t)(m > 0 ? m : 1) * sizeof(CullRec));
    /* GaussianCullRec prelude, cull_and_blend.cpp:723-777 */
    for (int64_t i = 0; i < m; ++i) {
        const float a = covs2d[i * 4 + 0], b = covs2d[i * 4 + 1], c = covs2d[i * 4 + 3];
        const float det = smax(a * c - b * b, 1e-6f);
        CullRec* r = &rec[i];
        r->mx = means2d[i * 2 + 0];
        r->my = means2d[i * 2 + 1];
        r->ci_a = c / det;
        r->ci_b = -b / det;
        r->ci_c = a / det;
        r->opacity = opac[i];
        r->cr = colors[i * 3 + 0];
        r->cg = colors[i * 3 + 1];
        r->cb = colors[i * 3 + 2];
        if (r->opacity <= mbf) {
            r->log_thresh = 0.0f;
            r->x_half = 0.0f;
            r->y_half = 0.0f;
        } else {
            const float lt = logf(mbf / r->opacity);
            r->log_thresh = lt;
            const float rd = sqrtf(-2.0f * lt);
            r->x_half = rd * sqrtf(smax(a, 0.0f));
            r->y_half = rd * sqrtf(smax(c, 0.0f));
        }
    }
    int64_t dropped = 0, kept_total = 0;
    const int64_t T = (int64_t)tiles_x * tiles_y;
    int64_t cap = 0;
    uint32_t* kept = NULL;
    for (int64_t tile = 0; tile < T; ++tile) {
        const int64_t start = tile_ranges[tile * 2 + 0], end = tile_ranges[tile * 2 + 1];
        if (start == end) continue;
        const int ty = (int)(tile / tiles_x), tx = (int)(tile % tiles_x);
        const float tx_tile = (float)(tx * tile_size);
        const float ty_tile = (float)(ty * tile_size);
        const int py_tile = ty * tile_size, px_tile = tx * tile_size;
        const int py_end_tile = imin(py_tile + tile_size, height);
        const int px_end_tile = imin(px_tile + tile_size, width);
        const int64_t L = end - start;
        if (32 * L > cap) {
            cap = 32 * L;
            kept = (uint32_t*)realloc(kept, (size_t)cap * sizeof(uint32_t));
        }
        int64_t cnt[32] = {0};
        for (int64_t l = 0; l < L; ++l) {
            const int64_t g = sorted_ids[start + l];
            const CullRec* r = &rec[g];
            const float lt = r->log_thresh;
            if (lt >= 0.0f) { ++dropped; continue; }
            const float bx0 = r->mx - r->x_half, bx1 = r->mx + r->x_half;
            const float by0 = r->my - r->y_half, by1 = r->my + r->y_half;
            const int mx_lo = imax(0, (int)floorf((bx0 - tx_tile) / 8.0f));
            const int mx_hi = imin(3, (int)floorf((bx1 - tx_tile) / 8.0f));
            const int my_lo = imax(0, (int)floorf((by0 - ty_tile) / 4.0f));
            const int my_hi = imin(7, (int)floorf((by1 - ty_tile) / 4.0f));
            if (mx_lo > mx_hi || my_lo > my_hi) { ++dropped; continue; }
            const float thresh_m2 = -2.0f * lt;
            const float ca_safe = smax(r->ci_a, 1e-12f);
            const float cc_safe = smax(r->ci_c, 1e-12f);
            int any = 0;
            for (int my = my_lo; my <= my_hi; ++my) {
                const float mb_oy = ty_tile + (float)(my * 4);
                const float v_lo = mb_oy - r->my;
                const float v_hi = v_lo + 4.0f;
                const int y_in = (v_lo <= 0.0f) && (0.0f <= v_hi);
                const float v_fix = (v_lo > 0.0f) ? v_lo : v_hi;
                for (int mx = mx_lo; mx <= mx_hi; ++mx) {
                    const float mb_ox = tx_tile + (float)(mx * 8);
                    const float u_lo = mb_ox - r->mx;
                    const float u_hi = u_lo + 8.0f;
                    const int x_in = (u_lo <= 0.0f) && (0.0f <= u_hi);
                    float m2_min;
                    if (cull_disabled || (x_in && y_in)) {
                        m2_min = 0.0f;
                    } else {
                        float m2_v = INFINITY, m2_h = INFINITY;
                        if (!x_in) {
                            const float uf = (u_lo > 0.0f) ? u_lo : u_hi;
                            float vs = -r->ci_b * uf / cc_safe;
                            vs = sclamp(vs, v_lo, v_hi);
                            m2_v = r->ci_a * uf * uf + 2.0f * r->ci_b * uf * vs +
                                   r->ci_c * vs * vs;
                        }
                        if (!y_in) {
                            float us = -r->ci_b * v_fix / ca_safe;
                            us = sclamp(us, u_lo, u_hi);
                            m2_h = r->ci_a * us * us + 2.0f * r->ci_b * us * v_fix +
                                   r->ci_c * v_fix * v_fix;
                        }
                        m2_min = smin(m2_v, m2_h);
                    }
                    if (m2_min <= thresh_m2) {
                        const int mb = (my << 2) | mx;
                        kept[(int64_t)mb * L + cnt[mb]++] = (uint32_t)g;
                        any = 1;
                        ++kept_total;
                    }
                }
            }
            if (!any) ++dropped;
        }
        for (int mb = 0; mb < 32; ++mb) {
            const int64_t kn = cnt[mb];
            if (kn == 0) continue;
            const uint32_t* kg = kept + (int64_t)mb * L;
            const int py_start = py_tile + (mb >> 2) * 4;
            const int px_start = px_tile + (mb & 3) * 8;
            const int py_end = imin(py_start + 4, py_end_tile);
            const int px_end = imin(px_start + 8, px_end_tile);
            if (py_start >= py_end || px_start >= px_end) continue;
            const int mb_h = py_end - py_start, mb_w = px_end - px_start;
            float Tr[32], ar[32], ag[32], ab[32];
            for (int k = 0; k < 32; ++k) { Tr[k] = 1.0f; ar[k] = ag[k] = ab[k] = 0.0f; }
            if (mb_h == 4 && mb_w == 8) {
                for (int64_t k = 0; k < kn; ++k) {
                    const CullRec* r = &rec[kg[k]];
                    const float A = -0.5f * r->ci_a, B = -r->ci_b, C = -0.5f * r->ci_c;
                    const float px_base = (float)px_start - r->mx;
                    for (int i = 0; i < 4; ++i) {
                        const float py = (float)(py_start + i) + 0.5f;
                        const float dy = py - r->my;
                        const float y_term = C * dy * dy;
                        const float xy_coef = B * dy;
                        for (int j = 0; j < 8; ++j) {
                            const float dx = px_base + ((float)j + 0.5f);
                            const float dx_sq = dx * dx;
                            float pwr = fmaf(xy_coef, dx, y_term);
                            pwr = fmaf(A, dx_sq, pwr);
                            pwr = (pwr < 0.0f) ? pwr : 0.0f;     /* _mm_min_ps */
                            pwr = (pwr > -30.0f) ? pwr : -30.0f; /* _mm_max_ps */
                            const float gw = orc_exp4(pwr);
                            float al = r->opacity * gw;
                            al = (al < 0.99f) ? al : 0.99f;
                            const int ij = i * 8 + j;
                            const float at = al * Tr[ij];
                            ar[ij] = fmaf(at, r->cr, ar[ij]);
                            ag[ij] = fmaf(at, r->cg, ag[ij]);
                            ab[ij] = fmaf(at, r->cb, ab[ij]);
                            Tr[ij] = Tr[ij] - at;
                        }
                    }
                    if (((k + 1) & 3) == 0) {
                        float tm = Tr[0];
                        for (int q = 1; q < 32; ++q) tm = (tm > Tr[q]) ? tm : Tr[q];
                        if (tm < thr) break;
                    }
                }
            } else {
                const int npix = mb_h * mb_w;
                for (int64_t k = 0; k < kn; ++k) {
                    const CullRec* r = &rec[kg[k]];
                    for (int i = 0; i < mb_h; ++i) {
                        const float py = (float)(py_start + i) + 0.5f;
                        for (int j = 0; j < mb_w; ++j) {
                            const float px = (float)(px_start + j) + 0.5f;
                            const float dx = px - r->mx;
                            const float dy = py - r->my;
                            const float power =
                                -0.5f * (r->ci_a * dx * dx + 2.0f * r->ci_b * dx * dy +
                                         r->ci_c * dy * dy);
                            const float gw = expf(smin(power, 0.0f));
                            const float al = smin(r->opacity * gw, 0.99f);
                            const int ij = i * mb_w + j;
                            const float t = Tr[ij];
                            const float at = al * t;
                            ar[ij] += at * r->cr;
                            ag[ij] += at * r->cg;
                            ab[ij] += at * r->cb;
                            Tr[ij] = t * (1.0f - al);
                        }
                    }
                    float tm = 0.0f;
                    for (int q = 0; q < npix; ++q) tm = smax(tm, Tr[q]);
                    if (tm < thr) break;
                }
            }
            for (int i = 0; i < mb_h; ++i) {
                for (int j = 0; j < mb_w; ++j) {
                    const int ij = (mb_h == 4 && mb_w == 8) ? i * 8 + j : i * mb_w + j;
                    const int64_t o = ((int64_t)(py_start + i) * width + (px_start + j)) * 3;
                    image[o + 0] = ar[ij];
                    image[o + 1] = ag[ij];
                    image[o + 2] = ab[ij];
                }
            }
        }
    }
    free(kept);
    free(rec);
    if (stats3 != NULL) {
        stats3[0] = p;
        stats3[1] = dropped;
        stats3[2] = kept_total;
    }
}

/* ------------------------------------------------------ stable u64 sort --
 * Complete specification of the tile/depth key sort (sort.cpp:24-85 is a
 * stable LSD radix; a stable sort by the 64-bit key is the same order):
 * LSD radix, 16-bit digits, passes whose digit is constant are skipped. */
void orc_stable_sort_u64(const uint64_t* keys, const uint32_t* vals, int64_t n,
                         uint64_t* keys_out, uint32_t* vals_out) {
    memcpy(keys_out, keys, (size_t)n * 8);
    memcpy(vals_out, vals, (size_t)n * 4);
    if (n <= 1) return;
    uint64_t* tk = (uint64_t*)malloc((size_t)n * 8);
    uint32_t* tv = (uint32_t*)malloc((size_t)n * 4);
    int64_t* cnt = (int64_t*)malloc(65537 * sizeof(int64_t));
    uint64_t* ik = keys_out; uint32_t* iv = vals_out;
    uint64_t* ok = tk; uint32_t* ov = tv;
    for (int shift = 0; shift < 64; shift += 16) {
        memset(cnt, 0, 65537 * sizeof(int64_t));
        for (int64_t i = 0; i < n; ++i) cnt[((ik[i] >> shift) & 0xFFFFu) + 1]++;
        int single = 0;
        for (int d = 0; d < 65536; ++d) if (cnt[d + 1] == n) single = 1;
        if (single) continue;
        for (int d = 0; d < 65536; ++d) cnt[d + 1] += cnt[d];
        for (int64_t i = 0; i < n; ++i) {
            const int64_t pos = cnt[(ik[i] >> shift) & 0xFFFFu]++;
            ok[pos] = ik[i];
            ov[pos] = iv[i];
        }
        uint64_t* sk = ik; ik = ok; ok = sk;
        uint32_t* sv = iv; iv = ov; ov = sv;
    }
    if (ik != keys_out) {
        memcpy(keys_out, ik, (size_t)n * 8);
        memcpy(vals_out, iv, (size_t)n * 4);
    }
    free(tk); free(tv); free(cnt);
}
