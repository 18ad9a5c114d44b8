/*
 * gs_oracle.h - CPU oracle of the Gaussian-splat forward pipeline.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C, single-threaded restatement of
 * the reference CPU renderer (src/gsplat_cpu, driven by
 * backends/cpu_cpp/pybind_module.cpp:1149-1575 render_full_py). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
 * as the checker. Nothing in the product links or calls it.
 *
 * Every function states the reference lines it follows. All arithmetic is
 * compiled with -ffp-contract=off, like the reference library
 * (src/CMakeLists.txt:90), so the float results are the reference's bit for
 * bit wherever the reference itself is deterministic.
 *
 * Parity status per function (how each one is pinned):
 *   orc_cov3d          closed forms (identity / axis rotations) + oracle/_ref
 *   orc_sh_rgb         reference training fixtures benchmarks/train_oracle/t0_*
 *   orc_project        KATs of tests/unit/test_project.cpp + oracle/_ref
 *   orc_tile_assign    KATs of tests/unit/test_tile_assign.cpp + brute force + oracle/_ref
 *   orc_sort_and_bin   KATs of tests/unit/test_sort.cpp + numpy stable sort + oracle/_ref
 *   orc_cull_and_blend closed forms of tests/unit/test_blend.cpp + oracle/_ref
 *   orc_stable_sort_u64 numpy argsort(kind="stable")
 */
#ifndef GS_ORACLE_H
#define GS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void orc_cov3d(const float* scales, const float* quats, int64_t n, float* cov3d9);

void orc_sh_rgb(const float* means, const float* sh, int64_t n, int degree,
                const float* w2c, int clamp_hi, float* rgb);

int64_t orc_project(const float* means, const float* cov3d9, const float* w2c,
                    const float* intr, const float* colors, const float* opac,
                    float min_opacity, int64_t n, int height, int width,
                    int max_radius_param, float contrib_floor, float k_cap,
                    int use_isoellipse,
                    uint8_t* valid_mask, float* means2d, float* covs2d,
                    float* depths, float* radii, float* colors_out,
                    float* opac_out);

int64_t orc_tile_count(const float* means2d, const float* radii, int64_t m,
                       int height, int width, int tile_size);

int64_t orc_tile_assign(const float* means2d, const float* radii, int64_t m,
                        int height, int width, int tile_size,
                        const float* covs2d, const float* opac, float contrib_floor,
                        int64_t* gids, int64_t* tids);

void orc_sort_and_bin(const int64_t* gids, const int64_t* tids, const float* depths,
                      int64_t p, int tiles_x, int tiles_y,
                      int64_t* sorted_ids, int64_t* tile_ranges);

void orc_cull_and_blend(const float* means2d, const float* covs2d,
                        const float* colors, const float* opac,
                        const int64_t* sorted_ids, const int64_t* tile_ranges,
                        int64_t m, int64_t p, int tiles_x, int tiles_y,
                        int tile_size, int height, int width,
                        float mb_contrib_floor, int cull_disabled,
                        float transmittance_threshold, float* image,
                        int64_t* stats3);

void orc_stable_sort_u64(const uint64_t* keys, const uint32_t* vals, int64_t n,
                         uint64_t* keys_out, uint32_t* vals_out);

float orc_exp4(float x);

#ifdef __cplusplus
}
#endif
#endif
