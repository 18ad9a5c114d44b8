/*
 * gsplat_hip.h - C ABI of the MI355X (gfx950) Gaussian-splat rasterizer.
 *
 * Plain pointers and sizes only; no exceptions cross this boundary. Every
 * entry point returns GS_OK (0) or a negative GS_E* status, with a message in
 * gs_last_error() (thread-local). One context = one GPU + one HIP stream;
 * calls on one context must not overlap (the Python module serialises them
 * with a mutex, like the reference's render_view_mutex,
 * render/host/render.cpp:73-75).
 *
 * Host-pointer entry points copy their inputs to HBM and their outputs back;
 * the *_dev variants take device pointers and never touch host memory.
 */
#ifndef GSPLAT_HIP_H
#define GSPLAT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_OK 0
#define GS_E_INVALID -1   /* bad argument (-> std::invalid_argument / ValueError) */
#define GS_E_DEVICE -2    /* HIP runtime / kernel failure (-> RuntimeError) */
#define GS_E_CAPACITY -3  /* a size limit of this build was exceeded */

#define GS_OUT_U8 0       /* u8 of the bf16 image: uint8(clip(float(bf16(rgb)),0,1)*255),
                           truncation (render/kernels/dataflow/img_pack_u8.h:9-14) */
#define GS_OUT_BF16 1     /* bf16, round to nearest even */
#define GS_OUT_F32 2

typedef struct gs_ctx gs_ctx;

/* Scene description. Host pointers, read during gs_scene_set only.
 * Replaces the per-scene caches of render/host/render.cpp:96-118
 * (cov3d_unique, keyed by pointer, N and scene version). */
typedef struct gs_scene {
    const float* means;     /* (n,3) world positions */
    const float* cov3d;     /* (n,9) row-major 3x3, or (n,6) c00 c01 c02 c11 c12 c22 */
    int cov3d_stride;       /* 9 or 6 */
    const float* opacities; /* (n) activated opacity, or NULL (k = 3, no opacity tests) */
    const float* colors;    /* sh_degree < 0: (n,3) RGB; else (n,(d+1)^2,3) SH coefficients */
    int sh_degree;          /* -1 (RGB) or 0..3 */
    int64_t n;
    uint64_t version;       /* caller's scene version; any change forces a re-upload */
} gs_scene;

/* One view. Mirrors the argument list of render_clean.render_view
 * (render/host/render.cpp:263-273) and _gsplat_cpu.render_full
 * (backends/cpu_cpp/pybind_module.cpp:2071-2091). */
typedef struct gs_view {
    float extrinsics[16];   /* world-to-camera 4x4, row-major, R | t in column 3 */
    float intrinsics[9];    /* 3x3, fx = [0], cx = [2], fy = [4], cy = [5] */
    int image_height, image_width;
    int tile_size;          /* 16 or 32 */
    float min_opacity;
    float contrib_floor;    /* radius k and per-pair tile cull floor */
    float mb_contrib_floor; /* microblock cull floor */
    int cull_disabled;
    float transmittance_threshold;
    int max_radius;         /* 0: min(H,W)/2, > 0: explicit, < 0: unlimited */
    float k_cap;            /* <= 0: uncapped */
    int use_isoellipse;
    int out_format;         /* GS_OUT_* */
    int sh_clamp_hi;        /* SH colour clamp to [0,1] (display) when 1, >= 0 only when 0 */
} gs_view;

typedef struct gs_stats {
    int64_t num_visible;    /* M */
    int64_t num_entries;    /* P, tile-Gaussian pairs after the per-pair cull */
    int64_t pairs_pre;      /* rectangle pairs before the cull */
    float ms_project;       /* device time per stage (events), when timing is on */
    float ms_depth_sort;
    float ms_tile_assign;
    float ms_tile_sort;
    float ms_blend;
    float ms_total;         /* host wall clock of the whole call */
    int64_t blend_evals;    /* pixel x Gaussian evaluations blended (gs_set_timing 2) */
    int64_t blend_batches;  /* wave x 32-entry batches culled (gs_set_timing 2) */
    int64_t blend_iters;    /* wave apply iterations (gs_set_timing 2) */
    int64_t blend_kept;     /* kept (entry, microblock) pairs seen (gs_set_timing 2) */
    int64_t blend_max_iters; /* longest wave's apply iterations (gs_set_timing 2) */
    int64_t chunks_skipped;  /* projection partitions the chunk frustum skip ruled out */
    /* The reference's microblock-cull counts (cull_and_blend.cpp:835-836, the
     * pairs_dropped / pairs_kept_per_mb of render_full's stats), when
     * gs_set_cull_stats is on; -1 otherwise. */
    int64_t pairs_dropped_mb;  /* pairs that no microblock keeps */
    int64_t pairs_kept_mb;     /* kept (pair, microblock) pairs */
    /* The contribution floor the frame was rendered at: the view's, or a
     * coarser one after floor_retries re-renders because its candidate pairs
     * exceeded the pair limit (gs_set_pair_limit; render/host/render.cpp:537-565). */
    float contrib_floor;
    int32_t floor_retries;
} gs_stats;

/* ---- context -------------------------------------------------------- */
int gs_create(int device, gs_ctx** out);
void gs_destroy(gs_ctx* ctx);
const char* gs_last_error(void);
/* on: 0 off, 1 per-stage hipEvent times in gs_stats (ms_project ..), 2 also
 * the blend's evaluation counters (blend_evals ..; device atomics per wave).
 * Frames with either are enqueued directly, never replayed from a graph. */
int gs_set_timing(gs_ctx* ctx, int on);
int gs_device_info(gs_ctx* ctx, int* num_cus, int* arch_minor);

/* ---- frame ----------------------------------------------------------
 * gs_scene_set: makes `scene` resident (no-op when pointers, n and version
 * are unchanged). gs_render: the five stages of render_view
 * (render/host/render.cpp:263-615): project+SH -> visibility compaction ->
 * tile assign + pair cull -> tile/depth sort -> microblock cull + blend.
 * `out` is (H,W,3) of the requested format, host memory unless
 * out_on_device. M == 0 gives a black image. */
int gs_scene_set(gs_ctx* ctx, const gs_scene* scene);
int gs_render(gs_ctx* ctx, const gs_view* view, void* out, int out_on_device, gs_stats* stats);
/* n views of the scene (a camera path), as n gs_render calls, with up to four
 * frames in flight on four streams: a view is enqueued before the earlier ones
 * are waited for, so one frame's last stages overlap the next frame's first
 * ones (the cross-view pipelining of render/host/xview.h and the next_extrinsics
 * argument of render/host/render.cpp:263-273, for a known list of views).
 * outs[i] receives view i; stats (optional) is an array of n. Every view must
 * share contrib_floor, mb_contrib_floor and k_cap. When a frame fails, every
 * frame of the batch still in flight has finished writing its output before
 * the error is returned. */
int gs_render_batch(gs_ctx* ctx, const gs_view* views, int n, void* const* outs,
                    int out_on_device, gs_stats* stats);
/* gs_render of `view`, and - with next_view - the next view's frame enqueued on
 * the context's second slot before this one is waited for (render/host/
 * render.cpp:316-322, the next_extrinsics argument of render_view): the next
 * call whose view equals next_view (and whose scene is unchanged) completes
 * that frame instead of starting one. Any other call first completes and
 * drops an announced frame. */
int gs_render_next(gs_ctx* ctx, const gs_view* view, void* out, int out_on_device,
                   const gs_view* next_view, gs_stats* stats);

/* The last frame of this context's first slot, read back for parity checks (the
 * SortResult of src/gsplat_cpu/sort.cpp:146-165,217-257 after the frame's
 * tile_assign, backends/cpu_cpp/pybind_module.cpp:1149-1575). counts (3):
 * M, candidate pairs before the per-pair cull, P. sorted_ids (ids_cap >= P):
 * the tile-sorted compact ids (compact id = rank among the visible Gaussians
 * in source order, the reference's m), stable by (tile, depth bits, id).
 * tile_ranges (num_tiles x 2, num_tiles = the frame's tile count): [start,
 * end), (0, 0) for empty tiles. Any NULL output is skipped. GS_E_INVALID when
 * no frame is held (a later call reused the frame buffers). After
 * gs_render_batch the held frame is the last one of the context's first slot
 * (views i with i % 4 == 0); gs_frame_readback_info says which. */
int gs_frame_readback(gs_ctx* ctx, int64_t* counts, int64_t* sorted_ids, int64_t ids_cap,
                      int64_t* tile_ranges, int64_t num_tiles);
/* No counterpart in the reference: what gs_frame_readback would read. info (6):
 * M, candidate pairs, P, the frame's tile count, its index in the last
 * gs_render_batch (-1 when another call rendered it), 1 when it was replayed
 * from a captured graph. GS_E_INVALID when no frame is held. */
int gs_frame_readback_info(gs_ctx* ctx, int64_t* info);
/* Per-frame counts of the reference's microblock cull (gs_stats.pairs_dropped_mb,
 * pairs_kept_mb; cull_and_blend.cpp:384-504,835-836): one more pass over the
 * frame's pairs after the blend, off by default. */
int gs_set_cull_stats(gs_ctx* ctx, int on);
/* Spin limit of every bounded look-back wait of this context's kernels (0: the
 * default, 2^20 polls, about 0.45 s). A wait that reaches it goes on without the missing
 * prefix and the call returns GS_E_DEVICE ("look-back wait gave up") instead of
 * results; every kernel still exits normally. A tiny limit is for tests of that
 * error path only. */
int gs_set_spin_limit(gs_ctx* ctx, uint32_t limit);
/* The most candidate pairs a rendered frame's pair buffer may hold (0: the
 * default, 2^32-1; training steps are not limited). The buffer grows to a
 * frame's count up to this limit; a frame with
 * more candidates is rendered again, the whole frame at a coarser contribution
 * floor (both floors set to gs_overflow_next_floor of the coarser one), up to
 * 8 times and while the floor is below 1/2, the floor used reported in
 * gs_stats (render/host/overflow_retry.h:26-61, render.cpp:537-565, where the
 * limit is a sort bucket's record capacity). With the cull disabled, or past
 * the ladder, the call fails with GS_E_CAPACITY. The opacity terms of the
 * coarser floor are computed for that frame only (every frame slot is waited
 * for first, since the slots share them). */
int gs_set_pair_limit(gs_ctx* ctx, uint32_t limit);
/* The next contribution floor after a frame of max_n candidates against a
 * capacity of cap (max_n > cap): L = ln(1 / floor) scaled by 0.9 cap / max_n,
 * and at least twice the floor, at most 1/2 (render/host/overflow_retry.h:35-42). */
float gs_overflow_next_floor(float floor, uint32_t max_n, uint32_t cap);
/* gs_render_batch frames replayed from HIP graphs (on by default): each frame
 * slot captures its frame's kernels once per frame shape and replays them for
 * its later frames of that shape with the new camera (no counterpart in the
 * reference, whose device path is not HIP; for callers of many small frames,
 * whose launches cost host time). Results are identical either way; off
 * enqueues every kernel directly. Completes frames in flight. */
int gs_set_graphs(gs_ctx* ctx, int on);
/* Frame graphs captured and replayed so far by the context's frame slots (no
 * counterpart in the reference; for tests and tuning of gs_set_graphs). */
int gs_graph_counts(gs_ctx* ctx, int64_t* captures, int64_t* replays);

/* Chunk frustum skip (render/host/chunk_cull.h; GSPLAT_TT_CHUNK_CULL and
 * GSPLAT_TT_CHUNK_K of render/host/pfwc_device.cpp:214-240): per scene, the box of
 * mean +- k * 3 sqrt(trace cov3d) over each partition of 2048 consecutive
 * Gaussians; per frame, partitions behind the near plane or beyond a side plane
 * of the image (5 px pad) are not read. Images and counts are unchanged; it pays
 * off when the scene is spatially ordered (Morton order, gsplat_tt_amd.prep).
 * Off by default; k <= 0 selects 1.5. Not applied to views with k_cap > 3. */
int gs_set_chunk_cull(gs_ctx* ctx, int on, double k);

/* ---- zero-copy output ring (render/host/out_ring.h; render/host/render.cpp:
 * 334-340,598-612, GSPLAT_TT_OUT_ZEROCOPY) ------------------------------
 * gs_render_out_ring is gs_render_next whose image lands (by DMA from HBM) in
 * a pinned host buffer of the context's ring; the caller gets that buffer, no
 * host copy, and a lease. The ring never writes a buffer whose lease is held:
 * it takes the first free slot after the last one written, else grows up to
 * its cap, else gives the slot after the last one written a new buffer (the
 * held one stays valid until released). gs_out_release ends a lease; it may be
 * called from any thread and after gs_destroy (the buffer is then freed). */
typedef struct gs_out_image {
    const void* data;   /* (H, W, 3) of the view's out_format, pinned host memory */
    int64_t bytes;
    int64_t pitch;      /* bytes per image row: W * 3 * element size */
    uint64_t lease;     /* nonzero; pass to gs_out_release when done with data */
} gs_out_image;
int gs_render_out_ring(gs_ctx* ctx, const gs_view* view, const gs_view* next_view,
                       gs_out_image* image, gs_stats* stats);
int gs_out_release(uint64_t lease);
/* most buffers the ring keeps (default 4, GSPLAT_TT_OUT_ZEROCOPY_SLOTS of
 * render/host/env_config.h:272-277); a smaller cap lets go of surplus slots */
int gs_out_ring_config(gs_ctx* ctx, int cap);
int gs_out_ring_info(gs_ctx* ctx, int* size, int* held, int64_t* grows, int64_t* replaced);

/* ---- stages on host arrays (parity entry points) ----------------------
 * gs_project: project_full_fused, src/gsplat_cpu/project.cpp:484-798.
 * Outputs sized for n; *m_out = M. colors_out is (M,3) RGB (SH evaluated). */
int gs_project(gs_ctx* ctx, const gs_scene* scene, const gs_view* view,
               uint8_t* valid_mask, float* means2d, float* covs2d, float* depths,
               float* radii, float* colors_out, float* opac_out, int64_t* m_out);

/* gs_tile_assign: tile_assign, src/gsplat_cpu/tile_assign.cpp:26-368.
 * covs2d (m,4) and opac (m) may be NULL (no per-pair cull). Pairs are
 * Gaussian-major. Writes at most `cap` pairs; *p_out = P, *p_pre_out =
 * pairs before the cull (cap < P -> GS_E_CAPACITY, nothing written).
 * At most 65535 tiles per row and per column (also for views). */
int gs_tile_assign(gs_ctx* ctx, const float* means2d, const float* radii, int64_t m,
                   int image_height, int image_width, int tile_size, const float* covs2d,
                   const float* opac, float contrib_floor, int64_t* gids, int64_t* tids,
                   int64_t cap, int64_t* p_out, int64_t* p_pre_out);

/* gs_sort_and_bin: sort_and_bin, src/gsplat_cpu/sort.cpp:89-263. Stable by
 * (tile, fp32 depth bits); tile_ranges (T,2) with (0,0) for empty tiles. */
int gs_sort_and_bin(gs_ctx* ctx, const int64_t* gids, const int64_t* tids,
                    const float* depths, int64_t p, int64_t m, int tiles_x, int tiles_y,
                    int64_t* sorted_ids, int64_t* tile_ranges);

/* gs_cull_and_blend: cull_and_blend, src/gsplat_cpu/cull_and_blend.cpp:678-838.
 * Writes (H,W,3) in view->out_format; only tile_size, image size, floors,
 * cull_disabled, transmittance_threshold and out_format of `view` are read. */
int gs_cull_and_blend(gs_ctx* ctx, const float* means2d, const float* covs2d,
                      const float* colors, const float* opac, const int64_t* sorted_ids,
                      const int64_t* tile_ranges, int64_t m, int64_t p, const gs_view* view,
                      void* image_out);

/* ---- standalone tile/depth key sort (device pointers) -----------------
 * Stable LSD radix sort of (u64 key, u32 value) pairs by key bits
 * [begin_bit, end_bit), in place. Replaces the per-tile stable radix of
 * src/gsplat_cpu/sort.cpp:24-85 / render/kernels/dataflow/sort_radix_tile.cpp
 * for a whole (tile<<32 | depth_bits) key array. *passes_out = digit passes
 * executed (passes whose digit is constant are skipped). */
int gs_sort_pairs_u64_dev(gs_ctx* ctx, uint64_t* keys, uint32_t* vals, int64_t n,
                          int begin_bit, int end_bit, int* passes_out);
/* Average device time (ms) of each onesweep pass kernel of the last
 * gs_sort_pairs_u64_dev call when timing is on; returns the pass count. */
int gs_last_sort_pass_ms(gs_ctx* ctx, float* ms, int max_passes);
/* The standalone tile/depth sort with its per-tile ranges: the stable sort of
 * (u64 key, u32 value) by key bits [0, 32 + ceil(log2 num_tiles)) - keys are
 * (tile << 32) | fp32 depth bits, tile < num_tiles - then tile_ranges (device,
 * num_tiles x 2 u32) = [start, end) of each tile in the sorted keys, (0, 0)
 * when empty. Replaces the bin + per-tile radix + range table of
 * src/gsplat_cpu/sort.cpp:124-165,217-257 for a whole key array. A key with a
 * tile id >= num_tiles gives GS_E_INVALID. */
int gs_sort_tile_depth_dev(gs_ctx* ctx, uint64_t* keys, uint32_t* vals, int64_t n,
                           int64_t num_tiles, uint32_t* tile_ranges, int* passes_out);
/* The same sort with the outputs of the reference's sort_and_bin
 * (src/gsplat_cpu/sort.h:11-31, sort.cpp:89-165): the sorted values (ids, in
 * place: the input values in, the values in sorted key order out) and
 * tile_ranges; the sorted keys are not produced and `keys` is overwritten
 * (scratch). num_gaussians is sort_and_bin's M: every id is below it (0: any
 * 32-bit id). The key bits of the digits already sorted are dropped as soon as
 * the rest and the id fit 64 bits: the later passes move each key's remaining
 * bits and its id as one 8-byte word (one store stream instead of two), and
 * the last writes only the ids (it counts each tile's keys instead of writing
 * keys). A key with a tile id >= num_tiles, or with any bit set above the tile
 * field, or an id >= num_gaussians gives GS_E_INVALID. More than 2^24 tiles:
 * sorted as by gs_sort_tile_depth_dev (the ids are not checked). */
int gs_sort_tile_depth_ids_dev(gs_ctx* ctx, uint64_t* keys, uint32_t* ids, int64_t n,
                               int64_t num_gaussians, int64_t num_tiles, uint32_t* tile_ranges,
                               int* passes_out);
/* Device time (ms) of the range extraction of the last gs_sort_tile_depth_dev
 * or gs_sort_tile_depth_ids_dev call when timing is on (0 otherwise). */
float gs_last_ranges_ms(gs_ctx* ctx);
/* gs_sort_tile_depth_dev with no allocation of any kind. It has no counterpart
 * in the reference: it is for callers that cannot allocate (tight serving
 * loops, harnesses that forbid hipMalloc). It waits for the context's stream
 * (the error word is read back), so it cannot sit under HIP graph capture: a
 * call while the stream is capturing returns GS_E_INVALID, nothing done. Its
 * scratch (ping-pong keys and values, look-back descriptors, digit histograms,
 * control words) is one file-scope device array of 12.5 MiB per GPU, held
 * until the process ends, so n is at most 2^20 keys (larger n: GS_E_CAPACITY,
 * nothing done). Calls that overlap on one GPU share that array and race;
 * each call clears what must start at zero. Same results as
 * gs_sort_tile_depth_dev on the context's stream. */
int gs_sort_tile_depth_noalloc(gs_ctx* ctx, uint64_t* keys, uint32_t* vals, int64_t n,
                               int64_t num_tiles, uint32_t* tile_ranges, int* passes_out);

/* ---- training (3DGS rules: forward, L1, backward, sparse Adam) ---------
 * Follows the reference's training oracle gsplat/train_oracle.py (forward
 * :125-233, sparse Adam :434-470), the L1 gradient of gsplat/train_loss.py:166-171,
 * the blend backward of gsplat/blend_backward_ref.py:134-250 and the projection
 * backward of gsplat/t2_param_backward.py:123-192 (extended to SH degrees 1-3).
 * Parameters live on the device in optimizer space; one step = forward + L1 +
 * backward + sparse Adam, fp32 throughout. tile_size of the view must be 16. */

/* Host arrays in optimizer space (row-major, the reference's shapes). */
typedef struct gs_train_arrays {
    float* means;           /* (n,3) */
    float* log_scales;      /* (n,3) */
    float* quats;           /* (n,4) w x y z, unnormalised */
    float* opacity_logits;  /* (n) */
    float* sh;              /* (n,(d+1)^2,3) */
} gs_train_arrays;

typedef struct gs_train_cfg {
    float near_plane;       /* 0.2 */
    float lowpass;          /* 0.3, added to the 2D covariance diagonal */
    float alpha_max;        /* 0.99 */
    float alpha_min;        /* 1/255: pairs below are skipped */
    float t_min;            /* 1e-4: a pixel stops before T (1 - alpha) drops below */
    float background[3];
    float loss_scale;       /* scale of the whole loss (1: the reference's) */
    float lambda_dssim;     /* 0: loss = loss_scale * mean |image - target| (L1);
                             * > 0: loss_scale * ((1 - l) L1 + l (1 - SSIM)), the full
                             * 3DGS loss at l = 0.2 (train_oracle.py:253-279: 11-tap
                             * Gaussian window, sigma 1.5, zero padding) */
    /* Adam hyper-parameters in double, as the reference forms its fp32 step sizes
     * (float(lr / (1 - beta1^t)), float(1 - beta1), ...) from Python floats. */
    double lr_means, lr_log_scales, lr_quats, lr_opacity, lr_sh_dc, lr_sh_rest;
    double beta1, beta2, eps;
} gs_train_cfg;

typedef struct gs_train_stats {
    int64_t num_blendable;  /* Gaussians that reach alpha_min somewhere (M) */
    int64_t num_entries;    /* tile-Gaussian pairs after the cull (P) */
    int64_t step;           /* Adam steps taken so far */
    double loss;            /* the loss of cfg (with a target) */
    float ms_forward;       /* device time: projection + tiles + forward + L1 */
    float ms_backward;      /* blend backward + projection backward */
    float ms_adam;
    float ms_total;         /* host wall clock of the call */
    double l1;              /* mean |image - target| */
    double ssim;            /* mean SSIM (computed when lambda_dssim > 0) */
    int64_t pairs_pre;      /* candidate tile-Gaussian pairs before the cull */
    int64_t pair_capacity;  /* candidate-pair capacity after the call (grown on overflow) */
    int64_t pixel_pairs;    /* (pixel, entry) pairs the forward considered (up to each
                               pixel's stop); the backward evaluates the same pairs */
    int64_t pixel_blended;  /* of those, the pairs blended (alpha >= alpha_min) */
} gs_train_stats;

/* Gaussian-indexed projection values of the last forward (parity tests). */
typedef struct gs_train_proj {
    float* means2d;         /* (n,2) */
    float* conic;           /* (n,3) A B C, power = -0.5 (A dx^2 + 2B dx dy + C dy^2) */
    float* opacity;         /* (n) */
    float* colors;          /* (n,3) max(SH + 0.5, 0) */
    float* depth;           /* (n) */
    uint8_t* valid;         /* (n) z > near */
    uint8_t* visible;       /* (n) sparse-Adam rows */
} gs_train_proj;

/* Uploads the parameters (n Gaussians, SH degree 0..3), zeroes the Adam
 * moments and the step count. */
int gs_train_init(gs_ctx* ctx, const gs_train_arrays* params, int64_t n, int sh_degree);
/* which: 0 parameters, 1 first moments, 2 second moments, 3 gradients of the
 * last backward. Read copies device -> host; write replaces the device copy. */
int gs_train_read(gs_ctx* ctx, int which, gs_train_arrays* out);
int gs_train_write(gs_ctx* ctx, int which, const gs_train_arrays* in);
int gs_train_set_step(gs_ctx* ctx, int64_t step);
/* Storage of the Adam moments: 0 fp32 (default), 1 bf16 - the moments are read
 * exactly into fp32, updated in fp32 and stored rounded to nearest even
 * (gsplat/train_oracle.py:434-470 with moment_dtype bfloat16, the default of
 * the reference's device step, gsplat/t2_param_backward.py:195-224). Stored
 * moments are carried over (rounded when going to bf16); gs_train_read/write of
 * moments take and return fp32 arrays either way. Kept across gs_train_init. */
int gs_train_set_moments(gs_ctx* ctx, int bf16);
/* Replaces the sparse-Adam row mask (n bytes) of the last forward. */
int gs_train_set_visible(gs_ctx* ctx, const uint8_t* visible);

/* Forward of the current parameters for `view` (camera, image size, tile 16).
 * With a target (H,W,3) it also forms the L1 gradient and the loss. Outputs are
 * optional host arrays: image (H,W,3), final_T (H,W), projection values. */
int gs_train_forward(gs_ctx* ctx, const gs_view* view, const gs_train_cfg* cfg,
                     const float* target, float* image, float* final_T,
                     gs_train_proj* proj, gs_train_stats* stats);
/* Backward of the last forward. dimage (H,W,3) replaces the L1 gradient when
 * given. Writes the gradients (gs_train_read(ctx, 3, ...)); g2d (n,9) receives
 * the Gaussian-indexed 2D gradients dmx dmy dA dB dC dop dr dg db when given. */
int gs_train_backward(gs_ctx* ctx, const gs_train_cfg* cfg, const float* dimage, float* g2d,
                      gs_train_stats* stats);
/* Sparse Adam over the rows visible in the last forward (or set), with the
 * gradients of the last backward; the step count then increments. */
int gs_train_adam(gs_ctx* ctx, const gs_train_cfg* cfg, gs_train_stats* stats);
/* One whole step: forward + L1 against `target` (H,W,3; host memory unless
 * target_on_device) + backward + sparse Adam, one host synchronisation. */
int gs_train_step(gs_ctx* ctx, const gs_view* view, const gs_train_cfg* cfg,
                  const float* target, int target_on_device, gs_train_stats* stats);

/* Loss and image gradient of an (H,W,3) image against a target, both host
 * arrays: loss_scale ((1 - lambda_dssim) L1 + lambda_dssim (1 - SSIM)) and
 * dL/dimage (H,W,3), the device form of the reference's
 * gsplat/train_loss.py:126-163 loss_and_grad_device (fp32). loss3 (optional)
 * receives {loss, mean L1, mean SSIM}. */
int gs_train_loss(gs_ctx* ctx, const float* image, const float* target, int height, int width,
                  float lambda_dssim, float loss_scale, float* dimage, double* loss3);

/* ---- device memory helpers (for callers without a GPU framework) ------ */
int gs_dev_alloc(gs_ctx* ctx, int64_t bytes, void** ptr);
int gs_dev_free(gs_ctx* ctx, void* ptr);
int gs_memcpy_h2d(gs_ctx* ctx, void* dst, const void* src, int64_t bytes);
int gs_memcpy_d2h(gs_ctx* ctx, void* dst, const void* src, int64_t bytes);
/* Device-to-device copy; also the plain copy kernel of known size that HBM
 * traffic counters are calibrated against. */
int gs_memcpy_d2d(gs_ctx* ctx, void* dst, const void* src, int64_t bytes);
int gs_sync(gs_ctx* ctx);

#ifdef __cplusplus
}
#endif
#endif
