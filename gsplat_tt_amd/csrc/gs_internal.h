// gs_internal.h - types shared by the host orchestration (gs_api.cpp) and the
// kernel translation units, plus the kernel launchers each unit exports.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

struct gs_ctx;  // include/gsplat_hip.h

namespace gs {

// Error flags that kernels raise in ctl[0], the first of a launch's two
// control words (ctl[1]: the spin limit of a bounded look-back wait, 0 for the
// default). The host clears the flags before a launch sequence and turns any
// raised flag into an error status.
constexpr uint32_t kErrLookback = 1u;  // a look-back wait gave up: a prefix may be wrong
constexpr uint32_t kErrKeyRange = 2u;  // a sorted key's tile id is past the tile count
// the frame's candidate pairs exceed its pair capacity: the later kernels skip
// their work and the host runs the frame again with a larger capacity
constexpr uint32_t kErrCapacity = 4u;
constexpr uint32_t kErrValRange = 8u;  // a sorted value is past its stated bound

// Scene resident in HBM, structure-of-arrays (one coalesced dword stream per
// attribute). `sh` holds (d+1)^2*3 planes of n floats, plane index k*3+c.
struct SceneDev {
    int64_t n = 0;
    int sh_degree = -1;        // -1: plain RGB colours in col[0..2]
    float* mean[3] = {nullptr, nullptr, nullptr};
    float* cov[6] = {};        // c00 c01 c02 c11 c12 c22
    float* opac = nullptr;
    // per-Gaussian colour record, n x 3K floats as the scene gives it: RGB
    // (K = 1, sh_degree -1) or SH coefficient k channel c at [i*3K + k*3 + c]
    float* sh = nullptr;
    // Per-Gaussian terms that depend only on opacity and the floors; they
    // are computed on the host with the C library's logf so every log on the
    // pair path is the reference's bit for bit.
    float* kfac = nullptr;     // min(sqrt(2 ln max(op/floor,1)), k_cap)
    float* m2thr = nullptr;    // -2 ln(floor/op) or -1 (drop) [tile cull]
    float* lthr = nullptr;     // ln(mb_floor/op) or 0 (drop)  [microblock cull]
    // chunk frustum skip: per projection partition boxes (chunk_box_doubles(n)),
    // nullptr when off; chunk_k = the box's multiple of rho
    const double* chunk_box = nullptr;
    double chunk_k = 1.5;
};

struct ProjParams {
    float r[9];
    float t[3];
    float fx, fy, cx, cy;
    float ccx, ccy, ccz;       // camera centre -R^T t (SH view direction)
    float max_radius;          // already resolved (0 -> min(H,W)/2, <0 -> INT_MAX)
    float min_opacity;
    int height, width;
    int use_iso;
    int has_opac;
    int sh_clamp_hi;
    int write_src;             // also write compact->source index
    // depth-sort values (dval_pack: compact index | tile count << idx_bits) of
    // the frame's tile grid, written when dvals is set (idx_bits > 0)
    int tiles_x, tiles_y, tile_size, idx_bits;
    uint32_t* dvals;
    // per projection partition: nonzero = no Gaussian of it can reach the image
    // (its loads are skipped); nullptr = no partition is skipped
    const uint8_t* skip;
    uint32_t* ctl;             // control words (gs_common.h), may be null
};

// Compact (visible-only) Gaussian records, index m in [0, M).
struct Compact {
    // 2 x float4 per Gaussian, adjacent so that one 32-byte read gathers both
    // in rank order: (px, py, rx, ry) (a, b, c, m2thr)
    float4* rc;
    uint32_t* dkey;    // fp32 depth bits
    float4* brec;      // 3 x float4 per Gaussian: (mx,my,xh,yh) (ci_a,ci_b,ci_c,lt) (op,r,g,b)
    uint32_t* src;     // source index (optional)
};

// ---- project.hip
// part_hist (optional): per-partition digit histograms of the visible depth
// keys, [project_partitions(n)][4][256], summed by launch_reduce_rows.
hipError_t launch_project(const SceneDev& s, const ProjParams& p, Compact out,
                          uint8_t* valid_mask, uint64_t* lb_state, uint32_t* ticket,
                          uint32_t* count_out, uint32_t* part_hist, hipStream_t st);
// Captured frames (HIP graphs): the k_project instance launch_project uses for
// an SH degree, and an update of a captured k_project node's view parameters
// in an instantiated graph (the node's other arguments are kept).
const void* project_kernel(int sh_degree);
// The captured k_project node's scene and view arguments are s and p (its
// argument layout is what graph_set_project_params assumes).
bool graph_project_args_are(hipGraphNode_t node, const SceneDev& s, const ProjParams& p);
hipError_t graph_set_project_params(hipGraphExec_t exec, hipGraphNode_t node, const ProjParams& p);
// Chunk frustum skip (render/host/chunk_cull.h): per projection partition of the
// scene, the box of mean +- k rho, rho = 3 sqrt(trace cov3d), the largest rho and
// a non-finite flag (8 doubles per partition); per view, the partitions that lie
// behind the near plane or beyond a padded side plane of the image.
size_t chunk_box_doubles(int64_t n);
hipError_t launch_chunk_boxes(const SceneDev& s, double k, double* box, hipStream_t st);
hipError_t launch_chunk_cull(const double* box, int64_t n, const ProjParams& p, double k,
                             uint8_t* skip, uint32_t* n_skipped, hipStream_t st);
hipError_t launch_soa_transpose(const float* aos, int64_t n, int cols, const int* col_map,
                                int planes, float* soa, hipStream_t st);
size_t project_partitions(int64_t n);
hipError_t launch_brec_from_arrays(const float* means2d, const float* covs2d,
                                   const float* colors, const float* opac, const float* lthr,
                                   int64_t m, float4* brec, hipStream_t st);

// ---- sort.hip: onesweep LSD radix sort (stable), 8-bit digits.
struct SortTemp {
    void* keys_alt = nullptr;      // ping-pong key buffer (n keys)
    uint32_t* vals_alt = nullptr;  // ping-pong value buffer (n values)
    uint32_t* hist = nullptr;      // sort_hist_words(): [8][256] histograms + 8 tickets
    uint64_t* state = nullptr;     // sort_state_bytes(n): look-back descriptors
    uint32_t epoch = 0;            // bumped per pass; tags descriptors (no clearing)
    // 32-bit descriptors (below 2^30 keys) use the two halves of `state` in
    // turn: a pass clears, row by row, the half that the next pass uses, so no
    // pass needs a clearing kernel. Rows [clean[h], dirty[h]) of half h may
    // hold descriptors; a pass clears by a kernel those of them below its own
    // row count before it uses the half.
    size_t state_parts = 0;        // partition rows per half (state bytes / 2048)
    uint32_t dirty[2] = {0u, 0u};
    uint32_t clean[2] = {0u, 0u};
    int half = 0;
    hipEvent_t* pass_events = nullptr;  // optional: 2 per pass (start, stop)
    int max_timed_passes = 0;
    uint32_t* ctl = nullptr;       // control words of the passes (gs_common.h)
};
size_t sort_partitions(int64_t n);
// Adds the digit histograms of every pass of radix_sort_pairs_dev over 64-bit
// keys (digits of sort_digit_width(end_bit - begin_bit) bits, 256 words per
// pass) into hist, which the caller clears.
hipError_t launch_digit_hist_u64(const uint64_t* keys, int64_t n, int begin_bit, int end_bit,
                                 uint32_t* hist, hipStream_t st);
size_t sort_state_bytes(int64_t n);
size_t sort_hist_words();
// Stable sort of (keys, vals) by key bits [begin_bit, end_bit). key_bytes = 4
// or 8. With vals_iota the input values are taken as 0..n-1 (vals unread).
// Passes whose digit is constant are skipped; the result is left in either
// the caller's buffers or the SortTemp alternates: *keys_final / *vals_final.
// Reads the histogram back to the host (one stream synchronisation).
hipError_t radix_sort_pairs(void* keys, uint32_t* vals, int64_t n, int key_bytes,
                            int begin_bit, int end_bit, SortTemp& tmp, uint32_t* host_hist,
                            hipStream_t st, int* passes_run, bool vals_iota,
                            void** keys_final, uint32_t** vals_final);
// Same sort with no host synchronisation: the key count is min(n_cap, *n_dev)
// (n_dev may be null), `hist` holds the [pass][256] digit histograms of the
// keys (built by their producer), `tickets` one zeroed word per pass. Every
// pass runs; the result buffer follows from the pass count alone.
// n_kept_dev (u32 keys only, optional): the first pass drops every key equal
// to kPairDrop (its value is not read) and stably compacts the rest; later
// passes sort min(n_cap, *n_kept_dev) keys, and `hist` counts kept keys only.
// run_cnt (u32 keys only, optional): the sorted keys are not written (*keys_final = nullptr); run_cnt[k] (cleared by the caller) gains
// the number of keys equal to k, for launch_ranges_from_counts.
// keys_out = false (u32 keys): the last pass writes the sorted values only
// (*keys_final = nullptr).
// first_offs (u32 keys only, optional): the first pass's output positions per
// partition of kSortPartition32 keys and digit (2^w words per partition, w the
// pass's digit width; launch_part_offsets): that pass needs no look-back.
constexpr uint32_t kPairDrop = 0xFFFFFFFFu;
constexpr uint32_t kSortPartition32 = 8192;  // keys per partition of a 32-bit-key pass
hipError_t radix_sort_pairs_dev(void* keys, uint32_t* vals, int64_t n_cap, const uint32_t* n_dev,
                                int key_bytes, int begin_bit, int end_bit, const uint32_t* hist,
                                uint32_t* tickets, SortTemp& tmp, hipStream_t st, bool vals_iota,
                                void** keys_final, uint32_t** vals_final,
                                const uint32_t* n_kept_dev = nullptr,
                                uint32_t* run_cnt = nullptr,
                                const uint32_t* first_offs = nullptr,
                                uint32_t run_limit = 0xFFFFFFFFu, bool keys_out = true);

// The 64-bit-key sort of radix_sort_pairs_dev over exactly n keys, with no
// producer histogram: a histogram kernel counts the first pass's digits and
// each pass adds the next pass's digit counts from the keys it holds, into
// `hist` ([pass][256], cleared by the caller). Every pass runs.
hipError_t radix_sort_pairs_dev_chain(uint64_t* keys, uint32_t* vals, int64_t n, int begin_bit,
                                      int end_bit, uint32_t* hist, uint32_t* tickets,
                                      SortTemp& tmp, hipStream_t st, void** keys_final,
                                      uint32_t** vals_final);

// The same stable sort of (tile << 32 | depth bits) keys below 2^(32 +
// tile_bits) with values below val_limit (0: any 32-bit value; the values take
// val_bits = the bits of val_limit - 1 in the words below), when only the values and the runs
// of each tile are wanted: once the key bits left to sort and the value fit
// 64 bits (after q passes of w-bit digits, the q-th writing each key's bits
// [q * w, ...) above its value as one 64-bit word), the later passes move
// those words, one store stream instead of two, and the last pass writes the
// sorted values into vals and counts each tile's keys into run_cnt[tile]
// (num_tiles words, cleared by the caller) instead of writing keys. The keys
// buffer is overwritten (scratch). A key with a tile id >= num_tiles or a bit
// set above the tile field flags kErrKeyRange, a value >= val_limit
// kErrValRange, in *key_err (a word other than tmp.ctl[0], cleared by the
// caller: the passes go on).
// hipErrorNotSupported: the key bits and the value never fit one word before
// the last pass; the caller sorts the keys whole instead.
hipError_t radix_sort_ids_dev_chain(uint64_t* keys, uint32_t* vals, int64_t n, int tile_bits,
                                    uint64_t val_limit, uint32_t num_tiles, uint32_t* run_cnt,
                                    uint32_t* key_err, uint32_t* hist, uint32_t* tickets,
                                    SortTemp& tmp, hipStream_t st, int* passes_out);

// Device and stream of a context (gs_api.cpp), for entry points in other units.
struct CtxInfo {
    int device;
    hipStream_t stream;
};
CtxInfo ctx_info(const ::gs_ctx* ctx);
// Sets the calling thread's gs_last_error() message.
void set_last_error(const char* msg);

// ---- tiles.hip
struct TileParams {
    int tiles_x, tiles_y, tile_size;
    int cull;          // per-pair Mahalanobis cull on
    uint32_t* ctl;     // control words (gs_common.h), may be null
    // the rank order holds packed depth-sort values (dval_pack) with this many
    // index bits; 0: plain compact indices
    int idx_bits;
};
// offs: exclusive scan of rectangle areas in `order`; bstart[b]: rank owning
// candidate b*emit_part (b < bstart_cap).
// Sizes: m / p_pre / p are host capacities sizing the grids; when the *_dev
// pointer is given the real count is read on the device (min with the
// capacity) and partitions beyond it exit at once.
// Rank r's rectangle is rect[order[r] * stride] (order null: rect[r * stride]);
// stride is in float4 (2 for the interleaved rectangle + conic records).
// cap (0: none): a total above it raises kErrCapacity in tp.ctl.
// reduce_scan: three kernels that never wait on each other's partitions
// (lb_state then holds rect_scan_partitions(m) partition sums) instead of one
// kernel chained by a look-back (lb_state: its cleared descriptors, ticket).
hipError_t launch_rect_count_scan(const float4* rect, int stride, const uint32_t* order,
                                  int64_t m, const uint32_t* m_dev, TileParams tp, uint32_t* offs,
                                  uint32_t* bstart, uint32_t bstart_cap, uint64_t* lb_state,
                                  uint32_t* ticket, uint32_t* total_out, uint32_t cap,
                                  bool reduce_scan, hipStream_t st);
// Digit width of a device sort over `bits` key bits: the fewest 8-bit-or-less
// passes, with the bits spread evenly over them (12 tile bits: two passes of 6,
// whose 64 digits give longer runs per digit than 256 would).
inline int sort_digit_width(int bits) {
    const int passes = (bits + 7) / 8;
    return passes > 0 ? (bits + passes - 1) / passes : 8;
}
// Tile-id digit histograms that the pair emission produces, one row per emit
// partition: two digits for up to 16 tile bits, three above, each of
// 2^sort_digit_width(tile_bits) words, the row padded with zeros to a power of
// two (12 tile bits: 2 x 64 = 128 words).
inline int tile_hist_cols(int tile_bits) {
    return (tile_bits > 16 ? 4 : 2) << sort_digit_width(tile_bits);
}
// Rank r's rectangle and conic are rect / cov[e * stride] with e = order[r]
// when by_order (records in compact order, as the projection writes them),
// else e = r (records already in rank order); pair ids are order[r] (r when
// order is null). part_hist (optional): per-partition digit histograms of the
// kept pairs' tile ids, one row of tile_hist_cols(tile_bits) words per emit
// partition: 2^w words per digit of w = sort_digit_width(tile_bits) bits, lowest
// digit first (launch_reduce_rows with dig_w = w spreads them to 256-word rows).
hipError_t launch_pair_emit(const float4* rect, const float4* cov, int stride, bool by_order,
                            const uint32_t* order, const uint32_t* offs, const uint32_t* bstart, int64_t m,
                            const uint32_t* m_dev, uint32_t p_pre, const uint32_t* p_pre_dev,
                            TileParams tp, uint32_t* pair_tile, uint32_t* pair_id, uint32_t cap,
                            uint64_t* lb_state, uint32_t* ticket, uint32_t* total_out,
                            uint32_t* part_hist, int tile_bits, bool compact, hipStream_t st);
hipError_t launch_tile_ranges(const uint32_t* sorted_tile, uint32_t p, const uint32_t* p_dev,
                              uint32_t* ranges, int64_t num_tiles, hipStream_t st);
// ranges[t] = [start, end) from per-tile pair counts (an exclusive scan in tile
// order; (0, 0) for an empty tile), one workgroup.
hipError_t launch_ranges_from_counts(const uint32_t* counts, int64_t num_tiles, uint32_t* ranges,
                                     hipStream_t st);
// Same ranges by per-tile binary search over the sorted tile keys (reads
// O(tiles * log p) keys instead of all p; no clearing pass).
hipError_t launch_tile_bounds(const uint32_t* sorted_tile, uint32_t p_cap, const uint32_t* p_dev,
                              uint32_t* ranges, int64_t num_tiles, hipStream_t st);
// The same ranges over (tile << 32 | depth bits) keys sorted ascending; a tile
// id >= num_tiles is flagged kErrKeyRange in ctl[0] (its keys get no range).
hipError_t launch_tile_bounds64(const uint64_t* sorted_keys, uint32_t p, uint32_t* ranges,
                                int64_t num_tiles, uint32_t* ctl, hipStream_t st);
// out[c] += sum over rows of part[r][c] (out must be cleared by the caller);
// with dig_w > 0 the columns are digit rows of 2^dig_w words and column c adds
// into out[(c >> dig_w) * 256 + (c & (2^dig_w - 1))].
// chunk_out (optional, reduce_chunks(rows_cap) x cols words): the column sums
// of each workgroup's rows, for launch_part_offsets. ctl (optional): the
// kernel does nothing when an upstream kernel raised an error flag there.
hipError_t launch_reduce_rows(const uint32_t* part, int cols, uint32_t rows_cap,
                              const uint32_t* count_dev, uint32_t count_cap, uint32_t per_row,
                              int dig_w, uint32_t* out, hipStream_t st,
                              uint32_t* chunk_out = nullptr, const uint32_t* ctl = nullptr);
size_t reduce_chunks(uint32_t rows_cap);
// After launch_reduce_rows with chunk_out over the same rows: per partition of
// rows_per_part rows and per digit d < 2^dig_w (columns 0 .. 2^dig_w - 1 of a
// row), offs[s << dig_w | d] = (sum of hist[d'] over d' < d) + (sum of
// part[e][d] over rows e < s * rows_per_part): the output position of the
// partition's first key of digit d in a sort pass over those keys (hist: that
// pass's digit histogram). ceil(rows in use / rows_per_part) << dig_w words.
// Nothing is done when an upstream kernel raised an error flag in ctl.
hipError_t launch_part_offsets(const uint32_t* part, int cols, uint32_t rows_cap,
                               const uint32_t* count_dev, uint32_t count_cap, uint32_t per_row,
                               int rows_per_part, int dig_w, const uint32_t* chunks,
                               const uint32_t* hist, uint32_t* offs, hipStream_t st,
                               const uint32_t* ctl = nullptr);
constexpr uint32_t kEmitPartition = 2048;   // candidates per emit partition
constexpr uint32_t kProjPartition = 2048;   // Gaussians per project partition
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t st);
// Up to six fills (n[r] words at p[r] set to v[r]) in one launch.
hipError_t launch_fill_ranges(uint32_t* const* p, const uint32_t* v, const uint32_t* n, int count,
                              hipStream_t st);
hipError_t launch_make_keys64(const uint32_t* gid, const uint32_t* tid, const float* depths,
                              uint32_t p, uint64_t* keys, hipStream_t st);
hipError_t launch_tile_ranges64(const uint64_t* keys, uint32_t p, uint32_t* ranges,
                                int64_t num_tiles, hipStream_t st);
size_t rect_scan_partitions(int64_t m);
size_t emit_partitions(uint64_t p_pre);

// ---- blend.hip
struct BlendParams {
    int tiles_x, tiles_y, tile_size;
    int height, width;
    int cull_disabled;
    float thr;
    int out_format;    // 0 u8, 1 bf16, 2 f32
    // optional counters, 64 slot groups of 8 (summed by the host): pixel-Gaussian
    // evaluations, entry batches, apply iterations, kept (entry, microblock)
    // pairs, max apply iterations of one wave
    unsigned long long* evals;
    const uint32_t* ctl;  // control words of the frame (nothing is read after an error)
};
hipError_t launch_blend(const float4* brec, const uint32_t* sorted_id, const uint32_t* ranges,
                        BlendParams bp, void* out, hipStream_t st);
// Counts of the reference's microblock cull over the tile-sorted pairs (ids
// `sid`, tile ids `stile`, min(p_cap, *p_dev) of them): out[0] += pairs kept by
// no microblock, out[1] += kept (pair, microblock) pairs.
hipError_t launch_mb_stats(const float4* brec, const uint32_t* sid, const uint32_t* stile,
                           uint32_t p_cap, const uint32_t* p_dev, int tiles_x, int tile_size,
                           int cull_disabled, unsigned long long* out, const uint32_t* ctl,
                           hipStream_t st);

// ---- train.hip: training step (3DGS forward rules, L1, backward, sparse Adam)
constexpr int kMaxTrainPlanes = 64;  // 11 geometry/opacity planes + 3 (d+1)^2 SH planes

// Optimizer-space parameters (or gradients / moments of the same shape) as SoA
// planes of n floats: mean x y z, log-scale 0..2, quaternion w x y z, opacity
// logit, then SH plane 3k+c for coefficient k, channel c.
struct TrainParamsDev {
    float* mean[3];
    float* ls[3];
    float* quat[4];
    float* ol;
    float* sh;
    int64_t n;
    int sh_degree;
};

struct TrainCam {
    float r[9], t[3];          // world-to-camera rotation (row-major) and translation
    float fx, fy, cx, cy;
    float ccx, ccy, ccz;       // camera centre -R^T t
    float near, lowpass, alpha_min;
    int H, W;
    uint32_t* ctl;             // control words (gs_common.h), may be null
};

// Optional Gaussian-indexed copies of the projection values (parity tests).
struct TrainDebug {
    float* means2d;   // (n,2)
    float* conic;     // (n,3)
    float* opacity;
    float* colors;    // (n,3)
    float* depth;
    uint8_t* valid;
};

struct TrainFwdParams {
    int tiles_x, tiles_y, width, height;
    float alpha_max, alpha_min, t_min;
    float bg[3];
    float* image;          // (H,W,3)
    float* final_T;        // (H,W)
    uint32_t* stop;        // (H,W) entries of the tile list the pixel considered
    const float* target;   // (H,W,3) or null (no loss)
    float* dimage;         // dL/dimage (H,W,3), written with a target
    float grad_scale;      // loss_scale / (3HW)
    double* loss;          // accumulates sum |image - target|
    // (pixel, entry) pairs: [0] considered (each pixel's entries up to its
    // stop), [1] blended; accumulated (the backward evaluates the same pairs)
    unsigned long long* pairs;
    const uint32_t* ctl;   // control words of the forward (nothing is read after an error)
};

// Full 3DGS loss terms (1 - lambda) L1 + lambda (1 - SSIM) on an (H,W,3) image.
struct SsimParams {
    int width, height;
    float g[11];           // normalised Gaussian taps (sigma 1.5)
    float w;               // -lambda * loss_scale / (3HW): scale of the SSIM terms
    const float* image;    // (H,W,3)
    const float* target;   // (H,W,3)
    float* maps;           // 3 x (H,W,3): w dS/dmu_x, w dS/dE_xx, w dS/dE_xy
    float* dimage;         // (H,W,3): the SSIM gradient is added
    double* ssim_sum;      // accumulates sum of S over the 3HW values
};
hipError_t launch_ssim(const SsimParams& sp, hipStream_t st);
// dimage = scale * sign(image - target); *l1_sum += sum |image - target|.
hipError_t launch_l1(const float* image, const float* target, int64_t count, float scale,
                     float* dimage, double* l1_sum, hipStream_t st);

struct TrainBwdParams {
    int tiles_x, tiles_y, width, height;
    float alpha_max, alpha_min;
    float bg[3];
    const float* final_T;
    const uint32_t* stop;
    const float* dimage;
    float* grad2d;         // (M,9) per compact Gaussian: dmx dmy dA dB dC dop dr dg db
};

struct AdamParams {
    float beta1, beta2, one_minus_beta1, one_minus_beta2, sqrt_bc2, eps;
    float step[kMaxTrainPlanes];  // learning rate / (1 - beta1^t), per plane
};

// Compact outputs: rect (u, v, rx, ry), cov (a, b, c, 2 ln(op/alpha_min)), depth
// keys, src (compact -> Gaussian) and the forward record trec (3 float4 per
// compact Gaussian: (u, v, op), (A, B, C), (r, g, b)); cidx maps Gaussian ->
// compact index or 0xFFFFFFFF; visible marks the sparse-Adam rows.
hipError_t launch_train_project(const TrainParamsDev& P, const TrainCam& cam, Compact out,
                                float4* trec, uint32_t* cidx, uint8_t* visible,
                                uint64_t* lb_state, uint32_t* ticket, uint32_t* count_out,
                                uint32_t* part_hist, const TrainDebug& dbg, hipStream_t st);
hipError_t launch_train_fwd(const float4* trec, const uint32_t* sid, const uint32_t* ranges,
                            const TrainFwdParams& fp, hipStream_t st);
hipError_t launch_train_bwd(const float4* trec, const uint32_t* sid, const uint32_t* ranges,
                            const TrainBwdParams& bp, hipStream_t st);
hipError_t launch_train_param_grads(const TrainParamsDev& P, const TrainCam& cam,
                                    const uint32_t* cidx, const float* grad2d,
                                    const TrainParamsDev& G, hipStream_t st);
// m, v: float planes, or bf16 bits (uint16_t planes) with bf16_moments.
hipError_t launch_sparse_adam(float* p, void* m, void* v, const float* g,
                              const uint8_t* visible, int64_t n, int planes, const AdamParams& ap,
                              bool bf16_moments, hipStream_t st);

}  // namespace gs
