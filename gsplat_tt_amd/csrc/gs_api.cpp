// gs_api.cpp - host orchestration behind the C ABI of include/gsplat_hip.h.
//
// Mirrors the stage order and failure policy of the reference's render_view
// (render/host/render.cpp:263-615): project -> visibility gather ->
// tile_assign -> sort -> cull+blend, all resident in HBM, no CPU fallback
// (a device failure is an error, render.cpp:252-259,570-578), M == 0 gives a
// black image (:389-396). The frame path sorts the visible Gaussians by depth
// once and then emits their pairs in depth order, so a stable sort of the
// pairs by tile id alone yields the reference's (tile, depth, id) order.
//
// Compiled with -ffp-contract=off: the per-Gaussian log terms computed here
// are the C library's logf values the reference uses (types.h:141-144,
// tile_assign.cpp:174-183, cull_and_blend.cpp:743-753).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/gsplat_hip.h"
#include "gs_internal.h"
#include "out_ring.h"

namespace {

thread_local std::string g_err;

struct GsError : std::runtime_error {
    int code;
    GsError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define HIPCHK(x)                                                                        \
    do {                                                                                 \
        hipError_t e_ = (x);                                                             \
        if (e_ != hipSuccess)                                                            \
            throw GsError(GS_E_DEVICE, std::string(#x) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define REQUIRE(cond, msg)                                  \
    do {                                                    \
        if (!(cond)) throw GsError(GS_E_INVALID, (msg));    \
    } while (0)

template <class F>
int guard(F&& f) {
    try {
        f();
        return GS_OK;
    } catch (const GsError& e) {
        g_err = e.what();
        return e.code;
    } catch (const std::exception& e) {
        g_err = e.what();
        return GS_E_DEVICE;
    }
}


struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    // Grows to at least `bytes`; callers guarantee the stream is idle.
    void ensure(size_t bytes) {
        if (bytes <= cap && p != nullptr) return;
        size_t want = std::max<size_t>(bytes, 256);
        if (cap > 0) want = std::max(want, cap + cap / 2);
        want = (want + 4095) & ~size_t(4095);
        if (p) HIPCHK(hipFree(p));
        p = nullptr;
        cap = 0;
        HIPCHK(hipMalloc(&p, want));
        cap = want;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
    template <class T>
    T* as() const { return static_cast<T*>(p); }
};

template <class F>
void parallel_for(int64_t n, F&& f) {
    const int64_t hw = std::max(1u, std::thread::hardware_concurrency());
    const int64_t workers = std::min<int64_t>(hw, std::max<int64_t>(1, n / 65536));
    if (workers <= 1) {
        f(0, n);
        return;
    }
    std::vector<std::thread> ts;
    const int64_t chunk = (n + workers - 1) / workers;
    for (int64_t w = 0; w < workers; ++w) {
        const int64_t lo = w * chunk, hi = std::min(n, lo + chunk);
        if (lo < hi) ts.emplace_back([&f, lo, hi] { f(lo, hi); });
    }
    for (auto& t : ts) t.join();
}

// Per-Gaussian opacity terms with the C library's logf (types.h:141-176,
// tile_assign.cpp:171-197, cull_and_blend.cpp:743-753).
void opacity_terms(const float* op, int64_t n, bool has_opac, float cf, float mbf, float k_cap,
                   float* kfac, float* m2thr, float* lthr) {
    parallel_for(n, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i) {
            float k = 3.0f;
            if (has_opac) {
                const float q = op[i] / cf;
                const float arg = (q < 1.0f) ? 1.0f : q;
                k = std::sqrt(2.0f * std::log(arg));
            }
            if (k_cap > 0.0f) k = (k_cap < k) ? k_cap : k;
            kfac[i] = k;
            if (m2thr) {
                const float o = has_opac ? op[i] : 1.0f;
                m2thr[i] = (o > cf) ? -2.0f * std::log(cf / o) : -1.0f;
            }
            if (lthr) {
                const float o = has_opac ? op[i] : 1.0f;
                lthr[i] = (o <= mbf) ? 0.0f : std::log(mbf / o);
            }
        }
    });
}

int tile_bits(int64_t num_tiles) {
    int b = 0;
    while (((int64_t)1 << b) < num_tiles) ++b;
    return std::max(b, 1);
}

// Candidate-pair capacity a scene of n Gaussians starts with: 8 per Gaussian
// (scene-scale views reach 6-7: 35-40M at 6M Gaussians), so a camera path does
// not stall mid-way to grow its buffers and re-run a frame; at most 2^29.
uint64_t default_pair_cap(int64_t n) {
    return std::min<uint64_t>((uint64_t)1 << 29, std::max<uint64_t>(1u << 20, (uint64_t)n * 8));
}

// Index bits of the frame's packed depth-sort values over n Gaussians (the
// tile count takes the rest of the word), 0 when too few bits would be left.
int dval_idx_bits(int64_t n) {
    const int b = tile_bits(n);
    return b <= 28 ? b : 0;
}

// The coarser-floor ladder of a frame whose candidate pairs exceed the pair
// limit (render/host/overflow_retry.h:26-61): a Gaussian reaches a tile while
// 2 ln(o / floor) >= d^2, so the pair count grows roughly with L = ln(1 / floor);
// the next floor scales L by 0.9 cap / max_n and at least doubles the floor.
constexpr int kFloorRetries = 8;
constexpr float kFloorMax = 0.5f;
float next_contrib_floor(float floor, uint32_t max_n, uint32_t cap) {
    const double f = std::min(std::max((double)floor, 1.0 / 1048576.0), (double)kFloorMax);
    const double scale = 0.9 * (double)cap / (double)std::max(max_n, cap);
    const double by_model = std::exp(std::log(f) * scale);  // exp(-L scale)
    return (float)std::min(std::max(by_model, 2.0 * f), (double)kFloorMax);
}

}  // namespace

struct gs_ctx {
    int device = 0;
    hipStream_t st = nullptr;
    bool timing = false;        // per-stage hipEvents (gs_set_timing >= 1)
    bool blend_counts = false;  // the blend's evaluation counters (gs_set_timing 2)
    hipEvent_t ev[12] = {};
    hipEvent_t sort_ev[16] = {};
    int last_sort_passes = 0;
    float last_ranges_ms = 0.0f;  // tile-range extraction of the last gs_sort_tile_depth_dev
    int num_cus = 0;

    // scene
    struct {
        const void *means = nullptr, *cov = nullptr, *opac = nullptr, *col = nullptr;
        int64_t n = -1;
        int stride = 0, deg = -2;
        uint64_t ver = 0;
        bool valid = false;
    } skey;
    struct {
        float cf = 0, mbf = 0, kcap = 0;
        bool has_opac = false;
        uint64_t gen = 0;
        bool valid = false;
    } tkey;
    uint64_t scene_gen = 0;
    gs::SceneDev sd;
    bool has_opac = false;
    std::vector<float> h_opac;
    DevBuf b_mean, b_cov, b_opac, b_col, b_terms, b_upload;

    // frame
    DevBuf b_rc, b_dkey, b_brec, b_src, b_valid;
    DevBuf b_offs, b_bstart, b_pair_tile, b_pair_id, b_ranges, b_out;
    DevBuf b_kalt, b_valt, b_hist, b_state, b_lb, b_cnt;
    DevBuf b_tmp_a, b_tmp_b, b_tmp_c, b_evals;
    DevBuf b_tcnt;  // per-tile key counts of gs_sort_tile_depth_ids_dev
    std::vector<uint64_t> h_evals = std::vector<uint64_t>(64 * 8);
    uint32_t* h_pin = nullptr;  // pinned: counters + histograms
    gs::SortTemp sort;

    // Control words of the kernels (ctl[0] error flags, ctl[1] look-back spin
    // limit): words C_CTL.. of the frame counters, or of b_cnt for the stage
    // entry points.
    uint32_t spin_limit = 0;   // 0: the kernels' default (gs_set_spin_limit)
    uint32_t pair_limit = 0xFFFFFFFFu;  // most candidate pairs a frame holds (gs_set_pair_limit)
    gs_ctx* owner = nullptr;   // a frame slot's first slot, whose opacity terms it shares
    bool cull_stats = false;   // microblock-cull statistics per frame (gs_set_cull_stats)
    bool graphs = true;        // batch frames replayed from captured graphs (gs_set_graphs)
    bool batch_frame = false;  // render_begin is enqueueing a gs_render_batch frame
    int64_t graph_captures = 0, graph_replays = 0;  // gs_graph_counts
    // Enqueues the reset of a pair of control words (flags 0, spin limit).
    void ctl_reset(uint32_t* ctl) {
        HIPCHK(gs::launch_fill_u32(ctl, 0u, 1, st));
        HIPCHK(gs::launch_fill_u32(ctl + 1, spin_limit, 1, st));
    }
    // Turns raised error flags into an error: the outputs are not trusted.
    static void ctl_check(uint32_t flags, const char* what) {
        if (flags & gs::kErrKeyRange)
            throw GsError(GS_E_INVALID, std::string(what) + ": a key's tile id is >= num_tiles");
        if (flags & gs::kErrValRange)
            throw GsError(GS_E_INVALID, std::string(what) + ": an id is >= num_gaussians");
        if (flags & gs::kErrCapacity)
            throw GsError(GS_E_CAPACITY, std::string(what) + ": candidate pairs past the capacity");
        if (flags != 0u)
            throw GsError(GS_E_DEVICE, std::string(what) +
                                           ": a bounded look-back wait gave up (outputs discarded)");
    }

    // The last gs_render frame of this context, for gs_frame_readback: its
    // tile-sorted compact ids and tile ids live in the frame buffers until the
    // next call that reuses them.
    bool rb_valid = false, rb_empty = false;
    uint32_t* rb_ids = nullptr;
    int64_t rb_T = 0, rb_M = 0, rb_ppre = 0, rb_P = 0;
    int64_t rb_batch = -1;     // its index in the last gs_render_batch (-1: another call)
    bool rb_replayed = false;  // it was replayed from a captured graph

    ~gs_ctx() {
        for (gs_ctx* p : peers) delete p;
        if (st) (void)hipStreamSynchronize(st);
        // an announced frame's ring image (its writer has finished: both
        // slots' streams are synchronised above)
        if (spec_lease) gs::LeaseTable::get().release(spec_lease);
        drop_graph();
        for (DevBuf* b : {&b_mean, &b_cov, &b_opac, &b_col, &b_terms, &b_upload, &b_rc,
                          &b_dkey, &b_brec, &b_src, &b_valid, &b_offs, &b_bstart, &b_pair_tile, &b_pair_id,
                          &b_ranges, &b_out, &b_kalt, &b_valt, &b_hist, &b_state, &b_lb, &b_cnt,
                          &b_tmp_a, &b_tmp_b, &b_tmp_c, &b_evals, &b_frame, &b_phist_proj,
                          &b_phist_emit, &b_pchunk, &b_poffs, &b_spec, &b_chunk_box,
                          &b_skip, &b_tcnt})
            b->release();
        if (h_pin) (void)hipHostFree(h_pin);
        ring.reset();  // held images stay valid until their leases are released
        for (auto& e : ev)
            if (e) (void)hipEventDestroy(e);
        for (auto& e : sort_ev)
            if (e) (void)hipEventDestroy(e);
        for (auto& e : tev)
            if (e) (void)hipEventDestroy(e);
        for (DevBuf* b : {&t_p, &t_m, &t_v, &t_g, &t_cidx, &t_vis, &t_grad2d, &t_img, &t_T, &t_stop,
                          &t_dimg, &t_tgt, &t_loss, &t_dbg, &t_ssim})
            b->release();
        if (st) (void)hipStreamDestroy(st);
    }

    void sync() { HIPCHK(hipStreamSynchronize(st)); }
    // Drops a frame that an error interrupted: waits for what it enqueued
    // (a copy into its output may be in flight) without throwing, so that the
    // caller can then hand its output buffer back.
    void abandon_frame() noexcept {
        if (!pend.active) return;
        pend.active = false;
        (void)hipStreamSynchronize(st);
    }

    // ------------------------------------------------------------ scene
    void set_scene(const gs_scene* s) {
        REQUIRE(s != nullptr && s->means != nullptr && s->cov3d != nullptr, "scene: null arrays");
        REQUIRE(s->n >= 0 && s->n < ((int64_t)1 << 31), "scene: n out of range");
        REQUIRE(s->cov3d_stride == 9 || s->cov3d_stride == 6, "scene: cov3d_stride must be 9 or 6");
        REQUIRE(s->sh_degree >= -1 && s->sh_degree <= 3, "scene: sh_degree must be -1..3");
        REQUIRE(s->colors != nullptr || s->n == 0, "scene: colors required");
        if (skey.valid && skey.means == s->means && skey.cov == s->cov3d &&
            skey.opac == s->opacities && skey.col == s->colors && skey.n == s->n &&
            skey.stride == s->cov3d_stride && skey.deg == s->sh_degree && skey.ver == s->version)
            return;
        drain_spec();  // an announced frame reads the buffers about to change
        const int64_t n = s->n;
        sync();
        if (n != sd.n) {
            // the frame's launch grids follow the pair capacity: a scene of another
            // size starts again from its own default (buffers keep their memory)
            pair_cap = 0;
            for (gs_ctx* p : peers) p->pair_cap = 0;
        }
        const int K = s->sh_degree < 0 ? 1 : (s->sh_degree + 1) * (s->sh_degree + 1);
        const int col_planes = 3 * K;
        b_mean.ensure(std::max<int64_t>(n, 1) * 3 * 4);
        b_cov.ensure(std::max<int64_t>(n, 1) * 6 * 4);
        b_opac.ensure(std::max<int64_t>(n, 1) * 4);
        b_col.ensure(std::max<int64_t>(n, 1) * col_planes * 4);
        b_terms.ensure(std::max<int64_t>(n, 1) * 3 * 4);
        const int max_cols = std::max(3, s->cov3d_stride);
        b_upload.ensure(std::max<int64_t>(n, 1) * max_cols * 4);
        float* up = b_upload.as<float>();
        auto transpose = [&](const float* host, int cols, const int* map, int planes, float* dst) {
            if (n == 0) return;
            HIPCHK(hipMemcpyAsync(up, host, (size_t)n * cols * 4, hipMemcpyHostToDevice, st));
            HIPCHK(gs::launch_soa_transpose(up, n, cols, map, planes, dst, st));
            sync();
        };
        const int id3[3] = {0, 1, 2};
        transpose(s->means, 3, id3, 3, b_mean.as<float>());
        const int u9[6] = {0, 1, 2, 4, 5, 8};
        const int u6[6] = {0, 1, 2, 3, 4, 5};
        transpose(s->cov3d, s->cov3d_stride, s->cov3d_stride == 9 ? u9 : u6, 6, b_cov.as<float>());
        // colour records stay per Gaussian (only visible ones are read)
        if (n > 0)
            HIPCHK(hipMemcpyAsync(b_col.p, s->colors, (size_t)n * col_planes * 4,
                                  hipMemcpyHostToDevice, st));
        has_opac = s->opacities != nullptr;
        h_opac.assign(has_opac ? (size_t)n : 0, 0.0f);
        if (has_opac && n > 0) {
            std::memcpy(h_opac.data(), s->opacities, (size_t)n * 4);
            HIPCHK(hipMemcpyAsync(b_opac.p, s->opacities, (size_t)n * 4, hipMemcpyHostToDevice, st));
        }
        sync();
        sd = gs::SceneDev{};
        sd.n = n;
        sd.sh_degree = s->sh_degree;
        for (int c = 0; c < 3; ++c) sd.mean[c] = b_mean.as<float>() + (size_t)c * n;
        for (int c = 0; c < 6; ++c) sd.cov[c] = b_cov.as<float>() + (size_t)c * n;
        sd.opac = has_opac ? b_opac.as<float>() : nullptr;
        sd.sh = b_col.as<float>();
        sd.kfac = b_terms.as<float>();
        sd.m2thr = b_terms.as<float>() + (size_t)n;
        sd.lthr = b_terms.as<float>() + 2 * (size_t)n;
        skey.means = s->means;
        skey.cov = s->cov3d;
        skey.opac = s->opacities;
        skey.col = s->colors;
        skey.n = n;
        skey.stride = s->cov3d_stride;
        skey.deg = s->sh_degree;
        skey.ver = s->version;
        skey.valid = true;
        ++scene_gen;
        tkey.valid = false;
        if (chunk_on) build_chunk_boxes();
    }

    // Chunk frustum skip (render/host/chunk_cull.h, GSPLAT_TT_CHUNK_CULL): boxes
    // per projection partition, built once per scene; each frame flags the
    // partitions that cannot reach the image and the projection skips them. The
    // frame is unchanged by it; it pays off on spatially ordered scenes (Morton
    // order), whose partitions are compact.
    bool chunk_on = false;
    double chunk_k = 1.5;
    DevBuf b_chunk_box, b_skip;
    void build_chunk_boxes() {
        sd.chunk_box = nullptr;
        sd.chunk_k = chunk_k;
        if (!chunk_on || !skey.valid || sd.n <= 0) return;
        b_chunk_box.ensure(gs::chunk_box_doubles(sd.n) * 8);
        HIPCHK(gs::launch_chunk_boxes(sd, chunk_k, b_chunk_box.as<double>(), st));
        sync();
        sd.chunk_box = b_chunk_box.as<double>();
    }
    void set_chunk_cull(bool on, double k) {
        REQUIRE(std::isfinite(k) && k >= 0.0, "chunk cull: k must be finite and >= 0");
        drain_spec();
        chunk_on = on;
        chunk_k = k > 0.0 ? k : 1.5;
        build_chunk_boxes();
    }

    void ensure_terms(const gs_view* v) {
        REQUIRE(skey.valid, "no scene set");
        if (tkey.valid && tkey.gen == scene_gen && tkey.cf == v->contrib_floor &&
            tkey.mbf == v->mb_contrib_floor && tkey.kcap == v->k_cap && tkey.has_opac == has_opac)
            return;
        const int64_t n = sd.n;
        std::vector<float> h(std::max<int64_t>(n, 1) * 3);
        opacity_terms(has_opac ? h_opac.data() : nullptr, n, has_opac, v->contrib_floor,
                      v->mb_contrib_floor, v->k_cap, h.data(), h.data() + n, h.data() + 2 * n);
        sync();
        if (n > 0)
            HIPCHK(hipMemcpyAsync(b_terms.p, h.data(), (size_t)n * 3 * 4, hipMemcpyHostToDevice, st));
        sync();
        tkey = {v->contrib_floor, v->mb_contrib_floor, v->k_cap, has_opac, scene_gen, true};
    }

    // --------------------------------------------------------- helpers
    void check_view(const gs_view* v) {
        REQUIRE(v != nullptr, "view: null");
        REQUIRE(v->image_height > 0 && v->image_width > 0, "view: image size must be positive");
        REQUIRE((int64_t)v->image_height * v->image_width <= ((int64_t)1 << 28),
                "view: image too large");
        REQUIRE(v->tile_size == 16 || v->tile_size == 32, "view: tile_size must be 16 or 32");
        REQUIRE((v->image_width + v->tile_size - 1) / v->tile_size <= 65535 &&
                    (v->image_height + v->tile_size - 1) / v->tile_size <= 65535,
                "view: at most 65535 tiles per row and per column");
        REQUIRE(v->out_format >= GS_OUT_U8 && v->out_format <= GS_OUT_F32, "view: bad out_format");
        REQUIRE(v->contrib_floor > 0.0f && v->mb_contrib_floor > 0.0f, "view: floors must be > 0");
    }

    gs::ProjParams proj_params(const gs_view* v) {
        const float* e = v->extrinsics;
        const float* K = v->intrinsics;
        gs::ProjParams p{};
        const int ri[9] = {0, 1, 2, 4, 5, 6, 8, 9, 10};
        for (int j = 0; j < 9; ++j) p.r[j] = e[ri[j]];
        p.t[0] = e[3];
        p.t[1] = e[7];
        p.t[2] = e[11];
        p.fx = K[0];
        p.fy = K[4];
        p.cx = K[2];
        p.cy = K[5];
        p.ccx = -(e[0] * p.t[0] + e[4] * p.t[1] + e[8] * p.t[2]);
        p.ccy = -(e[1] * p.t[0] + e[5] * p.t[1] + e[9] * p.t[2]);
        p.ccz = -(e[2] * p.t[0] + e[6] * p.t[1] + e[10] * p.t[2]);
        const int H = v->image_height, W = v->image_width;
        const int mr = (v->max_radius < 0) ? INT_MAX
                       : (v->max_radius > 0 ? v->max_radius : std::min(H, W) / 2);
        p.max_radius = (float)mr;
        p.min_opacity = v->min_opacity;
        p.height = H;
        p.width = W;
        p.use_iso = v->use_isoellipse ? 1 : 0;
        p.has_opac = has_opac ? 1 : 0;
        p.sh_clamp_hi = v->sh_clamp_hi ? 1 : 0;
        return p;
    }

    void ensure_counters() {
        b_cnt.ensure(64 * 4);
        if (!h_pin) HIPCHK(hipHostMalloc((void**)&h_pin, (gs::sort_hist_words() + 64) * 4));
    }

    void ensure_sort(int64_t n, int key_bytes) {
        b_kalt.ensure(std::max<int64_t>(n, 1) * key_bytes);
        b_valt.ensure(std::max<int64_t>(n, 1) * 4);
        b_hist.ensure(gs::sort_hist_words() * 4);
        const size_t sb = gs::sort_state_bytes(std::max<int64_t>(n, 1));
        if (b_state.cap < sb) {
            b_state.ensure(sb);
            HIPCHK(hipMemsetAsync(b_state.p, 0, b_state.cap, st));
            sort.epoch = 0;
            sort.dirty[0] = sort.dirty[1] = 0u;
            sort.clean[0] = sort.clean[1] = 0u;
            sort.half = 0;
        }
        sort.state_parts = b_state.cap / (256 * sizeof(uint64_t));
        sort.keys_alt = b_kalt.p;
        sort.vals_alt = b_valt.as<uint32_t>();
        sort.hist = b_hist.as<uint32_t>();
        sort.state = b_state.as<uint64_t>();
        if (timing) {
            for (auto& e : sort_ev)
                if (!e) HIPCHK(hipEventCreate(&e));
            sort.pass_events = sort_ev;
            sort.max_timed_passes = 8;
        } else {
            sort.pass_events = nullptr;
            sort.max_timed_passes = 0;
        }
    }

    void record(int i) {
        if (!timing) return;
        if (!ev[i]) HIPCHK(hipEventCreate(&ev[i]));
        HIPCHK(hipEventRecord(ev[i], st));
    }
    float elapsed(int a, int b) {
        if (!timing) return 0.0f;
        float ms = 0.0f;
        HIPCHK(hipEventElapsedTime(&ms, ev[a], ev[b]));
        return ms;
    }

    // Project + compaction. Returns M; compact arrays in b_rc/b_dkey/b_brec.
    int64_t run_project(const gs_view* v, bool want_valid, bool want_src) {
        const int64_t n = sd.n;
        ensure_counters();
        b_rc.ensure(std::max<int64_t>(n, 1) * 32);
        b_dkey.ensure(std::max<int64_t>(n, 1) * 4);
        b_brec.ensure(std::max<int64_t>(n, 1) * 48);
        if (want_src) b_src.ensure(std::max<int64_t>(n, 1) * 4);
        if (want_valid) b_valid.ensure(std::max<int64_t>(n, 1));
        const size_t parts = gs::project_partitions(std::max<int64_t>(n, 1));
        b_lb.ensure(parts * 8);
        HIPCHK(gs::launch_fill_u32(b_cnt.as<uint32_t>(), 0u, 64, st));
        HIPCHK(gs::launch_fill_u32(b_lb.as<uint32_t>(), 0u, parts * 2, st));
        if (n == 0) return 0;
        uint32_t* ctl = b_cnt.as<uint32_t>() + C_CTL;
        if (spin_limit) ctl_reset(ctl);
        gs::ProjParams p = proj_params(v);
        p.ctl = ctl;
        gs::Compact c{b_rc.as<float4>(), b_dkey.as<uint32_t>(),
                      b_brec.as<float4>(), want_src ? b_src.as<uint32_t>() : nullptr};
        HIPCHK(gs::launch_project(sd, p, c, want_valid ? b_valid.as<uint8_t>() : nullptr,
                                  b_lb.as<uint64_t>(), b_cnt.as<uint32_t>() + 0,
                                  b_cnt.as<uint32_t>() + 1, nullptr, st));
        HIPCHK(hipMemcpyAsync(h_pin, b_cnt.p, 64 * 4, hipMemcpyDeviceToHost, st));
        sync();
        ctl_check(h_pin[C_CTL], "project");
        return h_pin[1];
    }

    // Candidate count scan + pair emission (+ per-pair cull) over `order`
    // (nullptr = identity). Returns P; pairs in b_pair_tile / b_pair_id.
    uint32_t run_tile_assign(const float4* rect, const float4* cov, const uint32_t* order,
                             int64_t m, const gs::TileParams& tp, uint64_t* p_pre_out) {
        ensure_counters();
        b_offs.ensure(std::max<int64_t>(m, 1) * 4);
        const size_t rparts = gs::rect_scan_partitions(std::max<int64_t>(m, 1));
        b_lb.ensure(rparts * 8);
        if (b_bstart.cap < 4096 * 4) b_bstart.ensure(4096 * 4);
        uint32_t p_pre = 0;
        uint32_t* ctl = b_cnt.as<uint32_t>() + C_CTL;
        gs::TileParams tpc = tp;
        tpc.ctl = ctl;
        ctl_reset(ctl);
        for (int attempt = 0; attempt < 2; ++attempt) {
            HIPCHK(gs::launch_fill_u32(b_cnt.as<uint32_t>() + 8, 0u, 8, st));
            HIPCHK(gs::launch_fill_u32(b_lb.as<uint32_t>(), 0u, rparts * 2, st));
            HIPCHK(gs::launch_rect_count_scan(rect, 1, order, m, nullptr, tpc,
                                              b_offs.as<uint32_t>(), b_bstart.as<uint32_t>(),
                                              (uint32_t)(b_bstart.cap / 4), b_lb.as<uint64_t>(),
                                              b_cnt.as<uint32_t>() + 8, b_cnt.as<uint32_t>() + 9,
                                              0u, false, st));
            HIPCHK(hipMemcpyAsync(h_pin, b_cnt.p, 64 * 4, hipMemcpyDeviceToHost, st));
            sync();
            ctl_check(h_pin[C_CTL], "tile_assign");
            p_pre = h_pin[9];
            if (p_pre == 0xFFFFFFFFu)
                throw GsError(GS_E_CAPACITY, "tile_assign: more than 2^32-1 candidate pairs");
            const size_t need = gs::emit_partitions(p_pre) + 1;
            if (need * 4 <= b_bstart.cap) break;
            b_bstart.ensure(need * 4);  // partition table too small: grow, count again
        }
        *p_pre_out = p_pre;
        if (p_pre == 0) return 0;
        b_pair_tile.ensure((size_t)p_pre * 4);
        b_pair_id.ensure((size_t)p_pre * 4);
        const size_t eparts = gs::emit_partitions(p_pre);
        b_lb.ensure(eparts * 8);
        HIPCHK(gs::launch_fill_u32(b_lb.as<uint32_t>(), 0u, eparts * 2, st));
        HIPCHK(gs::launch_pair_emit(rect, cov, 1, false, order, b_offs.as<uint32_t>(),
                                    b_bstart.as<uint32_t>(), m, nullptr, p_pre, nullptr, tpc,
                                    b_pair_tile.as<uint32_t>(), b_pair_id.as<uint32_t>(), p_pre,
                                    b_lb.as<uint64_t>(), b_cnt.as<uint32_t>() + 10,
                                    b_cnt.as<uint32_t>() + 11, nullptr,
                                    tile_bits((int64_t)tp.tiles_x * tp.tiles_y), true, st));
        HIPCHK(hipMemcpyAsync(h_pin, b_cnt.p, 64 * 4, hipMemcpyDeviceToHost, st));
        sync();
        ctl_check(h_pin[C_CTL], "tile_assign");
        return h_pin[11];
    }

    // --------------------------------------------------------- render
    // Frame-scratch layout (u32 words): counters, histograms, look-back states.
    static constexpr size_t kFrCnt = 0;         // 64 counters (below)
    static constexpr size_t kFrDepthHist = 64;  // [4][256] depth-key digits
    static constexpr size_t kFrTileHist = 64 + 1024;  // [2 or 4][256] tile-id digits
    static constexpr size_t kFrLb = 64 + 1024 + 1024;  // look-back states (u64 each)
    enum : int {
        C_PROJ_TICKET = 0, C_M = 1, C_SKIPPED = 2, C_CTL = 4, C_RECT_TICKET = 8, C_PPRE = 9,
        C_EMIT_TICKET = 10, C_P = 11, C_DSORT_TICKETS = 16, C_TSORT_TICKETS = 24,
        C_MBSTAT = 40  // two u64: pairs no microblock keeps, kept (pair, microblock)
    };
    uint64_t pair_cap = 0;  // candidate-pair capacity of the frame buffers
    DevBuf b_frame, b_phist_proj, b_phist_emit;
    DevBuf b_pchunk, b_poffs;  // tile sort's first pass: emit row chunk sums, offsets
    static constexpr size_t kEmitPerSort = gs::kSortPartition32 / gs::kEmitPartition;
    static_assert(gs::kSortPartition32 % gs::kEmitPartition == 0,
                  "a sort partition is whole emit partitions");

    // One frame with no host synchronisation until the end: every size that
    // only the device knows (visible count, candidate and kept pairs) is read
    // by the kernels from the counters; grids are sized for capacities (the
    // scene size, the pair capacity) and partitions beyond the real count exit
    // at once. If the candidates overflow the pair capacity the frame is run
    // again with a larger one. render_begin enqueues the frame and returns;
    // render_end waits for it (and re-runs it after an overflow).
    struct Pending {
        bool active = false, empty = false;
        gs_view v{};
        void* out = nullptr;
        void* dout = nullptr;
        bool out_dev = false;
        size_t bytes = 0;
        int64_t T = 0;
        int tiles_x = 0, tiles_y = 0, attempt = 0;
        int floor_retries = 0;     // re-renders at a coarser contribution floor
        gs_view asked{};           // the view as the caller gave it
        int64_t batch_index = -1;  // index in the gs_render_batch call (-1: another call)
        bool replayed = false;     // the last attempt replayed a captured graph
        gs_stats* stats = nullptr;
        std::chrono::steady_clock::time_point t0;
    } pend;
    // further frame slots (peer contexts sharing the scene): slot 0 is this one
    std::vector<gs_ctx*> peers;
    // slots of gs_render_batch: four streams, one per hardware queue of the
    // process (orbit 964 frames/s with two, 1027 with three, 1047 with four,
    // 981 with five, whose streams share queues)
    static constexpr int kFramesInFlight = 4;

    void render(const gs_view* v, void* out, bool out_dev, gs_stats* stats) {
        drain_spec();
        render_begin(v, out, out_dev, stats, false);
        render_end();
    }

    // shared_terms: the opacity terms of the scene descriptor are another
    // context's (the batch's first slot computed them for this view's floors).
    void render_begin(const gs_view* v, void* out, bool out_dev, gs_stats* stats,
                      bool shared_terms) {
        if (pend.active) {  // an earlier frame that was never completed
            sync();
            pend.active = false;
        }
        pend = Pending{};
        pend.t0 = std::chrono::steady_clock::now();
        tr.fwd_valid = false;  // the frame buffers are about to be reused
        rb_valid = false;
        check_view(v);
        pend.asked = *v;
        REQUIRE(out != nullptr, "render: null output");
        if (!shared_terms) ensure_terms(v);
        if (timing)
            for (auto& e : ev)
                if (!e) HIPCHK(hipEventCreate(&e));
        const int H = v->image_height, W = v->image_width, ts = v->tile_size;
        pend.v = *v;
        pend.tiles_x = (W + ts - 1) / ts;
        pend.tiles_y = (H + ts - 1) / ts;
        pend.T = (int64_t)pend.tiles_x * pend.tiles_y;
        const size_t px = (size_t)H * W * 3;
        const size_t ebytes = v->out_format == GS_OUT_F32 ? 4 : (v->out_format == GS_OUT_BF16 ? 2 : 1);
        pend.bytes = px * ebytes;
        pend.out = out;
        pend.out_dev = out_dev;
        pend.dout = out;
        if (!out_dev) {
            b_out.ensure(pend.bytes);
            pend.dout = b_out.p;
        }
        pend.stats = stats;
        pend.active = true;
        ensure_counters();
        if (sd.n == 0) {
            pend.empty = true;
            HIPCHK(gs::launch_fill_u32(static_cast<uint32_t*>(pend.dout), 0u, pend.bytes / 4, st));
            if (pend.bytes % 4)
                HIPCHK(hipMemsetAsync(static_cast<char*>(pend.dout) + pend.bytes / 4 * 4, 0,
                                      pend.bytes % 4, st));
            if (!out_dev) HIPCHK(hipMemcpyAsync(out, pend.dout, pend.bytes, hipMemcpyDeviceToHost, st));
            return;
        }
        if (pair_cap == 0) pair_cap = std::min<uint64_t>(default_pair_cap(sd.n), pair_limit);
        enqueue_attempt();
    }

    void enqueue_attempt() {
        pend.replayed = false;
        if (!graph_frame()) frame(&pend.v, pend.dout, pend.T, pend.tiles_x, pend.tiles_y);
        if (!pend.out_dev)
            HIPCHK(hipMemcpyAsync(pend.out, pend.dout, pend.bytes, hipMemcpyDeviceToHost, st));
        HIPCHK(hipMemcpyAsync(h_pin, b_frame.p, 64 * 4, hipMemcpyDeviceToHost, st));
        if (blend_counts)
            HIPCHK(hipMemcpyAsync(h_evals.data(), b_evals.p, 64 * 8 * 8, hipMemcpyDeviceToHost, st));
    }

    void render_end() {
        REQUIRE(pend.active, "render: no frame in flight");
        try {
            settle_attempts();
        } catch (...) {
            // no frame stays pending (a re-run that an error interrupted is
            // waited for), and the caller's floor's terms are back
            abandon_frame();
            restore_terms();
            throw;
        }
        finish_frame();
    }

    // Waits for the frame, re-running it while its candidate pairs do not fit:
    // with a grown pair buffer up to the pair limit, past it at a coarser floor.
    void settle_attempts() {
        for (;;) {
            sync();
            if (pend.empty) break;
            // candidates of the last attempt (0xFFFFFFFF: more than 2^32-2)
            const uint32_t p_pre = h_pin[C_PPRE];
            if (p_pre != 0xFFFFFFFFu && p_pre <= pair_cap) break;
            if (pend.attempt > 2 * kFloorRetries + 2)
                throw GsError(GS_E_INVALID, "render: pair capacity did not converge");
            ++pend.attempt;
            if (p_pre != 0xFFFFFFFFu && p_pre <= pair_limit) {
                // the same frame again with room for its pairs
                pair_cap = std::min<uint64_t>(pair_limit, (uint64_t)p_pre + p_pre / 8 + 4096);
                enqueue_attempt();
                continue;
            }
            // more candidates than the limit: the whole frame again at a
            // coarser floor (render/host/render.cpp:537-565)
            const float f = std::max(pend.v.contrib_floor, pend.v.mb_contrib_floor);
            if (pend.v.cull_disabled || pend.floor_retries >= kFloorRetries || !(f < kFloorMax))
                throw GsError(GS_E_CAPACITY,
                              p_pre == 0xFFFFFFFFu
                                  ? "render: more than 2^32-1 candidate pairs"
                                  : "render: more candidate pairs than the pair limit");
            const float next = next_contrib_floor(f, p_pre, pair_limit);
            pend.v.contrib_floor = next;
            pend.v.mb_contrib_floor = next;
            ++pend.floor_retries;
            // every slot reads the one set of opacity terms: none may be running
            gs_ctx* o = owner ? owner : this;
            o->sync_slots();
            o->ensure_terms(&pend.v);
            enqueue_attempt();
        }
    }

    // The frame's statistics and readback state, once its last attempt fit.
    void finish_frame() {
        gs_stats s{};
        restore_terms();
        pend.active = false;
        s.pairs_dropped_mb = -1;
        s.pairs_kept_mb = -1;
        if (!pend.empty) {
            ctl_check(h_pin[C_CTL], "render");
            s.num_visible = h_pin[C_M];
            s.pairs_pre = h_pin[C_PPRE];
            s.num_entries = h_pin[C_P];
            s.chunks_skipped = h_pin[C_SKIPPED];
            if (cull_stats) {
                uint64_t mb[2];
                std::memcpy(mb, h_pin + C_MBSTAT, sizeof(mb));
                s.pairs_dropped_mb = (int64_t)mb[0];
                s.pairs_kept_mb = (int64_t)mb[1];
            }
            if (timing) {
                s.ms_project = elapsed(0, 1);
                s.ms_depth_sort = elapsed(1, 2);
                s.ms_tile_assign = elapsed(2, 3);
                s.ms_tile_sort = elapsed(3, 4);
                s.ms_blend = elapsed(4, 5);
            }
            if (blend_counts) blend_diag(s);
        }
        s.ms_total = std::chrono::duration<float, std::milli>(std::chrono::steady_clock::now() -
                                                               pend.t0).count();
        rb_valid = true;
        rb_empty = pend.empty;
        rb_T = pend.T;
        rb_batch = pend.batch_index;
        rb_replayed = pend.replayed;
        rb_M = pend.empty ? 0 : (int64_t)h_pin[C_M];
        rb_ppre = pend.empty ? 0 : (int64_t)h_pin[C_PPRE];
        rb_P = pend.empty ? 0 : (int64_t)h_pin[C_P];
        if (pend.empty) {
            s.pairs_dropped_mb = cull_stats ? 0 : -1;
            s.pairs_kept_mb = cull_stats ? 0 : -1;
        }
        s.contrib_floor = pend.v.contrib_floor;
        s.floor_retries = pend.floor_retries;
        if (pend.stats) *pend.stats = s;
    }

    // After a frame rendered at a coarser floor: the opacity terms of the floor
    // the caller asked for (later frames, and the other slots, expect them).
    void restore_terms() {
        if (pend.floor_retries == 0) return;
        gs_ctx* o = owner ? owner : this;
        o->sync_slots();
        o->ensure_terms(&pend.asked);
    }
    void sync_slots() {
        sync();
        for (gs_ctx* p : peers) p->sync();
    }

    // Frame slots 1..count-1: each its own stream and frame buffers, with this
    // context's scene planes and opacity terms (refreshed at every use).
    void ensure_peers(int count) {
        while ((int)peers.size() < count - 1) {
            auto* p = new gs_ctx();
            p->device = device;
            p->num_cus = num_cus;
            hipError_t e = hipStreamCreateWithFlags(&p->st, hipStreamNonBlocking);
            if (e != hipSuccess) {
                delete p;
                throw GsError(GS_E_DEVICE, std::string("hipStreamCreate: ") + hipGetErrorString(e));
            }
            peers.push_back(p);
        }
        for (gs_ctx* p : peers) {
            p->timing = timing;
            p->blend_counts = blend_counts;
            p->spin_limit = spin_limit;
            p->pair_limit = pair_limit;
            p->owner = this;
            p->cull_stats = cull_stats;
            p->graphs = graphs;
            p->sd = sd;
            p->has_opac = has_opac;
            p->skey.valid = true;
            p->pair_cap = std::max(p->pair_cap, pair_cap);
        }
    }
    gs_ctx* slot(int k) { return k == 0 ? this : peers[k - 1]; }

    // Cross-view pipelining for render_view(..., next_extrinsics): the next
    // view's whole frame is enqueued on the other slot, into that slot's own
    // output buffer, before the current view is waited for; the next call
    // takes it when its view equals the announced one and the scene is the
    // same (render/host/render.cpp:316-322, 439-492). Any other entry point
    // first completes and drops such a frame (drain_spec).
    gs_ctx* spec_slot = nullptr;  // the slot holding the announced frame
    gs_view spec_view{};
    uint64_t spec_gen = 0;
    DevBuf b_spec;                // output of an announced frame (per slot)
    gs_stats spec_st{};
    // An announced frame of render_out_ring writes its image by DMA straight
    // into a ring buffer leased for it when it is enqueued (no copy when the
    // next call takes it; the lease passes to the caller then, and is released
    // when the frame is dropped instead).
    gs::PinnedImage* spec_im = nullptr;
    uint64_t spec_lease = 0;

    // Zero-copy output (render/host/out_ring.h, render.cpp:598-612): the frame's
    // image is copied by DMA into a pinned buffer of the ring and handed over
    // with a lease; the ring never rewrites a held buffer.
    std::unique_ptr<gs::OutRing> ring;
    size_t ring_cap = 4;
    static void* pinned_alloc(size_t bytes) {
        void* p = nullptr;
        return hipHostMalloc(&p, bytes) == hipSuccess ? p : nullptr;
    }
    static void pinned_free(void* p) { (void)hipHostFree(p); }

    static size_t view_pitch(const gs_view* v) {
        const size_t eb = v->out_format == GS_OUT_F32 ? 4 : (v->out_format == GS_OUT_BF16 ? 2 : 1);
        return (size_t)v->image_width * 3 * eb;
    }

    // A ring image of `bytes`, leased at once so that no other acquire hands
    // it out while a frame writes it.
    gs::PinnedImage* ring_take(size_t bytes, uint64_t* lease) {
        gs::PinnedImage* im = nullptr;
        try {
            im = ring->acquire(bytes);
        } catch (const std::bad_alloc&) {
            throw GsError(GS_E_DEVICE, "render_out_ring: pinned host allocation failed");
        }
        *lease = gs::LeaseTable::get().lease(im);
        return im;
    }

    // render_next into the output ring: the view's image is a ring buffer
    // filled by DMA, and the announced next view's frame writes into a ring
    // buffer of its own, so a call that takes the announced frame only waits
    // for it (its image is already in host memory).
    void render_out_ring(const gs_view* v, const gs_view* next, gs_out_image* img,
                         gs_stats* stats) {
        REQUIRE(img != nullptr, "render_out_ring: null image");
        check_view(v);
        if (next) check_view(next);
        if (!ring) ring.reset(new gs::OutRing(pinned_alloc, pinned_free, ring_cap));
        const size_t pitch = view_pitch(v);
        const size_t bytes = pitch * v->image_height;
        ensure_peers(2);
        gs_ctx* peer = peers[0];
        const bool hit = spec_slot != nullptr && spec_im != nullptr && spec_gen == scene_gen &&
                         std::memcmp(&spec_view, v, sizeof(gs_view)) == 0;
        gs_ctx* cur;
        gs::PinnedImage* im;
        uint64_t lease = 0;
        if (hit) {
            cur = spec_slot;  // this view's frame is already in flight there
            im = spec_im;
            lease = spec_lease;
            spec_slot = nullptr;
            spec_im = nullptr;
            spec_lease = 0;
        } else {
            drain_spec();
            cur = this;
            im = ring_take(bytes, &lease);
            try {
                cur->render_begin(v, im->p, false, stats, false);
            } catch (...) {
                cur->abandon_frame();
                gs::LeaseTable::get().release(lease);
                throw;
            }
            peer->sd = sd;  // terms for v's floors
        }
        try {
            // announce the next view on the other slot (same floors: shared terms)
            if (next != nullptr && next->contrib_floor == v->contrib_floor &&
                next->mb_contrib_floor == v->mb_contrib_floor && next->k_cap == v->k_cap) {
                gs_ctx* other = cur == this ? peer : this;
                uint64_t nl = 0;
                gs::PinnedImage* nim = ring_take(view_pitch(next) * next->image_height, &nl);
                try {
                    other->render_begin(next, nim->p, false, &other->spec_st, true);
                } catch (...) {
                    other->abandon_frame();
                    gs::LeaseTable::get().release(nl);
                    throw;
                }
                spec_slot = other;
                spec_view = *next;
                spec_gen = scene_gen;
                spec_im = nim;
                spec_lease = nl;
            }
            cur->render_end();
        } catch (...) {
            cur->abandon_frame();  // the view's frame is dropped with its image
            gs::LeaseTable::get().release(lease);
            throw;
        }
        if (hit && stats) *stats = cur->spec_st;
        img->data = im->p;
        img->bytes = (int64_t)bytes;
        img->pitch = (int64_t)pitch;
        img->lease = lease;
    }

    void drain_spec() {
        if (spec_slot == nullptr) return;
        gs_ctx* s = spec_slot;
        const uint64_t lease = spec_lease;
        spec_slot = nullptr;
        spec_im = nullptr;
        spec_lease = 0;
        try {
            s->render_end();
        } catch (...) {
            if (lease) gs::LeaseTable::get().release(lease);
            throw;
        }
        if (lease) gs::LeaseTable::get().release(lease);
    }

    void render_next(const gs_view* v, void* out, bool out_dev, const gs_view* next,
                     gs_stats* stats) {
        check_view(v);
        REQUIRE(out != nullptr, "render: null output");
        if (next) check_view(next);
        ensure_peers(2);
        gs_ctx* peer = peers[0];
        gs_ctx* cur;
        // (a frame announced by render_out_ring writes into its ring image,
        // not b_spec: it is dropped like any other miss)
        const bool hit = spec_slot != nullptr && spec_im == nullptr && spec_gen == scene_gen &&
                         std::memcmp(&spec_view, v, sizeof(gs_view)) == 0;
        if (hit) {
            cur = spec_slot;  // this view's frame is already in flight there
            spec_slot = nullptr;
        } else {
            drain_spec();
            cur = this;
            cur->render_begin(v, out, out_dev, stats, false);
            peer->sd = sd;  // terms for v's floors
        }
        // announce the next view on the other slot (same floors: shared terms)
        if (next != nullptr && next->contrib_floor == v->contrib_floor &&
            next->mb_contrib_floor == v->mb_contrib_floor && next->k_cap == v->k_cap) {
            gs_ctx* other = cur == this ? peer : this;
            const size_t eb = next->out_format == GS_OUT_F32 ? 4 : (next->out_format == GS_OUT_BF16 ? 2 : 1);
            other->b_spec.ensure((size_t)next->image_height * next->image_width * 3 * eb);
            other->render_begin(next, other->b_spec.p, true, &other->spec_st, true);
            spec_slot = other;
            spec_view = *next;
            spec_gen = scene_gen;
        }
        cur->render_end();
        if (hit) {
            const size_t eb = v->out_format == GS_OUT_F32 ? 4 : (v->out_format == GS_OUT_BF16 ? 2 : 1);
            const size_t bytes = (size_t)v->image_height * v->image_width * 3 * eb;
            HIPCHK(hipMemcpyAsync(out, cur->b_spec.p, bytes,
                                  out_dev ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, cur->st));
            cur->sync();
            if (stats) *stats = cur->spec_st;
        }
    }

    // Renders views[0..n) keeping kFramesInFlight frames in flight, one per
    // slot (this context and its peers, which share the scene and have their
    // own streams and frame buffers): frame i+1.. are enqueued before frame i
    // is waited for, so one frame's memory-bound stages run beside another's
    // VALU-bound blend.
    void render_batch(const gs_view* views, int n, void* const* outs, bool out_dev,
                      gs_stats* stats) {
        REQUIRE(views != nullptr && outs != nullptr && n >= 0, "render_batch: bad arguments");
        drain_spec();
        if (n == 0) return;
        for (int i = 0; i < n; ++i) {
            check_view(&views[i]);
            REQUIRE(views[i].contrib_floor == views[0].contrib_floor &&
                        views[i].mb_contrib_floor == views[0].mb_contrib_floor &&
                        views[i].k_cap == views[0].k_cap,
                    "render_batch: every view must share the floors and k_cap");
        }
        ensure_terms(&views[0]);
        const int S = std::min(n, kFramesInFlight);
        ensure_peers(S);
        try {
            for (int i = 0; i < n; ++i) {
                gs_ctx* c = slot(i % S);
                if (i >= S) c->render_end();  // frame i-S used this slot
                c->batch_frame = true;
                try {
                    c->render_begin(&views[i], outs[i], out_dev, stats ? &stats[i] : nullptr,
                                    true);
                } catch (...) {
                    c->batch_frame = false;
                    throw;
                }
                c->batch_frame = false;
                c->pend.batch_index = i;
            }
            for (int i = std::max(0, n - S); i < n; ++i) slot(i % S)->render_end();
        } catch (...) {
            // the other frames still in flight write into the caller's
            // outputs: they are finished before the error returns
            for (int k = 0; k < S; ++k) slot(k)->abandon_frame();
            throw;
        }
    }

    // Enqueues one frame (project -> depth sort -> tile assign -> tile sort ->
    // ranges -> blend) on the stream; no host synchronisation.
    // Frame buffers for N Gaussians, T tiles and the current pair capacity, all
    // allocated before the first launch of a frame.
    struct FrameLayout {
        uint32_t* fr;
        uint32_t* cnt;
        uint64_t *lb_proj, *lb_rect, *lb_emit;
        uint32_t* tcnt;  // pairs per tile (the tile sort's last pass counts them)
        size_t fwords, pparts, rparts, eparts;
        uint32_t pcap;
    };
    FrameLayout frame_prepare(int64_t N, int64_t T) {
        FrameLayout L{};
        L.pcap = (uint32_t)pair_cap;
        L.pparts = gs::project_partitions(N);
        L.rparts = gs::rect_scan_partitions(N);
        L.eparts = gs::emit_partitions(L.pcap);
        b_rc.ensure((size_t)N * 32);
        b_dkey.ensure((size_t)N * 4);
        b_brec.ensure((size_t)N * 48);
        b_src.ensure((size_t)N * 4);
        b_tmp_a.ensure((size_t)N * 4);
        b_offs.ensure((size_t)N * 4);
        b_bstart.ensure((L.eparts + 1) * 4);
        b_pair_tile.ensure((size_t)L.pcap * 4);
        b_pair_id.ensure((size_t)L.pcap * 4);
        b_ranges.ensure((size_t)T * 8);
        b_phist_proj.ensure(L.pparts * 1024 * 4);
        b_phist_emit.ensure(L.eparts * gs::tile_hist_cols(tile_bits(T)) * 4);
        b_pchunk.ensure(gs::reduce_chunks((uint32_t)L.eparts) * gs::tile_hist_cols(tile_bits(T)) *
                        4);
        b_poffs.ensure(((L.eparts + kEmitPerSort - 1) / kEmitPerSort)
                       << gs::sort_digit_width(tile_bits(T))
                       << 2);
        const size_t lb_words = 2 * (L.pparts + L.rparts + L.eparts);
        L.fwords = kFrLb + lb_words + (size_t)T;
        b_frame.ensure(L.fwords * 4);
        ensure_sort(std::max<int64_t>(N, L.pcap), 4);
        if (blend_counts) b_evals.ensure(64 * 8 * 8);
        L.fr = b_frame.as<uint32_t>();
        L.lb_proj = reinterpret_cast<uint64_t*>(L.fr + kFrLb);
        L.lb_rect = L.lb_proj + L.pparts;
        L.lb_emit = L.lb_rect + L.rparts;
        L.tcnt = L.fr + kFrLb + lb_words;
        L.cnt = L.fr + kFrCnt;
        return L;
    }

    // From the compact records of the M visible Gaussians (count on the device at
    // cnt[C_M], depth-key histograms reduced) to the tile-sorted compact ids and
    // tile ranges: depth sort, candidate scan, pair emission + cull, tile sort,
    // tile bounds. Returns the sorted compact ids.
    uint32_t* frame_tiles(const FrameLayout& L, int64_t N, int64_t T, const gs::TileParams& tp,
                          uint32_t** tiles_out) {
        // without a caller for the tile-sorted keys, the tile sort's last pass
        // counts the pairs per tile instead of writing them, and the ranges come
        // from the counts
        const bool want_keys = tiles_out != nullptr;
        uint32_t* fr = L.fr;
        uint32_t* cnt = L.cnt;
        sort.ctl = cnt + C_CTL;
        // depth order of the visible Gaussians (stable: ties keep index order)
        // (values: the projection's packed ones when tp.idx_bits is set, else
        // the compact indices 0..M-1); the sorted depth keys are not needed, so
        // the last pass writes the values only
        void* kf = nullptr;
        uint32_t* order = nullptr;
        HIPCHK(gs::radix_sort_pairs_dev(b_dkey.p, b_tmp_a.as<uint32_t>(), N, cnt + C_M, 4, 0, 32,
                                        fr + kFrDepthHist, cnt + C_DSORT_TICKETS, sort, st,
                                        tp.idx_bits == 0, &kf, &order, nullptr, nullptr, nullptr,
                                        0xFFFFFFFFu, false));
        record(2);
        HIPCHK(gs::launch_rect_count_scan(b_rc.as<float4>(), 2, order, N, cnt + C_M, tp,
                                          b_offs.as<uint32_t>(), b_bstart.as<uint32_t>(),
                                          (uint32_t)(L.eparts + 1), L.lb_rect,
                                          cnt + C_RECT_TICKET, cnt + C_PPRE, L.pcap, true, st));
        HIPCHK(gs::launch_pair_emit(b_rc.as<float4>(), b_rc.as<float4>() + 1, 2, true, order,
                                    b_offs.as<uint32_t>(), b_bstart.as<uint32_t>(), N, cnt + C_M,
                                    L.pcap, cnt + C_PPRE, tp, b_pair_tile.as<uint32_t>(),
                                    b_pair_id.as<uint32_t>(), L.pcap, L.lb_emit,
                                    cnt + C_EMIT_TICKET, cnt + C_P, b_phist_emit.as<uint32_t>(),
                                    tile_bits(T), false, st));
        const int hcols = gs::tile_hist_cols(tile_bits(T));
        const int dw = gs::sort_digit_width(tile_bits(T));
        HIPCHK(gs::launch_reduce_rows(b_phist_emit.as<uint32_t>(), hcols, (uint32_t)L.eparts,
                                      cnt + C_PPRE, L.pcap, gs::kEmitPartition, dw,
                                      fr + kFrTileHist, st, b_pchunk.as<uint32_t>(),
                                      cnt + C_CTL));
        // the first tile pass's output positions per partition, from the emit
        // rows (four emit partitions per sort partition): no look-back
        HIPCHK(gs::launch_part_offsets(b_phist_emit.as<uint32_t>(), hcols, (uint32_t)L.eparts,
                                       cnt + C_PPRE, L.pcap, gs::kEmitPartition, kEmitPerSort,
                                       dw, b_pchunk.as<uint32_t>(), fr + kFrTileHist,
                                       b_poffs.as<uint32_t>(), st, cnt + C_CTL));
        record(3);
        // stable tile sort of the depth-ordered candidate slots; its first pass
        // drops the culled ones (kPairDrop), so the kept pairs come out compact
        void* tiles_sorted = nullptr;
        uint32_t* ids_sorted = nullptr;
        HIPCHK(gs::radix_sort_pairs_dev(b_pair_tile.p, b_pair_id.as<uint32_t>(), L.pcap,
                                        cnt + C_PPRE, 4, 0, tile_bits(T), fr + kFrTileHist,
                                        cnt + C_TSORT_TICKETS, sort, st, false, &tiles_sorted,
                                        &ids_sorted, cnt + C_P, want_keys ? nullptr : L.tcnt,
                                        b_poffs.as<uint32_t>(), (uint32_t)T));
        if (want_keys) {
            HIPCHK(gs::launch_tile_bounds(static_cast<uint32_t*>(tiles_sorted), L.pcap, cnt + C_P,
                                          b_ranges.as<uint32_t>(), T, st));
            *tiles_out = static_cast<uint32_t*>(tiles_sorted);
        } else {
            HIPCHK(gs::launch_ranges_from_counts(L.tcnt, T, b_ranges.as<uint32_t>(), st));
        }
        return ids_sorted;
    }

    // The projection's parameters for a frame of view v in layout L.
    gs::ProjParams frame_proj_params(const gs_view* v, const FrameLayout& L, int64_t N,
                                     int tiles_x, int tiles_y) {
        gs::ProjParams p = proj_params(v);
        p.ctl = L.cnt + C_CTL;
        // depth-sort values carry each Gaussian's tile count
        p.tiles_x = tiles_x;
        p.tiles_y = tiles_y;
        p.tile_size = v->tile_size;
        p.idx_bits = dval_idx_bits(N);
        p.dvals = p.idx_bits ? b_tmp_a.as<uint32_t>() : nullptr;
        return p;
    }

    // ------------------------------------------------------------ frame graphs
    // A gs_render_batch frame's kernels (everything frame() enqueues) captured
    // once per frame slot and shape and replayed for the slot's later frames of
    // that shape, with the view set on the graph's k_project node: one launch
    // instead of ~20 per frame (100K-Gaussian orbit 12.9K -> 13.4K frames/s; a
    // single frame, whose host waits for it, gains nothing and stays direct). A
    // shape is everything the captured launches depend on besides the view's
    // camera: the view's other fields, the output, the scene size and SH
    // degree, the pair capacity, the spin limit, the slot's device buffers
    // (their addresses) and the sort's look-back state — the state-
    // clearing launches of the passes are baked into the graph, so a graph is
    // kept only if the frame leaves that state as it found it (a frame's six
    // passes do from the second frame of a shape on; the first frame's capture
    // is redone from the state it leaves, so a slot replays from its second
    // frame). Frames with timing,
    // microblock statistics or the chunk skip, a capacity re-run and sorts of
    // 2^30 keys or more (epoch-tagged descriptors) are enqueued directly.
    // The sort's look-back bookkeeping (the half in use, each half's rows that
    // may hold descriptors): the clearing launches of a captured frame follow
    // from it, so a graph replays only from the bookkeeping it was captured in.
    using SortMarks = std::array<uint32_t, 5>;
    SortMarks sort_marks() const {
        return {(uint32_t)sort.half, sort.dirty[0], sort.dirty[1], sort.clean[0], sort.clean[1]};
    }
    struct FrameGraph {
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        hipGraphNode_t proj = nullptr;  // null: not replayable (the sort state moved)
        gs_view shape{};
        gs::SceneDev sd{};  // the scene's device pointers, held by the projection node
        void* dout = nullptr;
        int64_t n = -1, T = -1;
        int deg = -2;
        uint64_t pcap = 0, gen = 0;
        uint32_t spin = 0;
        SortMarks marks{};
        int misses = 0;  // captures of this shape in a row that were not replayable
    } fg;

    void drop_graph() {
        if (fg.exec) (void)hipGraphExecDestroy(fg.exec);
        if (fg.graph) (void)hipGraphDestroy(fg.graph);
        fg = FrameGraph{};
    }

    static bool same_scene(const gs::SceneDev& a, const gs::SceneDev& b) {
        return a.n == b.n && a.sh_degree == b.sh_degree && a.opac == b.opac && a.sh == b.sh &&
               a.kfac == b.kfac && a.m2thr == b.m2thr && a.lthr == b.lthr &&
               a.chunk_box == b.chunk_box && a.chunk_k == b.chunk_k &&
               std::equal(a.mean, a.mean + 3, b.mean) && std::equal(a.cov, a.cov + 6, b.cov);
    }

    static gs_view graph_shape(const gs_view* v) {
        gs_view k = *v;
        std::memset(k.extrinsics, 0, sizeof(k.extrinsics));
        std::memset(k.intrinsics, 0, sizeof(k.intrinsics));
        return k;
    }

    // The addresses of this slot's frame buffers: a captured frame graph holds
    // them and is replayed only while none moved (the scene planes and opacity
    // terms, which a slot shares with the first one, are compared through the
    // scene descriptor; another slot's allocations do not matter).
    uint64_t buffers_key() const {
        uint64_t h = 1469598103934665603ull;
        for (const DevBuf* b : {&b_rc, &b_dkey, &b_brec, &b_src, &b_tmp_a, &b_offs, &b_bstart,
                                &b_pair_tile, &b_pair_id, &b_ranges, &b_phist_proj, &b_phist_emit,
                                &b_pchunk, &b_poffs, &b_frame, &b_kalt, &b_valt, &b_hist,
                                &b_state, &b_out}) {
            h ^= (uint64_t)(uintptr_t)b->p;
            h *= 1099511628211ull;
        }
        return h;
    }

    // Enqueues pend's frame through a graph; false when it must be enqueued
    // directly (frame()).
    bool graph_frame() {
        const int64_t N = sd.n;
        if (!graphs || !batch_frame || timing || blend_counts || cull_stats || pend.attempt != 0)
            return false;
        if (sd.chunk_box != nullptr && pend.v.k_cap <= 3.0f) return false;
        if (N >= ((int64_t)1 << 30) || pair_cap >= (1ull << 30)) return false;
        const FrameLayout L = frame_prepare(N, pend.T);  // every allocation before a capture
        const gs_view shape = graph_shape(&pend.v);
        const uint64_t gen = buffers_key();
        const bool same_shape = fg.dout == pend.dout && fg.n == N && fg.T == pend.T &&
                                fg.deg == sd.sh_degree && fg.pcap == pair_cap && fg.gen == gen &&
                                fg.spin == spin_limit && same_scene(fg.sd, sd) &&
                                std::memcmp(&fg.shape, &shape, sizeof(shape)) == 0;
        // a shape whose frames never leave the sort state as they found it (an
        // odd pass count flips its half every frame: above 2^16 tiles the tile
        // sort has three passes) is enqueued directly after two such captures
        if (same_shape && fg.proj == nullptr && fg.misses >= 2) return false;
        if (fg.exec != nullptr && fg.proj != nullptr && same_shape && fg.marks == sort_marks()) {
            const gs::ProjParams p = frame_proj_params(&pend.v, L, N, pend.tiles_x, pend.tiles_y);
            HIPCHK(gs::graph_set_project_params(fg.exec, fg.proj, p));
            HIPCHK(hipGraphLaunch(fg.exec, st));
            ++graph_replays;
            pend.replayed = true;
            return true;
        }
        const int misses = same_shape && fg.proj == nullptr ? fg.misses : 0;
        drop_graph();  // the stream is idle: this slot's last frame was waited for
        FrameGraph g;
        g.misses = misses;
        g.shape = shape;
        g.sd = sd;
        g.dout = pend.dout;
        g.n = N;
        g.T = pend.T;
        g.deg = sd.sh_degree;
        g.pcap = pair_cap;
        g.gen = gen;
        g.spin = spin_limit;
        g.marks = sort_marks();
        auto capture = [&](hipGraph_t* out) {
            HIPCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            try {
                frame(&pend.v, pend.dout, pend.T, pend.tiles_x, pend.tiles_y);
            } catch (...) {
                hipGraph_t dead = nullptr;
                (void)hipStreamEndCapture(st, &dead);
                if (dead) (void)hipGraphDestroy(dead);
                throw;
            }
            HIPCHK(hipStreamEndCapture(st, out));
        };
        capture(&g.graph);
        if (sort_marks() != g.marks && buffers_key() == gen) {
            // The frame moved the sort's look-back bookkeeping (a slot's first
            // frame of a shape leaves more rows marked than it found). The
            // graph is dropped unlaunched, the whole descriptor buffer is
            // cleared directly (a clean buffer is within any marking), and the
            // frame is captured again from the moved bookkeeping, which a
            // steady shape's frames leave as they find it: the slot replays
            // from its next frame on instead of capturing twice.
            (void)hipGraphDestroy(g.graph);
            g.graph = nullptr;
            HIPCHK(gs::launch_fill_u32(b_state.as<uint32_t>(), 0u, b_state.cap / 4, st));
            g.marks = sort_marks();
            capture(&g.graph);
        }
        hipError_t e = hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(g.graph);
            HIPCHK(e);
        }
        fg = g;
        HIPCHK(hipGraphLaunch(fg.exec, st));  // this frame
        ++graph_captures;
        // replayable only from the sort state it was captured in, with the
        // buffers it captured, and with a projection node to set the view on
        ++fg.misses;  // until a projection node is found below
        if (sort_marks() == g.marks && buffers_key() == gen) {
            size_t nn = 0;
            HIPCHK(hipGraphGetNodes(fg.graph, nullptr, &nn));
            std::vector<hipGraphNode_t> nodes(nn);
            if (nn) HIPCHK(hipGraphGetNodes(fg.graph, nodes.data(), &nn));
            const void* fn = gs::project_kernel(sd.sh_degree);
            for (hipGraphNode_t node : nodes) {
                hipGraphNodeType ty;
                HIPCHK(hipGraphNodeGetType(node, &ty));
                if (ty != hipGraphNodeTypeKernel) continue;
                hipKernelNodeParams kp;
                HIPCHK(hipGraphKernelNodeGetParams(node, &kp));
                if (kp.func == fn && kp.kernelParams != nullptr) {
                    const gs::ProjParams p =
                        frame_proj_params(&pend.v, L, N, pend.tiles_x, pend.tiles_y);
                    if (gs::graph_project_args_are(node, sd, p)) {
                        fg.proj = node;
                        fg.misses = 0;
                    }
                    break;
                }
            }
        }
        return true;
    }

    // Enqueues one frame (project -> depth sort -> tile assign -> tile sort ->
    // ranges -> blend) on the stream; no host synchronisation.
    void frame(const gs_view* v, void* dout, int64_t T, int tiles_x, int tiles_y) {
        const int64_t N = sd.n;
        const FrameLayout L = frame_prepare(N, T);
        record(0);
        HIPCHK(gs::launch_fill_u32(L.fr, 0u, L.fwords, st));
        if (spin_limit) HIPCHK(gs::launch_fill_u32(L.cnt + C_CTL + 1, spin_limit, 1, st));
        if (blend_counts)
            HIPCHK(gs::launch_fill_u32(b_evals.as<uint32_t>(), 0u, 64 * 8 * 2, st));
        gs::ProjParams p = frame_proj_params(v, L, N, tiles_x, tiles_y);
        // the boxes bound three standard deviations: no skipping for wider k
        if (sd.chunk_box != nullptr && v->k_cap <= 3.0f) {
            b_skip.ensure(gs::project_partitions(N));
            HIPCHK(gs::launch_chunk_cull(sd.chunk_box, N, p, sd.chunk_k, b_skip.as<uint8_t>(),
                                         L.cnt + C_SKIPPED, st));
            p.skip = b_skip.as<uint8_t>();
        }
        gs::Compact c{b_rc.as<float4>(), b_dkey.as<uint32_t>(),
                      b_brec.as<float4>(), nullptr};
        HIPCHK(gs::launch_project(sd, p, c, nullptr, L.lb_proj, L.cnt + C_PROJ_TICKET,
                                  L.cnt + C_M, b_phist_proj.as<uint32_t>(), st));
        HIPCHK(gs::launch_reduce_rows(b_phist_proj.as<uint32_t>(), 1024, (uint32_t)L.pparts,
                                      nullptr, 0, 0, 0, L.fr + kFrDepthHist, st, nullptr,
                                      L.cnt + C_CTL));
        record(1);
        gs::TileParams tp{tiles_x, tiles_y, v->tile_size, v->cull_disabled ? 0 : 1,
                          L.cnt + C_CTL, p.idx_bits};
        uint32_t* tiles_sorted = nullptr;
        uint32_t* ids_sorted = frame_tiles(L, N, T, tp, cull_stats ? &tiles_sorted : nullptr);
        record(4);
        gs::BlendParams bp{tiles_x, tiles_y, v->tile_size, v->image_height, v->image_width,
                           v->cull_disabled ? 1 : 0, v->transmittance_threshold, v->out_format,
                           blend_counts ? b_evals.as<unsigned long long>() : nullptr,
                           L.cnt + C_CTL};
        HIPCHK(gs::launch_blend(b_brec.as<float4>(), ids_sorted, b_ranges.as<uint32_t>(), bp,
                                dout, st));
        record(5);
        if (cull_stats)
            HIPCHK(gs::launch_mb_stats(b_brec.as<float4>(), ids_sorted, tiles_sorted, L.pcap,
                                       L.cnt + C_P, tiles_x, v->tile_size, v->cull_disabled,
                                       reinterpret_cast<unsigned long long*>(L.cnt + C_MBSTAT),
                                       L.cnt + C_CTL, st));
        rb_ids = ids_sorted;
    }

    // ------------------------------------------------------------ training
    struct TrainState {
        int64_t n = 0;
        int deg = -1;
        int planes = 0;
        int64_t step = 0;
        bool ready = false;
        bool fwd_valid = false;   // the frame buffers hold the last training forward
        bool has_dimage = false;
        bool grads_valid = false;
        int H = 0, W = 0, tiles_x = 0, tiles_y = 0;
        gs::TrainCam cam{};
        uint32_t M = 0, P = 0, p_pre = 0;
        int64_t pixel_pairs = 0, pixel_blended = 0;
        uint32_t* ids = nullptr;  // tile-sorted compact ids of the last forward
        double loss = 0.0, l1 = 0.0, ssim = 0.0;
    } tr;
    // Adam moments stored as bf16 bits (gs_train_set_moments), kept across
    // gs_train_init; fp32 by default
    bool t_bf16_mom = false;
    DevBuf t_p, t_m, t_v, t_g, t_cidx, t_vis, t_grad2d, t_img, t_T, t_stop, t_dimg, t_tgt,
        t_loss, t_dbg, t_ssim;
    std::vector<float> t_host;
    hipEvent_t tev[6] = {};

    gs::TrainParamsDev tplanes(DevBuf& b) {
        gs::TrainParamsDev d{};
        float* base = b.as<float>();
        const size_t n = (size_t)tr.n;
        for (int c = 0; c < 3; ++c) d.mean[c] = base + c * n;
        for (int c = 0; c < 3; ++c) d.ls[c] = base + (3 + c) * n;
        for (int c = 0; c < 4; ++c) d.quat[c] = base + (6 + c) * n;
        d.ol = base + 10 * n;
        d.sh = base + 11 * n;
        d.n = tr.n;
        d.sh_degree = tr.deg;
        return d;
    }

    // AoS host arrays <-> SoA planes (mean 3, log-scale 3, quat 4, logit 1, SH 3K).
    // bf16 bits of x, round to nearest even (a NaN stays a quiet NaN), as
    // torch's float -> bfloat16 conversion rounds
    static uint16_t bf16_rne(float x) {
        uint32_t u;
        std::memcpy(&u, &x, 4);
        if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
        u += 0x7FFFu + ((u >> 16) & 1u);
        return (uint16_t)(u >> 16);
    }
    // Moments are bf16 planes when t_bf16_mom (gs_train_set_moments).
    bool bf16_planes(const DevBuf& b) const { return t_bf16_mom && (&b == &t_m || &b == &t_v); }

    void train_upload(DevBuf& b, const gs_train_arrays* a) {
        REQUIRE(a && a->means && a->log_scales && a->quats && a->opacity_logits && a->sh,
                "train: null parameter array");
        const int64_t n = tr.n;
        const int K = (tr.deg + 1) * (tr.deg + 1);
        t_host.resize((size_t)tr.planes * (size_t)std::max<int64_t>(n, 1));
        float* h = t_host.data();
        parallel_for(n, [&](int64_t lo, int64_t hi) {
            for (int64_t i = lo; i < hi; ++i) {
                for (int c = 0; c < 3; ++c) {
                    h[c * n + i] = a->means[3 * i + c];
                    h[(3 + c) * n + i] = a->log_scales[3 * i + c];
                }
                for (int c = 0; c < 4; ++c) h[(6 + c) * n + i] = a->quats[4 * i + c];
                h[10 * n + i] = a->opacity_logits[i];
                for (int k = 0; k < K; ++k)
                    for (int c = 0; c < 3; ++c)
                        h[(11 + 3 * k + c) * n + i] = a->sh[(i * K + k) * 3 + c];
            }
        });
        if (bf16_planes(b)) {
            std::vector<uint16_t> hb((size_t)tr.planes * (size_t)n);
            parallel_for((int64_t)hb.size(), [&](int64_t lo, int64_t hi) {
                for (int64_t i = lo; i < hi; ++i) hb[(size_t)i] = bf16_rne(h[i]);
            });
            HIPCHK(hipMemcpyAsync(b.p, hb.data(), hb.size() * 2, hipMemcpyHostToDevice, st));
            sync();
            return;
        }
        HIPCHK(hipMemcpyAsync(b.p, h, (size_t)tr.planes * n * 4, hipMemcpyHostToDevice, st));
        sync();
    }
    void train_download(DevBuf& b, gs_train_arrays* a) {
        REQUIRE(a && a->means && a->log_scales && a->quats && a->opacity_logits && a->sh,
                "train: null output array");
        const int64_t n = tr.n;
        const int K = (tr.deg + 1) * (tr.deg + 1);
        t_host.resize((size_t)tr.planes * (size_t)std::max<int64_t>(n, 1));
        float* h = t_host.data();
        if (bf16_planes(b)) {
            std::vector<uint16_t> hb((size_t)tr.planes * (size_t)n);
            HIPCHK(hipMemcpyAsync(hb.data(), b.p, hb.size() * 2, hipMemcpyDeviceToHost, st));
            sync();
            parallel_for((int64_t)hb.size(), [&](int64_t lo, int64_t hi) {
                for (int64_t i = lo; i < hi; ++i) {
                    const uint32_t u = (uint32_t)hb[(size_t)i] << 16;
                    std::memcpy(&h[i], &u, 4);
                }
            });
        } else {
            HIPCHK(hipMemcpyAsync(h, b.p, (size_t)tr.planes * n * 4, hipMemcpyDeviceToHost, st));
            sync();
        }
        parallel_for(n, [&](int64_t lo, int64_t hi) {
            for (int64_t i = lo; i < hi; ++i) {
                for (int c = 0; c < 3; ++c) {
                    a->means[3 * i + c] = h[c * n + i];
                    a->log_scales[3 * i + c] = h[(3 + c) * n + i];
                }
                for (int c = 0; c < 4; ++c) a->quats[4 * i + c] = h[(6 + c) * n + i];
                a->opacity_logits[i] = h[10 * n + i];
                for (int k = 0; k < K; ++k)
                    for (int c = 0; c < 3; ++c)
                        a->sh[(i * K + k) * 3 + c] = h[(11 + 3 * k + c) * n + i];
            }
        });
    }

    void train_init(const gs_train_arrays* a, int64_t n, int deg) {
        REQUIRE(n >= 0 && n < ((int64_t)1 << 31), "train: n out of range");
        REQUIRE(deg >= 0 && deg <= 3, "train: sh_degree must be 0..3");
        sync();
        tr = TrainState{};
        tr.n = n;
        tr.deg = deg;
        tr.planes = 11 + 3 * (deg + 1) * (deg + 1);
        const size_t bytes = (size_t)tr.planes * (size_t)std::max<int64_t>(n, 1) * 4;
        for (DevBuf* b : {&t_p, &t_m, &t_v, &t_g}) b->ensure(bytes);
        HIPCHK(gs::launch_fill_u32(t_m.as<uint32_t>(), 0u, bytes / 4, st));
        HIPCHK(gs::launch_fill_u32(t_v.as<uint32_t>(), 0u, bytes / 4, st));
        HIPCHK(gs::launch_fill_u32(t_g.as<uint32_t>(), 0u, bytes / 4, st));
        t_cidx.ensure((size_t)std::max<int64_t>(n, 1) * 4);
        t_vis.ensure((size_t)std::max<int64_t>(n, 1));
        HIPCHK(hipMemsetAsync(t_vis.p, 0, (size_t)std::max<int64_t>(n, 1), st));
        train_upload(t_p, a);
        tr.ready = true;
    }

    gs::TrainCam train_cam(const gs_view* v, const gs_train_cfg* c) {
        gs::TrainCam cam{};
        const float* e = v->extrinsics;
        const float* K = v->intrinsics;
        const int ri[9] = {0, 1, 2, 4, 5, 6, 8, 9, 10};
        for (int j = 0; j < 9; ++j) cam.r[j] = e[ri[j]];
        cam.t[0] = e[3];
        cam.t[1] = e[7];
        cam.t[2] = e[11];
        cam.fx = K[0];
        cam.fy = K[4];
        cam.cx = K[2];
        cam.cy = K[5];
        cam.ccx = -(e[0] * cam.t[0] + e[4] * cam.t[1] + e[8] * cam.t[2]);
        cam.ccy = -(e[1] * cam.t[0] + e[5] * cam.t[1] + e[9] * cam.t[2]);
        cam.ccz = -(e[2] * cam.t[0] + e[6] * cam.t[1] + e[10] * cam.t[2]);
        cam.near = c->near_plane;
        cam.lowpass = c->lowpass;
        cam.alpha_min = c->alpha_min;
        cam.H = v->image_height;
        cam.W = v->image_width;
        return cam;
    }

    void train_check(const gs_view* v, const gs_train_cfg* c) {
        REQUIRE(tr.ready, "train: gs_train_init first");
        REQUIRE(c != nullptr, "train: null cfg");
        check_view(v);
        REQUIRE(v->tile_size == 16, "train: tile_size must be 16");
        REQUIRE(c->alpha_min > 0.0f && c->alpha_max >= c->alpha_min && c->alpha_max < 1.0f,
                "train: need 0 < alpha_min <= alpha_max < 1");
        REQUIRE(c->t_min > 0.0f, "train: t_min must be > 0");
        REQUIRE(c->lambda_dssim >= 0.0f && c->lambda_dssim <= 1.0f,
                "train: lambda_dssim must be in [0, 1]");
    }

    // SSIM part of the full loss on device images: adds its gradient to dimage
    // (which holds the L1 part) and its S sum to *ssim_sum.
    void enqueue_ssim(const float* image, const float* target, int H, int W, float lambda,
                      float loss_scale, float* dimage, double* ssim_sum) {
        const size_t px = (size_t)H * W;
        t_ssim.ensure(px * 36);
        gs::SsimParams sp{};
        sp.width = W;
        sp.height = H;
        double g[11], gs = 0.0;
        for (int k = 0; k < 11; ++k) gs += (g[k] = std::exp(-(double)((k - 5) * (k - 5)) / 4.5));
        for (int k = 0; k < 11; ++k) sp.g[k] = (float)(g[k] / gs);
        sp.w = (float)(-(double)lambda * (double)loss_scale / (3.0 * (double)px));
        sp.image = image;
        sp.target = target;
        sp.maps = t_ssim.as<float>();
        sp.dimage = dimage;
        sp.ssim_sum = ssim_sum;
        HIPCHK(gs::launch_ssim(sp, st));
    }

    // Enqueues projection, tiles and the forward (+ L1 with a device target).
    void train_forward_enqueue(const gs_view* v, const gs_train_cfg* c, const float* tgt_dev,
                               const gs::TrainDebug& dbg) {
        const int64_t N = tr.n;
        const int H = v->image_height, W = v->image_width;
        tr.H = H;
        tr.W = W;
        tr.tiles_x = (W + 15) / 16;
        tr.tiles_y = (H + 15) / 16;
        const int64_t T = (int64_t)tr.tiles_x * tr.tiles_y;
        tr.cam = train_cam(v, c);
        const FrameLayout L = frame_prepare(std::max<int64_t>(N, 1), T);
        const size_t px = (size_t)H * W;
        t_img.ensure(px * 12);
        t_T.ensure(px * 4);
        t_stop.ensure(px * 4);
        t_dimg.ensure(px * 12);
        t_loss.ensure(32);  // L1 sum, SSIM sum (f64), considered and blended pairs (u64)
        if (timing)
            for (auto& e : tev)
                if (!e) HIPCHK(hipEventCreate(&e));
        if (timing) HIPCHK(hipEventRecord(tev[0], st));
        HIPCHK(gs::launch_fill_u32(L.fr, 0u, L.fwords, st));
        if (spin_limit) HIPCHK(gs::launch_fill_u32(L.cnt + C_CTL + 1, spin_limit, 1, st));
        tr.cam.ctl = L.cnt + C_CTL;
        HIPCHK(gs::launch_fill_u32(t_loss.as<uint32_t>(), 0u, 8, st));
        gs::Compact cpt{b_rc.as<float4>(), b_dkey.as<uint32_t>(),
                        nullptr, b_src.as<uint32_t>()};
        HIPCHK(gs::launch_train_project(tplanes(t_p), tr.cam, cpt, b_brec.as<float4>(),
                                        t_cidx.as<uint32_t>(), t_vis.as<uint8_t>(), L.lb_proj,
                                        L.cnt + C_PROJ_TICKET, L.cnt + C_M,
                                        b_phist_proj.as<uint32_t>(), dbg, st));
        HIPCHK(gs::launch_reduce_rows(b_phist_proj.as<uint32_t>(), 1024, (uint32_t)L.pparts,
                                      nullptr, 0, 0, 0, L.fr + kFrDepthHist, st, nullptr,
                                      L.cnt + C_CTL));
        gs::TileParams tp{tr.tiles_x, tr.tiles_y, 16, 1, L.cnt + C_CTL};
        tr.ids = frame_tiles(L, std::max<int64_t>(N, 1), T, tp, nullptr);
        gs::TrainFwdParams fp{};
        fp.tiles_x = tr.tiles_x;
        fp.tiles_y = tr.tiles_y;
        fp.width = W;
        fp.height = H;
        fp.alpha_max = c->alpha_max;
        fp.alpha_min = c->alpha_min;
        fp.t_min = c->t_min;
        for (int k = 0; k < 3; ++k) fp.bg[k] = c->background[k];
        fp.image = t_img.as<float>();
        fp.final_T = t_T.as<float>();
        fp.stop = t_stop.as<uint32_t>();
        fp.target = tgt_dev;
        fp.dimage = t_dimg.as<float>();
        fp.grad_scale = (float)((double)c->loss_scale * (1.0 - (double)c->lambda_dssim) /
                                (3.0 * (double)px));
        fp.loss = reinterpret_cast<double*>(t_loss.p);
        fp.pairs = reinterpret_cast<unsigned long long*>(t_loss.p) + 2;
        fp.ctl = L.cnt + C_CTL;
        HIPCHK(gs::launch_train_fwd(b_brec.as<float4>(), tr.ids, b_ranges.as<uint32_t>(), fp, st));
        if (tgt_dev != nullptr && c->lambda_dssim > 0.0f)
            enqueue_ssim(t_img.as<float>(), tgt_dev, H, W, c->lambda_dssim, c->loss_scale,
                         t_dimg.as<float>(), reinterpret_cast<double*>(t_loss.p) + 1);
        if (timing) HIPCHK(hipEventRecord(tev[1], st));
    }

    // Forward with the pair-capacity retry; one host synchronisation.
    void train_forward(const gs_view* v, const gs_train_cfg* c, const float* target,
                       bool target_dev, const gs::TrainDebug& dbg) {
        const size_t px = (size_t)v->image_height * v->image_width;
        const float* tgt = nullptr;
        if (target != nullptr) {
            if (target_dev) {
                tgt = target;
            } else {
                t_tgt.ensure(px * 12);
                HIPCHK(hipMemcpyAsync(t_tgt.p, target, px * 12, hipMemcpyHostToDevice, st));
                tgt = t_tgt.as<float>();
            }
        }
        ensure_counters();
        tr.fwd_valid = false;
        tr.grads_valid = false;
        rb_valid = false;
        if (pair_cap == 0) pair_cap = default_pair_cap(tr.n);
        for (int attempt = 0;; ++attempt) {
            train_forward_enqueue(v, c, tgt, dbg);
            HIPCHK(hipMemcpyAsync(h_pin, b_frame.p, 64 * 4, hipMemcpyDeviceToHost, st));
            HIPCHK(hipMemcpyAsync(h_pin + 64, t_loss.p, 32, hipMemcpyDeviceToHost, st));
            sync();
            // The capacity test comes first: an attempt past the capacity has
            // kErrCapacity raised by the count scan, and is re-run (its fill
            // clears the word) rather than reported.
            const uint32_t p_pre = h_pin[C_PPRE];
            if (p_pre == 0xFFFFFFFFu)
                throw GsError(GS_E_CAPACITY, "train: more than 2^32-1 candidate pairs");
            if (p_pre <= pair_cap) {
                ctl_check(h_pin[C_CTL], "train forward");
                break;
            }
            REQUIRE(attempt == 0, "train: pair capacity did not converge");
            pair_cap = std::min<uint64_t>(0xFFFFFFFFull, (uint64_t)p_pre + p_pre / 8 + 4096);
        }
        tr.M = h_pin[C_M];
        tr.p_pre = h_pin[C_PPRE];
        uint64_t pp[2];
        std::memcpy(pp, h_pin + 68, 16);
        tr.pixel_pairs = (int64_t)pp[0];
        tr.pixel_blended = (int64_t)pp[1];
        tr.P = h_pin[C_P];
        double sums[2];
        std::memcpy(sums, h_pin + 64, 16);
        const double lam = c->lambda_dssim;
        tr.l1 = tgt ? sums[0] / (3.0 * (double)px) : 0.0;
        tr.ssim = (tgt && lam > 0.0) ? sums[1] / (3.0 * (double)px) : 0.0;
        tr.loss = tgt ? (double)c->loss_scale * ((1.0 - lam) * tr.l1 + lam * (1.0 - tr.ssim))
                      : 0.0;
        tr.fwd_valid = true;
        tr.has_dimage = tgt != nullptr;
    }

    // Enqueues the blend backward and the projection backward (gradients in t_g).
    void train_backward_enqueue(const gs_train_cfg* c) {
        const int64_t N = tr.n;
        t_grad2d.ensure((size_t)std::max<uint32_t>(tr.M, 1) * 36);
        if (timing) HIPCHK(hipEventRecord(tev[2], st));
        HIPCHK(gs::launch_fill_u32(t_grad2d.as<uint32_t>(), 0u, (size_t)tr.M * 9, st));
        gs::TrainBwdParams bp{};
        bp.tiles_x = tr.tiles_x;
        bp.tiles_y = tr.tiles_y;
        bp.width = tr.W;
        bp.height = tr.H;
        bp.alpha_max = c->alpha_max;
        bp.alpha_min = c->alpha_min;
        for (int k = 0; k < 3; ++k) bp.bg[k] = c->background[k];
        bp.final_T = t_T.as<float>();
        bp.stop = t_stop.as<uint32_t>();
        bp.dimage = t_dimg.as<float>();
        bp.grad2d = t_grad2d.as<float>();
        if (tr.M > 0 && tr.P > 0)
            HIPCHK(gs::launch_train_bwd(b_brec.as<float4>(), tr.ids, b_ranges.as<uint32_t>(), bp, st));
        HIPCHK(gs::launch_train_param_grads(tplanes(t_p), tr.cam, t_cidx.as<uint32_t>(),
                                            t_grad2d.as<float>(), tplanes(t_g), st));
        if (timing) HIPCHK(hipEventRecord(tev[3], st));
        (void)N;
    }

    void train_adam_enqueue(const gs_train_cfg* c) {
        const double b1 = c->beta1, b2 = c->beta2;
        const int64_t t = tr.step + 1;
        const double bc1 = 1.0 - std::pow(b1, (double)t), bc2 = 1.0 - std::pow(b2, (double)t);
        gs::AdamParams ap{};
        ap.beta1 = (float)b1;
        ap.beta2 = (float)b2;
        ap.one_minus_beta1 = (float)(1.0 - b1);
        ap.one_minus_beta2 = (float)(1.0 - b2);
        ap.sqrt_bc2 = (float)std::sqrt(bc2);
        ap.eps = (float)c->eps;
        const double lr_geo[4] = {c->lr_means, c->lr_log_scales, c->lr_quats, c->lr_opacity};
        const int geo_planes[4] = {3, 3, 4, 1};
        int j = 0;
        for (int gidx = 0; gidx < 4; ++gidx)
            for (int k = 0; k < geo_planes[gidx]; ++k) ap.step[j++] = (float)(lr_geo[gidx] / bc1);
        const int K = (tr.deg + 1) * (tr.deg + 1);
        for (int k = 0; k < K; ++k)
            for (int ch = 0; ch < 3; ++ch)
                ap.step[j++] = (float)(k == 0 ? c->lr_sh_dc : c->lr_sh_rest) / (float)bc1;
        if (timing) HIPCHK(hipEventRecord(tev[4], st));
        HIPCHK(gs::launch_sparse_adam(t_p.as<float>(), t_m.p, t_v.p, t_g.as<float>(),
                                      t_vis.as<uint8_t>(), tr.n, tr.planes, ap, t_bf16_mom, st));
        if (timing) HIPCHK(hipEventRecord(tev[5], st));
        ++tr.step;
    }

    void train_stats(gs_train_stats* s, bool fwd, bool bwd, bool adam,
                     std::chrono::steady_clock::time_point t0) {
        if (!s) return;
        gs_train_stats o{};
        o.num_blendable = tr.M;
        o.num_entries = tr.P;
        o.step = tr.step;
        o.loss = tr.loss;
        o.l1 = tr.l1;
        o.ssim = tr.ssim;
        o.pairs_pre = tr.p_pre;
        o.pair_capacity = (int64_t)pair_cap;
        o.pixel_pairs = tr.pixel_pairs;
        o.pixel_blended = tr.pixel_blended;
        if (timing) {
            float ms = 0.0f;
            if (fwd && hipEventElapsedTime(&ms, tev[0], tev[1]) == hipSuccess) o.ms_forward = ms;
            if (bwd && hipEventElapsedTime(&ms, tev[2], tev[3]) == hipSuccess) o.ms_backward = ms;
            if (adam && hipEventElapsedTime(&ms, tev[4], tev[5]) == hipSuccess) o.ms_adam = ms;
        }
        o.ms_total = std::chrono::duration<float, std::milli>(std::chrono::steady_clock::now() - t0)
                         .count();
        *s = o;
    }

    void blend_diag(gs_stats& s) {
        uint64_t e[5] = {0, 0, 0, 0, 0};
        for (int k = 0; k < 64; ++k) {
            for (int c = 0; c < 4; ++c) e[c] += h_evals[k * 8 + c];
            e[4] = std::max<uint64_t>(e[4], h_evals[k * 8 + 4]);
        }
        s.blend_evals = (int64_t)e[0];
        s.blend_batches = (int64_t)e[1];
        s.blend_iters = (int64_t)e[2];
        s.blend_kept = (int64_t)e[3];
        s.blend_max_iters = (int64_t)e[4];
    }

};

gs::CtxInfo gs::ctx_info(const gs_ctx* ctx) { return gs::CtxInfo{ctx->device, ctx->st}; }
void gs::set_last_error(const char* msg) { g_err = msg ? msg : ""; }

extern "C" {

const char* gs_last_error(void) { return g_err.c_str(); }

int gs_create(int device, gs_ctx** out) {
    return guard([&] {
        REQUIRE(out != nullptr, "gs_create: null out");
        int count = 0;
        HIPCHK(hipGetDeviceCount(&count));
        REQUIRE(device >= 0 && device < count, "gs_create: no such device");
        HIPCHK(hipSetDevice(device));
        auto* c = new gs_ctx();
        c->device = device;
        hipError_t e = hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete c;
            throw GsError(GS_E_DEVICE, std::string("hipStreamCreate: ") + hipGetErrorString(e));
        }
        (void)hipDeviceGetAttribute(&c->num_cus, hipDeviceAttributeMultiprocessorCount, device);
        *out = c;
    });
}

void gs_destroy(gs_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    delete ctx;
}

int gs_set_timing(gs_ctx* ctx, int on) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        ctx->timing = on != 0;
        ctx->blend_counts = on >= 2;
    });
}

int gs_device_info(gs_ctx* ctx, int* num_cus, int* arch_minor) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        hipDeviceProp_t prop;
        HIPCHK(hipGetDeviceProperties(&prop, ctx->device));
        if (num_cus) *num_cus = prop.multiProcessorCount;
        if (arch_minor) *arch_minor = prop.minor;
    });
}

int gs_scene_set(gs_ctx* ctx, const gs_scene* scene) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->set_scene(scene);  // completes an announced frame only if the scene changes
    });
}

int gs_render(gs_ctx* ctx, const gs_view* view, void* out, int out_on_device, gs_stats* stats) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->render(view, out, out_on_device != 0, stats);
    });
}

int gs_frame_readback(gs_ctx* ctx, int64_t* counts, int64_t* sorted_ids, int64_t ids_cap,
                      int64_t* tile_ranges, int64_t num_tiles) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        REQUIRE(ctx->rb_valid, "frame_readback: no gs_render frame to read (or a later call "
                               "reused its buffers)");
        HIPCHK(hipSetDevice(ctx->device));
        if (counts) {
            counts[0] = ctx->rb_M;
            counts[1] = ctx->rb_ppre;
            counts[2] = ctx->rb_P;
        }
        const int64_t P = ctx->rb_P, T = ctx->rb_T;
        if (sorted_ids) REQUIRE(ids_cap >= P, "frame_readback: ids_cap is smaller than the pair count");
        if (tile_ranges) REQUIRE(num_tiles == T, "frame_readback: num_tiles is not the frame's tile count");
        std::vector<uint32_t> ids(sorted_ids && P > 0 ? (size_t)P : 0), rg(tile_ranges ? (size_t)T * 2 : 0);
        if (!ctx->rb_empty) {
            if (!ids.empty())
                HIPCHK(hipMemcpyAsync(ids.data(), ctx->rb_ids, (size_t)P * 4, hipMemcpyDeviceToHost,
                                      ctx->st));
            if (!rg.empty())
                HIPCHK(hipMemcpyAsync(rg.data(), ctx->b_ranges.p, (size_t)T * 8,
                                      hipMemcpyDeviceToHost, ctx->st));
            ctx->sync();
        }
        for (size_t i = 0; i < ids.size(); ++i) sorted_ids[i] = ids[i];
        if (tile_ranges)
            for (int64_t i = 0; i < T * 2; ++i) tile_ranges[i] = rg.empty() ? 0 : rg[(size_t)i];
    });
}

int gs_frame_readback_info(gs_ctx* ctx, int64_t* info) {
    return guard([&] {
        REQUIRE(ctx && info, "null argument");
        REQUIRE(ctx->rb_valid, "frame_readback_info: no frame to read (or a later call reused "
                               "its buffers)");
        info[0] = ctx->rb_M;
        info[1] = ctx->rb_ppre;
        info[2] = ctx->rb_P;
        info[3] = ctx->rb_T;
        info[4] = ctx->rb_batch;
        info[5] = ctx->rb_replayed ? 1 : 0;
    });
}

int gs_set_cull_stats(gs_ctx* ctx, int on) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        ctx->drain_spec();
        ctx->cull_stats = on != 0;
    });
}

int gs_set_graphs(gs_ctx* ctx, int on) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->graphs = on != 0;
        for (gs_ctx* p : ctx->peers) {
            if (p->pend.active) p->render_end();
            p->graphs = ctx->graphs;
            p->drop_graph();
        }
        if (ctx->pend.active) ctx->render_end();
        ctx->drop_graph();
    });
}

int gs_graph_counts(gs_ctx* ctx, int64_t* captures, int64_t* replays) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        int64_t c = ctx->graph_captures, r = ctx->graph_replays;
        for (gs_ctx* p : ctx->peers) {
            c += p->graph_captures;
            r += p->graph_replays;
        }
        if (captures) *captures = c;
        if (replays) *replays = r;
    });
}

int gs_set_spin_limit(gs_ctx* ctx, uint32_t limit) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        ctx->drain_spec();
        ctx->spin_limit = limit;
    });
}

int gs_set_pair_limit(gs_ctx* ctx, uint32_t limit) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        ctx->drain_spec();
        ctx->pair_limit = limit == 0 ? 0xFFFFFFFFu : limit;
        ctx->pair_cap = std::min<uint64_t>(ctx->pair_cap, ctx->pair_limit);
        for (gs_ctx* p : ctx->peers) p->pair_cap = std::min<uint64_t>(p->pair_cap, ctx->pair_limit);
    });
}

float gs_overflow_next_floor(float floor, uint32_t max_n, uint32_t cap) {
    return next_contrib_floor(floor, max_n, cap);
}

int gs_render_next(gs_ctx* ctx, const gs_view* view, void* out, int out_on_device,
                   const gs_view* next_view, gs_stats* stats) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->render_next(view, out, out_on_device != 0, next_view, stats);
    });
}

int gs_set_chunk_cull(gs_ctx* ctx, int on, double k) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->set_chunk_cull(on != 0, k);
    });
}

int gs_render_out_ring(gs_ctx* ctx, const gs_view* view, const gs_view* next_view,
                       gs_out_image* image, gs_stats* stats) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->render_out_ring(view, next_view, image, stats);
    });
}

int gs_out_release(uint64_t lease) {
    return guard([&] {
        REQUIRE(gs::LeaseTable::get().release(lease), "gs_out_release: unknown or released lease");
    });
}

int gs_out_ring_config(gs_ctx* ctx, int cap) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        REQUIRE(cap >= 1, "gs_out_ring_config: cap must be at least 1");
        ctx->ring_cap = (size_t)cap;
        if (ctx->ring) ctx->ring->set_cap((size_t)cap);
    });
}

int gs_out_ring_info(gs_ctx* ctx, int* size, int* held, int64_t* grows, int64_t* replaced) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        const gs::OutRing* r = ctx->ring.get();
        if (size) *size = r ? (int)r->size() : 0;
        if (held) *held = r ? (int)r->held() : 0;
        if (grows) *grows = r ? (int64_t)r->grows() : 0;
        if (replaced) *replaced = r ? (int64_t)r->replaced() : 0;
    });
}

int gs_render_batch(gs_ctx* ctx, const gs_view* views, int n, void* const* outs,
                    int out_on_device, gs_stats* stats) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->render_batch(views, n, outs, out_on_device != 0, stats);
    });
}

int gs_project(gs_ctx* ctx, const gs_scene* scene, const gs_view* view, uint8_t* valid_mask,
               float* means2d, float* covs2d, float* depths, float* radii, float* colors_out,
               float* opac_out, int64_t* m_out) {
    return guard([&] {
        REQUIRE(ctx && m_out, "null argument");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->rb_valid = false;
        ctx->set_scene(scene);
        ctx->check_view(view);
        ctx->ensure_terms(view);
        const int64_t n = ctx->sd.n;
        const int64_t M = ctx->run_project(view, valid_mask != nullptr, false);
        *m_out = M;
        if (valid_mask && n > 0)
            HIPCHK(hipMemcpyAsync(valid_mask, ctx->b_valid.p, (size_t)n, hipMemcpyDeviceToHost, ctx->st));
        std::vector<float> rc((size_t)M * 8), brec((size_t)M * 12);
        std::vector<uint32_t> dk((size_t)M);
        if (M > 0) {
            HIPCHK(hipMemcpyAsync(rc.data(), ctx->b_rc.p, (size_t)M * 32, hipMemcpyDeviceToHost, ctx->st));
            HIPCHK(hipMemcpyAsync(brec.data(), ctx->b_brec.p, (size_t)M * 48, hipMemcpyDeviceToHost, ctx->st));
            HIPCHK(hipMemcpyAsync(dk.data(), ctx->b_dkey.p, (size_t)M * 4, hipMemcpyDeviceToHost, ctx->st));
        }
        ctx->sync();
        for (int64_t m = 0; m < M; ++m) {
            if (means2d) {
                means2d[m * 2 + 0] = rc[m * 8 + 0];
                means2d[m * 2 + 1] = rc[m * 8 + 1];
            }
            if (radii) {
                radii[m * 2 + 0] = rc[m * 8 + 2];
                radii[m * 2 + 1] = rc[m * 8 + 3];
            }
            if (covs2d) {
                covs2d[m * 4 + 0] = rc[m * 8 + 4];
                covs2d[m * 4 + 1] = rc[m * 8 + 5];
                covs2d[m * 4 + 2] = rc[m * 8 + 5];
                covs2d[m * 4 + 3] = rc[m * 8 + 6];
            }
            if (depths) std::memcpy(&depths[m], &dk[m], 4);
            if (opac_out) opac_out[m] = brec[m * 12 + 11];
            if (colors_out) {
                colors_out[m * 3 + 0] = brec[m * 12 + 8];
                colors_out[m * 3 + 1] = brec[m * 12 + 9];
                colors_out[m * 3 + 2] = brec[m * 12 + 10];
            }
        }
    });
}

int gs_tile_assign(gs_ctx* ctx, const float* means2d, const float* radii, int64_t m,
                   int image_height, int image_width, int tile_size, const float* covs2d,
                   const float* opac, float contrib_floor, int64_t* gids, int64_t* tids,
                   int64_t cap, int64_t* p_out, int64_t* p_pre_out) {
    return guard([&] {
        REQUIRE(ctx && p_out, "null argument");
        REQUIRE(m >= 0 && m < ((int64_t)1 << 31), "m out of range");
        REQUIRE(image_height > 0 && image_width > 0 && tile_size > 0, "bad image/tile size");
        REQUIRE(((int64_t)image_width + tile_size - 1) / tile_size <= 65535 &&
                    ((int64_t)image_height + tile_size - 1) / tile_size <= 65535,
                "at most 65535 tiles per row and per column");
        REQUIRE(m == 0 || (means2d && radii), "null means2d/radii");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->rb_valid = false;
        const bool cull = covs2d != nullptr && opac != nullptr;
        *p_out = 0;
        if (p_pre_out) *p_pre_out = 0;
        if (m == 0) return;
        std::vector<float> rect((size_t)m * 4), cov((size_t)m * 4, 0.0f);
        for (int64_t i = 0; i < m; ++i) {
            rect[i * 4 + 0] = means2d[i * 2 + 0];
            rect[i * 4 + 1] = means2d[i * 2 + 1];
            rect[i * 4 + 2] = radii[i * 2 + 0];
            rect[i * 4 + 3] = radii[i * 2 + 1];
            if (cull) {
                cov[i * 4 + 0] = covs2d[i * 4 + 0];
                cov[i * 4 + 1] = covs2d[i * 4 + 1];
                cov[i * 4 + 2] = covs2d[i * 4 + 3];
                const float o = opac[i];
                cov[i * 4 + 3] = (o > contrib_floor) ? -2.0f * std::log(contrib_floor / o) : -1.0f;
            }
        }
        ctx->sync();
        ctx->b_tmp_a.ensure((size_t)m * 16);
        ctx->b_tmp_b.ensure((size_t)m * 16);
        HIPCHK(hipMemcpyAsync(ctx->b_tmp_a.p, rect.data(), (size_t)m * 16, hipMemcpyHostToDevice, ctx->st));
        HIPCHK(hipMemcpyAsync(ctx->b_tmp_b.p, cov.data(), (size_t)m * 16, hipMemcpyHostToDevice, ctx->st));
        const int tx = (image_width + tile_size - 1) / tile_size;
        const int ty = (image_height + tile_size - 1) / tile_size;
        gs::TileParams tp{tx, ty, tile_size, cull ? 1 : 0};
        uint64_t p_pre = 0;
        const uint32_t P = ctx->run_tile_assign(ctx->b_tmp_a.as<float4>(), ctx->b_tmp_b.as<float4>(),
                                                nullptr, m, tp, &p_pre);
        if (p_pre_out) *p_pre_out = (int64_t)p_pre;
        *p_out = P;
        if ((int64_t)P > cap) throw GsError(GS_E_CAPACITY, "tile_assign: output capacity too small");
        std::vector<uint32_t> t(P), g(P);
        if (P > 0) {
            HIPCHK(hipMemcpyAsync(t.data(), ctx->b_pair_tile.p, (size_t)P * 4, hipMemcpyDeviceToHost, ctx->st));
            HIPCHK(hipMemcpyAsync(g.data(), ctx->b_pair_id.p, (size_t)P * 4, hipMemcpyDeviceToHost, ctx->st));
        }
        ctx->sync();
        for (uint32_t i = 0; i < P; ++i) {
            gids[i] = g[i];
            tids[i] = t[i];
        }
    });
}

int gs_sort_and_bin(gs_ctx* ctx, const int64_t* gids, const int64_t* tids, const float* depths,
                    int64_t p, int64_t m, int tiles_x, int tiles_y, int64_t* sorted_ids,
                    int64_t* tile_ranges) {
    return guard([&] {
        REQUIRE(ctx && tile_ranges, "null argument");
        REQUIRE(tiles_x > 0 && tiles_y > 0, "bad tile grid");
        REQUIRE(p >= 0 && p < ((int64_t)1 << 32) - 1, "p out of range");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->rb_valid = false;
        const int64_t T = (int64_t)tiles_x * tiles_y;
        REQUIRE(T < ((int64_t)1 << 31), "too many tiles");
        std::vector<uint32_t> g((size_t)p), t((size_t)p);
        for (int64_t i = 0; i < p; ++i) {
            REQUIRE(gids[i] >= 0 && gids[i] < m, "gaussian id out of range");
            REQUIRE(tids[i] >= 0 && tids[i] < T, "tile id out of range");
            g[i] = (uint32_t)gids[i];
            t[i] = (uint32_t)tids[i];
        }
        if (p == 0) {
            std::memset(tile_ranges, 0, (size_t)T * 16);
            return;
        }
        ctx->sync();
        ctx->ensure_counters();
        ctx->b_tmp_a.ensure((size_t)p * 4);
        ctx->b_tmp_b.ensure((size_t)p * 4);
        ctx->b_tmp_c.ensure((size_t)std::max<int64_t>(m, 1) * 4);
        ctx->b_pair_tile.ensure((size_t)p * 8);
        ctx->b_ranges.ensure((size_t)T * 8);
        HIPCHK(hipMemcpyAsync(ctx->b_tmp_a.p, g.data(), (size_t)p * 4, hipMemcpyHostToDevice, ctx->st));
        HIPCHK(hipMemcpyAsync(ctx->b_tmp_b.p, t.data(), (size_t)p * 4, hipMemcpyHostToDevice, ctx->st));
        if (m > 0)
            HIPCHK(hipMemcpyAsync(ctx->b_tmp_c.p, depths, (size_t)m * 4, hipMemcpyHostToDevice, ctx->st));
        uint64_t* keys = ctx->b_pair_tile.as<uint64_t>();
        HIPCHK(gs::launch_make_keys64(ctx->b_tmp_a.as<uint32_t>(), ctx->b_tmp_b.as<uint32_t>(),
                                      ctx->b_tmp_c.as<float>(), (uint32_t)p, keys, ctx->st));
        ctx->ensure_sort(p, 8);
        uint32_t* ctl = ctx->b_cnt.as<uint32_t>() + gs_ctx::C_CTL;
        ctx->ctl_reset(ctl);
        ctx->sort.ctl = ctl;
        ctx->sync();
        int passes = 0;
        void* kf = nullptr;
        uint32_t* vf = nullptr;
        HIPCHK(gs::radix_sort_pairs(keys, ctx->b_tmp_a.as<uint32_t>(), p, 8, 0,
                                    32 + tile_bits(T), ctx->sort, ctx->h_pin + 64, ctx->st,
                                    &passes, false, &kf, &vf));
        HIPCHK(gs::launch_tile_bounds64(static_cast<uint64_t*>(kf), (uint32_t)p,
                                        ctx->b_ranges.as<uint32_t>(), T, ctl, ctx->st));
        std::vector<uint32_t> sid((size_t)p), rg((size_t)T * 2);
        uint32_t flags = 0;
        HIPCHK(hipMemcpyAsync(sid.data(), vf, (size_t)p * 4, hipMemcpyDeviceToHost, ctx->st));
        HIPCHK(hipMemcpyAsync(rg.data(), ctx->b_ranges.p, (size_t)T * 8, hipMemcpyDeviceToHost, ctx->st));
        HIPCHK(hipMemcpyAsync(&flags, ctl, 4, hipMemcpyDeviceToHost, ctx->st));
        ctx->sync();
        gs_ctx::ctl_check(flags, "sort_and_bin");
        for (int64_t i = 0; i < p; ++i) sorted_ids[i] = sid[i];
        for (int64_t i = 0; i < T * 2; ++i) tile_ranges[i] = rg[i];
    });
}

int gs_cull_and_blend(gs_ctx* ctx, const float* means2d, const float* covs2d,
                      const float* colors, const float* opac, const int64_t* sorted_ids,
                      const int64_t* tile_ranges, int64_t m, int64_t p, const gs_view* view,
                      void* image_out) {
    return guard([&] {
        REQUIRE(ctx && view && image_out && tile_ranges, "null argument");
        REQUIRE(m >= 0 && m < ((int64_t)1 << 31) && p >= 0 && p < ((int64_t)1 << 32), "size out of range");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->rb_valid = false;
        ctx->check_view(view);
        const int H = view->image_height, W = view->image_width, ts = view->tile_size;
        const int tiles_x = (W + ts - 1) / ts, tiles_y = (H + ts - 1) / ts;
        const int64_t T = (int64_t)tiles_x * tiles_y;
        std::vector<uint32_t> sid((size_t)std::max<int64_t>(p, 1)), rg((size_t)T * 2);
        for (int64_t i = 0; i < p; ++i) {
            REQUIRE(sorted_ids[i] >= 0 && sorted_ids[i] < m, "sorted id out of range");
            sid[i] = (uint32_t)sorted_ids[i];
        }
        for (int64_t t = 0; t < T; ++t) {
            const int64_t a = tile_ranges[2 * t], b = tile_ranges[2 * t + 1];
            REQUIRE(a >= 0 && a <= b && b <= p, "tile range out of bounds");
            rg[2 * t] = (uint32_t)a;
            rg[2 * t + 1] = (uint32_t)b;
        }
        std::vector<float> lthr((size_t)std::max<int64_t>(m, 1));
        for (int64_t i = 0; i < m; ++i) {
            const float o = opac[i];
            lthr[i] = (o <= view->mb_contrib_floor) ? 0.0f : std::log(view->mb_contrib_floor / o);
        }
        ctx->sync();
        const size_t mm = (size_t)std::max<int64_t>(m, 1);
        ctx->b_tmp_a.ensure(mm * 4 * 11);
        float* base = ctx->b_tmp_a.as<float>();
        float *dm = base, *dc = base + mm * 2, *dcol = base + mm * 6, *dop = base + mm * 9,
              *dl = base + mm * 10;
        if (m > 0) {
            HIPCHK(hipMemcpyAsync(dm, means2d, (size_t)m * 8, hipMemcpyHostToDevice, ctx->st));
            HIPCHK(hipMemcpyAsync(dc, covs2d, (size_t)m * 16, hipMemcpyHostToDevice, ctx->st));
            HIPCHK(hipMemcpyAsync(dcol, colors, (size_t)m * 12, hipMemcpyHostToDevice, ctx->st));
            HIPCHK(hipMemcpyAsync(dop, opac, (size_t)m * 4, hipMemcpyHostToDevice, ctx->st));
            HIPCHK(hipMemcpyAsync(dl, lthr.data(), (size_t)m * 4, hipMemcpyHostToDevice, ctx->st));
        }
        ctx->b_brec.ensure(mm * 48);
        HIPCHK(gs::launch_brec_from_arrays(dm, dc, dcol, dop, dl, m, ctx->b_brec.as<float4>(), ctx->st));
        ctx->b_pair_id.ensure(sid.size() * 4);
        ctx->b_ranges.ensure((size_t)T * 8);
        HIPCHK(hipMemcpyAsync(ctx->b_pair_id.p, sid.data(), sid.size() * 4, hipMemcpyHostToDevice, ctx->st));
        HIPCHK(hipMemcpyAsync(ctx->b_ranges.p, rg.data(), (size_t)T * 8, hipMemcpyHostToDevice, ctx->st));
        const size_t ebytes = view->out_format == GS_OUT_F32 ? 4 : (view->out_format == GS_OUT_BF16 ? 2 : 1);
        const size_t bytes = (size_t)H * W * 3 * ebytes;
        ctx->b_out.ensure(bytes);
        gs::BlendParams bp{tiles_x, tiles_y, ts, H, W, view->cull_disabled ? 1 : 0,
                           view->transmittance_threshold, view->out_format, nullptr, nullptr};
        HIPCHK(gs::launch_blend(ctx->b_brec.as<float4>(), ctx->b_pair_id.as<uint32_t>(),
                                ctx->b_ranges.as<uint32_t>(), bp, ctx->b_out.p, ctx->st));
        HIPCHK(hipMemcpyAsync(image_out, ctx->b_out.p, bytes, hipMemcpyDeviceToHost, ctx->st));
        ctx->sync();
    });
}

// The standalone u64 sort, and with ranges != null the per-tile [start, end)
// of (tile << 32 | depth bits) keys (sort.cpp:146-165) from the sorted keys.
static void sort_u64_dev(gs_ctx* ctx, uint64_t* keys, uint32_t* vals, int64_t n, int begin_bit,
                         int end_bit, int64_t num_tiles, uint32_t* ranges, int* passes_out) {
    HIPCHK(hipSetDevice(ctx->device));
    ctx->drain_spec();
    ctx->rb_valid = false;
    ctx->ensure_counters();
    ctx->ensure_sort(n, 8);
    uint32_t* ctl = ctx->b_cnt.as<uint32_t>() + gs_ctx::C_CTL;
    ctx->ctl_reset(ctl);
    ctx->sort.ctl = ctl;
    ctx->sync();
    int passes = 0;
    void* kf = nullptr;
    uint32_t* vf = nullptr;
    if (ranges != nullptr) {
        // the tile/depth sort: no host round trip, every pass runs, each pass
        // counting the next one's digits
        HIPCHK(gs::launch_fill_u32(ctx->sort.hist, 0u, gs::sort_hist_words(), ctx->st));
        HIPCHK(gs::radix_sort_pairs_dev_chain(keys, vals, n, begin_bit, end_bit, ctx->sort.hist,
                                              ctx->sort.hist + 8 * 256, ctx->sort, ctx->st, &kf,
                                              &vf));
        passes = n > 0 ? (end_bit - begin_bit + 7) / 8 : 0;
    } else {
        HIPCHK(gs::radix_sort_pairs(keys, vals, n, 8, begin_bit, end_bit, ctx->sort,
                                    ctx->h_pin + 64, ctx->st, &passes, false, &kf, &vf));
    }
    if (kf != keys) {
        HIPCHK(hipMemcpyAsync(keys, kf, (size_t)n * 8, hipMemcpyDeviceToDevice, ctx->st));
        HIPCHK(hipMemcpyAsync(vals, vf, (size_t)n * 4, hipMemcpyDeviceToDevice, ctx->st));
    }
    if (ranges != nullptr) {
        const bool timed = ctx->timing;
        if (timed) HIPCHK(hipEventRecord(ctx->ev[6], ctx->st));
        HIPCHK(gs::launch_tile_bounds64(keys, (uint32_t)n, ranges, num_tiles, ctl, ctx->st));
        if (timed) HIPCHK(hipEventRecord(ctx->ev[7], ctx->st));
    }
    HIPCHK(hipMemcpyAsync(ctx->h_pin + 64 + 8 * 256, ctl, 4, hipMemcpyDeviceToHost, ctx->st));
    ctx->sync();
    ctx->last_sort_passes = passes;
    ctx->last_ranges_ms = 0.0f;
    if (ranges != nullptr && ctx->timing)
        (void)hipEventElapsedTime(&ctx->last_ranges_ms, ctx->ev[6], ctx->ev[7]);
    if (passes_out) *passes_out = passes;
    gs_ctx::ctl_check(ctx->h_pin[64 + 8 * 256], "sort");
}

int gs_sort_pairs_u64_dev(gs_ctx* ctx, uint64_t* keys, uint32_t* vals, int64_t n, int begin_bit,
                          int end_bit, int* passes_out) {
    return guard([&] {
        REQUIRE(ctx && keys && vals, "null argument");
        REQUIRE(n >= 0 && n < ((int64_t)1 << 32) - 1, "n out of range");
        REQUIRE(0 <= begin_bit && begin_bit < end_bit && end_bit <= 64, "bad bit range");
        sort_u64_dev(ctx, keys, vals, n, begin_bit, end_bit, 0, nullptr, passes_out);
    });
}

int gs_sort_tile_depth_dev(gs_ctx* ctx, uint64_t* keys, uint32_t* vals, int64_t n,
                           int64_t num_tiles, uint32_t* tile_ranges, int* passes_out) {
    return guard([&] {
        REQUIRE(ctx && keys && vals && tile_ranges, "null argument");
        REQUIRE(n >= 0 && n < ((int64_t)1 << 32) - 1, "n out of range");
        REQUIRE(num_tiles >= 1 && num_tiles <= ((int64_t)1 << 31), "num_tiles out of range");
        if (ctx->timing)
            for (int i : {6, 7})
                if (!ctx->ev[i]) HIPCHK(hipEventCreate(&ctx->ev[i]));
        sort_u64_dev(ctx, keys, vals, n, 0, 32 + tile_bits(num_tiles), num_tiles, tile_ranges,
                     passes_out);
    });
}

int gs_sort_tile_depth_ids_dev(gs_ctx* ctx, uint64_t* keys, uint32_t* ids, int64_t n,
                               int64_t num_gaussians, int64_t num_tiles, uint32_t* tile_ranges,
                               int* passes_out) {
    return guard([&] {
        REQUIRE(ctx && keys && ids && tile_ranges, "null argument");
        REQUIRE(n >= 0 && n < ((int64_t)1 << 32) - 1, "n out of range");
        REQUIRE(num_gaussians >= 0 && num_gaussians <= ((int64_t)1 << 32),
                "num_gaussians out of range");
        REQUIRE(num_tiles >= 1 && num_tiles <= ((int64_t)1 << 31), "num_tiles out of range");
        if (ctx->timing)
            for (int i : {6, 7})
                if (!ctx->ev[i]) HIPCHK(hipEventCreate(&ctx->ev[i]));
        const int tb = tile_bits(num_tiles);
        // the tile counts of the last pass give the ranges (one workgroup scan)
        if (num_tiles > ((int64_t)1 << 24)) {
            sort_u64_dev(ctx, keys, ids, n, 0, 32 + tb, num_tiles, tile_ranges, passes_out);
            return;
        }
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->rb_valid = false;
        ctx->ensure_counters();
        ctx->ensure_sort(n, 8);
        ctx->b_tcnt.ensure((size_t)num_tiles * 4);
        uint32_t* ctl = ctx->b_cnt.as<uint32_t>() + gs_ctx::C_CTL;
        ctx->sort.ctl = ctl;
        uint32_t* tcnt = ctx->b_tcnt.as<uint32_t>();
        uint32_t* key_err = ctl + 2;  // a key-range flag that does not stop the passes
        {
            // the control words (flags, spin limit, key-range flag), the
            // histograms with the pass tickets and the tile counts: one launch
            uint32_t* p[5] = {ctl, ctl + 1, key_err, ctx->sort.hist, tcnt};
            const uint32_t v[5] = {0u, ctx->spin_limit, 0u, 0u, 0u};
            const uint32_t w[5] = {1u, 1u, 1u, (uint32_t)gs::sort_hist_words(),
                                   (uint32_t)num_tiles};
            HIPCHK(gs::launch_fill_ranges(p, v, w, 5, ctx->st));
        }
        int passes = 0;
        const hipError_t e = gs::radix_sort_ids_dev_chain(
            keys, ids, n, tb, (uint64_t)num_gaussians, (uint32_t)num_tiles, tcnt, key_err,
            ctx->sort.hist, ctx->sort.hist + 8 * 256, ctx->sort, ctx->st, &passes);
        if (e == hipErrorNotSupported) {
            sort_u64_dev(ctx, keys, ids, n, 0, 32 + tb, num_tiles, tile_ranges, passes_out);
            return;
        }
        HIPCHK(e);
        const bool timed = ctx->timing;
        if (timed) HIPCHK(hipEventRecord(ctx->ev[6], ctx->st));
        HIPCHK(gs::launch_ranges_from_counts(tcnt, num_tiles, tile_ranges, ctx->st));
        if (timed) HIPCHK(hipEventRecord(ctx->ev[7], ctx->st));
        HIPCHK(hipMemcpyAsync(ctx->h_pin + 64 + 8 * 256, ctl, 12, hipMemcpyDeviceToHost, ctx->st));
        ctx->sync();
        ctx->last_sort_passes = passes;
        ctx->last_ranges_ms = 0.0f;
        if (timed) (void)hipEventElapsedTime(&ctx->last_ranges_ms, ctx->ev[6], ctx->ev[7]);
        if (passes_out) *passes_out = passes;
        const uint32_t* hw = ctx->h_pin + 64 + 8 * 256;
        gs_ctx::ctl_check(hw[0] | hw[2], "sort");
    });
}

float gs_last_ranges_ms(gs_ctx* ctx) { return ctx ? ctx->last_ranges_ms : 0.0f; }

int gs_last_sort_pass_ms(gs_ctx* ctx, float* ms, int max_passes) {
    if (!ctx || !ctx->timing) return 0;
    const int np = std::min(std::min(ctx->last_sort_passes, max_passes), 8);
    for (int i = 0; i < np; ++i) {
        float v = 0.0f;
        if (hipEventElapsedTime(&v, ctx->sort_ev[2 * i], ctx->sort_ev[2 * i + 1]) != hipSuccess)
            v = -1.0f;
        ms[i] = v;
    }
    return np;
}

int gs_train_init(gs_ctx* ctx, const gs_train_arrays* params, int64_t n, int sh_degree) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->train_init(params, n, sh_degree);
    });
}

int gs_train_read(gs_ctx* ctx, int which, gs_train_arrays* out) {
    return guard([&] {
        REQUIRE(ctx && ctx->tr.ready, "train: gs_train_init first");
        REQUIRE(which >= 0 && which <= 3, "train: which must be 0..3");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        DevBuf* b[4] = {&ctx->t_p, &ctx->t_m, &ctx->t_v, &ctx->t_g};
        ctx->train_download(*b[which], out);
    });
}

int gs_train_write(gs_ctx* ctx, int which, const gs_train_arrays* in) {
    return guard([&] {
        REQUIRE(ctx && ctx->tr.ready, "train: gs_train_init first");
        REQUIRE(which >= 0 && which <= 3, "train: which must be 0..3");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        DevBuf* b[4] = {&ctx->t_p, &ctx->t_m, &ctx->t_v, &ctx->t_g};
        ctx->sync();
        ctx->train_upload(*b[which], in);
        if (which == 0) ctx->tr.fwd_valid = false;
        if (which == 3) ctx->tr.grads_valid = true;
    });
}

int gs_train_set_moments(gs_ctx* ctx, int bf16) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        REQUIRE(bf16 == 0 || bf16 == 1, "train: moment format must be 0 (fp32) or 1 (bf16)");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        const bool want = bf16 != 0;
        if (want == ctx->t_bf16_mom) return;
        if (!ctx->tr.ready) {
            ctx->t_bf16_mom = want;
            return;
        }
        // the stored moments are carried over (rounded to nearest even into bf16)
        const int64_t n = ctx->tr.n;
        const int K = (ctx->tr.deg + 1) * (ctx->tr.deg + 1);
        const size_t nn = (size_t)std::max<int64_t>(n, 1);
        std::vector<float> buf[2][5];
        gs_train_arrays a[2];
        for (int w = 0; w < 2; ++w) {
            const size_t sz[5] = {nn * 3, nn * 3, nn * 4, nn, nn * K * 3};
            for (int q = 0; q < 5; ++q) buf[w][q].resize(sz[q]);
            a[w] = gs_train_arrays{buf[w][0].data(), buf[w][1].data(), buf[w][2].data(),
                                   buf[w][3].data(), buf[w][4].data()};
        }
        ctx->sync();
        ctx->train_download(ctx->t_m, &a[0]);
        ctx->train_download(ctx->t_v, &a[1]);
        ctx->t_bf16_mom = want;
        ctx->train_upload(ctx->t_m, &a[0]);
        ctx->train_upload(ctx->t_v, &a[1]);
    });
}

int gs_train_set_step(gs_ctx* ctx, int64_t step) {
    return guard([&] {
        REQUIRE(ctx && ctx->tr.ready, "train: gs_train_init first");
        REQUIRE(step >= 0, "train: step must be >= 0");
        ctx->tr.step = step;
    });
}

int gs_train_set_visible(gs_ctx* ctx, const uint8_t* visible) {
    return guard([&] {
        REQUIRE(ctx && ctx->tr.ready, "train: gs_train_init first");
        REQUIRE(visible != nullptr || ctx->tr.n == 0, "train: null mask");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        if (ctx->tr.n > 0)
            HIPCHK(hipMemcpyAsync(ctx->t_vis.p, visible, (size_t)ctx->tr.n, hipMemcpyHostToDevice,
                                  ctx->st));
        ctx->sync();
    });
}

int gs_train_forward(gs_ctx* ctx, const gs_view* view, const gs_train_cfg* cfg,
                     const float* target, float* image, float* final_T, gs_train_proj* proj,
                     gs_train_stats* stats) {
    return guard([&] {
        const auto t0 = std::chrono::steady_clock::now();
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->train_check(view, cfg);
        const int64_t n = ctx->tr.n;
        gs::TrainDebug dbg{};
        if (proj != nullptr) {
            const size_t nn = (size_t)std::max<int64_t>(n, 1);
            ctx->t_dbg.ensure(nn * 41);  // 10 floats + 1 byte per Gaussian
            float* f = ctx->t_dbg.as<float>();
            dbg.means2d = f;
            dbg.conic = f + 2 * nn;
            dbg.opacity = f + 5 * nn;
            dbg.colors = f + 6 * nn;
            dbg.depth = f + 9 * nn;
            dbg.valid = reinterpret_cast<uint8_t*>(f + 10 * nn);
        }
        ctx->train_forward(view, cfg, target, false, dbg);
        const size_t px = (size_t)view->image_height * view->image_width;
        if (image) HIPCHK(hipMemcpyAsync(image, ctx->t_img.p, px * 12, hipMemcpyDeviceToHost, ctx->st));
        if (final_T) HIPCHK(hipMemcpyAsync(final_T, ctx->t_T.p, px * 4, hipMemcpyDeviceToHost, ctx->st));
        if (proj != nullptr && n > 0) {
            const size_t nn = (size_t)n;
            struct { void* dst; const void* src; size_t bytes; } cp[7] = {
                {proj->means2d, dbg.means2d, nn * 8}, {proj->conic, dbg.conic, nn * 12},
                {proj->opacity, dbg.opacity, nn * 4}, {proj->colors, dbg.colors, nn * 12},
                {proj->depth, dbg.depth, nn * 4},     {proj->valid, dbg.valid, nn},
                {proj->visible, ctx->t_vis.p, nn}};
            for (auto& c : cp)
                if (c.dst) HIPCHK(hipMemcpyAsync(c.dst, c.src, c.bytes, hipMemcpyDeviceToHost, ctx->st));
        }
        ctx->sync();
        ctx->train_stats(stats, true, false, false, t0);
    });
}

int gs_train_backward(gs_ctx* ctx, const gs_train_cfg* cfg, const float* dimage, float* g2d,
                      gs_train_stats* stats) {
    return guard([&] {
        const auto t0 = std::chrono::steady_clock::now();
        REQUIRE(ctx && ctx->tr.ready, "train: gs_train_init first");
        REQUIRE(cfg != nullptr, "train: null cfg");
        REQUIRE(ctx->tr.fwd_valid, "train: no current forward (run gs_train_forward first)");
        REQUIRE(dimage != nullptr || ctx->tr.has_dimage,
                "train: no dL/dimage (forward without a target and none given)");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        const size_t px = (size_t)ctx->tr.H * ctx->tr.W;
        if (dimage)
            HIPCHK(hipMemcpyAsync(ctx->t_dimg.p, dimage, px * 12, hipMemcpyHostToDevice, ctx->st));
        ctx->train_backward_enqueue(cfg);
        if (g2d != nullptr) {
            const int64_t n = ctx->tr.n;
            const uint32_t M = ctx->tr.M;
            std::vector<float> gm((size_t)M * 9);
            std::vector<uint32_t> src(M);
            if (M > 0) {
                HIPCHK(hipMemcpyAsync(gm.data(), ctx->t_grad2d.p, (size_t)M * 36,
                                      hipMemcpyDeviceToHost, ctx->st));
                HIPCHK(hipMemcpyAsync(src.data(), ctx->b_src.p, (size_t)M * 4,
                                      hipMemcpyDeviceToHost, ctx->st));
            }
            ctx->sync();
            std::fill(g2d, g2d + (size_t)n * 9, 0.0f);
            for (uint32_t m = 0; m < M; ++m)
                std::memcpy(g2d + (size_t)src[m] * 9, gm.data() + (size_t)m * 9, 36);
        }
        ctx->sync();
        ctx->tr.grads_valid = true;
        ctx->train_stats(stats, false, true, false, t0);
    });
}

int gs_train_adam(gs_ctx* ctx, const gs_train_cfg* cfg, gs_train_stats* stats) {
    return guard([&] {
        const auto t0 = std::chrono::steady_clock::now();
        REQUIRE(ctx && ctx->tr.ready, "train: gs_train_init first");
        REQUIRE(cfg != nullptr, "train: null cfg");
        REQUIRE(ctx->tr.grads_valid, "train: no gradients (run gs_train_backward first)");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->train_adam_enqueue(cfg);
        ctx->sync();
        ctx->tr.fwd_valid = false;  // parameters changed
        ctx->tr.grads_valid = false;
        ctx->train_stats(stats, false, false, true, t0);
    });
}

int gs_train_step(gs_ctx* ctx, const gs_view* view, const gs_train_cfg* cfg, const float* target,
                  int target_on_device, gs_train_stats* stats) {
    return guard([&] {
        const auto t0 = std::chrono::steady_clock::now();
        REQUIRE(ctx, "null ctx");
        REQUIRE(target != nullptr, "train: null target");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->train_check(view, cfg);
        ctx->train_forward(view, cfg, target, target_on_device != 0, gs::TrainDebug{});
        ctx->train_backward_enqueue(cfg);
        ctx->train_adam_enqueue(cfg);
        ctx->sync();
        ctx->tr.fwd_valid = false;
        ctx->tr.grads_valid = false;
        ctx->train_stats(stats, true, true, true, t0);
    });
}

int gs_train_loss(gs_ctx* ctx, const float* image, const float* target, int height, int width,
                  float lambda_dssim, float loss_scale, float* dimage, double* loss3) {
    return guard([&] {
        REQUIRE(ctx && image && target && dimage, "null argument");
        REQUIRE(height > 0 && width > 0 && (int64_t)height * width <= ((int64_t)1 << 28),
                "train_loss: bad image size");
        REQUIRE(lambda_dssim >= 0.0f && lambda_dssim <= 1.0f,
                "train_loss: lambda_dssim must be in [0, 1]");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        const size_t px = (size_t)height * width;
        ctx->t_img.ensure(px * 12);
        ctx->t_tgt.ensure(px * 12);
        ctx->t_dimg.ensure(px * 12);
        ctx->t_loss.ensure(16);
        hipStream_t st = ctx->st;
        HIPCHK(hipMemcpyAsync(ctx->t_img.p, image, px * 12, hipMemcpyHostToDevice, st));
        HIPCHK(hipMemcpyAsync(ctx->t_tgt.p, target, px * 12, hipMemcpyHostToDevice, st));
        HIPCHK(gs::launch_fill_u32(ctx->t_loss.as<uint32_t>(), 0u, 4, st));
        double* sums = reinterpret_cast<double*>(ctx->t_loss.p);
        const float scale = (float)((double)loss_scale * (1.0 - (double)lambda_dssim) /
                                    (3.0 * (double)px));
        HIPCHK(gs::launch_l1(ctx->t_img.as<float>(), ctx->t_tgt.as<float>(), (int64_t)px * 3,
                             scale, ctx->t_dimg.as<float>(), sums, st));
        if (lambda_dssim > 0.0f)
            ctx->enqueue_ssim(ctx->t_img.as<float>(), ctx->t_tgt.as<float>(), height, width,
                              lambda_dssim, loss_scale, ctx->t_dimg.as<float>(), sums + 1);
        double h[2];
        HIPCHK(hipMemcpyAsync(dimage, ctx->t_dimg.p, px * 12, hipMemcpyDeviceToHost, st));
        HIPCHK(hipMemcpyAsync(h, sums, 16, hipMemcpyDeviceToHost, st));
        ctx->sync();
        ctx->tr.fwd_valid = false;  // t_dimg / t_img no longer hold a training forward
        if (loss3) {
            const double n = 3.0 * (double)px, lam = lambda_dssim;
            const double l1 = h[0] / n, ssim = lam > 0.0 ? h[1] / n : 0.0;
            loss3[0] = (double)loss_scale * ((1.0 - lam) * l1 + lam * (1.0 - ssim));
            loss3[1] = l1;
            loss3[2] = ssim;
        }
    });
}

int gs_dev_alloc(gs_ctx* ctx, int64_t bytes, void** ptr) {
    return guard([&] {
        REQUIRE(ctx && ptr && bytes >= 0, "bad argument");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        HIPCHK(hipMalloc(ptr, (size_t)std::max<int64_t>(bytes, 1)));
    });
}

int gs_dev_free(gs_ctx* ctx, void* ptr) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        HIPCHK(hipSetDevice(ctx->device));
        ctx->drain_spec();
        ctx->sync();
        if (ptr) HIPCHK(hipFree(ptr));
    });
}

int gs_memcpy_h2d(gs_ctx* ctx, void* dst, const void* src, int64_t bytes) {
    return guard([&] {
        REQUIRE(ctx && bytes >= 0, "bad argument");
        HIPCHK(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyHostToDevice, ctx->st));
        ctx->sync();
    });
}

int gs_memcpy_d2h(gs_ctx* ctx, void* dst, const void* src, int64_t bytes) {
    return guard([&] {
        REQUIRE(ctx && bytes >= 0, "bad argument");
        HIPCHK(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToHost, ctx->st));
        ctx->sync();
    });
}

int gs_memcpy_d2d(gs_ctx* ctx, void* dst, const void* src, int64_t bytes) {
    return guard([&] {
        REQUIRE(ctx && bytes >= 0, "bad argument");
        HIPCHK(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice, ctx->st));
        ctx->sync();
    });
}

int gs_sync(gs_ctx* ctx) {
    return guard([&] {
        REQUIRE(ctx, "null ctx");
        ctx->sync();
    });
}

}  // extern "C"
