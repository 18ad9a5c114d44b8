// render_clean.cpp - the drop-in `render_clean` Python module over the C ABI.
//
// Same surface as the reference's module (render/host/render.cpp:617-721):
// render_view(...) -> (uint8 (H,W,3), {"num_visible", "num_entries"}) plus
// pfwc_num_cores, bump_scene_version, scene_version, device_shutdown,
// stage_timings, reset_stage_timings. Device work runs with the GIL released
// under one module mutex (render.cpp:73-75, 351-354). No CPU fallback: a
// device failure raises RuntimeError (render.cpp:252-259).
//
// Extensions, all keyword-only with defaults that keep the reference's
// behaviour: `output` ("u8" default, "bf16" as uint16 bits, "f32") and SH
// colours (colors of shape (N, K, 3), K = (d+1)^2, evaluated on the GPU).
// The u8 image is the bf16 image packed as img_pack_u8.h:9-14 does
// (uint8(clip(float(bf16), 0, 1) * 255), truncation), the reference's
// render_view output.
//
// One deliberate difference: the reference's device render_view ignores
// contrib_floor, transmittance_threshold, k_cap and use_isoellipse
// (render.cpp:274-278; its device path bakes its own values). Here they act
// as in the CPU renderer that defines this path's results
// (_gsplat_cpu.render_full, backends/cpu_cpp/pybind_module.cpp:2071-2091):
// with the values run.py passes (contrib_floor = mb_contrib_floor, threshold
// 1/255, k_cap 3, no isoellipse) both agree.
//
// Zero-copy output, on by default as in the reference (render.cpp:334-340,
// 598-612; env_config.h:251-277): the returned image is a pinned buffer of the
// context's output ring, and the array keeps that buffer's lease, so the ring
// never writes it again while Python holds the image or any view of it.
// GSPLAT_TT_OUT_ZEROCOPY=0 (or GSPLAT_TT_OUT_PINNED=0) returns a fresh array
// instead; GSPLAT_TT_OUT_ZEROCOPY_SLOTS (default 4, at least 1) caps the ring.
// GSPLAT_TT_CHUNK_CULL=1 turns on the chunk frustum skip with box factor
// GSPLAT_TT_CHUNK_K (default 1.5), as render/host/pfwc_device.cpp:214-240 reads
// them; the images are the same either way.
//
// Stage timings (render/host/stage_timers.h:1-60): host wall-clock spans,
// always on and cheap: head (entry to the device call: argument checks, scene
// cache lookup), frame (the device call: enqueue, wait, image copy-out; the
// frame has one host wait, so its stages are not split on the host), tail
// (stats and return value) and view_total; head + frame + tail = view_total.
// GSPLAT_TT_STAGE_EVENTS=1 (a diagnostic, like the reference's
// GSPLAT_TT_SPLIT_BLEND) adds per-stage device times from hipEvents on the
// render stream under project, depth_sort, tile_assign, sort and blend; they
// are 0.0 otherwise.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "gsplat_hip.h"

namespace py = pybind11;

namespace {

std::mutex g_mutex;
gs_ctx* g_ctx = nullptr;
uint64_t g_scene_version = 0;

struct Timings {
    int64_t views = 0, xview_hits = 0, xview_misses = 0;
    double head = 0, frame = 0, tail = 0, view_total = 0;  // host spans
    double project = 0, depth_sort = 0, tile_assign = 0, tile_sort = 0, blend = 0;  // events
} g_t;
bool g_events = false;  // per-stage hipEvents on the context (GSPLAT_TT_STAGE_EVENTS)
using clk = std::chrono::steady_clock;
double ms_between(clk::time_point a, clk::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
}
// the view announced by the last call's next_extrinsics (xview hit accounting)
bool g_have_next = false;
gs_view g_next{};

void check(int rc) {
    if (rc == GS_OK) return;
    const std::string msg = std::string("render_clean: ") + gs_last_error();
    if (rc == GS_E_INVALID) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

gs_ctx* ctx_locked() {
    if (g_ctx == nullptr) {
        check(gs_create(0, &g_ctx));
        g_events = false;
    }
    return g_ctx;
}

using farr = py::array_t<float, py::array::c_style | py::array::forcecast>;

unsigned env_uint(const char* name, unsigned dflt) {
    const char* v = std::getenv(name);
    if (v == nullptr || *v == 0) return dflt;
    char* end = nullptr;
    const unsigned long x = std::strtoul(v, &end, 10);
    return (end != nullptr && *end == 0) ? (unsigned)x : dflt;
}
bool out_zerocopy() {
    return env_uint("GSPLAT_TT_OUT_ZEROCOPY", 1u) != 0u && env_uint("GSPLAT_TT_OUT_PINNED", 1u) != 0u;
}
double env_double(const char* name, double dflt) {
    const char* v = std::getenv(name);
    if (v == nullptr || *v == 0) return dflt;
    char* end = nullptr;
    const double x = std::strtod(v, &end);
    return (end != nullptr && *end == 0) ? x : dflt;
}
bool g_chunk_on = false;
double g_chunk_k = 1.5;
// GSPLAT_TT_PAIR_LIMIT: the pair limit of gs_set_pair_limit (0: none), for
// tests of the overflow floor ladder (the reference's GSPLAT_TT_TEST_TILE_CAP)
unsigned g_pair_limit = 0u;
int out_zerocopy_slots() {
    const unsigned n = env_uint("GSPLAT_TT_OUT_ZEROCOPY_SLOTS", 4u);
    return n < 1u ? 1 : (int)std::min(n, 1024u);
}

py::tuple render_view(farr means, farr cov3d, farr opacities, farr colors, farr extrinsics,
                      farr intrinsics, int image_height, int image_width, int tile_size,
                      float min_opacity, float contrib_floor, float mb_contrib_floor,
                      bool cull_disabled, float transmittance_threshold, int max_radius,
                      float k_cap, bool use_isoellipse, int blend_mode, py::object next_extrinsics,
                      const std::string& output, bool sh_clamp) {
    const clk::time_point t_entry = clk::now();
    (void)blend_mode;
    const auto mi = means.request();
    if (mi.ndim != 2 || mi.shape[1] != 3) throw std::invalid_argument("means must have shape (N, 3)");
    const int64_t N = mi.shape[0];
    const auto ci = cov3d.request();
    int stride = 0;
    if (ci.size == N * 9) stride = 9;
    else if (ci.size == N * 6) stride = 6;
    else throw std::invalid_argument("cov3d must have shape (N, 3, 3), (N, 9) or (N, 6)");
    const auto oi = opacities.request();
    if (oi.size != N) throw std::invalid_argument("opacities must have shape (N,)");
    const auto coli = colors.request();
    int deg = -1;
    if (coli.ndim == 2 && coli.shape[1] == 3 && coli.shape[0] == N) {
        deg = -1;
    } else if (coli.ndim == 3 && coli.shape[0] == N && coli.shape[2] == 3) {
        const int64_t K = coli.shape[1];
        deg = K == 1 ? 0 : K == 4 ? 1 : K == 9 ? 2 : K == 16 ? 3 : -2;
        if (deg == -2) throw std::invalid_argument("colors: SH coefficient count must be 1, 4, 9 or 16");
    } else {
        throw std::invalid_argument("colors must have shape (N, 3) or (N, K, 3)");
    }
    if (extrinsics.size() != 16) throw std::invalid_argument("extrinsics must be 4x4");
    if (intrinsics.size() != 9) throw std::invalid_argument("intrinsics must be 3x3");
    farr ne;
    if (!next_extrinsics.is_none()) {
        ne = farr::ensure(next_extrinsics);
        if (!ne || ne.size() != 16)
            throw std::invalid_argument("render_view: next_extrinsics must be 16 floats (4x4)");
    }
    int fmt;
    if (output == "u8") fmt = GS_OUT_U8;
    else if (output == "bf16") fmt = GS_OUT_BF16;
    else if (output == "f32") fmt = GS_OUT_F32;
    else throw std::invalid_argument("output must be 'u8', 'bf16' or 'f32'");

    gs_scene sc{};
    sc.means = static_cast<const float*>(mi.ptr);
    sc.cov3d = static_cast<const float*>(ci.ptr);
    sc.cov3d_stride = stride;
    sc.opacities = static_cast<const float*>(oi.ptr);
    sc.colors = static_cast<const float*>(coli.ptr);
    sc.sh_degree = deg;
    sc.n = N;
    gs_view v{};
    std::memcpy(v.extrinsics, extrinsics.data(), sizeof(v.extrinsics));
    std::memcpy(v.intrinsics, intrinsics.data(), sizeof(v.intrinsics));
    v.image_height = image_height;
    v.image_width = image_width;
    v.tile_size = tile_size;
    v.min_opacity = min_opacity;
    v.contrib_floor = contrib_floor;
    v.mb_contrib_floor = mb_contrib_floor;
    v.cull_disabled = cull_disabled ? 1 : 0;
    v.transmittance_threshold = transmittance_threshold;
    v.max_radius = max_radius;
    v.k_cap = k_cap;
    v.use_isoellipse = use_isoellipse ? 1 : 0;
    v.out_format = fmt;
    v.sh_clamp_hi = sh_clamp ? 1 : 0;
    if (image_height <= 0 || image_width <= 0) throw std::invalid_argument("image size must be positive");

    const bool zerocopy = out_zerocopy();
    const int slots = out_zerocopy_slots();
    py::array image;
    if (!zerocopy) {
        if (fmt == GS_OUT_U8) image = py::array_t<uint8_t>({image_height, image_width, 3});
        else if (fmt == GS_OUT_BF16) image = py::array_t<uint16_t>({image_height, image_width, 3});
        else image = py::array_t<float>({image_height, image_width, 3});
    }
    void* out = zerocopy ? nullptr : image.mutable_data();
    gs_out_image ring_img{};
    gs_stats st{};
    clk::time_point t_call, t_done;
    {
        py::gil_scoped_release nogil;
        std::lock_guard<std::mutex> lock(g_mutex);
        gs_ctx* c = ctx_locked();
        const bool events = env_uint("GSPLAT_TT_STAGE_EVENTS", 0u) != 0u;
        if (events != g_events) {
            check(gs_set_timing(c, events ? 1 : 0));
            g_events = events;
        }
        const bool chunk_on = env_uint("GSPLAT_TT_CHUNK_CULL", 0u) != 0u;
        const double chunk_k = env_double("GSPLAT_TT_CHUNK_K", 1.5);
        if (chunk_on != g_chunk_on || chunk_k != g_chunk_k) {
            check(gs_set_chunk_cull(c, chunk_on ? 1 : 0, chunk_k));
            g_chunk_on = chunk_on;
            g_chunk_k = chunk_k;
        }
        const unsigned pair_limit = env_uint("GSPLAT_TT_PAIR_LIMIT", 0u);
        if (pair_limit != g_pair_limit) {
            check(gs_set_pair_limit(c, pair_limit));
            g_pair_limit = pair_limit;
        }
        sc.version = g_scene_version;
        check(gs_scene_set(c, &sc));
        // the next view: this call's parameters at the announced pose
        gs_view nv = v;
        if (ne) std::memcpy(nv.extrinsics, ne.data(), sizeof(nv.extrinsics));
        t_call = clk::now();
        if (zerocopy) {
            check(gs_out_ring_config(c, slots));
            check(gs_render_out_ring(c, &v, ne ? &nv : nullptr, &ring_img, &st));
        } else {
            check(gs_render_next(c, &v, out, 0, ne ? &nv : nullptr, &st));
        }
        t_done = clk::now();
        g_t.views++;
        if (g_have_next) {
            if (std::memcmp(&g_next, &v, sizeof(gs_view)) == 0) g_t.xview_hits++;
            else g_t.xview_misses++;
        }
        g_have_next = (bool)ne;
        if (ne) g_next = nv;
        g_t.project += st.ms_project;
        g_t.depth_sort += st.ms_depth_sort;
        g_t.tile_assign += st.ms_tile_assign;
        g_t.tile_sort += st.ms_tile_sort;
        g_t.blend += st.ms_blend;
    }
    if (zerocopy) {
        // the array's base holds the lease: released when the image is collected
        auto* lease = new uint64_t(ring_img.lease);
        py::capsule keep(lease, [](void* p) {
            auto* l = static_cast<uint64_t*>(p);
            (void)gs_out_release(*l);
            delete l;
        });
        const py::ssize_t eb = fmt == GS_OUT_F32 ? 4 : (fmt == GS_OUT_BF16 ? 2 : 1);
        const std::vector<py::ssize_t> shape{image_height, image_width, 3};
        const std::vector<py::ssize_t> strides{(py::ssize_t)ring_img.pitch, 3 * eb, eb};
        const py::dtype dt = fmt == GS_OUT_U8 ? py::dtype::of<uint8_t>()
                             : fmt == GS_OUT_BF16 ? py::dtype::of<uint16_t>()
                                                  : py::dtype::of<float>();
        image = py::array(dt, shape, strides, ring_img.data, keep);
    }
    if (st.floor_retries > 0)
        std::fprintf(stderr,
                     "[render_clean] pair overflow: the view was rendered at contrib floor "
                     "1/%.0f after %d retries\n",
                     1.0 / st.contrib_floor, st.floor_retries);
    py::dict stats;
    stats["num_visible"] = st.num_visible;
    stats["num_entries"] = st.num_entries;
    py::tuple result = py::make_tuple(image, stats);
    const clk::time_point t_end = clk::now();
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        g_t.head += ms_between(t_entry, t_call);
        g_t.frame += ms_between(t_call, t_done);
        g_t.tail += ms_between(t_done, t_end);
        g_t.view_total += ms_between(t_entry, t_end);
    }
    return result;
}

}  // namespace

PYBIND11_MODULE(render_clean, m) {
    m.doc() = "MI355X (gfx950) Gaussian-splat renderer with the render_clean surface";
    m.def("render_view", &render_view, "Render one view on the GPU", py::arg("means"),
          py::arg("cov3d"), py::arg("opacities"), py::arg("colors"), py::arg("extrinsics"),
          py::arg("intrinsics"), py::arg("image_height"), py::arg("image_width"),
          py::arg("tile_size"), py::arg("min_opacity"), py::arg("contrib_floor"),
          py::arg("mb_contrib_floor"), py::arg("cull_disabled"),
          py::arg("transmittance_threshold"), py::arg("max_radius"), py::arg("k_cap"),
          py::arg("use_isoellipse"), py::arg("blend_mode") = 2,
          py::arg("next_extrinsics") = py::none(), py::kw_only(), py::arg("output") = "u8",
          py::arg("sh_clamp") = true);
    m.def("pfwc_num_cores", []() {
        py::gil_scoped_release nogil;
        std::lock_guard<std::mutex> lock(g_mutex);
        int cus = 0;
        check(gs_device_info(ctx_locked(), &cus, nullptr));
        return static_cast<int64_t>(cus);
    });
    m.def("bump_scene_version", []() {
        py::gil_scoped_release nogil;
        std::lock_guard<std::mutex> lock(g_mutex);
        return ++g_scene_version;
    });
    m.def("scene_version", []() { return g_scene_version; });
    m.def("device_shutdown", []() {
        py::gil_scoped_release nogil;
        std::lock_guard<std::mutex> lock(g_mutex);
        if (g_ctx) gs_destroy(g_ctx);
        g_ctx = nullptr;
        g_chunk_on = false;
        g_chunk_k = 1.5;
        g_have_next = false;
    });
    // Totals in ms over every render_view since reset_stage_timings, under the
    // reference's keys (render/host/render.cpp:662-720): head, tail and
    // view_total are host spans, as in the reference; frame (this path's own
    // key) is the device call, whose stages the host does not see apart (one
    // wait per frame). With GSPLAT_TT_STAGE_EVENTS=1, project (projection +
    // depth sort), tile_assign, sort (tile sort) and blend (microblock cull +
    // blend, one kernel) hold hipEvent device times, and depth_sort (this
    // path's own key) the depth sort alone; 0.0 otherwise. xview_hits /
    // xview_misses: calls whose view was / was not the one the previous call
    // announced. Keys of Tenstorrent sub-steps that this path does not have
    // (blend_setup, mat, cull, d2h, assemble, xview, sort_*, project_cov3d,
    // project_pfwc_*, project_gather_*, tile_assign_*) are present and stay 0.0.
    m.def("stage_timings", []() {
        std::lock_guard<std::mutex> lock(g_mutex);
        py::dict d;
        d["views"] = g_t.views;
        for (const char* k : {"blend_setup", "mat", "cull", "d2h", "assemble", "xview", "sort_pread", "sort_bin_count", "sort_bin_hist_d2h",
                              "sort_bin_layout", "sort_upload", "sort_bin_emit", "sort_kernel",
                              "sort_d2h", "sort_compact", "sort_publish_host",
                              "sort_publish_wait", "sort_mat", "sort_pre", "sort_log",
                              "sort_cont_prep", "sort_cont_rtargs", "sort_cont_other",
                              "project_cov3d", "project_pfwc_setup", "project_pfwc_rtargs",
                              "project_pfwc_chunkcull", "project_pfwc_enqueue",
                              "project_pfwc_finish", "project_gather_setup",
                              "project_gather_rtargs", "project_gather_enqueue",
                              "project_gather_wait", "project_gather_result",
                              "tile_assign_setup", "tile_assign_rtargs", "tile_assign_enqueue",
                              "tile_assign_scan_finish", "tile_assign_p_d2h",
                              "tile_assign_k2_finish", "tile_assign_publish"})
            d[k] = 0.0;
        d["head"] = g_t.head;
        d["frame"] = g_t.frame;
        d["tail"] = g_t.tail;
        d["project"] = g_t.project + g_t.depth_sort;
        d["depth_sort"] = g_t.depth_sort;
        d["tile_assign"] = g_t.tile_assign;
        d["sort"] = g_t.tile_sort;
        d["blend"] = g_t.blend;
        d["view_total"] = g_t.view_total;
        d["xview_hits"] = g_t.xview_hits;
        d["xview_misses"] = g_t.xview_misses;
        return d;
    });
    m.def("reset_stage_timings", []() {
        std::lock_guard<std::mutex> lock(g_mutex);
        g_t = Timings{};
    });
}
