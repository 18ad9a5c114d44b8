// Host-only checks of the output ring policy (gsplat_tt_amd/csrc/out_ring.h),
// built with g++ and malloc/free by tests/test_out_ring.py. The scenarios are
// those the reference's ring must satisfy (tests/unit/test_out_ring.cpp:1-10):
// a caller that keeps the previous frame cycles through two slots; a dropped
// frame's slot is reused; a frame kept for the whole run costs one more slot;
// past the cap slots are replaced while every held image stays intact; a cap-1
// ring reuses its one slot; a held image outlives the ring. Plus: growing
// frames, a smaller cap, bad releases, and no buffer leaked or freed twice.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "out_ring.h"

static int fails = 0;
#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            std::fprintf(stderr, "FAIL line %d: %s\n", __LINE__, #c);         \
            ++fails;                                                          \
        }                                                                     \
    } while (0)

static int g_allocs = 0, g_frees = 0;
static void* test_alloc(size_t n) {
    ++g_allocs;
    return std::malloc(n);
}
static void test_free(void* p) {
    ++g_frees;
    std::free(p);
}

struct Frame {
    int* px = nullptr;
    uint64_t lease = 0;
};
constexpr size_t kBytes = 4 * sizeof(int);

// "Render" frame f into the ring's next image and lease it to the caller.
static Frame frame(gs::OutRing& r, int f, size_t bytes = kBytes) {
    gs::PinnedImage* im = r.acquire(bytes);
    int* px = static_cast<int*>(im->p);
    for (size_t i = 0; i < bytes / sizeof(int); ++i) px[i] = f;
    return Frame{px, gs::LeaseTable::get().lease(im)};
}
static void release(const Frame& f) { CHECK(gs::LeaseTable::get().release(f.lease)); }

int main() {
    gs::LeaseTable& t = gs::LeaseTable::get();
    {  // keep frame f while f+1 renders: two slots, never the held one
        gs::OutRing r(test_alloc, test_free, 4);
        Frame held = frame(r, 0);
        for (int f = 1; f < 20; ++f) {
            Frame next = frame(r, f);
            CHECK(next.px != held.px);
            CHECK(held.px[0] == f - 1 && held.px[3] == f - 1);
            release(held);
            held = next;
        }
        CHECK(r.size() == 2 && r.grows() == 2 && r.replaced() == 0);
        CHECK(r.held() == 1);
        release(held);
        CHECK(r.held() == 0);
    }
    {  // dropped frames: the same slot comes back
        gs::OutRing r(test_alloc, test_free, 4);
        const void* first = nullptr;
        for (int f = 0; f < 5; ++f) {
            Frame x = frame(r, f);
            if (f == 0) first = x.px;
            CHECK(x.px == first);
            release(x);
        }
        CHECK(r.size() == 1 && r.grows() == 1);
    }
    {  // one frame kept for the whole run costs one more slot
        gs::OutRing r(test_alloc, test_free, 4);
        Frame hero = frame(r, 100);
        Frame held{};
        for (int f = 0; f < 10; ++f) {
            Frame next = frame(r, f);
            CHECK(next.px != hero.px);
            if (held.lease) release(held);
            held = next;
        }
        CHECK(hero.px[0] == 100);
        CHECK(r.size() == 3 && r.replaced() == 0);
        release(held);
        release(hero);
    }
    {  // hoarding past the cap: slots replaced, every held image intact
        gs::OutRing r(test_alloc, test_free, 3);
        const int a0 = g_allocs;
        std::vector<Frame> kept;
        for (int f = 0; f < 8; ++f) kept.push_back(frame(r, f));
        for (int f = 0; f < 8; ++f) CHECK(kept[f].px[0] == f && kept[f].px[3] == f);
        CHECK(r.size() == 3 && r.replaced() == 5 && g_allocs - a0 == 8);
        for (const Frame& k : kept) release(k);  // the 5 replaced ones are freed here
        kept.clear();
        for (int f = 0; f < 4; ++f) release(frame(r, f));
        CHECK(r.replaced() == 5 && g_allocs - a0 == 8);
    }
    {  // cap 1: the one slot is reused
        gs::OutRing r(test_alloc, test_free, 1);
        gs::PinnedImage* a = r.acquire(kBytes);
        for (int f = 0; f < 3; ++f) CHECK(r.acquire(kBytes) == a);
        CHECK(r.size() == 1 && r.replaced() == 0);
    }
    {  // a held image outlives the ring's slots (clear, then the ring itself)
        Frame held{};
        {
            gs::OutRing r(test_alloc, test_free, 2);
            held = frame(r, 7);
            r.clear();
            CHECK(r.size() == 0 && held.px[0] == 7);
            Frame other = frame(r, 8);
            CHECK(other.px != held.px && held.px[0] == 7);
            release(other);
        }
        CHECK(held.px[0] == 7);  // still allocated after the ring is gone
        release(held);
    }
    {  // a larger frame gets a larger buffer; a smaller cap lets go of slots
        gs::OutRing r(test_alloc, test_free, 4);
        Frame a = frame(r, 1);
        Frame b = frame(r, 2);
        release(a);
        Frame c = frame(r, 3, 4 * kBytes);  // a's slot, new buffer of 16 ints
        CHECK(c.px[15] == 3 && b.px[0] == 2);
        CHECK(r.size() == 2);
        r.set_cap(1);
        CHECK(r.size() == 1 && b.px[0] == 2 && c.px[15] == 3);
        release(b);
        release(c);
        CHECK(r.held() == 0);
    }
    {  // unknown and repeated releases are refused
        gs::OutRing r(test_alloc, test_free, 2);
        Frame a = frame(r, 5);
        CHECK(t.release(a.lease));
        CHECK(!t.release(a.lease));
        CHECK(!t.release(0));
        CHECK(!t.release(a.lease + 1000));
    }
    CHECK(t.live() == 0);
    CHECK(g_allocs == g_frees);
    if (fails) {
        std::fprintf(stderr, "%d check(s) failed\n", fails);
        return 1;
    }
    std::printf("ok allocs=%d frees=%d\n", g_allocs, g_frees);
    return 0;
}
