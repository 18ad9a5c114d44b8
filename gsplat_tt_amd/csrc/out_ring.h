// out_ring.h - the ring of pinned host images behind gs_render_out_ring.
//
// A frame is copied by DMA from HBM into one slot's pinned host buffer and the
// caller receives that buffer (no host copy) with a lease. A buffer whose lease
// is held is never written again. acquire() picks the slot for the next frame
// with the policy of render/host/out_ring.h:9-12: the first slot after the last
// one written whose lease is free; else a new slot while the ring is under its
// cap; else the slot after the last one written gets a new buffer, and the old
// buffer stays alive for the lease holder until it is released. Leases are
// process-wide ids kept in one table, so a lease may be released from any
// thread, also after the ring that made it is gone.
//
// Host-only code (no HIP types): the allocator is a pair of function pointers,
// pinned host memory in the library, malloc/free in the CPU unit test.
#pragma once

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <new>
#include <unordered_map>
#include <vector>

namespace gs {

struct PinnedImage {
    void* p = nullptr;
    size_t bytes = 0;
    uint64_t lease = 0;  // nonzero while a caller holds the image
    bool in_ring = false;
    void (*free_fn)(void*) = nullptr;
};

class LeaseTable {
public:
    static LeaseTable& get() {
        static LeaseTable* t = new LeaseTable();  // never destroyed: leases may outlive statics
        return *t;
    }
    uint64_t lease(PinnedImage* im) {
        std::lock_guard<std::mutex> g(mu_);
        im->lease = ++next_;
        live_[im->lease] = im;
        return im->lease;
    }
    bool held(const PinnedImage* im) {
        std::lock_guard<std::mutex> g(mu_);
        return im->lease != 0;
    }
    // false for an unknown (or already released) lease
    bool release(uint64_t id) {
        std::lock_guard<std::mutex> g(mu_);
        auto it = live_.find(id);
        if (it == live_.end()) return false;
        PinnedImage* im = it->second;
        live_.erase(it);
        im->lease = 0;
        if (!im->in_ring) destroy(im);
        return true;
    }
    // the ring lets go of an image: freed now, or at its lease's release
    void drop(PinnedImage* im) {
        std::lock_guard<std::mutex> g(mu_);
        im->in_ring = false;
        if (im->lease == 0) destroy(im);
    }
    size_t live() {
        std::lock_guard<std::mutex> g(mu_);
        return live_.size();
    }

private:
    static void destroy(PinnedImage* im) {
        if (im->p && im->free_fn) im->free_fn(im->p);
        delete im;
    }
    std::mutex mu_;
    uint64_t next_ = 0;
    std::unordered_map<uint64_t, PinnedImage*> live_;
};

class OutRing {
public:
    using AllocFn = void* (*)(size_t);
    using FreeFn = void (*)(void*);

    OutRing(AllocFn a, FreeFn f, size_t cap) : alloc_(a), free_(f), cap_(cap < 1 ? 1 : cap) {}
    ~OutRing() { clear(); }
    OutRing(const OutRing&) = delete;
    OutRing& operator=(const OutRing&) = delete;

    // The image for the next frame, with a buffer of at least `bytes`.
    PinnedImage* acquire(size_t bytes) {
        LeaseTable& t = LeaseTable::get();
        const size_t n = slots_.size();
        for (size_t k = 1; k <= n; ++k) {
            const size_t i = (last_ + k) % n;
            if (!t.held(slots_[i])) {
                last_ = i;
                if (slots_[i]->bytes < bytes) {  // a larger frame: new buffer, same slot
                    t.drop(slots_[i]);
                    slots_[i] = make(bytes);
                }
                return slots_[i];
            }
        }
        if (n < cap_) {
            slots_.push_back(make(bytes));
            ++grows_;
            last_ = n;
            return slots_.back();
        }
        const size_t i = (last_ + 1) % n;  // every slot is held: replace one
        t.drop(slots_[i]);
        slots_[i] = make(bytes);
        ++replaced_;
        last_ = i;
        return slots_[i];
    }

    // At most `cap` slots from now on (surplus slots are let go, last first).
    void set_cap(size_t cap) {
        cap_ = cap < 1 ? 1 : cap;
        while (slots_.size() > cap_) {
            LeaseTable::get().drop(slots_.back());
            slots_.pop_back();
        }
        if (last_ >= slots_.size()) last_ = 0;
    }
    // Every slot let go; images whose leases are held stay valid until released.
    void clear() {
        for (PinnedImage* im : slots_) LeaseTable::get().drop(im);
        slots_.clear();
        last_ = 0;
    }

    size_t size() const { return slots_.size(); }
    size_t cap() const { return cap_; }
    size_t grows() const { return grows_; }
    size_t replaced() const { return replaced_; }
    size_t held() const {
        size_t h = 0;
        for (const PinnedImage* im : slots_) h += LeaseTable::get().held(im) ? 1 : 0;
        return h;
    }

private:
    PinnedImage* make(size_t bytes) {
        auto* im = new PinnedImage();
        im->p = alloc_(bytes);
        if (im->p == nullptr) {
            delete im;
            throw std::bad_alloc();
        }
        im->bytes = bytes;
        im->in_ring = true;
        im->free_fn = free_;
        return im;
    }

    AllocFn alloc_;
    FreeFn free_;
    size_t cap_;
    std::vector<PinnedImage*> slots_;
    size_t last_ = 0;
    size_t grows_ = 0;
    size_t replaced_ = 0;
};

}  // namespace gs
