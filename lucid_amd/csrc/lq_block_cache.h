// lq_block_cache.h -- bookkeeping of the device caching allocator (host-only C++, no HIP
// types, so the CPU test suite compiles and drives it with fake completion markers).
//
// A freed block goes back to its device's size-ordered free list together with the stream
// it was last used on and a completion marker recorded on that stream at the free (a HIP
// event in the library).  A later request on stream S may take a cached block when
//   * it was freed on S: S executes in order, so S's earlier work on the block precedes
//     anything S does with it next; or
//   * its marker reports completion: the work queued on the freeing stream before the free
//     has finished, so no kernel still reads or writes the block.
// A block whose stream recorded no marker (a stream under graph capture) is reused on that
// stream only.  A live block may also be marked as used on other streams (record_use, the
// role of torch's record_stream): its free then records a marker on each of them too, and
// the block is reused -- on any stream, the freeing one included -- only once every one of
// those markers reports completion (a use stream that records no marker keeps the block out
// of circulation until drain).  A stream about to be destroyed is first dropped from those
// records (forget_stream, after its work has finished).  Requests are served from blocks of
// up to twice the rounded size.
#pragma once

#include <stddef.h>

#include <map>
#include <mutex>
#include <unordered_map>
#include <utility>
#include <vector>

namespace lq {

// How completion markers are made and read.  record() returns nullptr when no marker can be
// recorded on that stream; the cache then keeps the block bound to the stream.
struct MarkerOps {
    void* (*record)(void* stream);
    bool (*done)(void* marker);
    void (*release)(void* marker);
};

class BlockCache {
public:
    struct FreeBlock {
        void* ptr;
        void* stream;  // stream of the last use (the free's stream)
        void* marker;  // completion marker on that stream, or nullptr (stream-bound)
        std::vector<void*> uses;  // markers on the other streams that used it (nullptr: none recordable)
    };

    explicit BlockCache(MarkerOps ops) : ops_(ops) {}

    // Size class of a request: 512-byte granules up to 1 MiB, 2 MiB granules above.
    static size_t round_size(size_t bytes) {
        if (bytes == 0) bytes = 1;
        if (bytes <= (size_t(1) << 20)) return (bytes + 511) & ~size_t(511);
        return (bytes + (size_t(2) << 20) - 1) & ~((size_t(2) << 20) - 1);
    }

    // A cached block of at least `rounded` bytes (at most twice that) safe to use on
    // `stream`, registered as live; nullptr when none qualifies.
    void* take(int device, size_t rounded, void* stream) {
        std::lock_guard<std::mutex> g(mu_);
        auto& fl = free_[device];
        for (auto it = fl.lower_bound(rounded); it != fl.end() && it->first <= 2 * rounded; ++it) {
            FreeBlock& b = it->second;
            const bool same_stream = b.stream == stream;
            if (!same_stream && !(b.marker && ops_.done(b.marker))) continue;
            bool uses_done = true;
            for (void* m : b.uses) uses_done = uses_done && m && ops_.done(m);
            if (!uses_done) continue;
            void* p = b.ptr;
            const size_t got = it->first;
            if (b.marker) ops_.release(b.marker);
            for (void* m : b.uses) ops_.release(m);
            fl.erase(it);
            live_[p] = Live{got, device, {}};
            cached_ -= got;
            allocated_ += got;
            return p;
        }
        return nullptr;
    }

    // Registers a fresh allocation as live.
    void add_live(void* p, int device, size_t rounded) {
        std::lock_guard<std::mutex> g(mu_);
        live_[p] = Live{rounded, device, {}};
        allocated_ += rounded;
    }

    // Marks a live block as used on `stream` besides the one it will be freed on; false if
    // `p` is not live.
    bool record_use(void* p, void* stream) {
        std::lock_guard<std::mutex> g(mu_);
        auto it = live_.find(p);
        if (it == live_.end()) return false;
        auto& u = it->second.uses;
        bool seen = false;
        for (void* s : u) seen = seen || s == stream;
        if (!seen) u.push_back(stream);
        return true;
    }

    // Drops `stream` from every live block's recorded uses: the caller has waited for the
    // stream's work and is about to destroy it, and a free must not record a marker on a
    // destroyed stream.
    void forget_stream(void* stream) {
        std::lock_guard<std::mutex> g(mu_);
        for (auto& kv : live_) {
            auto& u = kv.second.uses;
            for (size_t i = 0; i < u.size();)
                if (u[i] == stream) u.erase(u.begin() + (long)i);
                else ++i;
        }
    }

    // Returns a live block to the cache as last used on `stream`; false if `p` is not live.
    bool put(void* p, void* stream) {
        std::lock_guard<std::mutex> g(mu_);
        auto it = live_.find(p);
        if (it == live_.end()) return false;
        const Live l = it->second;
        live_.erase(it);
        allocated_ -= l.size;
        cached_ += l.size;
        FreeBlock fb{p, stream, ops_.record(stream), {}};
        for (void* s : l.uses)
            if (s != stream) fb.uses.push_back(ops_.record(s));
        free_[l.device].emplace(l.size, std::move(fb));
        return true;
    }

    // Removes every cached block, releasing their markers; returns (device, pointer) pairs
    // for the caller to free.
    std::vector<std::pair<int, void*>> drain() {
        std::lock_guard<std::mutex> g(mu_);
        std::vector<std::pair<int, void*>> out;
        for (auto& kv : free_)
            for (auto& e : kv.second) {
                if (e.second.marker) ops_.release(e.second.marker);
                for (void* m : e.second.uses)
                    if (m) ops_.release(m);
                out.emplace_back(kv.first, e.second.ptr);
            }
        free_.clear();
        cached_ = 0;
        return out;
    }

    void stats(size_t* allocated, size_t* cached) {
        std::lock_guard<std::mutex> g(mu_);
        if (allocated) *allocated = allocated_;
        if (cached) *cached = cached_;
    }

private:
    struct Live {
        size_t size;
        int device;
        std::vector<void*> uses;  // streams recorded by record_use
    };
    MarkerOps ops_;
    std::mutex mu_;
    std::unordered_map<void*, Live> live_;
    std::map<int, std::multimap<size_t, FreeBlock>> free_;
    size_t allocated_ = 0;
    size_t cached_ = 0;
};

}  // namespace lq
