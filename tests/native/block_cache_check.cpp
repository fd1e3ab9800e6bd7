// CPU check of the caching allocator's bookkeeping (lucid_amd/csrc/lq_block_cache.h) with
// fake completion markers: same-stream reuse, cross-stream reuse only after completion,
// stream-bound blocks without a marker, side-stream uses (record_use), the size window,
// per-device lists, stats and drain.
// Built and run by tests/test_block_cache.py; prints "ok" and exits 0 on success.
#include <cstdio>
#include <cstdlib>
#include <set>

#include "lq_block_cache.h"

namespace {
struct FakeMarker {
    bool done;
    void* stream;
};
std::set<FakeMarker*> g_live_markers;
bool g_no_marker_streams = false;  // when set, record() refuses (as under graph capture)

void* rec(void* stream) {
    if (g_no_marker_streams) return nullptr;
    auto* m = new FakeMarker{false, stream};
    g_live_markers.insert(m);
    return m;
}
bool done(void* m) { return static_cast<FakeMarker*>(m)->done; }
void rel(void* m) {
    g_live_markers.erase(static_cast<FakeMarker*>(m));
    delete static_cast<FakeMarker*>(m);
}
void complete_all(void* stream) {
    for (auto* m : g_live_markers)
        if (m->stream == stream) m->done = true;
}

int g_fail = 0;
#define CHECK(c)                                                   \
    do {                                                           \
        if (!(c)) {                                                \
            std::fprintf(stderr, "FAIL line %d: %s\n", __LINE__, #c); \
            g_fail = 1;                                            \
        }                                                          \
    } while (0)
}  // namespace

int main() {
    using lq::BlockCache;
    BlockCache c(lq::MarkerOps{rec, done, rel});
    void* s1 = reinterpret_cast<void*>(0x10);
    void* s2 = reinterpret_cast<void*>(0x20);
    char pool[16];
    void* a = &pool[0];
    void* b = &pool[1];

    CHECK(BlockCache::round_size(0) == 512 && BlockCache::round_size(513) == 1024);
    CHECK(BlockCache::round_size((1u << 20) + 1) == (size_t(2) << 20));

    // a live block freed on s1: reusable on s1 at once, on s2 only after completion
    c.add_live(a, 0, 4096);
    CHECK(c.put(a, s1));
    CHECK(!c.put(a, s1));  // double free refused
    CHECK(c.take(0, 4096, s2) == nullptr);
    CHECK(c.take(0, 4096, s1) == a);
    CHECK(g_live_markers.empty());  // the marker is released on reuse
    CHECK(c.put(a, s1));
    complete_all(s1);
    CHECK(c.take(0, 4096, s2) == a);

    // size window: a cached 4096 block serves 2048..4096 requests, not 1024 or 8192
    CHECK(c.put(a, s1));
    CHECK(c.take(0, 1024, s1) == nullptr);
    CHECK(c.take(0, 8192, s1) == nullptr);
    CHECK(c.take(0, 2048, s1) == a);

    // per-device lists
    CHECK(c.put(a, s1));
    CHECK(c.take(1, 4096, s1) == nullptr);

    // a pending block on another stream is skipped in favour of a usable one
    c.add_live(b, 0, 4096);
    CHECK(c.put(b, s2));  // b pending on s2; a still cached on s1 (pending)
    void* got = c.take(0, 4096, s2);
    CHECK(got == b);

    // no marker (graph capture): stream-bound even after everything completes
    g_no_marker_streams = true;
    CHECK(c.put(b, s2));
    g_no_marker_streams = false;
    complete_all(s2);
    CHECK(c.take(0, 4096, s1) == a);  // a: freed on s1, same stream
    CHECK(c.put(a, s1));
    complete_all(s1);
    CHECK(c.take(0, 4096, reinterpret_cast<void*>(0x30)) == a);  // a completed: any stream
    CHECK(c.take(0, 4096, reinterpret_cast<void*>(0x30)) == nullptr);  // b: bound to s2
    CHECK(c.take(0, 4096, s2) == b);

    // side-stream use (record_use): a block freed on the null stream after work on s2 read
    // it is reused -- even on the null stream itself -- only after s2's work completes
    void* s0 = nullptr;
    CHECK(c.put(a, s1) && c.put(b, s2));
    complete_all(s1);
    complete_all(s2);
    CHECK(c.take(0, 4096, s0) != nullptr && c.take(0, 4096, s0) != nullptr);  // a and b, live again
    CHECK(!c.record_use(&pool[2], s2));  // not live
    CHECK(c.record_use(a, s2) && c.record_use(a, s2));  // recorded once
    CHECK(c.put(a, s0));
    CHECK(c.take(0, 4096, s0) == nullptr);  // s2's marker pending: not even on the free stream
    complete_all(s0);
    CHECK(c.take(0, 4096, s1) == nullptr);
    complete_all(s2);
    CHECK(c.take(0, 4096, s0) == a);
    // a use stream that cannot record a marker keeps the block out until drain
    CHECK(c.record_use(a, s2));
    g_no_marker_streams = true;
    CHECK(c.put(a, s1));  // neither s1 nor s2 can record
    g_no_marker_streams = false;
    CHECK(c.take(0, 4096, s1) == nullptr);
    // the use list does not survive a free: a's next life starts clean
    CHECK(c.put(b, s0));
    complete_all(s0);
    CHECK(c.take(0, 4096, s2) == b);
    CHECK(c.put(b, s2));
    CHECK(c.take(0, 4096, s2) == b);
    (void)c.drain();  // a (held back) goes to the caller; markers released
    CHECK(c.take(0, 4096, s1) == nullptr);
    c.add_live(a, 0, 4096);
    // a use stream destroyed before the free (forget_stream): no marker is recorded on it
    CHECK(c.record_use(a, s2));
    c.forget_stream(s2);
    const size_t before = g_live_markers.size();
    CHECK(c.put(a, s1));
    CHECK(g_live_markers.size() == before + 1);  // only s1's
    CHECK(c.take(0, 4096, s1) == a);

    // stats and drain
    size_t al = 0, ca = 0;
    c.stats(&al, &ca);
    CHECK(al == 8192 && ca == 0);
    CHECK(c.put(a, s1) && c.put(b, s2));
    c.stats(&al, &ca);
    CHECK(al == 0 && ca == 8192);
    auto v = c.drain();
    CHECK(v.size() == 2);
    CHECK(g_live_markers.empty());
    c.stats(&al, &ca);
    CHECK(al == 0 && ca == 0);
    CHECK(c.take(0, 4096, s1) == nullptr);

    if (g_fail) return 1;
    std::printf("ok\n");
    return 0;
}
