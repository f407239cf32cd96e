// Host-only check of the workspace growth rules (csrc/workspace_pool.hpp):
// no shrink, retire-not-free on growth, refusal while capturing, the
// allocator's error passed back with the pool unchanged.  Built with g++
// (address and undefined-behaviour sanitizers) by tests/test_workspace_pool.py.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "workspace_pool.hpp"

static int failures = 0;
#define CHECK(c)                                                    \
    do {                                                            \
        if (!(c)) {                                                 \
            std::fprintf(stderr, "FAILED %s:%d: %s\n", __FILE__, __LINE__, #c); \
            ++failures;                                             \
        }                                                           \
    } while (0)

struct FakeAlloc {
    std::vector<void*> live;   // every buffer handed out (never freed by the pool)
    std::vector<size_t> sizes;
    int fail_next = 0;
    int operator()(void** p, size_t n) {
        if (fail_next) {
            const int rc = fail_next;
            fail_next = 0;
            return rc;
        }
        *p = std::malloc(n);
        live.push_back(*p);
        sizes.push_back(n);
        return 0;
    }
};

int main() {
    rt_hip::WorkspacePool pool;
    FakeAlloc a;
    auto alloc = [&](void** p, size_t n) { return a(p, n); };

    CHECK(pool.reserve(0, false, alloc) == 0 && pool.cur == nullptr && a.live.empty());
    // first growth: at least the 1 MiB floor
    CHECK(pool.reserve(100, false, alloc) == 0);
    CHECK(pool.bytes == rt_hip::WorkspacePool::kMinBytes && a.sizes.back() == pool.bytes);
    void* first = pool.cur;
    // a smaller or equal request reuses the buffer, even while capturing
    CHECK(pool.reserve(pool.bytes, true, alloc) == 0 && pool.cur == first && a.live.size() == 1);
    // growth while capturing is refused and leaves the pool as it was
    CHECK(pool.reserve(pool.bytes + 1, true, alloc) == rt_hip::WorkspacePool::kRefused);
    CHECK(pool.cur == first && a.live.size() == 1 && pool.retired.empty());
    // growth outside capture: new buffer, the old one retired (still live)
    CHECK(pool.reserve(3u << 20, false, alloc) == 0);
    CHECK(pool.cur != first && pool.bytes == (3u << 20));
    CHECK(pool.retired.size() == 1 && pool.retired[0] == first);
    // a failing allocation passes its code back and changes nothing
    void* second = pool.cur;
    a.fail_next = 2;
    CHECK(pool.reserve(8u << 20, false, alloc) == 2);
    CHECK(pool.cur == second && pool.bytes == (3u << 20) && pool.retired.size() == 1);
    // every buffer ever handed out is either current or retired
    CHECK(pool.reserve(16u << 20, false, alloc) == 0 && pool.retired.size() == 2);
    for (void* p : a.live) {
        bool found = p == pool.cur;
        for (void* r : pool.retired) found = found || r == p;
        CHECK(found);
    }
    for (void* p : a.live) std::free(p);
    if (failures) return 1;
    std::printf("workspace pool: all checks passed\n");
    return 0;
}
