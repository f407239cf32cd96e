// workspace_pool.hpp -- the grow-only bookkeeping of a per-device workspace,
// kept apart from the HIP allocator so that its rules can be checked by a
// host-only test (tests/cpp/test_workspace_pool.cpp):
//  * a request no larger than the current buffer returns it unchanged;
//  * a larger one allocates a new buffer (at least kMinBytes) and RETIRES the
//    old one -- it is never freed, because a hipGraph captured while it was
//    current keeps writing it on every replay;
//  * growth is refused while the caller's stream is being captured, since an
//    allocation cannot become part of a graph.
#pragma once

#include <cstddef>
#include <vector>

namespace rt_hip {

struct WorkspacePool {
    static constexpr size_t kMinBytes = size_t{1} << 20;
    static constexpr int kRefused = -1;  // growth needed during capture

    void* cur = nullptr;
    size_t bytes = 0;
    std::vector<void*> retired;

    // Ensures at least `need` bytes.  `alloc(void** p, size_t n)` returns 0 on
    // success or its own nonzero error code, which is passed back.
    template <class Alloc>
    int reserve(size_t need, bool capturing, Alloc&& alloc) {
        if (need <= bytes) return 0;
        if (capturing) return kRefused;
        const size_t sz = need < kMinBytes ? kMinBytes : need;
        void* p = nullptr;
        const int rc = alloc(&p, sz);
        if (rc != 0) return rc;
        if (cur) retired.push_back(cur);
        cur = p;
        bytes = sz;
        return 0;
    }
};

}  // namespace rt_hip
