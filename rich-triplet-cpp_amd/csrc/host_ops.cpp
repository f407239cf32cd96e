// host_ops.cpp -- the host-facing layer of the C ABI:
//  * weight handles: a weight uploaded once (verbatim bytes, plus the tiled
//    copy of a Q4_K weight for the M = 1 GEMV) and run on device activations;
//  * host drop-ins: host activations in, host outputs out, the weight cached
//    on the device by (host pointer, byte length) -- the reference's Metal
//    ops (metal_gemv_q4k_t / metal_gemv_bf16_t / metal_matmul_q4_t and
//    cached_weights, src/metal_ops.mm:425-434, 578-675);
//  * hipGraph capture of a call sequence (the analogue of the decode
//    engine's one command buffer, src/metal_decode.mm:436-482).
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "rt_hip.h"
#include "rt_launch.hpp"

struct rt_hip_weight {
    int device = -1;
    int32_t format = 0;
    int64_t n = 0, k = 0, bytes = 0;
    void* data = nullptr;   // verbatim bytes
    void* tiled = nullptr;  // Q4_K: tiled copy for the M = 1 GEMV (or null)
};

struct rt_hip_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace rt_hip {
namespace {

int fail(int code, const std::string& msg) { return set_error(code, msg); }
int hip_fail(hipError_t e, const std::string& what) {
    return set_error(RT_HIP_E_HIP, what + ": " + hipGetErrorString(e));
}

// Bytes a weight of this format and shape occupies (-1: not valid).
int64_t format_bytes(int32_t format, int64_t n, int64_t k) {
    if (n <= 0 || k <= 0) return -1;
    switch (format) {
        case RT_HIP_F32: return n * k * 4;
        case RT_HIP_BF16: return n * k * 2;
        case RT_HIP_Q4K: return k % 256 ? -1 : n * (k / 256) * 144;
        case RT_HIP_Q4_0: return k % 32 ? -1 : n * (k / 32) * 18;
        case RT_HIP_Q4MAT: return rt_hip_q4mat_bytes(n, k);
        default: return -1;
    }
}

// ---- host drop-ins ----------------------------------------------------------

struct HostDevice {
    std::map<std::tuple<uintptr_t, int64_t, uintptr_t>, rt_hip_weight*> cache;
    int64_t cached_bytes = 0;
    hipStream_t stream = nullptr;
    float* act = nullptr;  // staged activations
    float* out = nullptr;  // outputs before the copy back
    size_t act_cap = 0, out_cap = 0;
};

constexpr int kMaxDevices = 64;
std::mutex g_host_mu;
HostDevice g_host[kMaxDevices];

int grow(float** buf, size_t* cap, size_t elems, const char* fn) {
    if (elems <= *cap) return RT_HIP_OK;
    if (*buf) (void)hipFree(*buf);  // host calls are synchronous: nothing uses it now
    *buf = nullptr;
    *cap = 0;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(buf), elems * 4);
    if (e != hipSuccess) return e == hipErrorOutOfMemory ? fail(RT_HIP_E_OOM, std::string(fn) + ": out of memory")
                                                          : hip_fail(e, fn);
    *cap = elems;
    return RT_HIP_OK;
}

}  // namespace
}  // namespace rt_hip

using namespace rt_hip;

extern "C" {

int rt_hip_weight_upload(int32_t format, const void* host, int64_t bytes, int64_t n, int64_t k, int32_t flags,
                         rt_hip_weight** out) {
    const char* fn = "rt_hip_weight_upload";
    if (!out) return fail(RT_HIP_E_ARG, std::string(fn) + ": null output");
    *out = nullptr;
    if (!host) return fail(RT_HIP_E_ARG, std::string(fn) + ": null host pointer");
    const int64_t want = format_bytes(format, n, k);
    if (want < 0) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": invalid format or shape");
    if (bytes != want)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": " + std::to_string(bytes) + " bytes given, the format needs " +
                                        std::to_string(want));
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, fn);
    auto* w = new rt_hip_weight();
    w->device = dev;
    w->format = format;
    w->n = n;
    w->k = k;
    w->bytes = bytes;
    e = hipMalloc(&w->data, static_cast<size_t>(bytes));
    if (e == hipSuccess) e = hipMemcpy(w->data, host, static_cast<size_t>(bytes), hipMemcpyHostToDevice);
    if (e == hipSuccess && format == RT_HIP_Q4K && (flags & RT_HIP_WEIGHT_TILED)) {
        const int64_t tb = rt_hip_q4k_tiled_bytes(n, k);
        e = hipMalloc(&w->tiled, static_cast<size_t>(tb));
        if (e == hipSuccess) {
            const int rc = rt_hip_q4k_tile(w->data, w->tiled, n, k, nullptr);
            if (rc) {
                rt_hip_weight_free(w);
                return rc;
            }
            e = hipDeviceSynchronize();
        }
    }
    if (e != hipSuccess) {
        rt_hip_weight_free(w);
        return e == hipErrorOutOfMemory ? fail(RT_HIP_E_OOM, std::string(fn) + ": out of device memory")
                                        : hip_fail(e, fn);
    }
    *out = w;
    return RT_HIP_OK;
}

int rt_hip_weight_free(rt_hip_weight* w) {
    if (!w) return RT_HIP_OK;
    if (w->data) (void)hipFree(w->data);
    if (w->tiled) (void)hipFree(w->tiled);
    delete w;
    return RT_HIP_OK;
}

const void* rt_hip_weight_data(const rt_hip_weight* w) { return w ? w->data : nullptr; }

int rt_hip_weight_linear(const rt_hip_weight* w, const float* x, const float* bias, float* y, int64_t m,
                         rt_hip_stream stream) {
    const char* fn = "rt_hip_weight_linear";
    if (!w) return fail(RT_HIP_E_ARG, std::string(fn) + ": null weight");
    if (w->format == RT_HIP_F32) return fail(RT_HIP_E_UNSUPPORTED, std::string(fn) + ": f32 weights are not run here");
    if (m == 1 && w->tiled) {
        int rc = rt_hip_gemv_q4k_tiled(w->tiled, x, y, w->n, w->k, stream);
        if (rc || !bias) return rc;
        const hipError_t e = launch_add_bias(y, bias, 1, w->n, static_cast<hipStream_t>(stream));
        return e == hipSuccess ? RT_HIP_OK : hip_fail(e, fn);
    }
    return rt_hip_linear_forward(w->format, w->data, bias, x, y, m, w->n, w->k, stream);
}

int rt_hip_host_matmul(int32_t format, const void* w_host, int64_t w_bytes, const void* w2_host, int64_t n,
                       int64_t k, const float* x_host, float* y_host, int64_t m) {
    const char* fn = "rt_hip_host_matmul";
    if (!w_host || !x_host || !y_host) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (m <= 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": m must be > 0");
    if (format == RT_HIP_F32) return fail(RT_HIP_E_UNSUPPORTED, std::string(fn) + ": f32 weights are not run here");
    if (format == RT_HIP_Q4MAT && !w2_host) return fail(RT_HIP_E_ARG, std::string(fn) + ": Q4Mat needs its scales");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, fn);
    if (dev < 0 || dev >= kMaxDevices) return fail(RT_HIP_E_UNSUPPORTED, std::string(fn) + ": device ordinal");
    std::lock_guard<std::mutex> lk(g_host_mu);
    HostDevice& hd = g_host[dev];
    if (!hd.stream) {
        e = hipStreamCreateWithFlags(&hd.stream, hipStreamNonBlocking);
        if (e != hipSuccess) return hip_fail(e, fn);
    }
    // The weight: uploaded once, found again by (host pointer, byte length)
    // (and, for Q4Mat, the scales' pointer): cached_weights,
    // src/metal_ops.mm:425-434.  The caller keeps the host buffer unchanged
    // at that address for as long as it uses the cache, as with the
    // reference; rt_hip_host_cache_clear drops every entry.
    const auto key = std::make_tuple(reinterpret_cast<uintptr_t>(w_host), w_bytes,
                                     reinterpret_cast<uintptr_t>(w2_host));
    rt_hip_weight* w = nullptr;
    const auto it = hd.cache.find(key);
    if (it != hd.cache.end()) {
        w = it->second;
        if (w->format != format || w->n != n || w->k != k)
            return fail(RT_HIP_E_ARG, std::string(fn) + ": a cached weight at this address has another format or shape");
    } else {
        int rc;
        if (format == RT_HIP_Q4MAT) {
            // Q4Mat's two arrays (packed nibbles, f32 scales) become one
            // RT_HIP_Q4MAT buffer.
            const int64_t total = rt_hip_q4mat_bytes(n, k);
            if (total < 0) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": Q4Mat needs k % 32 == 0");
            if (w_bytes != (n * k + 1) / 2) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": packed size mismatch");
            std::string buf(static_cast<size_t>(total), '\0');
            std::memcpy(&buf[0], w_host, static_cast<size_t>(w_bytes));
            std::memcpy(&buf[static_cast<size_t>(rt_hip_q4mat_scales_offset(n, k))], w2_host,
                        static_cast<size_t>(n * k / 32) * 4);
            rc = rt_hip_weight_upload(format, buf.data(), total, n, k, 0, &w);
        } else {
            rc = rt_hip_weight_upload(format, w_host, w_bytes, n, k, 0, &w);
        }
        if (rc) return rc;
        hd.cache.emplace(key, w);
        hd.cached_bytes += w->bytes;
    }
    int rc = grow(&hd.act, &hd.act_cap, static_cast<size_t>(m * k), fn);
    if (!rc) rc = grow(&hd.out, &hd.out_cap, static_cast<size_t>(m * n), fn);
    if (rc) return rc;
    e = hipMemcpyAsync(hd.act, x_host, static_cast<size_t>(m * k) * 4, hipMemcpyHostToDevice, hd.stream);
    if (e != hipSuccess) return hip_fail(e, fn);
    rc = rt_hip_linear_forward(format, w->data, nullptr, hd.act, hd.out, m, n, k, hd.stream);
    if (rc) return rc;
    e = hipMemcpyAsync(y_host, hd.out, static_cast<size_t>(m * n) * 4, hipMemcpyDeviceToHost, hd.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(hd.stream);
    if (e != hipSuccess) return hip_fail(e, fn);
    return RT_HIP_OK;
}

int rt_hip_host_cache_clear(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_host_cache_clear");
    if (dev < 0 || dev >= kMaxDevices) return RT_HIP_OK;
    std::lock_guard<std::mutex> lk(g_host_mu);
    HostDevice& hd = g_host[dev];
    if (hd.stream) (void)hipStreamSynchronize(hd.stream);
    for (auto& kv : hd.cache) rt_hip_weight_free(kv.second);
    hd.cache.clear();
    hd.cached_bytes = 0;
    return RT_HIP_OK;
}

int64_t rt_hip_host_cache_bytes(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
    std::lock_guard<std::mutex> lk(g_host_mu);
    return g_host[dev].cached_bytes;
}

// ---- graphs -------------------------------------------------------------------

int rt_hip_graph_begin(rt_hip_stream stream) {
    const hipError_t e = hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal);
    return e == hipSuccess ? RT_HIP_OK : hip_fail(e, "rt_hip_graph_begin");
}

int rt_hip_graph_end(rt_hip_stream stream, rt_hip_graph** out) {
    const char* fn = "rt_hip_graph_end";
    if (!out) return fail(RT_HIP_E_ARG, std::string(fn) + ": null output");
    *out = nullptr;
    auto* g = new rt_hip_graph();
    hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        rt_hip_graph_destroy(g);
        return hip_fail(e, fn);
    }
    *out = g;
    return RT_HIP_OK;
}

int rt_hip_graph_launch(const rt_hip_graph* g, rt_hip_stream stream) {
    if (!g || !g->exec) return fail(RT_HIP_E_ARG, "rt_hip_graph_launch: null graph");
    const hipError_t e = hipGraphLaunch(g->exec, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RT_HIP_OK : hip_fail(e, "rt_hip_graph_launch");
}

int rt_hip_graph_destroy(rt_hip_graph* g) {
    if (!g) return RT_HIP_OK;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return RT_HIP_OK;
}

}  // extern "C"
