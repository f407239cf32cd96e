// api.cpp -- the C ABI (include/rt_hip.h): argument validation, device
// bookkeeping, workspaces and dispatch to the kernel launchers.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "rt_hip.h"
#include "rt_launch.hpp"
#include "workspace_pool.hpp"

namespace rt_hip {
namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(RT_HIP_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

struct DeviceState {
    DeviceInfo info;
    bool ok = false;
    WorkspacePool ws;              // grow-only; replaced buffers are retired, never freed
    uint32_t* counters = nullptr;  // arrival counters, zero between launches
};

// Fixed storage: a DeviceState's address stays valid for the process.
constexpr int kMaxDevices = 64;
std::mutex g_mu;
DeviceState g_dev[kMaxDevices];

DeviceState* state_for_current(hipError_t* err) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *err = e;
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState& st = g_dev[dev];
    if (!st.ok) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) {
            *err = e;
            return nullptr;
        }
        st.info.ordinal = dev;
        st.info.cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
        st.info.lds_per_block = prop.sharedMemPerBlock;
        st.ok = true;
    }
    *err = hipSuccess;
    return &st;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Byte ranges [a, a + na) and [b, b + nb) intersect.
bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return pa < pb + static_cast<uintptr_t>(nb) && pb < pa + static_cast<uintptr_t>(na);
}

int check_stream_launch(hipError_t e, const char* what) {
    if (e == hipErrorStreamCaptureUnsupported)
        return fail(RT_HIP_E_HIP, std::string(what) +
                                      ": the workspace must grow, which cannot happen while the stream is "
                                      "captured (call rt_hip_reserve_workspace / rt_hip_init before capture)");
    if (e != hipSuccess) return hip_fail(e, what);
    return RT_HIP_OK;
}

// Common GEMV argument checks.  Returns 0 or an error code.
int gemv_args(const char* fn, const void* w, const float* x, const float* y, int64_t n,
              int64_t k, int32_t m, int64_t k_multiple) {
    if (!w || !x || !y) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (n <= 0 || k <= 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": n and k must be > 0");
    if (m < 1 || m > RT_HIP_GEMV_MAX_M)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": m must be in [1, 8]");
    if (k % k_multiple != 0)
        return fail(RT_HIP_E_ALIGN,
                    std::string(fn) + ": k must be a multiple of " + std::to_string(k_multiple));
    if (n > 0x7fffffffLL || k > 0x7fffffffLL)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": n and k must fit in int32");
    if (!aligned16(w) || !aligned16(x))
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": w and x must be 16-byte aligned");
    // Every workgroup reads all of x while others already store rows of y.
    if (overlaps(y, n * m * 4, x, k * m * 4)) return fail(RT_HIP_E_ARG, std::string(fn) + ": y overlaps x");
    return RT_HIP_OK;
}

// Runs a GEMV in batches of activation rows that fit the LDS budget.
template <typename F>
int gemv_batched(const char* fn, int fmt, const float* x, float* y, int64_t n, int64_t k,
                 int32_t m, F&& launch) {
    hipError_t e;
    DeviceState* st = state_for_current(&e);
    if (!st) return hip_fail(e, fn);
    const size_t cap = lds_cap();
    int mb = m;
    while (mb > 1 && gemv_lds_bytes(fmt, mb, k) > cap) --mb;
    if (gemv_lds_bytes(fmt, mb, k) > cap)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k too large for the LDS-staged GEMV");
    for (int32_t m0 = 0; m0 < m; m0 += mb) {
        const int32_t mm = (m - m0) < mb ? (m - m0) : mb;
        e = launch(x + static_cast<size_t>(m0) * k, y + static_cast<size_t>(m0) * n, mm);
        if (e != hipSuccess) return hip_fail(e, fn);
    }
    return RT_HIP_OK;
}

}  // namespace

int set_error(int code, const std::string& msg) { return fail(code, msg); }

const DeviceInfo& device_info() {
    hipError_t e;
    DeviceState* st = state_for_current(&e);
    static DeviceInfo fallback;
    return st ? st->info : fallback;
}

size_t lds_cap() {
    const size_t b = device_info().lds_per_block;
    return b >= 65536 ? b : 65536;
}

int tune_param(const char* name, int fallback) {
#ifdef RT_HIP_TUNING
    // Sweep builds only (make TUNING=1): RT_HIP_<name> overrides a launch
    // shape.  The library as shipped always runs the measured defaults.
    // The environment is read once per name; an unset name keeps every
    // call's own default (which differs between launch shapes).
    static std::mutex mu;
    static std::vector<std::pair<std::string, std::pair<bool, int>>> cache;
    std::lock_guard<std::mutex> lk(mu);
    for (const auto& kv : cache)
        if (kv.first == name) return kv.second.first ? kv.second.second : fallback;
    const std::string env = std::string("RT_HIP_") + name;
    const char* s = std::getenv(env.c_str());
    cache.emplace_back(name, std::make_pair(s != nullptr, s ? std::atoi(s) : 0));
    return s ? std::atoi(s) : fallback;
#else
    (void)name;
    return fallback;
#endif
}

namespace {

// True when `s` (or, for the legacy stream, any stream) is being captured
// into a hipGraph: no allocation or synchronisation may happen then.
bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) return false;
    return st != hipStreamCaptureStatusNone;
}

// Grows st's workspace to `bytes` (caller holds g_mu); `capture`: the
// caller's stream is being captured, so no allocation may happen.
hipError_t grow_workspace(DeviceState* st, size_t bytes, bool capture) {
    const int rc = st->ws.reserve(bytes, capture, [](void** p, size_t n) { return static_cast<int>(hipMalloc(p, n)); });
    if (rc == WorkspacePool::kRefused) return hipErrorStreamCaptureUnsupported;
    return static_cast<hipError_t>(rc);
}

// Allocates and zeroes st's arrival counters (caller holds g_mu; never
// while a stream is being captured).
hipError_t make_counters(DeviceState* st) {
    if (st->counters) return hipSuccess;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, kArrivalCounters * sizeof(uint32_t));
    if (e != hipSuccess) return e;
    e = hipMemset(p, 0, kArrivalCounters * sizeof(uint32_t));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(p);
        return e;
    }
    st->counters = static_cast<uint32_t*>(p);
    return hipSuccess;
}

}  // namespace

void* workspace(size_t bytes, hipStream_t s, hipError_t* err) {
    DeviceState* st = state_for_current(err);
    if (!st) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    if (st->ws.bytes < bytes) {
        *err = grow_workspace(st, bytes, capturing(s));
        if (*err != hipSuccess) return nullptr;
    }
    *err = hipSuccess;
    return st->ws.cur;
}

uint32_t* arrival_counters(hipStream_t s, hipError_t* err) {
    DeviceState* st = state_for_current(err);
    if (!st) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!st->counters) {
        if (capturing(s)) {
            *err = hipErrorStreamCaptureUnsupported;
            return nullptr;
        }
        *err = make_counters(st);
        if (*err != hipSuccess) return nullptr;
    }
    *err = hipSuccess;
    return st->counters;
}

}  // namespace rt_hip

using namespace rt_hip;

extern "C" {

const char* rt_hip_last_error(void) { return g_last_error.c_str(); }

const char* rt_hip_version(void) { return "rt_hip 0.1 gfx950"; }

int rt_hip_init(int ordinal) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_init");
    if (ordinal < 0 || ordinal >= count)
        return fail(RT_HIP_E_ARG, "rt_hip_init: no device " + std::to_string(ordinal));
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, ordinal);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_init");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(RT_HIP_E_UNSUPPORTED,
                    std::string("rt_hip_init: device is ") + prop.gcnArchName + ", not gfx950");
    e = hipSetDevice(ordinal);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_init");
    DeviceState* st = state_for_current(&e);
    if (!st) return hip_fail(e, "rt_hip_init");
    {
        std::lock_guard<std::mutex> lk(g_mu);
        e = make_counters(st);
    }
    if (e != hipSuccess) return hip_fail(e, "rt_hip_init: arrival counters");
    e = attention_scratch_setup(ordinal, nullptr);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_init: attention scratch address");
    return RT_HIP_OK;
}

int rt_hip_reserve_workspace(int64_t bytes) {
    const char* fn = "rt_hip_reserve_workspace";
    if (bytes < 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": bytes must be >= 0");
    hipError_t e;
    DeviceState* st = state_for_current(&e);
    if (!st) return hip_fail(e, fn);
    std::lock_guard<std::mutex> lk(g_mu);
    e = make_counters(st);
    if (e == hipSuccess) e = grow_workspace(st, static_cast<size_t>(bytes), false);
    if (e == hipErrorOutOfMemory) return fail(RT_HIP_E_OOM, std::string(fn) + ": device allocation failed");
    if (e != hipSuccess) return hip_fail(e, fn);
    return RT_HIP_OK;
}

int64_t rt_hip_gemm_workspace_bytes(int32_t format, int32_t a_dtype, int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || (a_dtype != RT_HIP_F32 && a_dtype != RT_HIP_BF16)) return -1;
    if ((format == RT_HIP_Q4_0 || format == RT_HIP_Q4MAT) &&
        gemm_dequant_in_kernel(format, a_dtype == RT_HIP_BF16, m, n, k))
        return static_cast<int64_t>(gemm_workspace_bytes(format, a_dtype == RT_HIP_BF16, m, n, k));
    if (format == RT_HIP_Q4_0 || format == RT_HIP_Q4MAT)
        return static_cast<int64_t>((gemm_workspace_bytes(RT_HIP_BF16, a_dtype == RT_HIP_BF16, m, n, k) + 255) /
                                        256 * 256 +
                                    static_cast<size_t>(n * k) * 2);
    if (format != RT_HIP_Q4K && format != RT_HIP_BF16) return -1;
    return static_cast<int64_t>(gemm_workspace_bytes(format, a_dtype == RT_HIP_BF16, m, n, k));
}

int64_t rt_hip_gemv_workspace_bytes(int32_t format, int64_t n, int64_t k, int32_t m) {
    if (n <= 0 || k <= 0 || m < 1 || m > RT_HIP_GEMV_MAX_M) return -1;
    if (m == 1 || (format != RT_HIP_Q4K && format != RT_HIP_BF16)) return 0;
    return static_cast<int64_t>(gemv_batch_workspace_bytes(format, n, k, m));
}

int64_t rt_hip_attention_workspace_bytes(int32_t n_q_heads, int32_t n_kv_heads, int64_t seq_len) {
    if (n_kv_heads < 1 || n_q_heads < n_kv_heads || seq_len < 1) return -1;
    return static_cast<int64_t>(attention_decode_workspace(n_q_heads, n_kv_heads, seq_len));
}

int64_t rt_hip_workspace_bytes(void) {
    hipError_t e;
    DeviceState* st = state_for_current(&e);
    if (!st) return -1;
    std::lock_guard<std::mutex> lk(g_mu);
    return static_cast<int64_t>(st->ws.bytes);
}

int rt_hip_gemv_q4k(const void* blocks, const float* x, float* y, int64_t n, int64_t k,
                    int32_t m, rt_hip_stream stream) {
    int rc = gemv_args("rt_hip_gemv_q4k", blocks, x, y, n, k, m, 256);
    if (rc) return rc;
    if (m > 1 && tune_param("GEMV_BATCH_MFMA", 1))
        return check_stream_launch(launch_gemv_batch(RT_HIP_Q4K, blocks, x, y, n, k, m, static_cast<hipStream_t>(stream)),
                                   "rt_hip_gemv_q4k");
    if (m == 1) {
        // the int8-MFMA kernel stages 3.5 bytes per value (the VALU kernel's
        // bound below is 4.25)
        hipError_t e;
        if (!state_for_current(&e)) return hip_fail(e, "rt_hip_gemv_q4k");
        if (q4k_m1_lds_bytes(k) > lds_cap())
            return fail(RT_HIP_E_SHAPE, "rt_hip_gemv_q4k: k too large for the LDS");
        return check_stream_launch(launch_gemv_q4k_mfma(blocks, x, y, n, k, static_cast<hipStream_t>(stream)),
                                   "rt_hip_gemv_q4k");
    }
    return gemv_batched("rt_hip_gemv_q4k", RT_HIP_Q4K, x, y, n, k, m,
                        [&](const float* xx, float* yy, int mm) {
                            return launch_gemv_q4k(blocks, xx, yy, n, k, mm,
                                                   static_cast<hipStream_t>(stream));
                        });
}

int rt_hip_gemv_q4k_multi(int32_t count, const void* const* blocks, float* const* y,
                          const int64_t* n, const float* x, int64_t k, rt_hip_stream stream) {
    if (count < 1 || count > RT_HIP_MULTI_MAX || !blocks || !y || !n)
        return fail(RT_HIP_E_ARG, "rt_hip_gemv_q4k_multi: count must be in [1, 4] with arrays");
    for (int32_t j = 0; j < count; ++j) {
        int rc = gemv_args("rt_hip_gemv_q4k_multi", blocks[j], x, y[j], n[j], k, 1, 256);
        if (rc) return rc;
    }
    if (q4k_m1_lds_bytes(k) > lds_cap())
        return fail(RT_HIP_E_SHAPE, "rt_hip_gemv_q4k_multi: k too large for the LDS");
    return check_stream_launch(launch_gemv_q4k_mfma_multi(count, blocks, y, n, x, k,
                                                          static_cast<hipStream_t>(stream), false),
                               "rt_hip_gemv_q4k_multi");
}

int64_t rt_hip_q4k_tiled_bytes(int64_t n, int64_t k) {
    if (n <= 0 || k <= 0 || k % 256 != 0 || n > 0x7fffffffLL || k > 0x7fffffffLL) return -1;
    return (n + 15) / 16 * 16 * (k / 256) * 144;
}

static int q4k_tile(const char* fn, const void* blocks, void* tiled, int64_t n, int64_t k, int32_t head_dim,
                    rt_hip_stream stream) {
    if (!blocks || !tiled) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (rt_hip_q4k_tiled_bytes(n, k) < 0)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": need n > 0, k > 0, k % 256 == 0, int32 sizes");
    if (!aligned16(blocks) || !aligned16(tiled))
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": blocks and tiled must be 16-byte aligned");
    if (blocks == tiled) return fail(RT_HIP_E_ARG, std::string(fn) + ": in-place tiling is not supported");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_q4k_tile(blocks, tiled, n, k, static_cast<hipStream_t>(stream), head_dim),
                               fn);
}

int rt_hip_q4k_tile(const void* blocks, void* tiled, int64_t n, int64_t k, rt_hip_stream stream) {
    return q4k_tile("rt_hip_q4k_tile", blocks, tiled, n, k, 0, stream);
}

int rt_hip_q4k_tile_rope_half(const void* blocks, void* tiled, int64_t n, int64_t k, int32_t head_dim,
                              rt_hip_stream stream) {
    const char* fn = "rt_hip_q4k_tile_rope_half";
    if (head_dim < 2 || head_dim % 2 != 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": head_dim must be even");
    if (n % head_dim != 0) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": n is not whole heads");
    return q4k_tile(fn, blocks, tiled, n, k, head_dim, stream);
}

int rt_hip_gemv_q4k_tiled_multi(int32_t count, const void* const* tiled, float* const* y,
                                const int64_t* n, const float* x, int64_t k, rt_hip_stream stream) {
    if (count < 1 || count > RT_HIP_MULTI_MAX || !tiled || !y || !n)
        return fail(RT_HIP_E_ARG, "rt_hip_gemv_q4k_tiled_multi: count must be in [1, 4] with arrays");
    for (int32_t j = 0; j < count; ++j) {
        int rc = gemv_args("rt_hip_gemv_q4k_tiled_multi", tiled[j], x, y[j], n[j], k, 1, 256);
        if (rc) return rc;
    }
    if (q4k_m1_lds_bytes(k) > lds_cap())
        return fail(RT_HIP_E_SHAPE, "rt_hip_gemv_q4k_tiled_multi: k too large for the LDS");
    return check_stream_launch(launch_gemv_q4k_mfma_multi(count, tiled, y, n, x, k,
                                                          static_cast<hipStream_t>(stream), true),
                               "rt_hip_gemv_q4k_tiled_multi");
}

namespace {
static int gemv_xop(const char* fn, int xop, int32_t count, const void* const* tiled, float* const* y, const int64_t* n,
             const float* x, const float* aux, float eps, int64_t k, rt_hip_stream stream,
             const float* inv_freq = nullptr, int pos = 0, int head_dim = 0, int rope_jobs = 0, bool add = false) {
    if (count < 1 || count > RT_HIP_MULTI_MAX || !tiled || !y || !n)
        return fail(RT_HIP_E_ARG, std::string(fn) + ": count must be in [1, 4] with arrays");
    for (int32_t j = 0; j < count; ++j) {
        int rc = gemv_args(fn, tiled[j], x, y[j], n[j], k, 1, 256);
        if (rc) return rc;
    }
    if (xop != 0 && !aux) return fail(RT_HIP_E_ARG, std::string(fn) + ": null gamma / up");
    if (xop != 0 && !aligned16(aux))
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": gamma / up must be 16-byte aligned");
    if (q4k_m1_lds_bytes(k) > lds_cap()) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k too large for the LDS");
    // Every workgroup reads all of x (and gamma / up) while others already
    // store rows of y, so no output may overlap an input.
    for (int32_t j = 0; j < count; ++j) {
        if (overlaps(y[j], n[j] * 4, x, k * 4) || (aux && overlaps(y[j], n[j] * 4, aux, k * 4)))
            return fail(RT_HIP_E_ARG, std::string(fn) + ": an output overlaps x, gamma or up");
    }
    if (!(eps >= 0.0f)) return fail(RT_HIP_E_ARG, std::string(fn) + ": eps must be >= 0");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_gemv_q4k_xop(xop, count, tiled, y, n, x, aux, eps, k,
                                                   static_cast<hipStream_t>(stream), inv_freq, pos, head_dim,
                                                   rope_jobs, add),
                               fn);
}
}  // namespace

int rt_hip_gemv_q4k_tiled_rmsnorm_multi(int32_t count, const void* const* tiled, float* const* y,
                                        const int64_t* n, const float* x, const float* gamma, float eps,
                                        int32_t gemma3, int64_t k, rt_hip_stream stream) {
    return gemv_xop("rt_hip_gemv_q4k_tiled_rmsnorm_multi", gemma3 ? 2 : 1, count, tiled, y, n, x, gamma, eps, k,
                    stream);
}

int rt_hip_gemv_q4k_tiled_rmsnorm_rope(int32_t count, const void* const* tiled, float* const* y, const int64_t* n,
                                       const float* x, const float* gamma, float eps, int32_t gemma3,
                                       const float* inv_freq, int32_t pos, int32_t head_dim, int32_t rope_jobs,
                                       int64_t k, rt_hip_stream stream) {
    const char* fn = "rt_hip_gemv_q4k_tiled_rmsnorm_rope";
    if (count < 1 || count > RT_HIP_MULTI_MAX || !tiled || !y || !n)
        return fail(RT_HIP_E_ARG, std::string(fn) + ": count must be in [1, 4] with arrays");
    if (!inv_freq) return fail(RT_HIP_E_ARG, std::string(fn) + ": null inv_freq");
    if (pos < 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": pos must be >= 0");
    if (head_dim < 2 || head_dim % 2 != 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": head_dim must be even");
    const int32_t mask = rope_jobs & ~RT_HIP_ROPE_HALF;
    if (mask <= 0 || mask >= (1 << count))
        return fail(RT_HIP_E_ARG, std::string(fn) + ": rope_jobs must name jobs in [0, count)");
    for (int32_t j = 0; j < count; ++j)
        if (((mask >> j) & 1) && n[j] % head_dim != 0)
            return fail(RT_HIP_E_SHAPE, std::string(fn) + ": a rotated output is not whole heads");
    return gemv_xop(fn, gemma3 ? 2 : 1, count, tiled, y, n, x, gamma, eps, k, stream, inv_freq, pos, head_dim,
                    rope_jobs);
}

int rt_hip_gemv_q4k_tiled_residual(const void* tiled, const float* x, float* resid, int64_t n, int64_t k,
                                   rt_hip_stream stream) {
    return gemv_xop("rt_hip_gemv_q4k_tiled_residual", 0, 1, &tiled, &resid, &n, x, nullptr, 0.0f, k, stream, nullptr,
                    0, 0, 0, true);
}

int rt_hip_gemv_q4k_tiled_swiglu_residual(const void* tiled, const float* gate, const float* up, float* resid,
                                          int64_t n, int64_t k, rt_hip_stream stream) {
    return gemv_xop("rt_hip_gemv_q4k_tiled_swiglu_residual", 3, 1, &tiled, &resid, &n, gate, up, 0.0f, k, stream,
                    nullptr, 0, 0, 0, true);
}

int rt_hip_gemv_bf16_swiglu_residual(const uint16_t* w, const float* gate, const float* up, float* resid, int64_t n,
                                     int64_t k, rt_hip_stream stream) {
    const char* fn = "rt_hip_gemv_bf16_swiglu_residual";
    int rc = gemv_args(fn, w, gate, resid, n, k, 1, 256);
    if (rc) return rc;
    if (!up) return fail(RT_HIP_E_ARG, std::string(fn) + ": null up");
    if (!aligned16(up)) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": up must be 16-byte aligned");
    if (overlaps(resid, n * 4, gate, k * 4) || overlaps(resid, n * 4, up, k * 4))
        return fail(RT_HIP_E_ARG, std::string(fn) + ": resid overlaps gate or up");
    if (bf16_m1_lds_bytes(k) > lds_cap()) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k too large for the LDS");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(
        launch_gemv_bf16_xop(3, w, gate, up, 0.0f, resid, n, k, static_cast<hipStream_t>(stream), true), fn);
}

namespace {
static int attention_args(const char* fn, const float* q, const float* k_cache, const float* v_cache, const float* out,
                   int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int64_t seq_len) {
    if (!q || !k_cache || !v_cache || !out) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (head_dim != 128) return fail(RT_HIP_E_UNSUPPORTED, std::string(fn) + ": head_dim must be 128");
    if (n_kv_heads < 1 || n_q_heads < n_kv_heads || n_q_heads % n_kv_heads != 0 || n_q_heads / n_kv_heads > 4)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": need n_q = g * n_kv with g in [1, 4]");
    if (seq_len < 1 || seq_len > 0x7fffffffLL) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": seq_len out of range");
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": buffers must be 16-byte aligned");
    return RT_HIP_OK;
}
}  // namespace

int rt_hip_attention_decode(const float* q, const float* k_cache, const float* v_cache, float* out,
                            int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int64_t seq_len, float scale,
                            rt_hip_stream stream) {
    const char* fn = "rt_hip_attention_decode";
    int rc = attention_args(fn, q, k_cache, v_cache, out, n_q_heads, n_kv_heads, head_dim, seq_len);
    if (rc) return rc;
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    float* part = static_cast<float*>(workspace(attention_decode_workspace(n_q_heads, n_kv_heads, seq_len),
                                                static_cast<hipStream_t>(stream), &e));
    if (!part) return check_stream_launch(e, fn);
    return check_stream_launch(launch_attention_decode(q, k_cache, v_cache, out, part, n_q_heads, n_kv_heads,
                                                       seq_len, scale, static_cast<hipStream_t>(stream)),
                               fn);
}

int rt_hip_attention_decode_noalloc(const float* q, const float* k_cache, const float* v_cache, float* out,
                                    int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int64_t seq_len,
                                    float scale, rt_hip_stream stream) {
    const char* fn = "rt_hip_attention_decode_noalloc";
    int rc = attention_args(fn, q, k_cache, v_cache, out, n_q_heads, n_kv_heads, head_dim, seq_len);
    if (rc) return rc;
    hipError_t e;
    DeviceState* st = state_for_current(&e);
    if (!st) return hip_fail(e, fn);
    const size_t need = attention_decode_workspace(n_q_heads, n_kv_heads, seq_len);
    if (need > attention_scratch_bytes())
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": this shape needs " + std::to_string(need) +
                                        " bytes of split partials, above the " +
                                        std::to_string(attention_scratch_bytes()) + "-byte scratch maximum");
    void* part = nullptr;
    e = attention_scratch_setup(st->info.ordinal, &part);
    if (e != hipSuccess) return hip_fail(e, fn);
    return check_stream_launch(launch_attention_decode(q, k_cache, v_cache, out, static_cast<float*>(part),
                                                       n_q_heads, n_kv_heads, seq_len, scale,
                                                       static_cast<hipStream_t>(stream)),
                               fn);
}

int rt_hip_flux_attention(const float* q, const float* k, const float* v, float* out, int64_t t, int32_t n_heads,
                          int32_t head_dim, rt_hip_stream stream) {
    const char* fn = "rt_hip_flux_attention";
    if (!q || !k || !v || !out) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (t < 0 || n_heads < 1) return fail(RT_HIP_E_ARG, std::string(fn) + ": need t >= 0 and n_heads >= 1");
    if (head_dim < 8 || head_dim > 128 || head_dim % 8 != 0)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": head_dim must be a multiple of 8 in [8, 128]");
    const int64_t row_bytes = static_cast<int64_t>(n_heads) * head_dim * 4;
    // a 32-key tile of a head is addressed with 32-bit offsets below 2^31
    if (t > 0x7fffffffLL || row_bytes > (int64_t{1} << 26) || row_bytes > (int64_t{1} << 40) / (t > 0 ? t : 1))
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": t * n_heads * head_dim out of range");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": buffers must be 16-byte aligned");
    const int64_t bytes = t * row_bytes;
    if (overlaps(out, bytes, q, bytes) || overlaps(out, bytes, k, bytes) || overlaps(out, bytes, v, bytes))
        return fail(RT_HIP_E_ARG, std::string(fn) + ": out overlaps q, k or v");
    if (t == 0) return RT_HIP_OK;
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    // the scale of flux.cpp:290 and metal_flux.mm:264, in f32
    const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
    const hipStream_t s = static_cast<hipStream_t>(stream);
    float* part = nullptr;
    uint32_t* counters = nullptr;
    if (const size_t need = flux_attention_workspace(t, n_heads, head_dim)) {
        part = static_cast<float*>(workspace(need, s, &e));
        if (!part) return hip_fail(e, fn);
        counters = arrival_counters(s, &e);
        if (!counters) return hip_fail(e, fn);
    }
    return check_stream_launch(launch_flux_attention(q, k, v, out, t, n_heads, head_dim, scale, part, counters, s),
                               fn);
}

int64_t rt_hip_flux_attention_workspace_bytes(int64_t t, int32_t n_heads, int32_t head_dim) {
    if (t < 0 || n_heads < 1 || head_dim < 8 || head_dim > 128 || head_dim % 8 != 0) return -1;
    hipError_t e;
    if (!state_for_current(&e)) return -1;
    return static_cast<int64_t>(flux_attention_workspace(t, n_heads, head_dim));
}

int rt_hip_gemv_q4k_tiled_swiglu(const void* tiled, const float* gate, const float* up, float* y, int64_t n,
                                 int64_t k, rt_hip_stream stream) {
    return gemv_xop("rt_hip_gemv_q4k_tiled_swiglu", 3, 1, &tiled, &y, &n, gate, up, 0.0f, k, stream);
}

static int q4k_bf16_rmsnorm(const char* fn, int32_t count, const void* const* tiled, float* const* y,
                            const int64_t* n, const uint16_t* w_bf16, float* y_bf16, int64_t n_bf16, const float* x,
                            const float* gamma, float eps, int32_t gemma3, int64_t k, rt_hip_stream stream,
                            const float* inv_freq, int32_t pos, int32_t head_dim, int32_t rope_jobs) {
    if (count < 1 || count > RT_HIP_MULTI_MAX || !tiled || !y || !n)
        return fail(RT_HIP_E_ARG, std::string(fn) + ": count must be in [1, 4] with arrays");
    for (int32_t j = 0; j < count; ++j) {
        int rc = gemv_args(fn, tiled[j], x, y[j], n[j], k, 1, 256);
        if (rc) return rc;
    }
    int rc = gemv_args(fn, w_bf16, x, y_bf16, n_bf16, k, 1, 256);
    if (rc) return rc;
    if (!gamma) return fail(RT_HIP_E_ARG, std::string(fn) + ": null gamma");
    if (!aligned16(gamma)) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": gamma must be 16-byte aligned");
    if (!(eps >= 0.0f)) return fail(RT_HIP_E_ARG, std::string(fn) + ": eps must be >= 0");
    for (int32_t j = 0; j <= count; ++j) {
        const void* yj = j < count ? static_cast<const void*>(y[j]) : static_cast<const void*>(y_bf16);
        const int64_t nj = j < count ? n[j] : n_bf16;
        if (overlaps(yj, nj * 4, gamma, k * 4))
            return fail(RT_HIP_E_ARG, std::string(fn) + ": an output overlaps gamma");
    }
    if (k > 8192 || q4k_bf16_fused_lds_bytes(k) > 65536)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k above 8192");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_gemv_q4k_bf16_fused(count, tiled, y, n, w_bf16, y_bf16, n_bf16, x, k,
                                                          static_cast<hipStream_t>(stream), gemma3 ? 2 : 1, gamma,
                                                          eps, inv_freq, pos, head_dim, rope_jobs),
                               fn);
}

int rt_hip_gemv_q4k_tiled_bf16_rmsnorm(int32_t count, const void* const* tiled, float* const* y,
                                       const int64_t* n, const uint16_t* w_bf16, float* y_bf16, int64_t n_bf16,
                                       const float* x, const float* gamma, float eps, int32_t gemma3, int64_t k,
                                       rt_hip_stream stream) {
    return q4k_bf16_rmsnorm("rt_hip_gemv_q4k_tiled_bf16_rmsnorm", count, tiled, y, n, w_bf16, y_bf16, n_bf16, x,
                            gamma, eps, gemma3, k, stream, nullptr, 0, 0, 0);
}

int rt_hip_gemv_q4k_tiled_bf16_rmsnorm_rope(int32_t count, const void* const* tiled, float* const* y,
                                            const int64_t* n, const uint16_t* w_bf16, float* y_bf16,
                                            int64_t n_bf16, const float* x, const float* gamma, float eps,
                                            int32_t gemma3, const float* inv_freq, int32_t pos, int32_t head_dim,
                                            int32_t rope_jobs, int64_t k, rt_hip_stream stream) {
    const char* fn = "rt_hip_gemv_q4k_tiled_bf16_rmsnorm_rope";
    if (count < 1 || count > RT_HIP_MULTI_MAX || !tiled || !y || !n)
        return fail(RT_HIP_E_ARG, std::string(fn) + ": count must be in [1, 4] with arrays");
    if (!inv_freq) return fail(RT_HIP_E_ARG, std::string(fn) + ": null inv_freq");
    if (pos < 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": pos must be >= 0");
    if (head_dim < 2 || head_dim % 2 != 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": head_dim must be even");
    const int32_t mask = rope_jobs & ~RT_HIP_ROPE_HALF;
    if (mask <= 0 || mask >= (1 << count))
        return fail(RT_HIP_E_ARG, std::string(fn) + ": rope_jobs must name Q4_K jobs in [0, count)");
    for (int32_t j = 0; j < count; ++j)
        if (((mask >> j) & 1) && n[j] % head_dim != 0)
            return fail(RT_HIP_E_SHAPE, std::string(fn) + ": a rotated output is not whole heads");
    return q4k_bf16_rmsnorm(fn, count, tiled, y, n, w_bf16, y_bf16, n_bf16, x, gamma, eps, gemma3, k, stream,
                            inv_freq, pos, head_dim, rope_jobs);
}

int rt_hip_gemv_bf16_swiglu(const uint16_t* w, const float* gate, const float* up, float* y, int64_t n, int64_t k,
                            rt_hip_stream stream) {
    const char* fn = "rt_hip_gemv_bf16_swiglu";
    int rc = gemv_args(fn, w, gate, y, n, k, 1, 256);
    if (rc) return rc;
    if (!up) return fail(RT_HIP_E_ARG, std::string(fn) + ": null up");
    if (!aligned16(up)) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": up must be 16-byte aligned");
    if (overlaps(y, n * 4, up, k * 4)) return fail(RT_HIP_E_ARG, std::string(fn) + ": y overlaps up");
    if (bf16_m1_lds_bytes(k) > lds_cap()) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k too large for the LDS");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_gemv_bf16_xop(3, w, gate, up, 0.0f, y, n, k, static_cast<hipStream_t>(stream)),
                               fn);
}

int rt_hip_gemv_q4k_tiled_bf16(int32_t count, const void* const* tiled, float* const* y,
                               const int64_t* n, const uint16_t* w_bf16, float* y_bf16,
                               int64_t n_bf16, const float* x, int64_t k, rt_hip_stream stream) {
    const char* fn = "rt_hip_gemv_q4k_tiled_bf16";
    if (count < 1 || count > RT_HIP_MULTI_MAX || !tiled || !y || !n)
        return fail(RT_HIP_E_ARG, std::string(fn) + ": count must be in [1, 4] with arrays");
    for (int32_t j = 0; j < count; ++j) {
        int rc = gemv_args(fn, tiled[j], x, y[j], n[j], k, 1, 256);
        if (rc) return rc;
    }
    int rc = gemv_args(fn, w_bf16, x, y_bf16, n_bf16, k, 1, 256);
    if (rc) return rc;
    if (k > 8192 || q4k_bf16_fused_lds_bytes(k) > 65536)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k above 8192");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_gemv_q4k_bf16_fused(count, tiled, y, n, w_bf16, y_bf16, n_bf16, x, k,
                                                          static_cast<hipStream_t>(stream)),
                               fn);
}

int rt_hip_gemv_q4k_tiled(const void* tiled, const float* x, float* y, int64_t n, int64_t k,
                          rt_hip_stream stream) {
    return rt_hip_gemv_q4k_tiled_multi(1, &tiled, &y, &n, x, k, stream);
}

int rt_hip_q4k_quantize_activation_q8(const float* a, int64_t k, int8_t* q8, float* scales, float* sums,
                                      rt_hip_stream stream) {
    const char* fn = "rt_hip_q4k_quantize_activation_q8";
    if (!a || !q8 || !scales || !sums) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (k <= 0 || k > 0x7fffffffLL) return fail(RT_HIP_E_ARG, std::string(fn) + ": k must be in [1, 2^31)");
    if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(sums)) &
        3u)
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": a, scales and sums must be 4-byte aligned");
    const int64_t nq = (k + 31) / 32;
    if (overlaps(q8, nq * 32, a, k * 4) || overlaps(scales, nq * 4, a, k * 4) || overlaps(sums, nq * 4, a, k * 4) ||
        overlaps(q8, nq * 32, scales, nq * 4) || overlaps(q8, nq * 32, sums, nq * 4) ||
        overlaps(scales, nq * 4, sums, nq * 4))
        return fail(RT_HIP_E_ARG, std::string(fn) + ": outputs overlap each other or a");
    return check_stream_launch(launch_quantize_q8(a, k, q8, scales, sums, static_cast<hipStream_t>(stream)), fn);
}

namespace {
static int gemv_q8(const char* fn, bool tiled, const void* w, const float* x, float* y, int64_t n, int64_t k,
            rt_hip_stream stream) {
    int rc = gemv_args(fn, w, x, y, n, k, 1, 256);
    if (rc) return rc;
    if (k > 16384) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k above 16384");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_gemv_q4k_q8(w, tiled, x, y, n, k, static_cast<hipStream_t>(stream)), fn);
}
}  // namespace

int rt_hip_gemv_q4k_q8(const void* blocks, const float* x, float* y, int64_t n, int64_t k, rt_hip_stream stream) {
    return gemv_q8("rt_hip_gemv_q4k_q8", false, blocks, x, y, n, k, stream);
}

int rt_hip_gemv_q4k_tiled_q8(const void* tiled, const float* x, float* y, int64_t n, int64_t k,
                             rt_hip_stream stream) {
    return gemv_q8("rt_hip_gemv_q4k_tiled_q8", true, tiled, x, y, n, k, stream);
}

}  // extern "C"

extern "C" {

int rt_hip_gemv_bf16(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                     int32_t m, rt_hip_stream stream) {
    int rc = gemv_args("rt_hip_gemv_bf16", w, x, y, n, k, m, 8);
    if (rc) return rc;
    if (m > 1 && tune_param("GEMV_BATCH_MFMA", 1))
        return check_stream_launch(launch_gemv_batch(RT_HIP_BF16, w, x, y, n, k, m, static_cast<hipStream_t>(stream)),
                                   "rt_hip_gemv_bf16");
    return gemv_batched("rt_hip_gemv_bf16", RT_HIP_BF16, x, y, n, k, m,
                        [&](const float* xx, float* yy, int mm) {
                            return launch_gemv_bf16(w, xx, yy, n, k, mm, nullptr,
                                                    static_cast<hipStream_t>(stream));
                        });
}

int64_t rt_hip_q4mat_bytes(int64_t n, int64_t k) {
    if (n <= 0 || k <= 0 || k % 32 != 0 || n > 0x7fffffffLL || k > 0x7fffffffLL) return -1;
    return static_cast<int64_t>(q4mat_bytes(n, k));
}

int64_t rt_hip_q4mat_scales_offset(int64_t n, int64_t k) {
    if (rt_hip_q4mat_bytes(n, k) < 0) return -1;
    return static_cast<int64_t>(q4mat_scales_offset(n, k));
}

int rt_hip_gemv_q4mat(const void* w, const float* x, float* y, int64_t n, int64_t k, int32_t m,
                      rt_hip_stream stream) {
    const char* fn = "rt_hip_gemv_q4mat";
    int rc = gemv_args(fn, w, x, y, n, k, m, 32);
    if (rc) return rc;
    if (q4mat_gemv_lds_bytes(1, k) > lds_cap()) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k too large for the LDS");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    int mb = m;
    while (mb > 1 && q4mat_gemv_lds_bytes(mb, k) > lds_cap()) --mb;
    for (int32_t m0 = 0; m0 < m; m0 += mb) {
        const int32_t mm = (m - m0) < mb ? (m - m0) : mb;
        e = launch_gemv_q4mat(w, x + static_cast<size_t>(m0) * k, y + static_cast<size_t>(m0) * n, n, k, mm,
                              static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail(e, fn);
    }
    return RT_HIP_OK;
}

int rt_hip_gemv_q4_0(const void* blocks, const float* x, float* y, int64_t n, int64_t k,
                     int32_t m, rt_hip_stream stream) {
    int rc = gemv_args("rt_hip_gemv_q4_0", blocks, x, y, n, k, m, 256);
    if (rc) return rc;
    return gemv_batched("rt_hip_gemv_q4_0", RT_HIP_Q4_0, x, y, n, k, m,
                        [&](const float* xx, float* yy, int mm) {
                            return launch_gemv_q4_0(blocks, xx, yy, n, k, mm,
                                                    static_cast<hipStream_t>(stream));
                        });
}

int rt_hip_dequant_q6k_bf16(const void* blocks, uint16_t* out, int64_t n, int64_t k, rt_hip_stream stream) {
    const char* fn = "rt_hip_dequant_q6k_bf16";
    if (!blocks || !out) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (n <= 0 || k <= 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": n and k must be > 0");
    if (k % 256 != 0) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": k must be a multiple of 256");
    if (n > 0x7fffffffLL || k > 0x7fffffffLL) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": n, k must fit in int32");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_q6k_to_bf16(blocks, out, n, k, static_cast<hipStream_t>(stream)), fn);
}

int64_t rt_hip_q6k_tiled_bytes(int64_t n, int64_t k) {
    if (n <= 0 || k <= 0 || k % 256 != 0 || n > 0x7fffffffLL || k > 0x7fffffffLL) return -1;
    return q6k_tiled_bytes(n, k);
}

int rt_hip_q6k_tile(const void* blocks, void* tiled, int64_t n, int64_t k, rt_hip_stream stream) {
    const char* fn = "rt_hip_q6k_tile";
    if (!blocks || !tiled) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (rt_hip_q6k_tiled_bytes(n, k) < 0) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": invalid n, k");
    if ((n + 15) / 16 > 65535) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": n too large");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_q6k_tile(blocks, tiled, n, k, static_cast<hipStream_t>(stream)), fn);
}

int rt_hip_gemv_q6k_tiled(const void* tiled, const float* x, float* y, int64_t n, int64_t k,
                          rt_hip_stream stream) {
    const char* fn = "rt_hip_gemv_q6k_tiled";
    int rc = gemv_args(fn, tiled, x, y, n, k, 1, 256);
    if (rc) return rc;
    if (k > 8192) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k above 8192");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_gemv_q6k(tiled, x, y, n, k, static_cast<hipStream_t>(stream)), fn);
}

int rt_hip_gemv_q6k_tiled_swiglu_residual(const void* tiled, const float* gate, const float* up, float* resid,
                                          int64_t n, int64_t k, rt_hip_stream stream) {
    const char* fn = "rt_hip_gemv_q6k_tiled_swiglu_residual";
    int rc = gemv_args(fn, tiled, gate, resid, n, k, 1, 256);
    if (rc) return rc;
    if (!up) return fail(RT_HIP_E_ARG, std::string(fn) + ": null up");
    if (!aligned16(up)) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": up must be 16-byte aligned");
    if (overlaps(resid, n * 4, gate, k * 4) || overlaps(resid, n * 4, up, k * 4))
        return fail(RT_HIP_E_ARG, std::string(fn) + ": resid overlaps gate or up");
    if (k > 8192) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": k above 8192");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(launch_gemv_q6k(tiled, gate, resid, n, k, static_cast<hipStream_t>(stream), up), fn);
}

int rt_hip_argmax(const float* logits, int64_t rows, int64_t cols, int64_t* idx, float* val,
                  rt_hip_stream stream) {
    if (!logits || !idx) return fail(RT_HIP_E_ARG, "rt_hip_argmax: null pointer");
    if (rows <= 0 || cols <= 0) return fail(RT_HIP_E_ARG, "rt_hip_argmax: rows, cols must be > 0");
    if (cols > 0xffffffffLL || rows > 65535)
        return fail(RT_HIP_E_SHAPE, "rt_hip_argmax: cols < 2^32 and rows <= 65535 required");
    hipError_t e;
    uint64_t* keys = static_cast<uint64_t*>(workspace(static_cast<size_t>(rows) * 8, static_cast<hipStream_t>(stream), &e));
    if (!keys) return check_stream_launch(e, "rt_hip_argmax: workspace");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if ((e = launch_argmax_init(keys, rows, s)) != hipSuccess) return hip_fail(e, "rt_hip_argmax");
    if ((e = launch_argmax_scan(logits, rows, cols, keys, s)) != hipSuccess)
        return hip_fail(e, "rt_hip_argmax");
    if ((e = launch_argmax_finalize(keys, rows, idx, val, s)) != hipSuccess)
        return hip_fail(e, "rt_hip_argmax");
    return RT_HIP_OK;
}

int rt_hip_gemv_bf16_argmax(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                            int64_t* idx, float* val, rt_hip_stream stream) {
    int rc = gemv_args("rt_hip_gemv_bf16_argmax", w, x, y, n, k, 1, 8);
    if (rc) return rc;
    if (!idx) return fail(RT_HIP_E_ARG, "rt_hip_gemv_bf16_argmax: null idx");
    hipError_t e;
    if (bf16_m1_lds_bytes(k) > lds_cap()) return fail(RT_HIP_E_SHAPE, "rt_hip_gemv_bf16_argmax: k too large for the LDS");
    const int64_t parts = bf16_argmax_partials(n, k);
    uint64_t* key = static_cast<uint64_t*>(workspace(static_cast<size_t>(parts) * 8, static_cast<hipStream_t>(stream), &e));
    if (!key) return check_stream_launch(e, "rt_hip_gemv_bf16_argmax: workspace");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if ((e = launch_gemv_bf16_m1(w, x, y, n, k, key, s)) != hipSuccess)
        return hip_fail(e, "rt_hip_gemv_bf16_argmax");
    if ((e = launch_argmax_reduce(key, parts, idx, val, s)) != hipSuccess)
        return hip_fail(e, "rt_hip_gemv_bf16_argmax");
    return RT_HIP_OK;
}

int rt_hip_dequant_q4k_f32(const void* blocks, float* out, int64_t n, int64_t k,
                           rt_hip_stream stream) {
    if (!blocks || !out) return fail(RT_HIP_E_ARG, "rt_hip_dequant_q4k_f32: null pointer");
    if (n <= 0 || k <= 0) return fail(RT_HIP_E_ARG, "rt_hip_dequant_q4k_f32: n, k must be > 0");
    if (k % 256) return fail(RT_HIP_E_ALIGN, "rt_hip_dequant_q4k_f32: k must be a multiple of 256");
    if (!aligned16(blocks) || !aligned16(out))
        return fail(RT_HIP_E_ALIGN, "rt_hip_dequant_q4k_f32: pointers must be 16-byte aligned");
    return check_stream_launch(
        launch_dequant_q4k(blocks, out, false, n, k, static_cast<hipStream_t>(stream)),
        "rt_hip_dequant_q4k_f32");
}

int rt_hip_dequant_q4k_bf16(const void* blocks, uint16_t* out, int64_t n, int64_t k,
                            rt_hip_stream stream) {
    if (!blocks || !out) return fail(RT_HIP_E_ARG, "rt_hip_dequant_q4k_bf16: null pointer");
    if (n <= 0 || k <= 0) return fail(RT_HIP_E_ARG, "rt_hip_dequant_q4k_bf16: n, k must be > 0");
    if (k % 256) return fail(RT_HIP_E_ALIGN, "rt_hip_dequant_q4k_bf16: k must be a multiple of 256");
    if (!aligned16(blocks) || !aligned16(out))
        return fail(RT_HIP_E_ALIGN, "rt_hip_dequant_q4k_bf16: pointers must be 16-byte aligned");
    return check_stream_launch(
        launch_dequant_q4k(blocks, out, true, n, k, static_cast<hipStream_t>(stream)),
        "rt_hip_dequant_q4k_bf16");
}

int rt_hip_quantize_q4k(const float* w, void* blocks, int64_t n, int64_t k,
                        rt_hip_stream stream) {
    if (!w || !blocks) return fail(RT_HIP_E_ARG, "rt_hip_quantize_q4k: null pointer");
    if (n <= 0 || k <= 0) return fail(RT_HIP_E_ARG, "rt_hip_quantize_q4k: n, k must be > 0");
    if (k % 256) return fail(RT_HIP_E_ALIGN, "rt_hip_quantize_q4k: k must be a multiple of 256");
    if (!aligned16(w) || !aligned16(blocks))
        return fail(RT_HIP_E_ALIGN, "rt_hip_quantize_q4k: pointers must be 16-byte aligned");
    return check_stream_launch(
        launch_quantize_q4k(w, blocks, n, k, static_cast<hipStream_t>(stream)),
        "rt_hip_quantize_q4k");
}

static int gemm_common(const char* fn, int w_fmt, const void* a, int32_t a_dtype, const void* w,
                       const float* bias, float* c, int64_t m, int64_t n, int64_t k,
                       int64_t k_multiple, rt_hip_stream stream) {
    if (!a || !w || !c) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (m <= 0 || n <= 0 || k <= 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": sizes must be > 0");
    if (a_dtype != RT_HIP_F32 && a_dtype != RT_HIP_BF16)
        return fail(RT_HIP_E_ARG, std::string(fn) + ": a_dtype must be RT_HIP_F32 or RT_HIP_BF16");
    if (k % k_multiple)
        return fail(RT_HIP_E_ALIGN,
                    std::string(fn) + ": k must be a multiple of " + std::to_string(k_multiple));
    if (m > 0x7fffffffLL || n > 0x7fffffffLL || k > 0x7fffffffLL)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": sizes must fit in int32");
    if (!aligned16(a) || !aligned16(w) || !aligned16(c))
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": a, w, c must be 16-byte aligned");
    if (n % 4) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": n must be a multiple of 4");
    return check_stream_launch(launch_gemm(w_fmt, a, a_dtype == RT_HIP_BF16, w, bias, c, m, n, k,
                                           static_cast<hipStream_t>(stream)),
                               fn);
}

int rt_hip_gemm_q4k(const void* a, int32_t a_dtype, const void* blocks, const float* bias,
                    float* c, int64_t m, int64_t n, int64_t k, rt_hip_stream stream) {
    return gemm_common("rt_hip_gemm_q4k", RT_HIP_Q4K, a, a_dtype, blocks, bias, c, m, n, k, 256,
                       stream);
}

int rt_hip_gemm_bf16(const void* a, int32_t a_dtype, const uint16_t* w, const float* bias,
                     float* c, int64_t m, int64_t n, int64_t k, rt_hip_stream stream) {
    return gemm_common("rt_hip_gemm_bf16", RT_HIP_BF16, a, a_dtype, w, bias, c, m, n, k, 64,
                       stream);
}

int rt_hip_gemm(int32_t format, const void* a, int32_t a_dtype, const void* w, const float* bias, float* c,
                int64_t m, int64_t n, int64_t k, rt_hip_stream stream) {
    const char* fn = "rt_hip_gemm";
    if (format == RT_HIP_Q4K) return rt_hip_gemm_q4k(a, a_dtype, w, bias, c, m, n, k, stream);
    if (format == RT_HIP_BF16)
        return rt_hip_gemm_bf16(a, a_dtype, static_cast<const uint16_t*>(w), bias, c, m, n, k, stream);
    if (format != RT_HIP_Q4_0 && format != RT_HIP_Q4MAT)
        return fail(RT_HIP_E_UNSUPPORTED, std::string(fn) + ": unsupported format");
    // Validate as the bf16 GEMM will (K % 64), then dequantize W once into
    // the workspace behind the GEMM's own scratch and run the bf16 path.
    if (!a || !w || !c) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (m <= 0 || n <= 0 || k <= 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": sizes must be > 0");
    if (a_dtype != RT_HIP_F32 && a_dtype != RT_HIP_BF16)
        return fail(RT_HIP_E_ARG, std::string(fn) + ": a_dtype must be RT_HIP_F32 or RT_HIP_BF16");
    if (k % 64) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": k must be a multiple of 64");
    if (m > 0x7fffffffLL || n > 0x7fffffffLL || k > 0x7fffffffLL)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": sizes must fit in int32");
    if (n % 4) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": n must be a multiple of 4");
    if (!aligned16(a) || !aligned16(w) || !aligned16(c))
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": a, w, c must be 16-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (gemm_dequant_in_kernel(format, a_dtype == RT_HIP_BF16, m, n, k))  // decoded inside the GEMM
        return check_stream_launch(launch_gemm(format, a, a_dtype == RT_HIP_BF16, w, bias, c, m, n, k, s), fn);
    const size_t own = (gemm_workspace_bytes(RT_HIP_BF16, a_dtype == RT_HIP_BF16, m, n, k) + 255) / 256 * 256;
    hipError_t e;
    auto* ws = static_cast<uint8_t*>(workspace(own + static_cast<size_t>(n * k) * 2, s, &e));
    if (!ws) return check_stream_launch(e, fn);
    uint16_t* wb = reinterpret_cast<uint16_t*>(ws + own);
    e = launch_dequant_4bit(format, w, wb, true, n, k, s);
    if (e != hipSuccess) return hip_fail(e, fn);
    return check_stream_launch(launch_gemm(RT_HIP_BF16, a, a_dtype == RT_HIP_BF16, wb, bias, c, m, n, k, s), fn);
}

int rt_hip_dequant(int32_t format, const void* w, void* out, int32_t out_dtype, int64_t n, int64_t k,
                   rt_hip_stream stream) {
    const char* fn = "rt_hip_dequant";
    if (out_dtype != RT_HIP_F32 && out_dtype != RT_HIP_BF16)
        return fail(RT_HIP_E_ARG, std::string(fn) + ": out_dtype must be RT_HIP_F32 or RT_HIP_BF16");
    if (format == RT_HIP_Q4K)
        return out_dtype == RT_HIP_BF16 ? rt_hip_dequant_q4k_bf16(w, static_cast<uint16_t*>(out), n, k, stream)
                                        : rt_hip_dequant_q4k_f32(w, static_cast<float*>(out), n, k, stream);
    if (format != RT_HIP_Q4_0 && format != RT_HIP_Q4MAT)
        return fail(RT_HIP_E_UNSUPPORTED, std::string(fn) + ": unsupported format");
    if (!w || !out) return fail(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (n <= 0 || k <= 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": n, k must be > 0");
    if (k % 32) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": k must be a multiple of 32");
    if (n > 0x7fffffffLL || k > 0x7fffffffLL) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": n, k must fit in int32");
    if (!aligned16(out) || (format == RT_HIP_Q4MAT && !aligned16(w)))
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": pointers must be 16-byte aligned");
    if (format == RT_HIP_Q4_0 && (reinterpret_cast<uintptr_t>(w) & 1u))
        return fail(RT_HIP_E_ALIGN, std::string(fn) + ": Q4_0 blocks must be 2-byte aligned");
    hipError_t e;
    if (!state_for_current(&e)) return hip_fail(e, fn);
    return check_stream_launch(
        launch_dequant_4bit(format, w, out, out_dtype == RT_HIP_BF16, n, k, static_cast<hipStream_t>(stream)), fn);
}

int rt_hip_linear_forward(int32_t format, const void* w, const float* bias, const float* x,
                          float* y, int64_t m, int64_t n, int64_t k, rt_hip_stream stream) {
    int rc;
    if (m <= RT_HIP_GEMV_MAX_M) {
        switch (format) {
            case RT_HIP_Q4K: rc = rt_hip_gemv_q4k(w, x, y, n, k, static_cast<int32_t>(m), stream); break;
            case RT_HIP_BF16:
                rc = rt_hip_gemv_bf16(static_cast<const uint16_t*>(w), x, y, n, k,
                                      static_cast<int32_t>(m), stream);
                break;
            case RT_HIP_Q4_0: rc = rt_hip_gemv_q4_0(w, x, y, n, k, static_cast<int32_t>(m), stream); break;
            case RT_HIP_Q4MAT: rc = rt_hip_gemv_q4mat(w, x, y, n, k, static_cast<int32_t>(m), stream); break;
            default: return fail(RT_HIP_E_UNSUPPORTED, "rt_hip_linear_forward: unsupported format");
        }
        if (rc || !bias) return rc;
        return check_stream_launch(launch_add_bias(y, bias, m, n, static_cast<hipStream_t>(stream)),
                                   "rt_hip_linear_forward");
    }
    if (format != RT_HIP_Q4K && format != RT_HIP_BF16 && format != RT_HIP_Q4_0 && format != RT_HIP_Q4MAT)
        return fail(RT_HIP_E_UNSUPPORTED, "rt_hip_linear_forward: unsupported format");
    return rt_hip_gemm(format, x, RT_HIP_F32, w, bias, y, m, n, k, stream);
}

}  // extern "C"
