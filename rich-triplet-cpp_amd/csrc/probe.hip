// probe.hip -- calibration kernels for the decode step's launch ceiling.
//
// Two launches that do no arithmetic of the path, so a graph of them shows
// what the launch structure alone costs on this device:
//   rt_hip_probe_read   streams `bytes` of a buffer with 16-byte loads,
//                       folds them into one word per workgroup and writes
//                       `out_bytes` of output from those words (a GEMV's
//                       rows after its reads);
//   rt_hip_probe_empty  a kernel that returns at once.
// A hipGraph of the decode step's launch sequence with each GEMV replaced by
// a read of its byte count, or by an empty launch, bounds from above what
// any GEMV of that launch structure can reach.
#include <hip/hip_runtime.h>

#include <string>

#include "rt_hip.h"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr uint32_t kNever = 0x9e3779b9u;

// Workgroup g reads the 16-byte words [g * per, (g + 1) * per) of the buffer
// in rounds of U words per thread (U * 4 KB per workgroup round), all U
// loads of a round issued before any is used.
template <int U>
__global__ __launch_bounds__(kThreads) void k_probe_read(const u32x4* __restrict__ p, int64_t words, int64_t per,
                                                         uint32_t* __restrict__ out, int64_t out_words) {
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * per;
    const int64_t hi = lo + per < words ? lo + per : words;
    uint32_t acc = 0;
    // every round issues its U loads (those past the range read word lo,
    // in bounds, and are not used) before it uses any, the last round too
    for (int64_t i = lo + threadIdx.x; i < hi; i += U * kThreads) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = p[i + u * kThreads < hi ? i + u * kThreads : lo];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (i + u * kThreads < hi) acc ^= (v[u][0] ^ v[u][1]) ^ (v[u][2] ^ v[u][3]);
    }
    // the output, as a GEMV stores its rows after its reads: workgroup g
    // writes words [g * ow, (g + 1) * ow) (acc itself, so the stores wait
    // for the reads); with out_words == 0 only a word that random data never
    // gives is stored
    if (out_words == 0) {
        if (acc == kNever) out[blockIdx.x] = acc;
        return;
    }
    const int64_t ow = (out_words + gridDim.x - 1) / gridDim.x;
    const int64_t o0 = static_cast<int64_t>(blockIdx.x) * ow;
    for (int64_t j = o0 + threadIdx.x; j < o0 + ow && j < out_words; j += kThreads) out[j] = acc;
}

__global__ void k_probe_empty() {}

}  // namespace
}  // namespace rt_hip

using namespace rt_hip;

extern "C" {

int rt_hip_probe_read(const void* buf, int64_t bytes, int32_t workgroups, uint32_t* out, int64_t out_bytes,
                      rt_hip_stream stream) {
    const char* fn = "rt_hip_probe_read";
    if (!buf || !out) return set_error(RT_HIP_E_ARG, std::string(fn) + ": null pointer");
    if (out_bytes < 0 || out_bytes % 4) return set_error(RT_HIP_E_ALIGN, std::string(fn) + ": out_bytes must be a multiple of 4");
    if (bytes <= 0 || bytes % 16) return set_error(RT_HIP_E_ALIGN, std::string(fn) + ": bytes must be a positive multiple of 16");
    if (reinterpret_cast<uintptr_t>(buf) & 15u) return set_error(RT_HIP_E_ALIGN, std::string(fn) + ": buf must be 16-byte aligned");
    if (workgroups < 1 || workgroups > 65536)
        return set_error(RT_HIP_E_SHAPE, std::string(fn) + ": workgroups must be in [1, 65536]");
    const int64_t words = bytes / 16;
    // whole 4 KB rounds per workgroup, so every workgroup's loads stay aligned
    int64_t per = (words + workgroups - 1) / workgroups;
    per = (per + kThreads - 1) / kThreads * kThreads;
    const unsigned grid = static_cast<unsigned>((words + per - 1) / per);
    hipLaunchKernelGGL(k_probe_read<8>, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       static_cast<const u32x4*>(buf), words, per, out, out_bytes / 4);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? RT_HIP_OK : set_error(RT_HIP_E_HIP, std::string(fn) + ": " + hipGetErrorString(e));
}

int rt_hip_probe_empty(int32_t workgroups, int32_t threads, rt_hip_stream stream) {
    const char* fn = "rt_hip_probe_empty";
    if (workgroups < 1 || workgroups > 65536 || threads < 1 || threads > 1024)
        return set_error(RT_HIP_E_SHAPE, std::string(fn) + ": workgroups in [1, 65536], threads in [1, 1024]");
    hipLaunchKernelGGL(k_probe_empty, dim3(static_cast<unsigned>(workgroups)), dim3(static_cast<unsigned>(threads)), 0,
                       static_cast<hipStream_t>(stream));
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? RT_HIP_OK : set_error(RT_HIP_E_HIP, std::string(fn) + ": " + hipGetErrorString(e));
}

}  // extern "C"
