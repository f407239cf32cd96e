// argmax.hip -- greedy token selection over logits rows.
//
// Semantics of the reference's greedy branch (src/transformer5.cpp:382-391):
// the first index of the strict maximum; NaN is never selected; a row with
// nothing above -inf yields index 0.
//
// Each (value, index) pair is packed into one u64 key: an order-preserving
// map of the f32 (with -0 folded onto +0, since -0 > +0 is false in the
// reference's comparison) in the high half and (0xffffffff - index) in the
// low half.  The maximum key is then the largest value with the lowest
// index.  Keys start at (-inf, index 0), which every finite value beats and
// no -inf beats, so an all -inf/NaN row keeps index 0.  Blocks combine with
// atomicMax (order-independent, so the result is deterministic).
#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

constexpr uint32_t kNegInfOrdered = ~0xff800000u;  // order map of -inf
constexpr uint64_t kInitKey = (static_cast<uint64_t>(kNegInfOrdered) << 32) | 0xffffffffull;

__global__ void k_argmax_init(uint64_t* keys, int64_t rows) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < rows) keys[i] = kInitKey;
}

// grid = (chunks, rows): block (c, r) scans a chunk of row r.
__global__ __launch_bounds__(256) void k_argmax_scan(const float* __restrict__ v, int64_t cols,
                                                     int64_t chunk, uint64_t* keys) {
    const int64_t r = blockIdx.y;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * chunk;
    int64_t c1 = c0 + chunk;
    if (c1 > cols) c1 = cols;
    const float* row = v + r * cols;
    uint64_t best = 0;
    // four independent loads per thread per round
    for (int64_t cb = c0 + threadIdx.x; cb < c1; cb += 4 * 256) {
        float x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t c = cb + u * 256;
            x[u] = c < c1 ? row[c] : __builtin_nanf("");
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (x[u] == x[u]) {
                const uint64_t k = argmax_key(x[u], static_cast<uint32_t>(cb + u * 256));
                best = k > best ? k : best;
            }
        }
    }
#pragma unroll
    for (int off = kWave / 2; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off, kWave);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & (kWave - 1)) == 0 && best != 0)
        atomicMax(reinterpret_cast<unsigned long long*>(keys + r),
                  static_cast<unsigned long long>(best));
}

__global__ void k_argmax_finalize(const uint64_t* keys, int64_t rows, int64_t* idx, float* val) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    const uint64_t k = keys[i];
    const uint32_t u = static_cast<uint32_t>(k >> 32);
    const uint32_t bits = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
    idx[i] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(k));
    if (val) val[i] = __uint_as_float(bits);
}

// Largest of `count` partial keys (0 = empty) -> idx[0], val[0]; one
// workgroup, order-independent.  U loads in flight per thread before any is
// compared (the launcher picks U so that one round covers the keys: 8016
// for the Q4_K lm_head of 128256 rows, 32768 for a BF16 one of 262144).
// Indices past the end repeat the thread's first key, which changes no
// maximum: loads behind a branch would each be waited for on their own.
template <int U>
__global__ __launch_bounds__(1024) void k_argmax_reduce(const uint64_t* __restrict__ part, int64_t count,
                                                        int64_t* idx, float* val) {
    __shared__ uint64_t wbest[1024 / kWave];
    uint64_t best = kInitKey;
    const int64_t first = threadIdx.x < count ? threadIdx.x : 0;
    for (int64_t i0 = threadIdx.x; i0 < count; i0 += U * 1024) {
        uint64_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + u * 1024;
            v[u] = part[i < count ? i : first];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) best = v[u] > best ? v[u] : best;
    }
#pragma unroll
    for (int off = kWave / 2; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off, kWave);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & (kWave - 1)) == 0) wbest[threadIdx.x / kWave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = wbest[0];
        for (int w = 1; w < 1024 / kWave; ++w) b = wbest[w] > b ? wbest[w] : b;
        const uint32_t u = static_cast<uint32_t>(b >> 32);
        const uint32_t bits = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
        idx[0] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(b));
        if (val) val[0] = __uint_as_float(bits);
    }
}

}  // namespace

hipError_t launch_argmax_reduce(const uint64_t* part, int64_t count, int64_t* idx, float* val, hipStream_t s) {
    if (count <= 8 * 1024)
        hipLaunchKernelGGL(k_argmax_reduce<8>, dim3(1), dim3(1024), 0, s, part, count, idx, val);
    else if (count <= 16 * 1024)
        hipLaunchKernelGGL(k_argmax_reduce<16>, dim3(1), dim3(1024), 0, s, part, count, idx, val);
    else
        hipLaunchKernelGGL(k_argmax_reduce<32>, dim3(1), dim3(1024), 0, s, part, count, idx, val);
    return hipGetLastError();
}

hipError_t launch_argmax_init(uint64_t* keys, int64_t rows, hipStream_t s) {
    const unsigned blocks = static_cast<unsigned>((rows + 255) / 256);
    hipLaunchKernelGGL(k_argmax_init, dim3(blocks), dim3(256), 0, s, keys, rows);
    return hipGetLastError();
}

hipError_t launch_argmax_scan(const float* v, int64_t rows, int64_t cols, uint64_t* keys,
                              hipStream_t s) {
    // About two blocks per CU over the whole matrix, each a whole number of
    // 1024-value rounds (at least one).
    const int64_t cus = device_info().cus;
    int64_t per_row = (2 * cus + rows - 1) / rows;
    per_row = per_row < 1 ? 1 : per_row;
    int64_t chunk = (cols + per_row - 1) / per_row;
    chunk = (chunk + 1023) / 1024 * 1024;
    int64_t chunks = (cols + chunk - 1) / chunk;
    if (chunks < 1) chunks = 1;
    hipLaunchKernelGGL(k_argmax_scan, dim3(static_cast<unsigned>(chunks),
                                           static_cast<unsigned>(rows)),
                       dim3(256), 0, s, v, cols, chunk, keys);
    return hipGetLastError();
}

hipError_t launch_argmax_finalize(uint64_t* keys, int64_t rows, int64_t* idx, float* val,
                                  hipStream_t s) {
    const unsigned blocks = static_cast<unsigned>((rows + 255) / 256);
    hipLaunchKernelGGL(k_argmax_finalize, dim3(blocks), dim3(256), 0, s, keys, rows, idx, val);
    return hipGetLastError();
}

}  // namespace rt_hip
