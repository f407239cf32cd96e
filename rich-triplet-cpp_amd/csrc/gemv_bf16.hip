// gemv_bf16.hip -- the M = 1 BF16 GEMV kernel (decode): one launch of the
// row body in gemv_bf16.hpp.
#include "gemv_bf16.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

using namespace bf16_gemv;

template <int RPW, int D, int XP, bool ARGMAX>
__global__ __launch_bounds__(kThreads) void k_gemv_bf16(const uint16_t* __restrict__ W,
                                                        const float* __restrict__ X,
                                                        float* __restrict__ Y, int N, int K,
                                                        uint64_t* __restrict__ key) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    rows<RPW, D, XP, ARGMAX>(static_cast<int>(blockIdx.x), W, X, Y, N, K, key, lds);
}

template <int RPW, int D, bool ARGMAX>
hipError_t run(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k, uint64_t* key,
               hipStream_t s) {
    const int64_t rows_per_wg = static_cast<int64_t>(kThreads / kWave) * RPW;
    const int64_t wgs = (n + rows_per_wg - 1) / rows_per_wg;
    const size_t lds = bf16_m1_lds_bytes(k);
    const int ik = static_cast<int>(k), in = static_cast<int>(n);
    if (k <= 4 * kThreads * 4)
        hipLaunchKernelGGL((k_gemv_bf16<RPW, D, 4, ARGMAX>), dim3(static_cast<unsigned>(wgs)),
                           dim3(kThreads), lds, s, w, x, y, in, ik, key);
    else
        hipLaunchKernelGGL((k_gemv_bf16<RPW, D, 8, ARGMAX>), dim3(static_cast<unsigned>(wgs)),
                           dim3(kThreads), lds, s, w, x, y, in, ik, key);
    return hipGetLastError();
}

template <bool ARGMAX>
hipError_t run_rows(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k, uint64_t* key,
                    hipStream_t s) {
    // One row per wave measured fastest at every decode shape (more, smaller
    // workgroups balance better over the CUs); RT_HIP_BF16_RPW overrides.
    const int rpw = tune_param("BF16_RPW", 1);
    const int ring = tune_param("BF16_RING", 8);
    if (rpw <= 1) return ring >= 16 ? run<1, 16, ARGMAX>(w, x, y, n, k, key, s) : run<1, 8, ARGMAX>(w, x, y, n, k, key, s);
    if (rpw == 2) return run<2, 8, ARGMAX>(w, x, y, n, k, key, s);
    if (rpw == 3) return run<3, 8, ARGMAX>(w, x, y, n, k, key, s);
    return run<4, 4, ARGMAX>(w, x, y, n, k, key, s);
}

}  // namespace

size_t bf16_m1_lds_bytes(int64_t k) { return bf16_gemv::lds_bytes(k); }

hipError_t launch_gemv_bf16_m1(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                               uint64_t* key, hipStream_t s) {
    return key ? run_rows<true>(w, x, y, n, k, key, s) : run_rows<false>(w, x, y, n, k, key, s);
}

}  // namespace rt_hip
