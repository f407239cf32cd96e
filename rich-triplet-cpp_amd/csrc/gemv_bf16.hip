// gemv_bf16.hip -- the M = 1 BF16 GEMV kernel (decode): one launch of the
// row body in gemv_bf16.hpp.
#include "gemv_bf16.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

using namespace bf16_gemv;

template <int D, int XP, bool ARGMAX, int T>
__global__ __launch_bounds__(T) void k_gemv_bf16(const uint16_t* __restrict__ W, const float* __restrict__ X,
                                                 float* __restrict__ Y, int N, int K,
                                                 uint64_t* __restrict__ key) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if constexpr (ARGMAX) {
        // The fused argmax: each wave's best key lands in LDS, the
        // workgroup's best goes to key[blockIdx.x], and a second launch folds
        // those partials (one atomic target for every wave serialized the
        // 262144-row lm_head).
        __shared__ uint64_t wbest[T / kWave];
        rows<D, XP, ARGMAX, T>(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), W, X, Y, N, K, wbest,
                               lds);
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t b = wbest[0];
            for (int w = 1; w < T / kWave; ++w) b = wbest[w] > b ? wbest[w] : b;
            key[blockIdx.x] = b;
        }
    } else {
        rows<D, XP, ARGMAX, T>(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), W, X, Y, N, K, key,
                               lds);
    }
}

// The same with a layer operation applied to x while it is staged (XOp);
// ARGMAX as above (the key of each row as stored, after the norm's scale).
template <int D, int XP, int T, int XOP, bool ADD, bool ARGMAX = false>
__global__ __launch_bounds__(T) void k_gemv_bf16_xop(const uint16_t* __restrict__ W, const float* __restrict__ X,
                                                    const float* __restrict__ aux, float* __restrict__ Y, int N,
                                                    int K, float eps, uint64_t* __restrict__ key = nullptr) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if constexpr (ARGMAX) {
        __shared__ uint64_t wbest[T / kWave];
        rows<D, XP, true, T, XOP, ADD>(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), W, X, Y, N, K,
                                       wbest, lds, aux, eps);
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t b = wbest[0];
            for (int w = 1; w < T / kWave; ++w) b = wbest[w] > b ? wbest[w] : b;
            key[blockIdx.x] = b;
        }
    } else {
        rows<D, XP, false, T, XOP, ADD>(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), W, X, Y, N, K,
                                        nullptr, lds, aux, eps);
    }
}

// T threads per workgroup, each wave looping over its rows; x is prefetched into registers before the
// weight prologue when XP * T covers K / 4 (else the rest is copied after).
// Rows per wave (at most 64: the row sums stay in lanes), measured: 4 for
// short rows (<= 3 pieces: one row alone leaves the ring part empty), 2 for
// long ones (x is staged by half as many workgroups), else 1.
int64_t bf16_workgroups(int64_t n, int64_t k, int T) {
    const int64_t waves = T / kWave, pieces = (k + kPiece - 1) / kPiece;
    int64_t rpw = tune_param("BF16_ROWS_PER_WAVE", pieces <= 3 ? 4 : (pieces >= 12 ? 2 : 1));
    rpw = rpw < 1 ? 1 : (rpw > 64 ? 64 : rpw);
    return (n + waves * rpw - 1) / (waves * rpw);
}

template <bool ARGMAX, int T>
hipError_t run(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k, uint64_t* key,
               hipStream_t s) {
    const int64_t wgs = bf16_workgroups(n, k, T);
    const size_t lds = bf16_m1_lds_bytes(k);
    const int ik = static_cast<int>(k), in = static_cast<int>(n);
    const int64_t per = (k / 4 + T - 1) / T;
    const dim3 g(static_cast<unsigned>(wgs)), b(T);
    if (tune_param("BF16_RING", 8) == 16) {
        if (per <= 2)
            hipLaunchKernelGGL((k_gemv_bf16<16, 2, ARGMAX, T>), g, b, lds, s, w, x, y, in, ik, key);
        else if (per <= 4)
            hipLaunchKernelGGL((k_gemv_bf16<16, 4, ARGMAX, T>), g, b, lds, s, w, x, y, in, ik, key);
        else
            hipLaunchKernelGGL((k_gemv_bf16<16, 8, ARGMAX, T>), g, b, lds, s, w, x, y, in, ik, key);
        return hipGetLastError();
    }
    if (per <= 2)
        hipLaunchKernelGGL((k_gemv_bf16<8, 2, ARGMAX, T>), g, b, lds, s, w, x, y, in, ik, key);
    else if (per <= 4)
        hipLaunchKernelGGL((k_gemv_bf16<8, 4, ARGMAX, T>), g, b, lds, s, w, x, y, in, ik, key);
    else
        hipLaunchKernelGGL((k_gemv_bf16<8, 8, ARGMAX, T>), g, b, lds, s, w, x, y, in, ik, key);
    return hipGetLastError();
}

template <bool ARGMAX>
hipError_t run_rows(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k, uint64_t* key,
                    hipStream_t s) {
    // One row per wave at a time, ring of 8 pieces; RT_HIP_BF16_WAVES (waves
    // per workgroup) overrides the measured default.
    const int waves = tune_param("BF16_WAVES", 8);
    if (waves == 4) return run<ARGMAX, 256>(w, x, y, n, k, key, s);
    if (waves == 12) return run<ARGMAX, 768>(w, x, y, n, k, key, s);
    if (waves == 16) return run<ARGMAX, 1024>(w, x, y, n, k, key, s);
    return run<ARGMAX, 512>(w, x, y, n, k, key, s);
}

}  // namespace

size_t bf16_m1_lds_bytes(int64_t k) { return bf16_gemv::lds_bytes(k); }

int64_t bf16_argmax_partials(int64_t n, int64_t k) {
    const int waves = tune_param("BF16_WAVES", 8);
    const int T = waves == 4 ? 256 : (waves == 12 ? 768 : (waves == 16 ? 1024 : 512));
    return bf16_workgroups(n, k, T);
}

hipError_t launch_gemv_bf16_m1(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                               uint64_t* key, hipStream_t s) {
    return key ? run_rows<true>(w, x, y, n, k, key, s) : run_rows<false>(w, x, y, n, k, key, s);
}

namespace {
// The default launch shape of run() (8 waves), with an x operation.
constexpr int kXopThreads = 512;
int64_t xop_workgroups(int64_t n, int64_t k) {
    const int64_t waves = kXopThreads / kWave, pieces = (k + kPiece - 1) / kPiece;
    const int64_t rpw = pieces <= 3 ? 4 : (pieces >= 12 ? 2 : 1);
    return (n + waves * rpw - 1) / (waves * rpw);
}

template <int XOP, bool ADD, bool ARGMAX = false>
hipError_t run_xop(const uint16_t* w, const float* x, const float* aux, float eps, float* y, int64_t n, int64_t k,
                   hipStream_t s, uint64_t* key = nullptr) {
    constexpr int T = kXopThreads;
    const int64_t wgs = xop_workgroups(n, k);
    const int64_t per = (k / 4 + T - 1) / T;
    const dim3 g(static_cast<unsigned>(wgs)), b(T);
    const size_t lds = bf16_m1_lds_bytes(k);
    const int ik = static_cast<int>(k), in = static_cast<int>(n);
    if (per <= 2)
        hipLaunchKernelGGL((k_gemv_bf16_xop<8, 2, T, XOP, ADD, ARGMAX>), g, b, lds, s, w, x, aux, y, in, ik, eps, key);
    else if (per <= 4)
        hipLaunchKernelGGL((k_gemv_bf16_xop<8, 4, T, XOP, ADD, ARGMAX>), g, b, lds, s, w, x, aux, y, in, ik, eps, key);
    else
        hipLaunchKernelGGL((k_gemv_bf16_xop<8, 8, T, XOP, ADD, ARGMAX>), g, b, lds, s, w, x, aux, y, in, ik, eps, key);
    return hipGetLastError();
}
}  // namespace

int64_t bf16_xop_argmax_partials(int64_t n, int64_t k) { return xop_workgroups(n, k); }

hipError_t launch_gemv_bf16_xop_argmax(int xop, const uint16_t* w, const float* x, const float* gamma, float eps,
                                       float* y, int64_t n, int64_t k, uint64_t* keys, hipStream_t s) {
    if (!keys) return hipErrorInvalidValue;
    switch (xop) {
        case kXRmsNorm: return run_xop<kXRmsNorm, false, true>(w, x, gamma, eps, y, n, k, s, keys);
        case kXRmsNorm1: return run_xop<kXRmsNorm1, false, true>(w, x, gamma, eps, y, n, k, s, keys);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_bf16_xop(int xop, const uint16_t* w, const float* x, const float* aux, float eps, float* y,
                                int64_t n, int64_t k, hipStream_t s, bool add) {
    if (add) return xop == kXSwiGlu ? run_xop<kXSwiGlu, true>(w, x, aux, eps, y, n, k, s) : hipErrorInvalidValue;
    switch (xop) {
        case kXRmsNorm: return run_xop<kXRmsNorm, false>(w, x, aux, eps, y, n, k, s);
        case kXRmsNorm1: return run_xop<kXRmsNorm1, false>(w, x, aux, eps, y, n, k, s);
        case kXSwiGlu: return run_xop<kXSwiGlu, false>(w, x, aux, eps, y, n, k, s);
        case kXGelu: return run_xop<kXGelu, false>(w, x, aux, eps, y, n, k, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rt_hip
