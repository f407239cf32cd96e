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

// Launch shape: waves per workgroup (T / 64), each wave looping over its
// rows; x is prefetched into registers before the weight prologue when
// XP * T covers K / 4 (else the rest is copied after).  Rows per wave (at
// most 64: the row sums stay in lanes), measured: 4 for short rows (<= 3
// pieces: one row alone leaves the ring part empty), 2 for long ones (x is
// staged by half as many workgroups), else 1, with 8 waves.  Long rows
// whose 16-row workgroups would leave CUs idle take 12 waves of one row
// each where that is one round: the K = 8192 BF16 down projection of
// 3072 rows in 256 workgroups instead of 192, the headline step 697-699
// against 702-704 us (4 waves of 3 rows, also 256 workgroups, 699-700).
// Outputs of more than 16 rounds of workgroups (the lm_heads) double the
// rows per wave up to 8, so each workgroup stages x for more rows: config
// 2b (262144 x 1152) 5214-5281 GB/s at 8 rows against 4880-4946 at 4 on
// one box (5104 at 16).
struct Bf16Shape {
    int waves;
    int64_t rpw;
};
int64_t amortized_rows(int64_t n, int waves, int64_t rpw) {
    const int64_t cus = device_info().cus;
    while (rpw < 8 && (n + waves * rpw - 1) / (waves * rpw) > 16 * cus) rpw *= 2;
    return rpw;
}
Bf16Shape bf16_shape(int64_t n, int64_t k) {
    const int64_t pieces = (k + kPiece - 1) / kPiece, cus = device_info().cus;
    Bf16Shape sh{8, amortized_rows(n, 8, pieces <= 3 ? 4 : (pieces >= 12 ? 2 : 1))};
    if (pieces >= 12 && (n + 15) / 16 < cus && (n + 11) / 12 <= cus) sh = Bf16Shape{12, 1};
    sh.waves = tune_param("BF16_WAVES", sh.waves);
    if (sh.waves != 4 && sh.waves != 12 && sh.waves != 16) sh.waves = 8;
    const int64_t r = tune_param("BF16_ROWS_PER_WAVE", static_cast<int>(sh.rpw));
    sh.rpw = r < 1 ? 1 : (r > 64 ? 64 : r);
    return sh;
}
int64_t bf16_workgroups(int64_t n, const Bf16Shape& sh) {
    return (n + sh.waves * sh.rpw - 1) / (sh.waves * sh.rpw);
}

template <bool ARGMAX, int T>
hipError_t run(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k, uint64_t* key,
               hipStream_t s, const Bf16Shape& sh) {
    const int64_t wgs = bf16_workgroups(n, sh);
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
    // One row per wave at a time, ring of 8 pieces.
    const Bf16Shape sh = bf16_shape(n, k);
    if (sh.waves == 4) return run<ARGMAX, 256>(w, x, y, n, k, key, s, sh);
    if (sh.waves == 12) return run<ARGMAX, 768>(w, x, y, n, k, key, s, sh);
    if (sh.waves == 16) return run<ARGMAX, 1024>(w, x, y, n, k, key, s, sh);
    return run<ARGMAX, 512>(w, x, y, n, k, key, s, sh);
}

}  // namespace

size_t bf16_m1_lds_bytes(int64_t k) { return bf16_gemv::lds_bytes(k); }

int64_t bf16_argmax_partials(int64_t n, int64_t k) { return bf16_workgroups(n, bf16_shape(n, k)); }

hipError_t launch_gemv_bf16_m1(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                               uint64_t* key, hipStream_t s) {
    return key ? run_rows<true>(w, x, y, n, k, key, s) : run_rows<false>(w, x, y, n, k, key, s);
}

namespace {
// run()'s default launch shape (8 waves) with an x operation.  The 12-wave
// shape of long rows measured slower here: the Llama-3.2-3B engine's BF16
// SwiGLU + down + residual 1124.6-1124.9 against 1116.0-1117.3 us/token.
// Nor do more rows per wave pay for the Gemma-3-4B lm_head (262144 x 2560
// with the final norm): engine token 1623-1627 us at 8 rows against
// 1608-1612 at 1, on one box.
Bf16Shape xop_shape(int64_t n, int64_t k) {
    const int64_t pieces = (k + kPiece - 1) / kPiece;
    const int r = tune_param("BF16_XOP_ROWS_PER_WAVE", pieces <= 3 ? 4 : (pieces >= 12 ? 2 : 1));
    return Bf16Shape{8, r < 1 ? 1 : (r > 64 ? 64 : r)};
}

template <int XOP, bool ADD, bool ARGMAX, int T>
hipError_t run_xop_t(const uint16_t* w, const float* x, const float* aux, float eps, float* y, int64_t n, int64_t k,
                     hipStream_t s, uint64_t* key, const Bf16Shape& sh) {
    const int64_t wgs = bf16_workgroups(n, sh);
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

template <int XOP, bool ADD, bool ARGMAX = false>
hipError_t run_xop(const uint16_t* w, const float* x, const float* aux, float eps, float* y, int64_t n, int64_t k,
                   hipStream_t s, uint64_t* key = nullptr) {
    return run_xop_t<XOP, ADD, ARGMAX, 512>(w, x, aux, eps, y, n, k, s, key, xop_shape(n, k));
}
}  // namespace

int64_t bf16_xop_argmax_partials(int64_t n, int64_t k) { return bf16_workgroups(n, xop_shape(n, k)); }

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
