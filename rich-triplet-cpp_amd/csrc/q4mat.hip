// q4mat.hip -- the reference's own 4-bit format, Q4Mat (include/rt/quant.hpp:
// 23-75, src/quant_q4.cpp:17-156), on the GPU: the M <= 8 GEMV, and the
// dequantization to bf16 / f32 that the any-M GEMM and the parity tests use;
// plus the GGUF Q4_0 dequantization for the same GEMM path.
//
// Q4Mat storage, one device buffer (rt_hip.h):
//   [0, ceil(N*K/2))          packed: flat element k = r*K + c is the low
//                             nibble of byte k/2 when k is even, the high
//                             nibble when odd; 4-bit two's complement
//   [scales_off, +4*N*K/32)   f32 scale per 32 flat elements
// With K % 32 == 0 (required here) a row is K/32 whole groups: group g of
// row r is packed bytes (r*K + 32g)/2 .. +16 (16-byte aligned) and scale
// (r*K)/32 + g.
//
// GEMV: w = s(nib) * scale with s(n) = (n ^ 8) - 8, so per group
//     sum_j x_j w_j = scale * (sum_j (nib_j ^ 8) x_j - 8 * sum_j x_j):
// the XOR flips bit 3 of every nibble at once (v ^ 0x88888888) and the
// group's sum of x is precomputed when x is staged.  A lane owns whole
// groups (one 16-byte and one 4-byte load), x [M][K] sits in LDS
// chunk-major (16-byte chunk c of group g at (c*NG + g)*16, so the lanes of
// one LDS read hit consecutive chunks), rows are reduced across the wave.
// Numerics: f32, factorized and reordered against the reference's
// sequential dequantize-and-dot (quant_q4.cpp:92-114): agreement to f32
// rounding (normwise 1e-5 in the tests).
//
// Dequantization: w = (float)s(nib) * scale, the reference's product
// (quant_q4.cpp:77), rounded to bf16 (RNE) for the GEMM; GGUF Q4_0:
// ((q & 15) - 8) * d for value j, ((q >> 4) - 8) * d for value j + 16
// (gguf.cpp:495-529), exact in f32.
#include "gemv_bf16.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

constexpr int kT = 256;  // 4 waves

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// x[M][K] -> LDS chunk-major per row, with the per-group sums.  Thread f
// handles 16-byte chunk f of the flattened x; a group's 8 chunks are 8
// consecutive threads (DPP sum within the aligned 8-lane group).
template <int M>
__device__ __forceinline__ void stage_x(const float* __restrict__ X, int K, f32x4* xs, float* sums) {
    const int NG = K >> 5, nx4 = K >> 2;
    for (int f0 = 0; f0 < M * nx4; f0 += kT) {
        const int f = f0 + static_cast<int>(threadIdx.x);
        const bool in = f < M * nx4;
        const f32x4 v = reinterpret_cast<const f32x4*>(X)[in ? f : 0];
        float s = (v[0] + v[1]) + (v[2] + v[3]);
        s += dpp_f<0xb1>(s);   // lane ^ 1
        s += dpp_f<0x4e>(s);   // lane ^ 2
        s += dpp_f<0x141>(s);  // half-row mirror: lane i <-> 7 - i
        if (in) {
            const int m = f / nx4, c = f - m * nx4;
            xs[m * nx4 + (c & 7) * NG + (c >> 3)] = v;
            if ((c & 7) == 0) sums[m * NG + (c >> 3)] = s;
        }
    }
    lds_barrier();
}

template <int M>
__global__ __launch_bounds__(kT) void k_gemv_q4mat(const uint8_t* __restrict__ P, const float* __restrict__ S,
                                                   const float* __restrict__ X, float* __restrict__ Y, int N,
                                                   int K) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int NG = K >> 5, nx4 = K >> 2;
    f32x4* const xs = reinterpret_cast<f32x4*>(lds);
    float* const sums = reinterpret_cast<float*>(lds + static_cast<size_t>(16) * M * nx4);
    stage_x<M>(X, K, xs, sums);

    const int lane = threadIdx.x & 63;
    const int NW = static_cast<int>(gridDim.x) * (kT / kWave);
    const int gw = static_cast<int>(blockIdx.x) * (kT / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int r = gw; r < N; r += NW) {
        const int64_t row0 = static_cast<int64_t>(r) * K;
        const BufRsrc rp = make_rsrc(P + row0 / 2, K / 2);
        const BufRsrc rs = make_rsrc(S + row0 / 32, static_cast<int64_t>(NG) * 4);
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = 0.0f;
        // Two groups per lane in flight: both loads issued before either is used.
        for (int g0 = 0; g0 < NG; g0 += 128) {
            u32x4 q[2];
            float sc[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int g = g0 + 64 * u + lane;
                q[u] = ld16(rp, static_cast<uint32_t>(g < NG ? 16 * g : 0x7ffffff0));
                sc[u] = __uint_as_float(
                    __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(g < NG ? 4 * g : 0x7ffffff0), 0, 0));
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int g = g0 + 64 * u + lane;
                const int gg = g < NG ? g : 0;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const f32x4* xm = xs + m * nx4;
                    float dc[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        // dword c: bytes 4c..4c+3 = values 8c..8c+7 (low nibble even)
                        const uint32_t v = q[u][c] ^ 0x88888888u;
                        const uint32_t lo = v & 0x0f0f0f0fu, hi = (v >> 4) & 0x0f0f0f0fu;
                        const f32x4 a = xm[(2 * c) * NG + gg], b = xm[(2 * c + 1) * NG + gg];
                        float t = ubyte_f32(lo, 0) * a[0];
                        t = __builtin_fmaf(ubyte_f32(hi, 0), a[1], t);
                        t = __builtin_fmaf(ubyte_f32(lo, 1), a[2], t);
                        t = __builtin_fmaf(ubyte_f32(hi, 1), a[3], t);
                        t = __builtin_fmaf(ubyte_f32(lo, 2), b[0], t);
                        t = __builtin_fmaf(ubyte_f32(hi, 2), b[1], t);
                        t = __builtin_fmaf(ubyte_f32(lo, 3), b[2], t);
                        t = __builtin_fmaf(ubyte_f32(hi, 3), b[3], t);
                        dc[c] = t;
                    }
                    const float dot = (dc[0] + dc[1]) + (dc[2] + dc[3]);
                    const float blk = sc[u] * __builtin_fmaf(-8.0f, sums[m * NG + gg], dot);
                    acc[m] += g < NG ? blk : 0.0f;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float v = bf16_gemv::wave_sum(acc[m], lane);
            if (lane == m) Y[static_cast<int64_t>(m) * N + r] = v;
        }
    }
}

template <int M>
hipError_t run_gemv(const uint8_t* p, const float* sc, const float* x, float* y, int64_t n, int64_t k, hipStream_t s) {
    const size_t lds = q4mat_gemv_lds_bytes(M, k);
    const int64_t waves = kT / kWave;
    const int64_t cus = device_info().cus;
    int64_t wgs = (n + waves - 1) / waves;
    const int64_t cap = 8 * cus;  // grid-stride beyond eight workgroups per CU
    wgs = wgs > cap ? cap : wgs;
    hipLaunchKernelGGL(k_gemv_q4mat<M>, dim3(static_cast<unsigned>(wgs)), dim3(kT), lds, s, p, sc, x, y,
                       static_cast<int>(n), static_cast<int>(k));
    return hipGetLastError();
}

// ---- dequantization --------------------------------------------------------
// One lane per 32-value group; 4 units per lane per round (grid-stride).
template <bool BF16>
__device__ __forceinline__ void store32(void* out, int64_t o, const float (&w)[32]) {
    if constexpr (BF16) {
        u32x4* d = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + o);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            d[c] = u32x4{bf16_pair(w[8 * c], w[8 * c + 1]), bf16_pair(w[8 * c + 2], w[8 * c + 3]),
                         bf16_pair(w[8 * c + 4], w[8 * c + 5]), bf16_pair(w[8 * c + 6], w[8 * c + 7])};
    } else {
        f32x4* d = reinterpret_cast<f32x4*>(static_cast<float*>(out) + o);
#pragma unroll
        for (int c = 0; c < 8; ++c) d[c] = f32x4{w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]};
    }
}

template <bool BF16>
__global__ __launch_bounds__(256) void k_dequant_q4mat(const uint8_t* __restrict__ P, const float* __restrict__ S,
                                                       void* __restrict__ out, int64_t groups) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; g < groups; g += stride) {
        const u32x4 q = *reinterpret_cast<const u32x4*>(P + 16 * g);
        const float sc = S[g];
        float w[32];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t byte = (q[c] >> (8 * e)) & 0xffu;
                const int lo = static_cast<int>((byte & 15u) ^ 8u) - 8, hi = static_cast<int>((byte >> 4) ^ 8u) - 8;
                w[8 * c + 2 * e] = static_cast<float>(lo) * sc;
                w[8 * c + 2 * e + 1] = static_cast<float>(hi) * sc;
            }
        store32<BF16>(out, 32 * g, w);
    }
}

// GGUF Q4_0: 18-byte blocks (2-byte aligned), read as nine u16.
template <bool BF16>
__global__ __launch_bounds__(256) void k_dequant_q4_0(const uint8_t* __restrict__ B, void* __restrict__ out,
                                                      int64_t blocks) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; b < blocks; b += stride) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(B + kQ40BlockBytes * b);
        const float d = f16_bits_to_f32(h[0]);
        float w[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t two = h[1 + i];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t byte = (two >> (8 * e)) & 0xffu;
                w[2 * i + e] = static_cast<float>(static_cast<int>(byte & 15u) - 8) * d;
                w[16 + 2 * i + e] = static_cast<float>(static_cast<int>(byte >> 4) - 8) * d;
            }
        }
        store32<BF16>(out, 32 * b, w);
    }
}

dim3 grid_for(int64_t units) {
    const int64_t cap = 16 * static_cast<int64_t>(device_info().cus);
    const int64_t want = (units + 255) / 256;
    return dim3(static_cast<unsigned>(want < cap ? (want < 1 ? 1 : want) : cap));
}

}  // namespace

size_t q4mat_scales_offset(int64_t n, int64_t k) {
    const int64_t packed = (n * k + 1) / 2;
    return static_cast<size_t>((packed + 255) / 256 * 256);
}

size_t q4mat_bytes(int64_t n, int64_t k) {
    return q4mat_scales_offset(n, k) + static_cast<size_t>((n * k + 31) / 32) * 4;
}

size_t q4mat_gemv_lds_bytes(int m, int64_t k) {
    return static_cast<size_t>(m) * (static_cast<size_t>(k) * 4 + static_cast<size_t>(k / 32) * 4);
}

hipError_t launch_gemv_q4mat(const void* w, const float* x, float* y, int64_t n, int64_t k, int m, hipStream_t s) {
    const auto* p = static_cast<const uint8_t*>(w);
    const auto* sc = reinterpret_cast<const float*>(p + q4mat_scales_offset(n, k));
    switch (m) {
        case 1: return run_gemv<1>(p, sc, x, y, n, k, s);
        case 2: return run_gemv<2>(p, sc, x, y, n, k, s);
        case 3: return run_gemv<3>(p, sc, x, y, n, k, s);
        case 4: return run_gemv<4>(p, sc, x, y, n, k, s);
        case 5: return run_gemv<5>(p, sc, x, y, n, k, s);
        case 6: return run_gemv<6>(p, sc, x, y, n, k, s);
        case 7: return run_gemv<7>(p, sc, x, y, n, k, s);
        case 8: return run_gemv<8>(p, sc, x, y, n, k, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dequant_4bit(int fmt, const void* w, void* out, bool bf16, int64_t n, int64_t k, hipStream_t s) {
    const auto* p = static_cast<const uint8_t*>(w);
    const int64_t groups = n * k / 32;
    if (fmt == RT_HIP_Q4MAT) {
        const auto* sc = reinterpret_cast<const float*>(p + q4mat_scales_offset(n, k));
        if (bf16)
            hipLaunchKernelGGL(k_dequant_q4mat<true>, grid_for(groups), dim3(256), 0, s, p, sc, out, groups);
        else
            hipLaunchKernelGGL(k_dequant_q4mat<false>, grid_for(groups), dim3(256), 0, s, p, sc, out, groups);
    } else if (fmt == RT_HIP_Q4_0) {
        if (bf16)
            hipLaunchKernelGGL(k_dequant_q4_0<true>, grid_for(groups), dim3(256), 0, s, p, out, groups);
        else
            hipLaunchKernelGGL(k_dequant_q4_0<false>, grid_for(groups), dim3(256), 0, s, p, out, groups);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rt_hip
