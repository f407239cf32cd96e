// gemm.hip -- prefill / FLUX GEMM on bf16 MFMA (gfx950), C = A * W^T (+ bias).
//
// W is Q4_K blocks or bf16 [N, K]; A is f32 or bf16 [M, K]; C is f32 [M, N].
// Operands are rounded to bf16 (RNE) where they enter LDS and contracted
// with v_mfma_f32_16x16x32_bf16, f32 accumulation.  A Q4_K weight is
// dequantized tile by tile straight into LDS (each K step of 64 values is
// one 32-byte qs chunk of every row's super-block), so no dequantized copy
// of the weight is ever written to HBM -- unlike the reference's FLUX path,
// which dequantizes the whole weight into a scratch buffer before its GEMM
// (src/metal_flux.mm:155-185).
//
// Block tile 128 x 128 x 64, 256 threads = 4 waves in 2 x 2, each wave a
// 64 x 64 sub-tile of 4 x 4 MFMA 16x16 tiles.
//
// MFMA operand layout: lane l supplies row (l % 16) of its A fragment and
// column (l % 16) of its B fragment, 8 bf16 K-values each, the K slot being
// selected by l / 16; A and B use the same K slots, so the contraction is
// independent of how the hardware orders K.  The f32 result: lane l holds
// C[4 * (l / 16) + r][l % 16], r = 0..3.
#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (16 B pad)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return static_cast<uint32_t>(f32_to_bf16_rne(a)) |
           (static_cast<uint32_t>(f32_to_bf16_rne(b)) << 16);
}

template <int WFMT, bool A_BF16>
__global__ __launch_bounds__(256) void k_gemm(const void* __restrict__ Ap,
                                              const void* __restrict__ Wp,
                                              const float* __restrict__ bias,
                                              float* __restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t sB[BN * LDS_STRIDE];
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Staging roles: thread -> (row, 32-value half) of the 128 x 64 tiles.
    const int sr = tid >> 1, shalf = tid & 1;
    const int gm = m0 + sr, gn = n0 + sr;
    const int nb = K >> 8;

    for (int k0 = 0; k0 < K; k0 += BK) {
        // ---- A tile: 32 values of row gm at k0 + 32*shalf -> bf16 in LDS.
        {
            u32x4 out[4];
            if (gm < M) {
                if constexpr (A_BF16) {
                    const uint16_t* src = static_cast<const uint16_t*>(Ap) +
                                          static_cast<size_t>(gm) * K + k0 + 32 * shalf;
#pragma unroll
                    for (int j = 0; j < 4; ++j) out[j] = ld16(src + 8 * j);
                } else {
                    const float* src = static_cast<const float*>(Ap) +
                                       static_cast<size_t>(gm) * K + k0 + 32 * shalf;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const f32x4 v0 = reinterpret_cast<const f32x4*>(src)[2 * j];
                        const f32x4 v1 = reinterpret_cast<const f32x4*>(src)[2 * j + 1];
                        out[j] = u32x4{pack_bf16x2(v0[0], v0[1]), pack_bf16x2(v0[2], v0[3]),
                                       pack_bf16x2(v1[0], v1[1]), pack_bf16x2(v1[2], v1[3])};
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = u32x4{0u, 0u, 0u, 0u};
            }
            u32x4* dst = reinterpret_cast<u32x4*>(sA + sr * LDS_STRIDE + 32 * shalf);
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[j] = out[j];
        }
        // ---- W tile.
        if constexpr (WFMT == RT_HIP_Q4K) {
            // Row gn, qs chunk c of super-block b, half shalf: 16 low-nibble
            // values at k0 + 16*shalf and 16 high-nibble values 32 later.
            u32x4 lo2[2], hi2[2];
            if (gn < N) {
                const int b = k0 >> 8, c = (k0 >> 6) & 3;
                const uint8_t* bp = static_cast<const uint8_t*>(Wp) +
                                    (static_cast<size_t>(gn) * nb + b) * kQ4kBlockBytes;
                const u32x4 hd = ld16(bp);
                const u32x4 q = ld16(bp + 16 + 32 * c + 16 * shalf);
                const float d = f16_bits_to_f32(hd[0] & 0xffffu);
                const float dm = f16_bits_to_f32(hd[0] >> 16);
                uint32_t sv1, mv1, sv2, mv2;
                decode_scale_min(make_scale_sel(2 * c), hd[1], hd[2], hd[3], sv1, mv1);
                decode_scale_min(make_scale_sel(2 * c + 1), hd[1], hd[2], hd[3], sv2, mv2);
                const float s1 = d * static_cast<float>(sv1), n1 = dm * static_cast<float>(mv1);
                const float s2 = d * static_cast<float>(sv2), n2 = dm * static_cast<float>(mv2);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w = q[j];
                    float l[4], h[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t byte = (w >> (8 * e)) & 0xffu;
                        l[e] = s1 * static_cast<float>(byte & 0x0fu) - n1;
                        h[e] = s2 * static_cast<float>(byte >> 4) - n2;
                    }
                    lo2[j >> 1][2 * (j & 1)] = pack_bf16x2(l[0], l[1]);
                    lo2[j >> 1][2 * (j & 1) + 1] = pack_bf16x2(l[2], l[3]);
                    hi2[j >> 1][2 * (j & 1)] = pack_bf16x2(h[0], h[1]);
                    hi2[j >> 1][2 * (j & 1) + 1] = pack_bf16x2(h[2], h[3]);
                }
            } else {
                lo2[0] = lo2[1] = hi2[0] = hi2[1] = u32x4{0u, 0u, 0u, 0u};
            }
            u32x4* dlo = reinterpret_cast<u32x4*>(sB + sr * LDS_STRIDE + 16 * shalf);
            u32x4* dhi = reinterpret_cast<u32x4*>(sB + sr * LDS_STRIDE + 32 + 16 * shalf);
            dlo[0] = lo2[0];
            dlo[1] = lo2[1];
            dhi[0] = hi2[0];
            dhi[1] = hi2[1];
        } else {
            u32x4 out[4];
            if (gn < N) {
                const uint16_t* src = static_cast<const uint16_t*>(Wp) +
                                      static_cast<size_t>(gn) * K + k0 + 32 * shalf;
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = ld16(src + 8 * j);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = u32x4{0u, 0u, 0u, 0u};
            }
            u32x4* dst = reinterpret_cast<u32x4*>(sB + sr * LDS_STRIDE + 32 * shalf);
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[j] = out[j];
        }
        __syncthreads();

        // ---- 2 MFMA K-steps of 32.
        const int fr = lane & 15, fk = 8 * (lane >> 4);
#pragma unroll
        for (int ks = 0; ks < BK; ks += 32) {
            bf16x8 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(sA + (wm + 16 * i + fr) * LDS_STRIDE + ks + fk);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bf[j] = *reinterpret_cast<const bf16x8*>(sB + (wn + 16 * j + fr) * LDS_STRIDE + ks + fk);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // ---- epilogue
    const int cr = 4 * (lane >> 4), cc = lane & 15;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = n0 + wn + 16 * j + cc;
        if (col >= N) continue;
        const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm + 16 * i + cr + r;
                if (row < M) C[static_cast<size_t>(row) * N + col] = acc[i][j][r] + bv;
            }
        }
    }
}

__global__ void k_add_bias(float* __restrict__ y, const float* __restrict__ bias, int64_t m,
                           int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < m * n) y[i] += bias[i % n];
}

}  // namespace

hipError_t launch_gemm(int w_fmt, const void* a, bool a_bf16, const void* w, const float* bias,
                       float* c, int64_t m, int64_t n, int64_t k, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((n + BN - 1) / BN), static_cast<unsigned>((m + BM - 1) / BM));
    if (k % BK) return hipErrorInvalidValue;
    if (w_fmt == RT_HIP_Q4K) {
        if (a_bf16)
            hipLaunchKernelGGL((k_gemm<RT_HIP_Q4K, true>), grid, dim3(256), 0, s, a, w, bias, c,
                               static_cast<int>(m), static_cast<int>(n), static_cast<int>(k));
        else
            hipLaunchKernelGGL((k_gemm<RT_HIP_Q4K, false>), grid, dim3(256), 0, s, a, w, bias, c,
                               static_cast<int>(m), static_cast<int>(n), static_cast<int>(k));
    } else if (w_fmt == RT_HIP_BF16) {
        if (a_bf16)
            hipLaunchKernelGGL((k_gemm<RT_HIP_BF16, true>), grid, dim3(256), 0, s, a, w, bias, c,
                               static_cast<int>(m), static_cast<int>(n), static_cast<int>(k));
        else
            hipLaunchKernelGGL((k_gemm<RT_HIP_BF16, false>), grid, dim3(256), 0, s, a, w, bias, c,
                               static_cast<int>(m), static_cast<int>(n), static_cast<int>(k));
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_add_bias(float* y, const float* bias, int64_t m, int64_t n, hipStream_t s) {
    const int64_t total = m * n;
    hipLaunchKernelGGL(k_add_bias, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                       s, y, bias, m, n);
    return hipGetLastError();
}

}  // namespace rt_hip
