// gemv_q8.hip -- the Q4_K x Q8-activation GEMV (M = 1): the reference's
// aarch64 gemv_mt path (quant_q4k.cpp:564-600), which quantizes the
// activation to int8 per 32 values once (Q4KMat::quantize_activation_q8,
// quant_q4k.cpp:525-562) and takes every row's dot product with integer dot
// products (dot_row_q8, quant_q4k.cpp:425-478).
//
// The integer part maps onto v_mfma_i32_16x16x64_i8 exactly as the f32
// GEMV's limbs do (q4k_mfma.hpp): one int8 plane instead of three, so row 4g
// of the A operand carries the q8 values of chunk g and lane (n, g) ends with
// the two exact chunk dots of row n.  The f32 part follows the reference
// operation by operation (the library builds with -ffp-contract=off, as the
// reference does):
//     term  = d*sv1*scale_lo*idot_lo - dmin*mv1*sum_lo
//           + d*sv2*scale_hi*idot_hi - dmin*mv2*sum_hi      (left to right)
//     total = ((0 + term_0) + term_1) + ...                (chunks in order)
// The terms of a 16-row tile go to LDS and one lane per row adds them in
// chunk order, so results are bit-identical to the reference's arithmetic.
#include <type_traits>

#include "q4k_mfma.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

using namespace q4k_mfma;

constexpr int kQ8Ring = 8;  // super-blocks per wave, all loaded up front

// One 32-value block of the activation, n <= 32 values present (the rest
// count as absent, not as zeros): the running maximum of |a| that NaN never
// wins (std::max(max_abs, fabs(a))), the sum in order from 0, scale =
// max_abs / 127 and inv = 1 / scale (both correctly rounded), and
// q = clamp(round(a * inv), -128, 127) with round half away from zero.  A
// zero block gets scale 0 and q = 0.  q holds the 32 bytes in order.
__device__ __forceinline__ void q8_block(const float (&v)[32], int n, uint32_t (&q)[8], float& scale,
                                         float& sum) {
    float mx = 0.0f, sm = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        if (i < n) {
            mx = fmaxf(mx, fabsf(v[i]));
            sm += v[i];
        }
    }
    sum = sm;
    scale = mx == 0.0f ? 0.0f : mx / 127.0f;
    const float inv = mx == 0.0f ? 0.0f : 1.0f / scale;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * w + e;
            float r = roundf(v[i] * inv);
            r = r < -128.0f ? -128.0f : (127.0f < r ? 127.0f : r);
            const uint32_t b = i < n && mx != 0.0f ? static_cast<uint32_t>(static_cast<int>(r)) & 0xffu : 0u;
            word |= b << (8 * e);
        }
        q[w] = word;
    }
}

// Standalone quantizer: one thread per 32-value block; q8 is padded with
// zeros to whole blocks.
__global__ __launch_bounds__(256) void k_quantize_q8(const float* __restrict__ a, int64_t k, int8_t* __restrict__ q8,
                                                     float* __restrict__ scales, float* __restrict__ sums,
                                                     int64_t nq) {
    const int64_t blk = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (blk >= nq) return;
    const int64_t s = 32 * blk;
    const int n = k - s < 32 ? static_cast<int>(k - s) : 32;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = i < n ? a[s + i] : 0.0f;
    uint32_t q[8];
    float sc, sm;
    q8_block(v, n, q, sc, sm);
#pragma unroll
    for (int i = 0; i < 32; ++i) q8[s + i] = static_cast<int8_t>((q[i >> 2] >> (8 * (i & 3))) & 0xffu);
    scales[blk] = sc;
    sums[blk] = sm;
}

// LDS layout of the GEMV (K % 256 == 0):
//   [0, K)                    q8 bytes
//   [K, K + 64)               zeros (the A operand of inactive lanes)
//   [K + 64, K + 64 + K/4)    {scale, sum} per 32-value block (f32 pairs)
//   then per tile slot 16 rows x (4 nb + 1) f32: the tile's chunk terms
//   (odd row stride: the 16 lanes of the ordered sum read distinct banks)
__host__ __device__ inline size_t q8_term_offset(int K) { return static_cast<size_t>(K) + 64 + K / 4; }
__host__ __device__ inline size_t q8_lds_bytes(int K, int tpw) {
    return q8_term_offset(K) + static_cast<size_t>(tpw) * 16 * static_cast<size_t>(4 * (K / 256) + 1) * 4;
}

// TPW 16-row tiles per workgroup, KS waves per tile; wave ks of a tile owns
// super-blocks [ks * bpw, min(nb, (ks + 1) * bpw)), bpw <= kQ8Ring.  The
// workgroup quantizes x once for its TPW tiles.
template <bool TILED>
__global__ __launch_bounds__(512) void k_gemv_q4k_q8(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                     float* __restrict__ Y, int N, int K, int bpw, int KS) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = K >> 8, nq = K >> 5;
    const int tslot = wave / KS, ks = wave - tslot * KS;
    const int TPW = static_cast<int>(blockDim.x >> 6) / KS;
    const int row0 = 16 * (static_cast<int>(blockIdx.x) * TPW + tslot);

    // x first: thread t < nq holds block t (K % 256 == 0: whole blocks).
    const f32x4* const X4 = reinterpret_cast<const f32x4*>(X);
    f32x4 xv[8];
    const int xb = tid < nq ? tid : 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = X4[8 * xb + i];
    __builtin_amdgcn_sched_barrier(0);

    // The wave's super-blocks, every ring slot issued (an empty resource
    // past the wave's range loads zeros without touching memory).
    const int b0 = ks * bpw;
    const int nbw = max(0, min(nb, b0 + bpw) - b0);
    Lane ln = make_lane(lane, K);
    const int64_t rb = static_cast<int64_t>(nb) * kQ4kBlockBytes;
    constexpr int64_t kStride = TILED ? kTiledBlockBytes : kQ4kBlockBytes;
    const int64_t off0 = TILED ? (static_cast<int64_t>(row0 >> 4) * nb + b0) * kTiledBlockBytes
                               : static_cast<int64_t>(row0) * rb + static_cast<int64_t>(b0) * kQ4kBlockBytes;
    const int64_t total = TILED ? static_cast<int64_t>((N + 15) >> 4) * 16 * rb : static_cast<int64_t>(N) * rb;
    const uint8_t* const tbase = W + off0;
    const uint32_t tl32 = rsrc_bytes(total - off0);
    const uint32_t roff = static_cast<uint32_t>(ln.n * rb);
    const TLane tl = make_tlane(lane);
    using B = typename std::conditional<TILED, BlkT, Blk>::type;
    B ring[kQ8Ring];
#pragma unroll
    for (int j = 0; j < kQ8Ring; ++j) {
        const uint32_t o = static_cast<uint32_t>(j) * static_cast<uint32_t>(kStride);
        const uint32_t left = static_cast<uint32_t>(
            __builtin_amdgcn_readfirstlane(static_cast<int>(j < nbw && o < tl32 ? tl32 - o : 0u)));
        const BufRsrc rs = make_rsrc_n(tbase + o, left);
        if constexpr (TILED)
            load_blk_t(rs, static_cast<uint32_t>(lane), ring[j]);
        else
            load_blk(rs, roff, ln, ring[j]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Quantize x into LDS while the weights are in flight (the x loads are
    // the oldest: wait for them alone).
    wait_vmcnt<3 * kQ8Ring>();
    if (tid < nq) {
        float v[32];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * i + e] = xv[i][e];
        uint32_t q[8];
        float sc, sm;
        q8_block(v, 32, q, sc, sm);
        u32x4* dst = reinterpret_cast<u32x4*>(lds + 32 * tid);
        dst[0] = u32x4{q[0], q[1], q[2], q[3]};
        dst[1] = u32x4{q[4], q[5], q[6], q[7]};
        reinterpret_cast<f32x2*>(lds + K + 64)[tid] = f32x2{sc, sm};
    }
    if (tid < 4) reinterpret_cast<u32x4*>(lds + K)[tid] = u32x4{0u, 0u, 0u, 0u};
    lds_barrier();

    // Only lambda-0 rows of the A operand are live: lane (m, g) supplies
    // row m = 4 g of chunk g.
    {
        const int m = lane & 15;
        const bool active = (m >> 2) == ln.g && (m & 3) == 0;
        ln.a_base = active ? static_cast<uint32_t>(64 * ln.g) : static_cast<uint32_t>(K);
        ln.a_mask = active ? 0xffffffffu : 0u;
    }
    const int stride = 4 * nb + 1;
    float* const terms = reinterpret_cast<float*>(lds + q8_term_offset(K)) + tslot * 16 * stride;
    wait_vmcnt<0>();
#pragma unroll
    for (int j = 0; j < kQ8Ring; ++j) {
        if (j < nbw) {
            Dec dc;
            if constexpr (TILED)
                dc = decode_t(ring[j], tl);
            else
                dc = decode(ring[j], ln);
            const int b = b0 + j;
            const uint32_t a_addr = ln.a_base + ((static_cast<uint32_t>(b) << 8) & ln.a_mask);
            const i32x4 A0 = *reinterpret_cast<const i32x4*>(lds + a_addr);
            const i32x4 A1 = *reinterpret_cast<const i32x4*>(lds + a_addr + 16);
            const i32x4 A2 = *reinterpret_cast<const i32x4*>(lds + a_addr + 32);
            const i32x4 A3 = *reinterpret_cast<const i32x4*>(lds + a_addr + 48);
            const i32x4 z = {0, 0, 0, 0};
            i32x4 clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, dc.B0, z, 0, 0, 0);
            clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, dc.B1, clo, 0, 0, 0);
            i32x4 chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, dc.B2, z, 0, 0, 0);
            chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(A3, dc.B3, chi, 0, 0, 0);
            // {scale, sum} of sub-blocks 8b + 2g (low nibbles) and 8b + 2g + 1
            const f32x4 c = *reinterpret_cast<const f32x4*>(lds + K + 64 + 64 * b + 16 * ln.g);
            const float t = dc.ds0 * c[0] * static_cast<float>(clo[0]) - dc.dm0 * c[1] +
                            dc.ds1 * c[2] * static_cast<float>(chi[0]) - dc.dm1 * c[3];
            terms[ln.n * stride + 4 * b + ln.g] = t;
        }
    }
    lds_barrier();
    if (ks == 0 && lane < 16) {
        const float* tr = terms + lane * stride;
        float acc = 0.0f;
        for (int c = 0; c < 4 * nb; ++c) acc += tr[c];
        if (row0 + lane < N) Y[row0 + lane] = acc;
    }
}

}  // namespace

hipError_t launch_quantize_q8(const float* a, int64_t k, int8_t* q8, float* scales, float* sums, hipStream_t s) {
    const int64_t nq = (k + 31) / 32;
    const int64_t grid = (nq + 255) / 256;
    hipLaunchKernelGGL(k_quantize_q8, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, a, k, q8, scales, sums,
                       nq);
    return hipGetLastError();
}

// Waves per tile and tiles per workgroup: with few tiles one tile per
// workgroup of min(8, nb) waves (the most loads in flight); with many (more
// than 8 per CU) up to four tiles per workgroup of ceil(nb / 8) waves each
// (at most 8 waves), so that x is quantized once for several tiles.  Either way the workgroup has at least
// one thread per 32-value block of x.
static void q8_split(int64_t n, int nb, int cus, int& ks, int& tpw) {
    const int64_t tiles = (n + 15) / 16;
    if (tiles > 8LL * cus) {
        ks = (nb + 7) / 8;
        tpw = ks <= 2 ? 4 : (ks <= 4 ? 2 : 1);
    } else {
        tpw = 1;
        ks = nb < 8 ? nb : 8;
    }
}

hipError_t launch_gemv_q4k_q8(const void* w, bool tiled, const float* x, float* y, int64_t n, int64_t k,
                              hipStream_t s) {
    const int nb = static_cast<int>(k / 256);
    int ks, tpw;
    q8_split(n, nb, device_info().cus, ks, tpw);
    const int bpw = (nb + ks - 1) / ks;
    if (nb < 1 || bpw > kQ8Ring || 8 * nb > 64 * ks * tpw || ks * tpw > 8) return hipErrorInvalidValue;
    const int64_t tiles = (n + 15) / 16;
    const dim3 grid(static_cast<unsigned>((tiles + tpw - 1) / tpw)), block(static_cast<unsigned>(64 * ks * tpw));
    const size_t lds = q8_lds_bytes(static_cast<int>(k), tpw);
    const auto* W = static_cast<const uint8_t*>(w);
    if (tiled)
        hipLaunchKernelGGL(k_gemv_q4k_q8<true>, grid, block, lds, s, W, x, y, static_cast<int>(n),
                           static_cast<int>(k), bpw, ks);
    else
        hipLaunchKernelGGL(k_gemv_q4k_q8<false>, grid, block, lds, s, W, x, y, static_cast<int>(n),
                           static_cast<int>(k), bpw, ks);
    return hipGetLastError();
}

}  // namespace rt_hip
