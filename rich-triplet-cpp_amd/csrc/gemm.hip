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

// ---------------------------------------------------------------------------
// Pipelined kernel (K % 256 == 0): bf16 A and W.
//
// LDS tiles are 128 rows x 64 bf16 (128 B per row, unpadded) with the 16-byte
// chunk c of row r stored at chunk slot c ^ (r & 7), so the MFMA fragment
// reads (16 rows x one chunk) are conflict-free and whole tiles can be
// written by direct-to-LDS buffer loads (1 KB per wave instruction: 8 rows).
//  * A and W stream through a ring of kStages LDS tiles each, copied by
//    buffer loads straight into LDS kStages-1 steps ahead; rows past M (N)
//    read as zeros through the buffer range check.
//  * One barrier per 64-wide K step.  Tiles are assigned XCD by XCD (a
//    workgroup's XCD is its id mod 8), each XCD getting a contiguous range
//    of a grouped tile order (8 M-tiles per N column), so the tiles resident
//    on an XCD at once share A rows and W rows in its L2.
constexpr int kPThreads = 256;
constexpr int kStages = 4;
constexpr int kTile = 128 * 128;    // bytes of one 128 x 64 bf16 tile
constexpr int kGroupM = 8;

__device__ __forceinline__ uint32_t swz(int r, int c) {
    return static_cast<uint32_t>(r * 128 + ((c ^ (r & 7)) << 4));
}

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    return __builtin_bit_cast(uint32_t, v);
}

// s_waitcnt vmcnt(N) alone (vmcnt bits [3:0] and [15:14]; expcnt, lgkmcnt
// left at their no-wait maxima).
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that waits for this wave's LDS traffic only (not for its
// global loads and copies in flight).
__device__ __forceinline__ void lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Epilogue through LDS.  A wave's accumulators hold C in the MFMA layout
// (lane l: rows 4 (l / 16) + r of each 16-row fragment, column l % 16), so
// storing them directly writes 64-byte pieces of four rows per instruction.
// Instead each wave writes 64 rows of its tile at a time, row-major, into its
// own LDS region of 64 x kEpiStride floats, and stores them back as whole
// 256-byte row segments (16 lanes x 16 bytes per row, 4 rows per
// instruction) plus the bias.  Measured on the FLUX shapes: 11-25% faster
// than the direct stores, identical results.  The caller has waited for its
// copies and passed a barrier, so no wave still writes or reads the ring.
constexpr int kEpiStride = 68;  // floats per LDS row: 64 + 4 (the 4 row groups of a write hit distinct banks)
constexpr int kEpiWaveBytes = 64 * kEpiStride * 4;

template <int NI>
__device__ __forceinline__ void store_tile_staged(const f32x4 (&acc)[NI][4], float* reg, float* __restrict__ C,
                                                  int M, int N, int row0, int col0, const float* __restrict__ bias,
                                                  int lane) {
    static_assert(NI % 4 == 0, "64-row halves");
    const int q = lane >> 4, c16 = lane & 15;
    const int col = col0 + 4 * c16;
    const bool full = (N & 3) == 0 && col + 3 < N;  // whole, 16-byte aligned groups of 4
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (bias) {
        if (full) {
            bv = f32x4{bias[col], bias[col + 1], bias[col + 2], bias[col + 3]};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[e] = col + e < N ? bias[col + e] : 0.f;
        }
    }
#pragma unroll
    for (int h = 0; h < NI / 4; ++h) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) reg[(16 * i + 4 * q + r) * kEpiStride + 16 * j + c16] = acc[4 * h + i][j][r];
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's writes are in
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int lr = 4 * k + q;
            const int row = row0 + 64 * h + lr;
            const f32x4 v = *reinterpret_cast<const f32x4*>(reg + lr * kEpiStride + 4 * c16) + bv;
            if (row >= M) continue;
            float* dst = C + static_cast<size_t>(row) * N + col;
            if (full) {
                *reinterpret_cast<f32x4*>(dst) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < N) dst[e] = v[e];
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // reads done before the region is rewritten
    }
}

__global__ __launch_bounds__(kPThreads) void k_gemm_pipe(const uint16_t* __restrict__ A,
                                                        const uint16_t* __restrict__ Wp,
                                                        const float* __restrict__ bias,
                                                        float* __restrict__ Cp, int M, int N, int K,
                                                        int mt, int ldk, int64_t c_split) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* const sA = lds;                        // [kStages][kTile]
    uint8_t* const sW = lds + kStages * kTile;      // [kStages][kTile]

    // XCD-contiguous tile id, then grouped order: consecutive ids walk
    // kGroupM M-tiles of one N column before the next column, so the tiles
    // resident together share A rows and W rows in L2.
    const int G = static_cast<int>(gridDim.x), bid = static_cast<int>(blockIdx.x);
    const int xcd = bid & 7, idx = bid >> 3, q8 = G >> 3, r8 = G & 7;
    const int tile = xcd < r8 ? xcd * (q8 + 1) + idx : r8 * (q8 + 1) + (xcd - r8) * q8 + idx;
    const int nt = G / mt;
    const int group = tile / (kGroupM * nt), first_m = group * kGroupM;
    const int gm = min(mt - first_m, kGroupM);
    const int m0 = (first_m + (tile % (kGroupM * nt)) % gm) * 128;
    const int n0 = ((tile % (kGroupM * nt)) / gm) * 128;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    // Split-K slice blockIdx.y: columns [k0, k0 + K) of rows of ldk
    // elements, into C + blockIdx.y * c_split (unsplit calls have one slice:
    // k0 = 0, ldk = K).
    const int k0 = static_cast<int>(blockIdx.y) * K;
    float* const C = Cp + static_cast<int64_t>(blockIdx.y) * c_split;
    const int S = K >> 6;
    const int64_t rowA = static_cast<int64_t>(ldk) * 2;

    // Copy roles: wave instruction i (0..3) covers tile rows 8*(4*wave+i) ..
    // +7; lane l fills chunk slot l%8 of row 8*(4*wave+i) + l/8, i.e. global
    // chunk (l%8) ^ (row & 7).
    uint32_t coff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * (4 * wave + i) + (lane >> 3);
        coff[i] = static_cast<uint32_t>(r * rowA + (((lane & 7) ^ (r & 7)) << 4));
    }
    const uint8_t* const Ab = reinterpret_cast<const uint8_t*>(A) + static_cast<int64_t>(m0) * rowA + 2 * k0;
    const int64_t Aleft = static_cast<int64_t>(M - m0) * rowA - 2 * k0;
    auto copy_tile = [&](uint8_t* dst, const uint8_t* base, int64_t left, int step) {
        const int64_t o = static_cast<int64_t>(step) * 128;  // 64 bf16 per step
        const BufRsrc rs = make_rsrc(base + o, step < S ? left - o : 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void*)(dst + (4 * wave + i) * 1024), 16,
                static_cast<int>(coff[i]), 0, 0, 0);
    };
    const uint8_t* const Wb16 = reinterpret_cast<const uint8_t*>(Wp) + static_cast<int64_t>(n0) * rowA + 2 * k0;
    const int64_t Wleft16 = static_cast<int64_t>(N - n0) * rowA - 2 * k0;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int fr = lane & 15, fc = lane >> 4;
    auto mfma_step = [&](const uint8_t* ta, const uint8_t* tw) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            bf16x8 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(ta + swz(wm + 16 * i + fr, 4 * ks + fc));
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bf[j] = *reinterpret_cast<const bf16x8*>(tw + swz(wn + 16 * j + fr, 4 * ks + fc));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    // Prologue: copies of steps 0 .. kStages-2.
#pragma unroll
    for (int j = 0; j < kStages - 1; ++j) {
        copy_tile(sA + j * kTile, Ab, Aleft, j);
        copy_tile(sW + j * kTile, Wb16, Wleft16, j);
    }
    wait_vm<0>();
    lds_sync();

    // Step s: copy step t = s+kStages-1 (A, then W); MFMAs of step s; wait
    // for this wave's copies that step s+1 needs, then the barrier.  Copies
    // are ordered and counted by vmcnt: after W of step s+1 this wave has
    // issued 16 more (A, W of s+2 and s+3).  kStages == 4 and S % 4 == 0:
    // the unrolled round keeps every ring index a compile-time constant.
    static_assert(kStages == 4, "the unrolled round assumes a 4-stage ring");
    for (int s0 = 0; s0 < S; s0 += 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int s = s0 + j;
            const int t = (j + kStages - 1) % kStages;
            copy_tile(sA + t * kTile, Ab, Aleft, s + kStages - 1);
            copy_tile(sW + t * kTile, Wb16, Wleft16, s + kStages - 1);
            mfma_step(sA + j * kTile, sW + j * kTile);
            wait_vm<16>();
            lds_sync();
        }
    }

    // Epilogue (+ bias) through LDS, once the copies issued for steps past
    // the end (zero fill) have landed in every wave.
    static_assert(4 * kEpiWaveBytes <= 2 * kStages * kTile, "the epilogue's LDS regions fit");
    wait_vm<0>();
    __syncthreads();
    store_tile_staged<4>(acc, reinterpret_cast<float*>(lds + wave * kEpiWaveBytes), C, M, N, m0 + wm, n0 + wn, bias,
                         lane);
}

// Q4_K W over several M tiles, warp-specialized (128 x 128 tiles, 8 waves).
//  * Waves 0-3 compute: the four 64 x 64 MFMA tiles of k_gemm_pipe with the
//    same fragment reads and MFMA order, so the result is bit-identical to
//    dequantizing W and converting A once and running k_gemm_pipe.
//  * Waves 4-7 produce: every K step's W tile is dequantized straight from
//    the Q4_K bytes in HBM (w = (d*sv)*q - dmin*mv, exact in f32, then
//    round-to-nearest-even bf16, as the reference's flux_dequant_q4k,
//    shaders/flux.msl:69-81) and its A tile converted from f32 (RNE) or
//    copied as bf16, into a two-stage LDS ring.  Their global loads run
//    kWsAhead steps ahead in registers.  Thread p of the producers owns row
//    p / 2 of both tiles, half p % 2 of the step's 64 values.
//  * One barrier per step: in round j the compute waves read stage j % 2
//    while the producers fill stage (j + 1) % 2 with step j + 1.
//  * Rows past M or N and steps past the slice read zeros (buffer range);
//    split-K slices start on super-block boundaries.
// Replaces the dequantize-into-HBM pre-pass for several M tiles: no weight
// copy, no extra launch; the dequantization of a W tile repeats per M tile,
// in waves of its own beside the MFMA waves.
constexpr int kWsThreads = 512;
constexpr int kWsAhead = 3;  // steps loaded ahead; kWsAhead + 1 register slots
constexpr size_t kWsLds = 4 * kEpiWaveBytes > 4 * kTile ? 4 * kEpiWaveBytes : 4 * kTile;

template <int WF, bool A_F32>
__global__ __launch_bounds__(kWsThreads) void k_gemm_ws(const void* __restrict__ Ap, const uint8_t* __restrict__ Wq,
                                                        const float* __restrict__ bias, float* __restrict__ Cp,
                                                        int M, int N, int K, int mt, int ldk, int64_t c_split,
                                                        int64_t sc_off) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* const stA = lds;              // [2][kTile]
    uint8_t* const stW = lds + 2 * kTile;  // [2][kTile]

    const int G = static_cast<int>(gridDim.x), bid = static_cast<int>(blockIdx.x);
    const int xcd = bid & 7, idx = bid >> 3, q8 = G >> 3, r8 = G & 7;
    const int tile = xcd < r8 ? xcd * (q8 + 1) + idx : r8 * (q8 + 1) + (xcd - r8) * q8 + idx;
    const int nt = G / mt;
    const int group = tile / (kGroupM * nt), first_m = group * kGroupM;
    const int gm = min(mt - first_m, kGroupM);
    const int m0 = (first_m + (tile % (kGroupM * nt)) % gm) * 128;
    const int n0 = ((tile % (kGroupM * nt)) / gm) * 128;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int k0 = static_cast<int>(blockIdx.y) * K;  // split-K slice: columns [k0, k0 + K) of rows of ldk
    float* const C = Cp + static_cast<int64_t>(blockIdx.y) * c_split;
    const int S = K >> 6;

    if (wave < 4) {
        const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
        const int fr = lane & 15, fc = lane >> 4;
        f32x4 acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        lds_sync();  // round -1: the producers fill stage 0
        for (int s0 = 0; s0 < S; s0 += 2) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint8_t* ta = stA + u * kTile;
                const uint8_t* tw = stW + u * kTile;
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    bf16x8 af[4], bf[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        af[i] = *reinterpret_cast<const bf16x8*>(ta + swz(wm + 16 * i + fr, 4 * ks + fc));
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        bf[j] = *reinterpret_cast<const bf16x8*>(tw + swz(wn + 16 * j + fr, 4 * ks + fc));
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
                }
                lds_sync();
            }
        }
        // After the last round's barrier no wave touches the ring again.
        store_tile_staged<4>(acc, reinterpret_cast<float*>(lds + wave * kEpiWaveBytes), C, M, N, m0 + wm, n0 + wn,
                             bias, lane);
        return;
    }

    // ---- producers ----
    // W: thread p decodes row p / 2, half p % 2 of the step.  A: load i of
    // thread p is row 16 i + p / 16, values 4 (p % 16) .. +3 of the step
    // (f32; bf16: 8 rows per load, 8 values) -- whole 256-byte row pieces per
    // 16 lanes.
    const int p = tid - 4 * kWave;
    const int r = p >> 1, h = p & 1;
    // W bytes per row and at the slice's first column, and this thread's
    // row offset, by format:
    //   Q4_K  144-byte super-blocks of 256 values;
    //   Q4Mat packed nibbles (two values per byte), then f32 scales per 32
    //         flat values at sc_off;
    //   Q4_0  18-byte GGUF blocks of 32 values (rows of K % 256 == 0 values
    //         start 16-byte aligned; block 2t + h starts 0 or 2 mod 4).
    const int64_t wrow = WF == RT_HIP_Q4K ? static_cast<int64_t>(ldk >> 8) * kQ4kBlockBytes
                       : WF == RT_HIP_Q4MAT ? static_cast<int64_t>(ldk >> 1)
                                            : static_cast<int64_t>(ldk >> 5) * kQ40BlockBytes;
    const int64_t wk0 = WF == RT_HIP_Q4K ? static_cast<int64_t>(k0 >> 8) * kQ4kBlockBytes
                      : WF == RT_HIP_Q4MAT ? static_cast<int64_t>(k0 >> 1)
                                           : static_cast<int64_t>(k0 >> 5) * kQ40BlockBytes;
    const uint8_t* const wbase = Wq + static_cast<int64_t>(n0) * wrow + wk0;
    const BufRsrc rw = make_rsrc(wbase, static_cast<int64_t>(N - n0) * wrow - wk0);
    // Q4Mat scales: one f32 per 32 values, rows of ldk / 32
    const int64_t srow = static_cast<int64_t>(ldk >> 5) * 4;
    const uint8_t* const sbase = Wq + sc_off + static_cast<int64_t>(n0) * srow + static_cast<int64_t>(k0 >> 5) * 4;
    const BufRsrc rs = make_rsrc(sbase, WF == RT_HIP_Q4MAT ? static_cast<int64_t>(N - n0) * srow - (k0 >> 5) * 4 : 0);
    constexpr int kAEl = A_F32 ? 4 : 2;
    const int64_t arow = static_cast<int64_t>(ldk) * kAEl;
    const uint8_t* const abase = static_cast<const uint8_t*>(Ap) + static_cast<int64_t>(m0) * arow +
                                 static_cast<int64_t>(k0) * kAEl;
    const BufRsrc ra = make_rsrc(abase, static_cast<int64_t>(M - m0) * arow - static_cast<int64_t>(k0) * kAEl);
    const uint32_t wro = static_cast<uint32_t>(static_cast<int64_t>(r) * wrow);
    const uint32_t sro = static_cast<uint32_t>(static_cast<int64_t>(r) * srow);
    constexpr int kAL = A_F32 ? 8 : 4;     // 16-byte A loads per thread and step
    constexpr int kRowsPerLoad = 256 / (A_F32 ? 16 : 8);  // rows one load instruction of all producers covers
    const int alane = A_F32 ? (p & 15) : (p & 7);          // 16-byte piece of the row's step
    const int arow0 = A_F32 ? (p >> 4) : (p >> 3);
    const uint32_t aro = static_cast<uint32_t>(static_cast<int64_t>(arow0) * arow) + static_cast<uint32_t>(alane) * 16u;
    const uint32_t a_load_stride = static_cast<uint32_t>(static_cast<int64_t>(kRowsPerLoad) * arow);
    // W registers of a step: Q4_K header and qs; Q4Mat packed bytes and the
    // scale (w1[0]); Q4_0 the five dwords covering the block.
    struct Slot {
        u32x4 w0;
        uint32_t w1[4];
        u32x4 a[kAL];
    };
    Slot slot[kWsAhead + 1];
    // Steps past the slice load nothing (an offset past the resource reads
    // zeros).
    auto issue = [&](Slot& sl, int t) {
        const bool in = t < S;
        if constexpr (WF == RT_HIP_Q4K) {
            const uint32_t bo = wro + static_cast<uint32_t>(t >> 2) * kQ4kBlockBytes;
            sl.w0 = ld16(rw, in ? bo : 0xfffffff0u);
            const u32x4 q = ld16(rw, in ? bo + 16u + 32u * static_cast<uint32_t>(t & 3) + 16u * static_cast<uint32_t>(h)
                                        : 0xfffffff0u);
#pragma unroll
            for (int e = 0; e < 4; ++e) sl.w1[e] = q[e];
        } else if constexpr (WF == RT_HIP_Q4MAT) {
            const uint32_t v = static_cast<uint32_t>(64 * t + 32 * h);  // first value of the thread's 32
            sl.w0 = ld16(rw, in ? wro + v / 2u : 0xfffffff0u);
            sl.w1[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(in ? sro + (v / 32u) * 4u : 0xfffffff0u),
                                                            0, 0);
        } else {
            const uint32_t bo = wro + static_cast<uint32_t>(2 * t + h) * kQ40BlockBytes;
            const uint32_t al = bo & ~3u;
            sl.w0 = ld16(rw, in ? al : 0xfffffff0u);
            sl.w1[0] = __builtin_amdgcn_raw_buffer_load_b32(rw, static_cast<int>(in ? al + 16u : 0xfffffff0u), 0, 0);
            sl.w1[1] = bo & 2u;  // the block's offset in its first dword (not a load)
        }
        const uint32_t ao = aro + static_cast<uint32_t>(t) * 64u * kAEl;
#pragma unroll
        for (int i = 0; i < kAL; ++i)
            sl.a[i] = ld16(ra, in ? ao + a_load_stride * static_cast<uint32_t>(i) : 0xfffffff0u);
    };
    auto produce = [&](const Slot& sl, int t, int stage) {
        uint8_t* const tw = stW + stage * kTile;
        uint8_t* const ta = stA + stage * kTile;
        if constexpr (WF == RT_HIP_Q4K) {
            // values 16 h .. +15 (low nibbles, sub-block 2c) and 32 + 16 h ..
            // +15 (high nibbles, sub-block 2c + 1): chunks 2h, 2h + 1, 4 + 2h,
            // 5 + 2h of the tile row
            const int c = t & 3;
            const float d = f16_bits_to_f32(sl.w0[0] & 0xffffu), dm = f16_bits_to_f32(sl.w0[0] >> 16);
            uint32_t sv1, mv1, sv2, mv2;
            decode_scale_min(make_scale_sel(2 * c), sl.w0[1], sl.w0[2], sl.w0[3], sv1, mv1);
            decode_scale_min(make_scale_sel(2 * c + 1), sl.w0[1], sl.w0[2], sl.w0[3], sv2, mv2);
            const float s1 = d * static_cast<float>(sv1), n1 = dm * static_cast<float>(mv1);
            const float s2 = d * static_cast<float>(sv2), n2 = dm * static_cast<float>(mv2);
            u32x4 lo[2], hi[2];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t wl = sl.w1[j] & 0x0f0f0f0fu, wh = (sl.w1[j] >> 4) & 0x0f0f0f0fu;
                lo[j >> 1][2 * (j & 1)] = pk_bf16(s1 * ubyte_f32(wl, 0) - n1, s1 * ubyte_f32(wl, 1) - n1);
                lo[j >> 1][2 * (j & 1) + 1] = pk_bf16(s1 * ubyte_f32(wl, 2) - n1, s1 * ubyte_f32(wl, 3) - n1);
                hi[j >> 1][2 * (j & 1)] = pk_bf16(s2 * ubyte_f32(wh, 0) - n2, s2 * ubyte_f32(wh, 1) - n2);
                hi[j >> 1][2 * (j & 1) + 1] = pk_bf16(s2 * ubyte_f32(wh, 2) - n2, s2 * ubyte_f32(wh, 3) - n2);
            }
            *reinterpret_cast<u32x4*>(tw + swz(r, 2 * h)) = lo[0];
            *reinterpret_cast<u32x4*>(tw + swz(r, 2 * h + 1)) = lo[1];
            *reinterpret_cast<u32x4*>(tw + swz(r, 4 + 2 * h)) = hi[0];
            *reinterpret_cast<u32x4*>(tw + swz(r, 5 + 2 * h)) = hi[1];
        } else if constexpr (WF == RT_HIP_Q4MAT) {
            // values 32 h .. +31 in order (chunks 4h .. 4h + 3): byte i of the
            // packed load holds values 2i (low nibble) and 2i + 1 (high),
            // signed 4-bit, times the group's scale (quant_q4.cpp:56-90)
            const float sc = __uint_as_float(sl.w1[0]);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t q = sl.w0[c];
                u32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // (the builtin's result is unsigned: the sign extension
                    // survives only through int)
                    const int nl = static_cast<int>(__builtin_amdgcn_sbfe(static_cast<int>(q), 8 * e, 4));
                    const int nh = static_cast<int>(__builtin_amdgcn_sbfe(static_cast<int>(q), 8 * e + 4, 4));
                    const float lo = static_cast<float>(nl) * sc;
                    const float hi = static_cast<float>(nh) * sc;
                    v[e] = pk_bf16(lo, hi);
                }
                *reinterpret_cast<u32x4*>(tw + swz(r, 4 * h + c)) = v;
            }
        } else {
            // GGUF Q4_0 block (gguf.cpp:495-529): d, then qs[16]; value j is
            // (qs[j] & 15) - 8, value 16 + j is (qs[j] >> 4) - 8, times d
            const bool odd = sl.w1[1] != 0;  // block at byte 2 of its first dword
            const uint32_t d0 = sl.w0[0], d1 = sl.w0[1], d2 = sl.w0[2], d3 = sl.w0[3], d4 = sl.w1[0];
            const float d = f16_bits_to_f32(odd ? d0 >> 16 : d0 & 0xffffu);
            // qs as four dwords: bytes 2..17 of the block
            const uint32_t qs[4] = {odd ? d1 : __builtin_amdgcn_alignbyte(d1, d0, 2),
                                    odd ? d2 : __builtin_amdgcn_alignbyte(d2, d1, 2),
                                    odd ? d3 : __builtin_amdgcn_alignbyte(d3, d2, 2),
                                    odd ? d4 : __builtin_amdgcn_alignbyte(d4, d3, 2)};
#pragma unroll
            for (int c = 0; c < 2; ++c) {  // chunks 4h + c (low nibbles), 4h + 2 + c (high)
                u32x4 lo, hi;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t q = qs[2 * c + (e >> 1)];
                    const int s0 = 16 * (e & 1);
                    lo[e] = pk_bf16(static_cast<float>(static_cast<int>(__builtin_amdgcn_ubfe(q, s0, 4)) - 8) * d,
                                    static_cast<float>(static_cast<int>(__builtin_amdgcn_ubfe(q, s0 + 8, 4)) - 8) * d);
                    hi[e] = pk_bf16(static_cast<float>(static_cast<int>(__builtin_amdgcn_ubfe(q, s0 + 4, 4)) - 8) * d,
                                    static_cast<float>(static_cast<int>(__builtin_amdgcn_ubfe(q, s0 + 12, 4)) - 8) * d);
                }
                *reinterpret_cast<u32x4*>(tw + swz(r, 4 * h + c)) = lo;
                *reinterpret_cast<u32x4*>(tw + swz(r, 4 * h + 2 + c)) = hi;
            }
        }
#pragma unroll
        for (int i = 0; i < kAL; ++i) {
            const int ar = arow0 + kRowsPerLoad * i;
            if constexpr (A_F32) {
                // 4 values -> 8 bytes: half (alane % 2) of 16-byte chunk alane / 2
                const f32x4 x = __builtin_bit_cast(f32x4, sl.a[i]);
                *reinterpret_cast<u32x2*>(ta + swz(ar, alane >> 1) + 8 * (alane & 1)) =
                    u32x2{bf16_pair(x[0], x[1]), bf16_pair(x[2], x[3])};
            } else {
                *reinterpret_cast<u32x4*>(ta + swz(ar, alane)) = sl.a[i];
            }
        }
    };
    constexpr int kL = 2 + kAL;  // loads per step (vmcnt)
    static_assert(kWsAhead == 3 && kWsAhead * kL < 64, "the unrolled round assumes four slots");
#pragma unroll
    for (int t = 0; t <= kWsAhead; ++t) {
        issue(slot[t], t);
        __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm<kWsAhead * kL>();
    produce(slot[0], 0, 0);
    lds_sync();  // round -1
    // Round j (S % 4 == 0): refill slot j % 4 (step j freed it) with step
    // j + 4, wait for step j + 1 (three steps' loads may still run),
    // produce it into stage (j + 1) % 2.
    for (int s0 = 0; s0 < S; s0 += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            issue(slot[u], s0 + u + kWsAhead + 1);
            __builtin_amdgcn_sched_barrier(0);
            wait_vm<kWsAhead * kL>();
            produce(slot[(u + 1) & 3], s0 + u + 1, (u + 1) & 1);
            lds_sync();
        }
    }
}

// Large-tile bf16 GEMM (both operands bf16 in HBM): C = A * W^T (+ bias).
//  * 256 x 256 workgroup tile, 8 waves of 128 x 64 (2 per SIMD): 384 B of
//    LDS fragment reads per 16x16x32 MFMA (a 64 x 64 wave tile needs 512 B,
//    more than the CU's LDS bandwidth at full MFMA rate).
//  * K steps of 32: a 4-stage ring of A and W tiles (16 KB each) filled by
//    direct-to-LDS buffer loads three steps ahead; one barrier per step.
//  * LDS rows are 64 bytes (32 bf16); chunk c of row r sits at chunk
//    c ^ ((r / 2) % 4).  A 16-byte-per-lane LDS read is served 8 lanes (one
//    128-byte bank line) at a time; the 8 lanes of a fragment read are 8
//    consecutive rows, two per 128 bytes, and the swizzle gives the rows of
//    each parity four different chunks: no bank conflicts.  The copies apply
//    the swizzle on the global side: lane l fills LDS chunk slot l % 4 of
//    row l / 4 with global chunk (l % 4) ^ f(row).
//  * Tile order: XCD-contiguous ranges of a grouped order (as k_gemm_pipe).
constexpr int kBThreads = 512;
constexpr int kBTile = 256 * 64;  // bytes of one 256 x 32 bf16 tile
constexpr int kBGroupM = 4;

__device__ __forceinline__ uint32_t swz64(int r, int c) {
    return static_cast<uint32_t>(r * 64 + ((c ^ ((r >> 1) & 3)) << 4));
}

// NS: ring stages (A and W tile pairs, 32 KB each); 8 waves of 128 x 64.
// (4 waves of 128 x 128, one per SIMD with the accumulators in AGPRs, have a
// third fewer fragment reads per MFMA but measured slower.)
template <int NS>
__global__ __launch_bounds__(kBThreads) void k_gemm_256(const uint16_t* __restrict__ A,
                                                        const uint16_t* __restrict__ W,
                                                        const float* __restrict__ bias,
                                                        float* __restrict__ C, int M, int N, int K, int mt) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* const sA = lds;                 // [NS][kBTile]
    uint8_t* const sW = lds + NS * kBTile;   // [NS][kBTile]

    const int G = static_cast<int>(gridDim.x), bid = static_cast<int>(blockIdx.x);
    const int xcd = bid & 7, idx = bid >> 3, q8 = G >> 3, r8 = G & 7;
    const int tile = xcd < r8 ? xcd * (q8 + 1) + idx : r8 * (q8 + 1) + (xcd - r8) * q8 + idx;
    const int nt = G / mt;
    const int group = tile / (kBGroupM * nt), first_m = group * kBGroupM;
    const int gm = min(mt - first_m, kBGroupM);
    const int m0 = (first_m + (tile % (kBGroupM * nt)) % gm) * 256;
    const int n0 = ((tile % (kBGroupM * nt)) / gm) * 256;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr int NJ = 4;  // 16-column fragments per wave
    constexpr int CP = 2;  // copy instructions per wave and operand
    static_assert(NS * 2 * kBTile >= 8 * kEpiWaveBytes, "the epilogue's LDS regions fit in the ring");
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
    const int S = K >> 5;
    const int64_t rowb = static_cast<int64_t>(K) * 2;

    // Copy roles: wave instruction i (0 .. CP - 1) covers tile rows
    // 16 (CP wave + i) .. +15.
    uint32_t coff[CP];
#pragma unroll
    for (int i = 0; i < CP; ++i) {
        const int r = 16 * (CP * wave + i) + (lane >> 2);
        coff[i] = static_cast<uint32_t>(r * rowb + (((lane & 3) ^ ((r >> 1) & 3)) << 4));
    }
    const uint8_t* const Ab = reinterpret_cast<const uint8_t*>(A) + static_cast<int64_t>(m0) * rowb;
    const uint8_t* const Wb = reinterpret_cast<const uint8_t*>(W) + static_cast<int64_t>(n0) * rowb;
    const int64_t Aleft = static_cast<int64_t>(M - m0) * rowb, Wleft = static_cast<int64_t>(N - n0) * rowb;
    auto copy = [&](uint8_t* dst, const uint8_t* base, int64_t left, int step) {
        const int64_t o = static_cast<int64_t>(step) * 64;  // 32 bf16 per step
        const BufRsrc rs = make_rsrc(base + o, step < S ? left - o : 0);
#pragma unroll
        for (int i = 0; i < CP; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void*)(dst + (CP * wave + i) * 1024), 16,
                static_cast<int>(coff[i]), 0, 0, 0);
    };

    f32x4 acc[8][NJ];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int fr = lane & 15, fc = lane >> 4;
    uint32_t aoff[8], woff[NJ];
#pragma unroll
    for (int i = 0; i < 8; ++i) aoff[i] = swz64(wm + 16 * i + fr, fc);
#pragma unroll
    for (int j = 0; j < NJ; ++j) woff[j] = swz64(wn + 16 * j + fr, fc);
    // Fragments are double-buffered in registers: step s reads step s + 1's
    // fragments while its own MFMAs run on the ones read during step s - 1,
    // so LDS reads and MFMAs overlap within every wave (the step barrier
    // aligns the waves, so they cannot rely on each other for it).
    bf16x8 af[2][8], bf[2][NJ];
    auto read_frags = [&](int buf, const uint8_t* ta, const uint8_t* tw) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) bf[buf][j] = *reinterpret_cast<const bf16x8*>(tw + woff[j]);
#pragma unroll
        for (int i = 0; i < 8; ++i) af[buf][i] = *reinterpret_cast<const bf16x8*>(ta + aoff[i]);
    };
    auto mfmas = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[buf][i], bf[buf][j], acc[i][j], 0, 0, 0);
    };

#pragma unroll
    for (int j = 0; j < NS - 1; ++j) {
        copy(sA + j * kBTile, Ab, Aleft, j);
        copy(sW + j * kBTile, Wb, Wleft, j);
    }
    wait_vm<0>();
    lds_sync();
    read_frags(0, sA, sW);

    // Step s: copy step s + NS - 1 into the stage of step s - 1 (last read
    // during step s - 2, before the barrier that ended it); read step s + 1's
    // fragments; MFMAs of step s; then wait for this wave's copies of step
    // s + 2 (2 CP (NS - 3) younger copy instructions: steps s + 3 .. s + NS - 1)
    // and the barrier, after which step s + 2's stage is complete for every
    // wave.  Two steps per round keep the fragment buffers compile-time;
    // S is even (K % 64 == 0).  Stage offsets are scalars.
    static_assert(NS >= 4, "fragments of step s + 1 are read one step early");
    int st_cur = 0;  // stage of step s
    for (int s = 0; s < S; s += 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int step = s + h;
            // This step's fragments (read a step ago) are in: saying so
            // here keeps the compiler from waiting for the reads issued
            // below before the MFMAs.
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) alone
            const int st_copy = st_cur == 0 ? NS - 1 : st_cur - 1;
            const int st_next = st_cur == NS - 1 ? 0 : st_cur + 1;
            copy(sA + st_copy * kBTile, Ab, Aleft, step + NS - 1);
            copy(sW + st_copy * kBTile, Wb, Wleft, step + NS - 1);
            if (step + 1 < S) read_frags(h ^ 1, sA + st_next * kBTile, sW + st_next * kBTile);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(h);
            __builtin_amdgcn_sched_barrier(0);  // the MFMAs stay ahead of the barrier
            wait_vm<2 * CP * (NS - 3)>();
            // A plain barrier: the fragment reads just issued may stay in
            // flight across it (their stage is overwritten two barriers
            // later).
            asm volatile("s_barrier" ::: "memory");
            st_cur = st_next;
        }
    }

    // Epilogue through LDS: the copies issued for steps past the end (zero
    // fill) land first, then every wave is past its last fragment read.
    wait_vm<0>();
    __syncthreads();
    store_tile_staged<8>(acc, reinterpret_cast<float*>(lds + wave * kEpiWaveBytes), C, M, N, m0 + wm, n0 + wn, bias,
                         lane);
}

// f32 -> bf16 round-to-nearest-even, 8 values per thread.
__global__ __launch_bounds__(256) void k_f32_to_bf16(const float* __restrict__ x,
                                                     uint16_t* __restrict__ y, int64_t n8) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n8) return;
    const f32x4 a = reinterpret_cast<const f32x4*>(x)[2 * i];
    const f32x4 b = reinterpret_cast<const f32x4*>(x)[2 * i + 1];
    reinterpret_cast<u32x4*>(y)[i] = u32x4{pk_bf16(a[0], a[1]), pk_bf16(a[2], a[3]),
                                           pk_bf16(b[0], b[1]), pk_bf16(b[2], b[3])};
}

// Split-K: C = sum of the `splits` partial products (in split order, so the
// result does not depend on scheduling) + bias.  mn % 4 == 0, n % 4 == 0.
__global__ __launch_bounds__(256) void k_splitk_sum(const float* __restrict__ parts, int splits,
                                                    const float* __restrict__ bias, float* __restrict__ C,
                                                    int64_t mn, int64_t n) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= mn) return;
    f32x4 v = *reinterpret_cast<const f32x4*>(parts + i);
    for (int q = 1; q < splits; ++q) v += *reinterpret_cast<const f32x4*>(parts + q * mn + i);
    if (bias) v += *reinterpret_cast<const f32x4*>(bias + i % n);
    *reinterpret_cast<f32x4*>(C + i) = v;
}

__global__ void k_add_bias(float* __restrict__ y, const float* __restrict__ bias, int64_t m,
                           int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < m * n) y[i] += bias[i % n];
}

}  // namespace

namespace {

// How one GEMM call runs (shared by the launcher and the workspace query).
struct GemmPlan {
    bool pipe = false;  // pipelined MFMA kernels (k % 256 == 0, Q4_K or BF16 W)
    bool big = false;   // 256 x 256 bf16 kernel
    bool ws = false;    // Q4_K W dequantized inside the GEMM by producer waves (k_gemm_ws)
    int splits = 1;     // split-K slices of the 128 x 128 kernels
    int64_t mt = 0, nt = 0, mt2 = 0, nt2 = 0;
    size_t a_bytes = 0, w_bytes = 0, p_bytes = 0;
};

GemmPlan plan_gemm(int w_fmt, bool a_bf16, int64_t m, int64_t n, int64_t k) {
    GemmPlan p;
    const bool four_bit = w_fmt == RT_HIP_Q4MAT || w_fmt == RT_HIP_Q4_0;
    p.pipe = k % 256 == 0 && (w_fmt == RT_HIP_Q4K || w_fmt == RT_HIP_BF16 || four_bit);
    if (!p.pipe) return p;
    // A Q4_K weight is dequantized (bf16, round-to-nearest-even of the exact
    // f32 value, as the reference's flux_dequant_q4k) either inside the GEMM
    // by producer waves, once per 128-row M tile, or once per call into the
    // workspace ahead of the bf16 kernels; Q4Mat and GGUF Q4_0 weights the
    // same way (their workspace route runs in the ABI layer).
    p.mt = (m + 127) / 128;
    p.nt = (n + 127) / 128;
    const int64_t cus = device_info().cus;
    p.mt2 = (m + 255) / 256;
    p.nt2 = (n + 255) / 256;
    p.big = 4 * p.mt2 * p.nt2 >= 3 * cus && tune_param("GEMM_BIG", 1);
    // Measured (Q4_K, Llama-3.2-3B and 4096-square shapes): inside wins up
    // to two M tiles (32 rows: 19 against 47 us for gate 8192 x 3072, 33
    // against 113 us for down 3072 x 8192; 256 rows: 36 against 42 us); up
    // to eight tiles when N >= 2K (gate, 768 rows: 68.5 against 76.1 us with
    // f32 A, 62.7 against 72.6 with bf16 A); up to four when N >= K with a
    // bf16 A (3072 x 3072, 384 rows: 26.7 against 28.2 us).  It loses for
    // square shapes beyond four tiles (4096 x 4096, 768 rows: 61 against
    // 53 us) and for the down shape beyond two (60 against 57 us at 512).
    // Up to two M tiles an f32 A is converted to bf16 inside k_gemm_ws;
    // beyond that once into the workspace first (read as f32 by every N
    // tile, its traffic made the in-GEMM route lose).
    const bool wide = p.mt <= 8 && (n >= 2 * k || (a_bf16 && n >= k && p.mt <= 4));
    p.ws = w_fmt != RT_HIP_BF16 && !p.big &&
           (p.mt <= tune_param("GEMM_WS_MT", 2) || (wide && tune_param("GEMM_WS_WIDE", 1)));
    if (four_bit && !p.ws) {
        p.pipe = false;  // Q4Mat / Q4_0 beyond two M tiles: the caller dequantizes into the workspace
        return p;
    }
    // Split-K for the 128 x 128 kernels when their tiles leave at least half
    // the CUs idle: up to 4 slices of K (8 for k_gemm_ws), summed afterwards
    // in a fixed order (deterministic).  Slices are multiples of 64 values
    // (256 for k_gemm_ws, whose slices start on super-blocks).
    if (!p.big && 2 * p.mt * p.nt <= cus && n % 4 == 0) {
        const int cap = p.ws ? 8 : 4, unit = p.ws ? 256 : 64;
        int splits = static_cast<int>(cus / (p.mt * p.nt));
        splits = splits > cap ? cap : splits;
        while (splits > 1 && k % (unit * splits) != 0) --splits;
        const int forced = tune_param("GEMM_SPLITK", 0);
        if (forced >= 1 && forced <= cap && k % (unit * forced) == 0) splits = forced;
        p.splits = splits;
    }
    p.a_bytes = a_bf16 || (p.ws && p.mt <= 2) ? 0 : static_cast<size_t>(m * k) * 2;
    p.w_bytes = w_fmt == RT_HIP_Q4K && !p.ws ? static_cast<size_t>(n * k) * 2 : 0;
    p.p_bytes = p.splits > 1 ? static_cast<size_t>(p.splits) * m * n * 4 : 0;
    return p;
}

}  // namespace

bool gemm_dequant_in_kernel(int w_fmt, bool a_bf16, int64_t m, int64_t n, int64_t k) {
    const GemmPlan p = plan_gemm(w_fmt, a_bf16, m, n, k);
    return p.pipe && p.ws;
}

size_t gemm_workspace_bytes(int w_fmt, bool a_bf16, int64_t m, int64_t n, int64_t k) {
    const GemmPlan p = plan_gemm(w_fmt, a_bf16, m, n, k);
    return p.a_bytes + p.w_bytes + p.p_bytes;
}

hipError_t launch_gemm(int w_fmt, const void* a, bool a_bf16, const void* w, const float* bias,
                       float* c, int64_t m, int64_t n, int64_t k, hipStream_t s) {
    if (k % BK) return hipErrorInvalidValue;
    const GemmPlan P = plan_gemm(w_fmt, a_bf16, m, n, k);
    if (P.pipe) {
        const int64_t mt = P.mt, nt = P.nt, mt2 = P.mt2, nt2 = P.nt2;
        const bool big = P.big;
        const int splits = P.splits;
        const size_t a_bytes = P.a_bytes, w_bytes = P.w_bytes, p_bytes = P.p_bytes;
        uint8_t* ws = nullptr;
        if (a_bytes + w_bytes + p_bytes) {
            hipError_t e;
            ws = static_cast<uint8_t*>(workspace(a_bytes + w_bytes + p_bytes, s, &e));
            if (!ws) return e;
        }
        if (P.ws) {
            // Both roles of k_gemm_ws run the same number of barriers only if
            // each slice is whole super-blocks (S % 4 == 0).
            if ((k / splits) % 256 != 0) return hipErrorInvalidValue;
            const int im = static_cast<int>(m), in = static_cast<int>(n), ik = static_cast<int>(k);
            const dim3 g(static_cast<unsigned>(mt * nt), static_cast<unsigned>(splits)), b(kWsThreads);
            const auto* wq = static_cast<const uint8_t*>(w);
            bool abf = a_bf16;
            const void* ain = a;
            if (a_bytes) {  // f32 A over more than two M tiles: once to bf16 first
                uint16_t* ab = reinterpret_cast<uint16_t*>(ws);
                const int64_t n8 = m * k / 8;
                hipLaunchKernelGGL(k_f32_to_bf16, dim3(static_cast<unsigned>((n8 + 255) / 256)), dim3(256), 0, s,
                                   static_cast<const float*>(a), ab, n8);
                ain = ab;
                abf = true;
            }
            float* out = splits > 1 ? reinterpret_cast<float*>(ws + a_bytes) : c;
            const float* bs = splits > 1 ? nullptr : bias;
            const int64_t cs = splits > 1 ? m * n : 0;
            const int64_t so = w_fmt == RT_HIP_Q4MAT ? static_cast<int64_t>(q4mat_scales_offset(n, k)) : 0;
            const int imt = static_cast<int>(mt), iks = ik / splits;
            auto go = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, g, b, kWsLds, s, ain, wq, bs, out, im, in, iks, imt, ik, cs, so);
            };
            if (w_fmt == RT_HIP_Q4K)
                abf ? go(k_gemm_ws<RT_HIP_Q4K, false>) : go(k_gemm_ws<RT_HIP_Q4K, true>);
            else if (w_fmt == RT_HIP_Q4MAT)
                abf ? go(k_gemm_ws<RT_HIP_Q4MAT, false>) : go(k_gemm_ws<RT_HIP_Q4MAT, true>);
            else
                abf ? go(k_gemm_ws<RT_HIP_Q4_0, false>) : go(k_gemm_ws<RT_HIP_Q4_0, true>);
            if (splits > 1) {
                const int64_t mn = m * n;
                hipLaunchKernelGGL(k_splitk_sum, dim3(static_cast<unsigned>((mn / 4 + 255) / 256)), dim3(256), 0, s,
                                   reinterpret_cast<const float*>(ws + a_bytes), splits, bias, c, mn, n);
            }
            return hipGetLastError();
        }
        const uint16_t* a16 = static_cast<const uint16_t*>(a);
        if (!a_bf16 && w_bytes) {
            // both conversions in one launch
            uint16_t* ab = reinterpret_cast<uint16_t*>(ws);
            const hipError_t e = launch_dequant_q4k_cvt(w, reinterpret_cast<uint16_t*>(ws + a_bytes), n, k,
                                                        static_cast<const float*>(a), ab, m * k, s);
            if (e != hipSuccess) return e;
            a16 = ab;
            w = ws + a_bytes;
        } else if (!a_bf16) {
            uint16_t* ab = reinterpret_cast<uint16_t*>(ws);
            const int64_t n8 = m * k / 8;
            hipLaunchKernelGGL(k_f32_to_bf16, dim3(static_cast<unsigned>((n8 + 255) / 256)), dim3(256), 0, s,
                               static_cast<const float*>(a), ab, n8);
            a16 = ab;
        } else if (w_bytes) {
            const hipError_t e = launch_dequant_q4k(w, ws + a_bytes, true, n, k, s);
            if (e != hipSuccess) return e;
            w = ws + a_bytes;
        }
        // Large outputs: the 256 x 256 kernel when its tiles cover at least
        // three quarters of the CUs (k % 64 == 0 always holds here).
        if (big) {
            const dim3 g(static_cast<unsigned>(mt2 * nt2)), b(kBThreads);
            const uint16_t* w16 = static_cast<const uint16_t*>(w);
            const int im = static_cast<int>(m), in = static_cast<int>(n), ik = static_cast<int>(k);
            const int imt = static_cast<int>(mt2);
            hipLaunchKernelGGL((k_gemm_256<5>), g, b, static_cast<size_t>(10) * kBTile, s, a16, w16, bias, c, im,
                               in, ik, imt);
            return hipGetLastError();
        }
        const size_t lds = static_cast<size_t>(2 * kStages) * kTile;
        const int im = static_cast<int>(m), in = static_cast<int>(n), ik = static_cast<int>(k);
        const dim3 g(static_cast<unsigned>(mt * nt)), b(kPThreads);
        const uint16_t* w16 = static_cast<const uint16_t*>(w);
        if (splits == 1) {
            hipLaunchKernelGGL(k_gemm_pipe, g, b, lds, s, a16, w16, bias, c, im, in, ik, static_cast<int>(mt), ik,
                               int64_t{0});
        } else {
            float* parts = reinterpret_cast<float*>(ws + a_bytes + w_bytes);
            const int64_t mn = m * n;
            hipLaunchKernelGGL(k_gemm_pipe, dim3(g.x, static_cast<unsigned>(splits)), b, lds, s, a16, w16, nullptr,
                               parts, im, in, ik / splits, static_cast<int>(mt), ik, mn);
            hipLaunchKernelGGL(k_splitk_sum, dim3(static_cast<unsigned>((mn / 4 + 255) / 256)), dim3(256), 0, s,
                               parts, splits, bias, c, mn, n);
        }
        return hipGetLastError();
    }
    const dim3 grid(static_cast<unsigned>((n + BN - 1) / BN), static_cast<unsigned>((m + BM - 1) / BM));
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
