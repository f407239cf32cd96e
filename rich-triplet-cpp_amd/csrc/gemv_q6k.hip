// gemv_q6k.hip -- GGUF Q6_K weights on the GPU without widening them in
// memory.
//
// The reference loads a Q6_K projection (the v / down of a Q4_K_M model) by
// decoding it to f32 and rounding every weight to bf16 (GgufFile::
// decode_q6k_to_f32, gguf.cpp:531-580, then f32s_to_bf16_and_drop,
// transformer4_load.cpp:33-41, 141-143), and runs the BF16 GEMV on 2 bytes
// per weight.  Here the weights stay Q6_K (210 bytes per 256, 0.82 byte per
// weight) and each weight is widened in registers to the same bf16 value:
//     w = bf16_rne((d * sc) * (q - 32)),
// where d * sc (f16 times int8, at most 19 significant bits) and its product
// with q - 32 (|q - 32| <= 32) are exact in f32, so the only rounding is the
// bf16 one, as in the reference.  The GEMV's products are then those of the
// BF16 GEMV on the widened weights; results agree with it to f32 rounding.
//
// Block (210 bytes): ql[128] | qh[64] | sc[16] (int8) | d (f16).  Value
// 128 j + 32 r + t (half j, quarter r, t < 32) takes, from ql_j = ql[64 j..]
// and qh_j = qh[32 j..]:
//     r = 0: ql_j[t] & 15        | (qh_j[t] & 3) << 4
//     r = 1: ql_j[32 + t] & 15   | (qh_j[t] >> 2 & 3) << 4
//     r = 2: ql_j[t] >> 4        | (qh_j[t] >> 4 & 3) << 4
//     r = 3: ql_j[32 + t] >> 4   | (qh_j[t] >> 6 & 3) << 4
// with scale sc[8 j + t / 16 + 2 r].
//
// Tiled layout (load-time, size-preserving, this build's own): a 16-row
// tile's block b is 3360 contiguous bytes in the GEMV's lane order
// (lane l = n + 16 g, row n of the tile, t-range [8 g, 8 g + 8)):
//   [0, 2048)     32 bytes per lane: for j = 0, 1: ql_j[8g, 8g+8), ql_j[32+8g, +8)
//   [2048, 3072)  16 bytes per lane: for j = 0, 1: qh_j[8g, 8g+8)
//   [3072, 3328)  16 bytes per row: sc[16]
//   [3328, 3360)  2 bytes per row: d
// Tiles follow one another, each as its K/256 blocks; rows past N are zero.
//
// GEMV (M = 1): one MFMA step is 32 values of K (a quarter r of a half j):
// lane (n, g) widens its 8 weights of row n at t = 8 g .. 8 g + 7 into the B
// operand of v_mfma_f32_16x16x32_bf16; A rows 0..2 hold x as three bf16
// limbs (h + m + l == x exactly), the other rows zero.  Products are exact,
// so C accumulates the whole K-range with no per-step epilogue; lane (n, 0)
// ends with the three limb dots of row n.
#include "gemv_bf16.hpp"
#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kBlk = 210;
constexpr int kTileBlk = 16 * kBlk;  // 3360
constexpr int kOffQh = 2048, kOffSc = 3072, kOffD = 3328;
constexpr int kThreads = 256;        // 4 waves (K splits up to 4)
constexpr int kMaxThreads = 1024;    // 16 waves (one tile split 6, 8, 12 or 16 ways)
constexpr int kStepBytes = 192;      // x limbs of one 32-value step: 3 limbs x 32 bf16
constexpr int kMaxK = 8192;

// ---- repack: row-major blocks -> tiled ------------------------------------
// One workgroup of 64 threads per (tile, block); thread l = n + 16 g.
__global__ __launch_bounds__(64) void k_q6k_tile(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int N,
                                                int nb) {
    const int tile = blockIdx.y, b = blockIdx.x, l = threadIdx.x;
    const int n = l & 15, g = l >> 4;
    const int row = tile * 16 + n;
    const bool in = row < N;
    const uint8_t* blk = src + (static_cast<int64_t>(in ? row : 0) * nb + b) * kBlk;
    uint8_t* out = dst + (static_cast<int64_t>(tile) * nb + b) * kTileBlk;
    uint8_t ql[32], qh[16];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            ql[16 * j + e] = in ? blk[64 * j + 8 * g + e] : 0;
            ql[16 * j + 8 + e] = in ? blk[64 * j + 32 + 8 * g + e] : 0;
            qh[8 * j + e] = in ? blk[128 + 32 * j + 8 * g + e] : 0;
        }
#pragma unroll
    for (int e = 0; e < 32; ++e) out[32 * l + e] = ql[e];
#pragma unroll
    for (int e = 0; e < 16; ++e) out[kOffQh + 16 * l + e] = qh[e];
    if (g == 0) {
#pragma unroll
        for (int e = 0; e < 16; ++e) out[kOffSc + 16 * n + e] = in ? blk[192 + e] : 0;
        out[kOffD + 2 * n] = in ? blk[208] : 0;
        out[kOffD + 2 * n + 1] = in ? blk[209] : 0;
    }
}

// ---- widening: row-major blocks -> bf16 [N][K] (the reference's load) ------
// One thread per (block, half j, t < 32): its four values.
__global__ __launch_bounds__(256) void k_q6k_to_bf16(const uint8_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                    int64_t nblocks) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= nblocks * 64) return;
    const int64_t b = i >> 6;
    const int j = static_cast<int>(i >> 5) & 1, t = static_cast<int>(i) & 31;
    const uint8_t* blk = src + b * kBlk;
    const float d = f16_bits_to_f32(static_cast<uint32_t>(blk[208]) | (static_cast<uint32_t>(blk[209]) << 8));
    const uint8_t a = blk[64 * j + t], a2 = blk[64 * j + 32 + t], h = blk[128 + 32 * j + t];
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * j + (t >> 4));
    const int q[4] = {(a & 15) | ((h & 3) << 4), (a2 & 15) | ((h >> 2 & 3) << 4), (a >> 4) | ((h >> 4 & 3) << 4),
                      (a2 >> 4) | ((h >> 6 & 3) << 4)};
    uint16_t* out = dst + b * 256 + 128 * j + t;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float s = d * static_cast<float>(sc[2 * r]);
        const float w = s * static_cast<float>(q[r] - 32);
        out[32 * r] = f32_to_bf16_rne(w);
    }
}

// ---- GEMV ------------------------------------------------------------------

struct Slot {
    u32x4 ql0, ql1, qh, sc;
    uint32_t d2;  // d of rows n & ~1 (low half) and n | 1 (high half)
};

__device__ __forceinline__ void load_slot(BufRsrc rs, int lane, Slot& s) {
    const uint32_t l = static_cast<uint32_t>(lane), n = l & 15u;
    s.ql0 = ld16(rs, 32u * l);
    s.ql1 = ld16(rs, 32u * l + 16u);
    s.qh = ld16(rs, kOffQh + 16u * l);
    s.sc = ld16(rs, kOffSc + 16u * n);
    s.d2 = __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(kOffD + 4u * (n >> 1)), 0, 0);
}

// B operand of step (j, r) for lane (n, g): bf16 of its 8 weights.
template <int J, int R>
__device__ __forceinline__ bf16x8 widen(const Slot& s, float d, uint32_t gsh) {
    const u32x4& qlv = J == 0 ? s.ql0 : s.ql1;
    const uint32_t a0 = (R & 1) ? qlv[2] : qlv[0], a1 = (R & 1) ? qlv[3] : qlv[1];
    const uint32_t n0 = R >= 2 ? (a0 >> 4) & 0x0f0f0f0fu : a0 & 0x0f0f0f0fu;
    const uint32_t n1 = R >= 2 ? (a1 >> 4) & 0x0f0f0f0fu : a1 & 0x0f0f0f0fu;
    const uint32_t h0 = s.qh[2 * J], h1 = s.qh[2 * J + 1];
    const uint32_t b0 = (R <= 2 ? (h0 << (4 - 2 * R)) : (h0 >> 2)) & 0x30303030u;
    const uint32_t b1 = (R <= 2 ? (h1 << (4 - 2 * R)) : (h1 >> 2)) & 0x30303030u;
    const uint32_t q0 = n0 | b0, q1 = n1 | b1;
    // scale byte 8 J + 2 R + g / 2: dword 2 J + R / 2, byte 2 (R & 1) + g / 2
    const int32_t scv = static_cast<int32_t>(s.sc[2 * J + (R >> 1)]);
    const int sc = __builtin_amdgcn_sbfe(scv, 16 * (R & 1) + gsh, 8);
    const float sf = d * static_cast<float>(sc);
    const float m = -32.0f * sf;
    u32x4 w;
    w[0] = bf16_pair(__builtin_fmaf(ubyte_f32(q0, 0), sf, m), __builtin_fmaf(ubyte_f32(q0, 1), sf, m));
    w[1] = bf16_pair(__builtin_fmaf(ubyte_f32(q0, 2), sf, m), __builtin_fmaf(ubyte_f32(q0, 3), sf, m));
    w[2] = bf16_pair(__builtin_fmaf(ubyte_f32(q1, 0), sf, m), __builtin_fmaf(ubyte_f32(q1, 1), sf, m));
    w[3] = bf16_pair(__builtin_fmaf(ubyte_f32(q1, 2), sf, m), __builtin_fmaf(ubyte_f32(q1, 3), sf, m));
    return __builtin_bit_cast(bf16x8, w);
}

// Workgroup of T threads: KS <= 4 runs 4 waves, TPW = 4 / KS tiles each
// split over KS waves by blocks; larger KS runs one tile on KS waves.  LDS:
// x limbs [K/32 steps][3][32] bf16, a zero line, then the KS partial rows.
// SWIGLU: x = silu(X) * UP while it is staged (swiglu1, the BF16 GEMV's
// form), and the finished rows are added to Y (the residual add of the MLP's
// down projection) instead of stored.
template <int D, int XP, int T, bool SWIGLU>
__global__ __launch_bounds__(T) void k_gemv_q6k(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                               const float* __restrict__ UP, float* __restrict__ Y, int N, int K,
                                               int KS) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = K >> 8;
    const int nthr = static_cast<int>(blockDim.x);
    const int tpw = (nthr >> 6) / KS;
    const int ks = wave % KS, tslot = wave / KS;
    const int tile = blockIdx.x * tpw + tslot;
    const int bpw = nb / KS;  // the host picks KS | nb
    const int b0 = ks * bpw;
    const int tiles = (N + 15) >> 4;
    const int64_t tb = static_cast<int64_t>(nb) * kTileBlk;
    const uint8_t* const base = W + static_cast<int64_t>(tile) * tb + static_cast<int64_t>(b0) * kTileBlk;
    const int64_t left = tile < tiles ? (tb - static_cast<int64_t>(b0) * kTileBlk) : 0;

    // x first: unit u = (step, g) is the 8 values 8u .. 8u + 7.
    const int units = K >> 3;
    f32x4 xa[XP], xb[XP], ua[XP], ub[XP];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int u = tid + nthr * i;
        const f32x4* src = reinterpret_cast<const f32x4*>(X) + 2 * (u < units ? u : 0);
        xa[i] = src[0];
        xb[i] = src[1];
        if constexpr (SWIGLU) {
            const f32x4* up = reinterpret_cast<const f32x4*>(UP) + 2 * (u < units ? u : 0);
            ua[i] = up[0];
            ub[i] = up[1];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    Slot ring[D];
    auto issue = [&](Slot& s, int i) {
        const int64_t o = static_cast<int64_t>(i) * kTileBlk;
        load_slot(make_rsrc(base + o, i < bpw ? left - o : 0), lane, s);
    };
#pragma unroll
    for (int j = 0; j < D; ++j) {
        issue(ring[j], j);
        __builtin_amdgcn_sched_barrier(0);
    }

    const uint32_t zoff = static_cast<uint32_t>((K >> 5) * kStepBytes);
    if (tid == 0) *reinterpret_cast<u32x4*>(lds + zoff) = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int u = tid + nthr * i;
        if constexpr (SWIGLU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xa[i][e] = swiglu1(xa[i][e], ua[i][e]);
                xb[i][e] = swiglu1(xb[i][e], ub[i][e]);
            }
        }
        u32x2 ha, ma, la, hb, mb, lb;
        bf16_limbs4(xa[i], ha, ma, la);
        bf16_limbs4(xb[i], hb, mb, lb);
        if (u < units) {
            u32x4* dst = reinterpret_cast<u32x4*>(lds + (u >> 2) * kStepBytes + (u & 3) * 16);
            dst[0] = u32x4{ha[0], ha[1], hb[0], hb[1]};
            dst[4] = u32x4{ma[0], ma[1], mb[0], mb[1]};
            dst[8] = u32x4{la[0], la[1], lb[0], lb[1]};
        }
    }
    lds_barrier();

    // A: rows 0..2 are the limbs (lane i = l % 16 < 3), the rest read zeros.
    const int ai = lane & 15, g = lane >> 4;
    const bool live = ai < 3;
    const uint32_t abase = live ? static_cast<uint32_t>(ai * 64 + g * 16) : zoff;
    const uint32_t amask = live ? 0xffffffffu : 0u;
    const uint32_t gsh = static_cast<uint32_t>(g >> 1) * 8u;
    const int n = lane & 15;
    f32x4 C = {0.0f, 0.0f, 0.0f, 0.0f};
    auto consume = [&](const Slot& s, int blk) {
        const uint32_t d2 = s.d2;
        const float d = f16_bits_to_f32((n & 1) ? (d2 >> 16) : (d2 & 0xffffu));
        const uint32_t sb = static_cast<uint32_t>(blk) * 8u * kStepBytes;
#define RT_Q6_STEP(J, R)                                                                                     \
        {                                                                                                    \
            const bf16x8 B = widen<J, R>(s, d, gsh);                                                         \
            const bf16x8 A = __builtin_bit_cast(                                                            \
                bf16x8, *reinterpret_cast<const u32x4*>(lds + abase + ((sb + (4 * J + R) * kStepBytes) & amask))); \
            C = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, C, 0, 0, 0);                                   \
        }
        RT_Q6_STEP(0, 0) RT_Q6_STEP(0, 1) RT_Q6_STEP(0, 2) RT_Q6_STEP(0, 3)
        RT_Q6_STEP(1, 0) RT_Q6_STEP(1, 1) RT_Q6_STEP(1, 2) RT_Q6_STEP(1, 3)
#undef RT_Q6_STEP
    };

    // Steady rounds (straight-line: consume slot j in place, then refill it
    // D blocks ahead -- a copy of the slot would make the compiler copy the
    // whole ring at the loop head and wait for every load), then the tail
    // of the last <= D blocks.
    int i = 0;
    for (; i + D < bpw; i += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            consume(ring[j], b0 + i + j);
            __builtin_amdgcn_sched_barrier(0);
            issue(ring[j], i + D + j);
        }
    }
#pragma unroll
    for (int j = 0; j < D; ++j)
        if (i + j < bpw) consume(ring[j], b0 + i + j);

    // Lane (n, 0): C[0..2][n] are the limb dots of row n.
    float v = (C[0] + C[1]) + C[2];
    const int row = tile * 16 + n;
    if (KS == 1) {
        if (lane < 16 && row < N) Y[row] = SWIGLU ? Y[row] + v : v;
    } else {
        float* red = reinterpret_cast<float*>(lds + zoff + 16);  // [tpw][KS][16], tpw * KS <= 16
        float* rp = red + tslot * KS * 16;
        if (lane < 16) rp[ks * 16 + lane] = v;
        lds_barrier();
        if (ks == 0 && lane < 16 && row < N) {
            float sum = rp[lane];
            for (int q = 1; q < KS; ++q) sum += rp[q * 16 + lane];
            Y[row] = SWIGLU ? Y[row] + sum : sum;
        }
    }
}

template <int D, int XP, int T>
hipError_t run(const void* w, const float* x, const float* up, float* y, int64_t n, int64_t k, int ks,
               hipStream_t s) {
    const int64_t tiles = (n + 15) / 16;
    const int waves = ks <= 4 ? 4 : ks;
    const int tpw = waves / ks;
    const int64_t wgs = (tiles + tpw - 1) / tpw;
    const dim3 g(static_cast<unsigned>(wgs)), b(static_cast<unsigned>(waves * kWave));
    const auto* wb = static_cast<const uint8_t*>(w);
    const int in = static_cast<int>(n), ik = static_cast<int>(k);
    if (up)
        hipLaunchKernelGGL((k_gemv_q6k<D, XP, T, true>), g, b, q6k_gemv_lds_bytes(k), s, wb, x, up, y, in, ik, ks);
    else
        hipLaunchKernelGGL((k_gemv_q6k<D, XP, T, false>), g, b, q6k_gemv_lds_bytes(k), s, wb, x, up, y, in, ik, ks);
    return hipGetLastError();
}

template <int D, int T>
hipError_t run_xp(const void* w, const float* x, const float* up, float* y, int64_t n, int64_t k, int ks,
                  hipStream_t s) {
    const int waves = ks <= 4 ? 4 : ks;
    const int64_t per = (k / 8 + waves * kWave - 1) / (waves * kWave);  // 8-value units of x per thread
    if (per <= 1) return run<D, 1, T>(w, x, up, y, n, k, ks, s);
    if (per <= 2) return run<D, 2, T>(w, x, up, y, n, k, ks, s);
    return run<D, 4, T>(w, x, up, y, n, k, ks, s);
}

}  // namespace

size_t q6k_gemv_lds_bytes(int64_t k) { return static_cast<size_t>(k / 32) * kStepBytes + 16 + 16 * 16 * sizeof(float); }

int64_t q6k_tiled_bytes(int64_t n, int64_t k) { return (n + 15) / 16 * (k / 256) * kTileBlk; }

hipError_t launch_q6k_tile(const void* blocks, void* tiled, int64_t n, int64_t k, hipStream_t s) {
    const int64_t nb = k / 256, tiles = (n + 15) / 16;
    if (tiles > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_q6k_tile, dim3(static_cast<unsigned>(nb), static_cast<unsigned>(tiles)), dim3(64), 0, s,
                       static_cast<const uint8_t*>(blocks), static_cast<uint8_t*>(tiled), static_cast<int>(n),
                       static_cast<int>(nb));
    return hipGetLastError();
}

hipError_t launch_q6k_to_bf16(const void* blocks, uint16_t* dst, int64_t n, int64_t k, hipStream_t s) {
    const int64_t nblocks = n * (k / 256);
    const int64_t threads = nblocks * 64;
    hipLaunchKernelGGL(k_q6k_to_bf16, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, s,
                       static_cast<const uint8_t*>(blocks), dst, nblocks);
    return hipGetLastError();
}

// K split per tile, as the Q4_K GEMV: the largest split of {1, 2, 3, 4, 6,
// 8, 12, 16} that divides the blocks, leaves every wave two of them and keeps
// one round of workgroups.  The widening makes this GEMV VALU-heavy (about
// four VALU per weight), so it wants more waves than the streaming GEMVs:
// splits above 4 run one tile on KS waves with a two-slot ring (<= 128 VGPRs,
// four waves per SIMD).
hipError_t launch_gemv_q6k(const void* tiled, const float* x, float* y, int64_t n, int64_t k, hipStream_t s,
                           const float* up) {
    if (k % 256 != 0 || k > kMaxK) return hipErrorInvalidValue;
    const int64_t nb = k / 256, tiles = (n + 15) / 16, cus = device_info().cus;
    static const int kSplits[] = {1, 2, 3, 4, 6, 8, 12, 16};
    auto wgs_for = [&](int c) {
        const int64_t tpw = c <= 4 ? 4 / c : 1;
        return (tiles + tpw - 1) / tpw;
    };
    int ks = 1;
    for (int c : kSplits) {
        if (nb % c != 0 || (c > 1 && 2 * c > nb) || (c == 3)) continue;
        if (wgs_for(c) <= cus) ks = c;
    }
    if (const int forced = tune_param("Q6K_KS", 0))
        for (int c : kSplits)
            if (c == forced && nb % c == 0 && c != 3) ks = c;
    if (ks <= 4) return run_xp<4, kThreads>(tiled, x, up, y, n, k, ks, s);
    return run_xp<2, kMaxThreads>(tiled, x, up, y, n, k, ks, s);
}

}  // namespace rt_hip
