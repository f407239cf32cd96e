// gemv_bf16.hpp -- the M = 1 BF16 GEMV body (y[n] = sum_k x[k] * W[n, k],
// W row-major bf16 (MatBf16, include/rt/mat.hpp), x and y f32), shared by
// the BF16 GEMV kernel and the fused q/k/v launch of gemv_mfma.hip.
//
// A wave owns RPW consecutive rows and walks them side by side, one "piece"
// (512 values = 1 KB of one row, 16 bytes per lane) per row per step, so a
// load instruction reads 1 KB of contiguous memory and one activation read
// from LDS feeds RPW rows.  Rows are never split across waves: a wave's
// partial sums only need a butterfly at the end.
//
// Pipeline: a ring of D slots (RPW pieces each) is loaded ahead of the
// compute; each slot is refilled as soon as it is consumed.  The steady loop
// is straight-line and the last <= D pieces are a tail that issues nothing,
// so the compiler keeps the ring in place and every wait is partial.  x is
// loaded into registers before the weight prologue and staged in LDS after
// it, so waiting for x never waits for weight loads.
//
// Loads go through per-(row, piece) buffer resources: rows past N and bytes
// past the end of a row (K % 512 != 0) read as zeros, with no clamping.
//
// Numerics: f32 FMA accumulation, lane-strided then butterfly-reduced; the
// order differs from the reference's sequential dot (mat.cpp:310-314), so
// results agree to f32 rounding, not bit-for-bit.
#pragma once

#include "rt_common.hpp"

namespace rt_hip {
namespace bf16_gemv {

constexpr int kThreads = 256;  // one workgroup: 4 waves
constexpr int kPiece = 512;  // bf16 values per wave-wide 16-byte-per-lane load

// LDS byte offset of x[4f .. 4f+3]: piece i = f / 128 holds, for lane
// l = (f / 2) % 64, the values 8l .. 8l+7 of the piece as two 16-byte halves
// h = f % 2, stored half-major: ((2i + h) * 64 + l) * 16.  A lane's two reads
// of a piece are then contiguous across the wave (no bank conflicts).
__device__ __forceinline__ uint32_t x_off(int f) {
    const int i = f >> 7, l = (f >> 1) & 63, h = f & 1;
    return static_cast<uint32_t>((((i << 1) + h) << 6) + l) << 4;
}

// Workgroup `blk` of a launch of kThreads-thread workgroups; `lds` holds
// lds_bytes(K).
template <int RPW, int D, int XP, bool ARGMAX>
__device__ __forceinline__ void rows(int blk, const uint16_t* __restrict__ W, const float* __restrict__ X,
                                     float* __restrict__ Y, int N, int K, uint64_t* __restrict__ key,
                                     uint8_t* lds) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int P = (K + kPiece - 1) / kPiece;  // pieces per row (the last may be partial)
    const int nx4 = P * (kPiece / 4);         // f32x4 slots of the zero-padded x
    const int kx4 = K >> 2;                   // f32x4 of x (K % 8 == 0)
    const f32x4* X4 = reinterpret_cast<const f32x4*>(X);

    f32x4 xv[XP];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int f = tid + kThreads * i;
        xv[i] = X4[f < kx4 ? f : 0];
    }
    __builtin_amdgcn_sched_barrier(0);

    const int row0 = (blk * (kThreads / kWave) + wave) * RPW;
    const int64_t rowb = static_cast<int64_t>(K) * 2;
    const uint8_t* const wb = reinterpret_cast<const uint8_t*>(W);
    const uint32_t loff = static_cast<uint32_t>(lane) * 16u;

    // Piece i of each of the wave's rows; empty resources past N or past
    // the last piece.
    auto issue = [&](u32x4 (&slot)[RPW], int i) {
        const int64_t o = static_cast<int64_t>(i) * (kPiece * 2);
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = row0 + r;
            const int64_t left = (row < N && i < P) ? rowb - o : 0;
            slot[r] = ld16(make_rsrc(wb + static_cast<int64_t>(row) * rowb + o, left), loff);
        }
    };

    u32x4 ring[D][RPW];
#pragma unroll
    for (int j = 0; j < D; ++j) {
        issue(ring[j], j);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Stage x (zeros past K, up to the whole last piece).
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int f = tid + kThreads * i;
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        if (f < nx4) *reinterpret_cast<f32x4*>(lds + x_off(f)) = f < kx4 ? xv[i] : z;
    }
    for (int f = tid + kThreads * XP; f < nx4; f += kThreads) {
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        *reinterpret_cast<f32x4*>(lds + x_off(f)) = f < kx4 ? X4[f] : z;
    }
    lds_barrier();

    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
    // Values 8l .. 8l+7 of piece i: dword e holds values 2e (low half) and
    // 2e + 1 (high half).
    auto fma_piece = [&](const u32x4 (&w)[RPW], int i) {
        const f32x4 xa = *reinterpret_cast<const f32x4*>(lds + ((((i << 1) + 0) << 6) + lane) * 16);
        const f32x4 xb = *reinterpret_cast<const f32x4*>(lds + ((((i << 1) + 1) << 6) + lane) * 16);
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            float a = acc[r];
            a = __builtin_fmaf(bf16_lo_to_f32(w[r][0]), xa[0], a);
            a = __builtin_fmaf(bf16_hi_to_f32(w[r][0]), xa[1], a);
            a = __builtin_fmaf(bf16_lo_to_f32(w[r][1]), xa[2], a);
            a = __builtin_fmaf(bf16_hi_to_f32(w[r][1]), xa[3], a);
            a = __builtin_fmaf(bf16_lo_to_f32(w[r][2]), xb[0], a);
            a = __builtin_fmaf(bf16_hi_to_f32(w[r][2]), xb[1], a);
            a = __builtin_fmaf(bf16_lo_to_f32(w[r][3]), xb[2], a);
            a = __builtin_fmaf(bf16_hi_to_f32(w[r][3]), xb[3], a);
            acc[r] = a;
        }
    };

    // Steady rounds (straight-line: compute slot j, then refill it with the
    // piece D steps ahead), then the tail of the last <= D pieces.
    int i = 0;
    for (; i + D < P; i += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            fma_piece(ring[j], i + j);
            __builtin_amdgcn_sched_barrier(0);
            issue(ring[j], i + D + j);
        }
    }
#pragma unroll
    for (int j = 0; j < D; ++j)
        if (i + j < P) fma_piece(ring[j], i + j);

    uint64_t best = 0;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float v = acc[r];
#pragma unroll
        for (int off = kWave / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
        const int row = row0 + r;
        if (row < N) {
            if (lane == 0) Y[row] = v;
            if constexpr (ARGMAX) {
                if (v == v) {
                    const uint64_t kk = argmax_key(v, static_cast<uint32_t>(row));
                    best = kk > best ? kk : best;
                }
            }
        }
    }
    if constexpr (ARGMAX) {
        if (lane == 0 && best != 0)
            atomicMax(reinterpret_cast<unsigned long long*>(key), static_cast<unsigned long long>(best));
    }
}

__host__ __device__ inline size_t lds_bytes(int64_t k) {
    return static_cast<size_t>((k + kPiece - 1) / kPiece) * kPiece * sizeof(float);
}

}  // namespace bf16_gemv
}  // namespace rt_hip
