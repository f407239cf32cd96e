// gemv_bf16.hpp -- the M = 1 BF16 GEMV body (y[n] = sum_k x[k] * W[n, k],
// W row-major bf16 (MatBf16, include/rt/mat.hpp), x and y f32), shared by
// the BF16 GEMV kernel and the fused q/k/v launch of gemv_mfma.hip.
//
// A wave walks its rows one "piece" (512 values = 1 KB of one row, 16 bytes
// per lane) at a time, so a load instruction reads 1 KB of contiguous
// memory.  Rows are never split across waves: a row's partial sums only
// need a butterfly once its last piece is in.
//
// Pipeline: a ring of D pieces is loaded ahead of the compute; each slot is
// refilled as soon as it is consumed, running on into the wave's next row.
// The steady loop is straight-line and the last <= D pieces are a tail that
// issues nothing, so the compiler keeps the ring in place and every wait is
// partial.  x is loaded into registers before the weight prologue and
// staged in LDS after it, so waiting for x never waits for weight loads.
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

// What a decode GEMV applies to its activation while staging it (the layer
// operations either side of the projection, fused into its launch):
//   kXNone     x as given;
//   kXRmsNorm  RMSNorm(x) * gamma            (tensor_node.cpp:320-344, 383);
//   kXRmsNorm1 RMSNorm(x) * (1 + gamma)      (the Gemma 3 form, :387);
//   kXSwiGlu   silu(gate) * up, x = gate     (tensor_node.cpp:391-402,
//              transformer5.cpp:186-190);
//   kXGelu     gelu_tanh(gate) * up, x = gate (the Gemma 3 MLP gating,
//              decode_gemma3.msl:128-158);
//   kXPostNorm1 the Gemma 3 residual step, then kXRmsNorm1 of its result:
//              x = a + RMSNorm(b) * (1 + g2) (the post-attention / post-FFN
//              norm and residual add, metal_decode.mm:467-480), x also
//              stored for the next residual add (Q4_K GEMV only).
// `aux` is gamma or up.  RMSNorm(x) * g = rms_inv * (x * g) with one scalar
// rms_inv per vector, so kernels stage x * g and scale the finished dot
// products by rms_inv (equal in exact arithmetic); the sum of squares is
// reduced per wave and across waves through LDS at the staging barrier.
enum XOp { kXNone = 0, kXRmsNorm = 1, kXRmsNorm1 = 2, kXSwiGlu = 3, kXGelu = 4, kXPostNorm1 = 5 };

// silu(g) * u in the reference's order, the sigmoid from the hardware exp2
// and reciprocal (about 1 ulp each; exp overflows to inf for g < -88 and
// the sigmoid is then 0, as the reference's is).
__device__ __forceinline__ float swiglu1(float g, float u) {
    const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
    return (g * sig) * u;
}

// gelu_tanh(g) * u as the Metal kernel forms it (decode_gemma3.msl:128-145):
// inner = 0.7978845608 (g + 0.044715 g^3), clamped to [-10, 10], then
// 0.5 g (1 + tanh(inner)), times up.  tanh(a) = 1 - 2 / (e^(2a) + 1) from
// the hardware exp2 and reciprocal (about 1 ulp each; |2a| <= 20 keeps e^(2a)
// finite), rather than the library tanhf (~20 VALU per value).
__device__ __forceinline__ float gelu1(float g, float u) {
    float inner = 0.7978845608f * (g + 0.044715f * (g * g * g));
    inner = fminf(fmaxf(inner, -10.0f), 10.0f);
    const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(inner * 2.88539008177792682f) + 1.0f);
    return (0.5f * g * (1.0f + t)) * u;
}

namespace bf16_gemv {

constexpr int kThreads = 256;  // default workgroup: 4 waves
constexpr int kPiece = 512;  // bf16 values per wave-wide 16-byte-per-lane load

// LDS byte offset of x[4f .. 4f+3]: piece i = f / 128 holds, for lane
// l = (f / 2) % 64, the values 8l .. 8l+7 of the piece as two 16-byte halves
// h = f % 2, stored half-major: ((2i + h) * 64 + l) * 16.  A lane's two reads
// of a piece are then contiguous across the wave (no bank conflicts).
__device__ __forceinline__ uint32_t x_off(int f) {
    const int i = f >> 7, l = (f >> 1) & 63, h = f & 1;
    return static_cast<uint32_t>((((i << 1) + h) << 6) + l) << 4;
}

// Staged x (zero-padded to whole pieces), then one float per wave (up to
// 16) for the RMSNorm partial sums.
__host__ __device__ inline size_t x_bytes(int64_t k) {
    return static_cast<size_t>((k + kPiece - 1) / kPiece) * kPiece * sizeof(float);
}
__host__ __device__ inline size_t lds_bytes(int64_t k) { return x_bytes(k) + 16 * sizeof(float); }

// Workgroup `blk` of `nblk` T-thread workgroups; `lds` holds lds_bytes(K).
// Wave gw = blk * (T / 64) + wave of the NW = nblk * (T / 64) waves takes
// rows gw, gw + NW, gw + 2 NW, ... (at most 64: the launcher sizes the
// grid); the pieces of its rows form one sequence that the ring streams
// without a break between rows, so a short row (small K) costs no pipeline
// ramp and x is staged once per workgroup, not once per row.  A row's sum is
// reduced as soon as its last piece is in and kept by lane r (the wave's
// r-th row); the sums are stored after the loop, since a store among the
// ring's loads makes the compiler wait for all of them.
// Sum over the 64 lanes, in VALU only: DPP within each row of 16 lanes
// (quad swaps, half-row and row mirrors), then the gfx950 permlane swaps
// across rows.  Every lane ends with the same bits.
__device__ __forceinline__ float wave_sum(float v, int lane) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false));   // l ^ 1
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false));   // l ^ 2
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));  // half mirror
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));  // row mirror
    const uint32_t u = __float_as_uint(v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v += __uint_as_float(((lane >> 4) & 1) ? r16[0] : r16[1]);  // lane ^ 16
    const uint32_t u2 = __float_as_uint(v);
    const auto r32 = __builtin_amdgcn_permlane32_swap(u2, u2, false, false);
    v += __uint_as_float(lane >= 32 ? r32[0] : r32[1]);  // lane ^ 32
    return v;
}

// ADD: the rows are added to what Y holds (the residual add) instead of
// stored.
template <int D, int XP, bool ARGMAX, int T = kThreads, int XOP = kXNone, bool ADD = false>
__device__ __forceinline__ void rows(int blk, int nblk, const uint16_t* __restrict__ W,
                                     const float* __restrict__ X, float* __restrict__ Y, int N, int K,
                                     uint64_t* __restrict__ key, uint8_t* lds,
                                     const float* __restrict__ aux = nullptr, float eps = 0.0f) {
    static_assert(!(ADD && ARGMAX), "the argmax epilogue keys stored rows, not added ones");
    constexpr bool kNorm = XOP == kXRmsNorm || XOP == kXRmsNorm1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int P = (K + kPiece - 1) / kPiece;  // pieces per row (the last may be partial)
    const int nx4 = P * (kPiece / 4);         // f32x4 slots of the zero-padded x
    const int kx4 = K >> 2;                   // f32x4 of x (K % 8 == 0)
    const f32x4* X4 = reinterpret_cast<const f32x4*>(X);

    const f32x4* A4 = reinterpret_cast<const f32x4*>(aux);
    f32x4 xv[XP], av[XP];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int f = tid + T * i;
        xv[i] = X4[f < kx4 ? f : 0];
    }
    if constexpr (XOP != kXNone) {
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int f = tid + T * i;
            av[i] = A4[f < kx4 ? f : 0];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    const int NW = nblk * (T / kWave);
    const int gw = blk * (T / kWave) + wave;
    const int R = gw < N ? (N - 1 - gw) / NW + 1 : 0;  // this wave's rows
    const int L = R * P;                                // and their pieces
    const int64_t rowb = static_cast<int64_t>(K) * 2;
    const int64_t stride = static_cast<int64_t>(NW) * rowb;
    const uint8_t* const wb = reinterpret_cast<const uint8_t*>(W) + static_cast<int64_t>(gw) * rowb;
    const uint32_t loff = static_cast<uint32_t>(lane) * 16u;
    auto* const Yg = (__attribute__((address_space(1))) float*)Y;

    // Cursors (wave-uniform, kept in SGPRs): the issue side is at row ir,
    // piece ip; the consume side at row cr, piece cp.  Past the last row the
    // resource is empty (zeros, no memory traffic).
    int ir = 0, ip = 0, cr = 0, cp = 0;
    u32x4 ring[D];
#pragma unroll
    for (int j = 0; j < D; ++j) {
        const int64_t o = static_cast<int64_t>(ip) * (kPiece * 2);
        ring[j] = ld16(make_rsrc(wb + ir * stride + o, ir < R ? rowb - o : 0), loff);
        const bool wrap = ip == P - 1;
        ip = __builtin_amdgcn_readfirstlane(wrap ? 0 : ip + 1);
        ir = __builtin_amdgcn_readfirstlane(wrap ? ir + 1 : ir);
        __builtin_amdgcn_sched_barrier(0);
    }
    // ADD: the values the rows add to, loaded behind the prologue so that
    // their latency passes while the weights stream.
    float y_old = 0.0f;
    if constexpr (ADD) y_old = lane < R ? Yg[gw + lane * NW] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);

    // Stage x (zeros past K, up to the whole last piece), with the x
    // operation applied.
    float sq = 0.0f;
    auto op = [&](f32x4 v, f32x4 a) {
        if constexpr (kNorm) {
            sq += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] *= XOP == kXRmsNorm1 ? 1.0f + a[e] : a[e];
        } else if constexpr (XOP == kXSwiGlu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = swiglu1(v[e], a[e]);
        } else if constexpr (XOP == kXGelu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu1(v[e], a[e]);
        }
        return v;
    };
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int f = tid + T * i;
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        if (f < nx4) *reinterpret_cast<f32x4*>(lds + x_off(f)) = f < kx4 ? op(xv[i], av[i]) : z;
    }
    for (int f = tid + T * XP; f < nx4; f += T) {
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        f32x4 a = z;
        if constexpr (XOP != kXNone) a = f < kx4 ? A4[f] : z;
        *reinterpret_cast<f32x4*>(lds + x_off(f)) = f < kx4 ? op(X4[f], a) : z;
    }
    float* const part = reinterpret_cast<float*>(lds + x_bytes(K));
    if constexpr (kNorm) {
        sq = wave_sum(sq, lane);
        if (lane == 0) part[wave] = sq;
    }
    lds_barrier();
    float out_scale = 1.0f;
    if constexpr (kNorm) {
        float tot = 0.0f;
        for (int w = 0; w < T / kWave; ++w) tot += part[w];
        out_scale = 1.0f / __builtin_sqrtf(tot * (1.0f / static_cast<float>(K)) + eps);
    }

    // Values 8l .. 8l+7 of a piece: dword e holds values 2e (low half) and
    // 2e + 1 (high half).  A row's sum stays with lane cr of the wave.
    float acc = 0.0f, res = 0.0f;
    uint64_t best = 0;
#define RT_BF16_CONSUME(w)                                                                                  \
    do {                                                                                                    \
        const f32x4 xa = *reinterpret_cast<const f32x4*>(lds + ((((cp << 1) + 0) << 6) + lane) * 16);       \
        const f32x4 xb = *reinterpret_cast<const f32x4*>(lds + ((((cp << 1) + 1) << 6) + lane) * 16);       \
        float a = acc;                                                                                      \
        a = __builtin_fmaf(bf16_lo_to_f32((w)[0]), xa[0], a);                                               \
        a = __builtin_fmaf(bf16_hi_to_f32((w)[0]), xa[1], a);                                               \
        a = __builtin_fmaf(bf16_lo_to_f32((w)[1]), xa[2], a);                                               \
        a = __builtin_fmaf(bf16_hi_to_f32((w)[1]), xa[3], a);                                               \
        a = __builtin_fmaf(bf16_lo_to_f32((w)[2]), xb[0], a);                                               \
        a = __builtin_fmaf(bf16_hi_to_f32((w)[2]), xb[1], a);                                               \
        a = __builtin_fmaf(bf16_lo_to_f32((w)[3]), xb[2], a);                                               \
        a = __builtin_fmaf(bf16_hi_to_f32((w)[3]), xb[3], a);                                               \
        acc = a;                                                                                            \
        if (cp == P - 1) {                                                                                  \
            const float v = wave_sum(acc, lane);                                                            \
            res = lane == cr ? v : res;                                                                     \
            if constexpr (ARGMAX) {                                                                         \
                /* the key of the value stored (scaled by the norm's rms_inv, the same product) */          \
                const float fv = kNorm ? v * out_scale : v;                                                 \
                if (fv == fv) {                                                                             \
                    const uint64_t kk = argmax_key(fv, static_cast<uint32_t>(gw + cr * NW));                \
                    best = kk > best ? kk : best;                                                           \
                }                                                                                           \
            }                                                                                               \
            acc = 0.0f;                                                                                     \
        }                                                                                                   \
        const bool cwrap = cp == P - 1;                                                                     \
        cp = __builtin_amdgcn_readfirstlane(cwrap ? 0 : cp + 1);                                            \
        cr = __builtin_amdgcn_readfirstlane(cwrap ? cr + 1 : cr);                                           \
    } while (0)

    // Steady rounds (straight-line: compute slot j, then refill it with the
    // piece D steps ahead), then the tail of the last <= D pieces.
    int i = 0;
    for (; i + D < L; i += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            RT_BF16_CONSUME(ring[j]);
            __builtin_amdgcn_sched_barrier(0);
            const int64_t o = static_cast<int64_t>(ip) * (kPiece * 2);
            ring[j] = ld16(make_rsrc(wb + ir * stride + o, ir < R ? rowb - o : 0), loff);
            const bool wrap = ip == P - 1;
            ip = __builtin_amdgcn_readfirstlane(wrap ? 0 : ip + 1);
            ir = __builtin_amdgcn_readfirstlane(wrap ? ir + 1 : ir);
        }
    }
#pragma unroll
    for (int j = 0; j < D; ++j)
        if (i + j < L) RT_BF16_CONSUME(ring[j]);
#undef RT_BF16_CONSUME

    if (lane < R) {
        const float out = kNorm ? res * out_scale : res;
        Yg[gw + lane * NW] = ADD ? y_old + out : out;
    }
    if constexpr (ARGMAX) {
        // the wave's best key (0: no row) into slot `wave` of the caller's
        // per-workgroup array (LDS), which the caller folds
        if (lane == 0) key[wave] = best;
    }
}


}  // namespace bf16_gemv
}  // namespace rt_hip
