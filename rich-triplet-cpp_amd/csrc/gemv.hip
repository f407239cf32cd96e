// gemv.hip -- decode GEMV (M <= 8 activation rows) for Q4_K, GGUF Q4_0 and
// BF16 weights on gfx950.
//
// y[m, n] = sum_k x[m, k] * W[n, k]
//
// Work decomposition (all three formats):
//  * A "piece" is the unit one lane loads per weight row: 16 bytes of Q4_K
//    qs (32 nibbles) plus its block header, 144 bytes of Q4_0 (8 blocks), or
//    16 bytes of BF16 (8 values).
//  * A row is split over L lanes (L = the largest power of two <= 64 that
//    divides the row's piece count), so each lane owns a fixed set of piece
//    positions for the whole kernel: its Q4_K sub-block selector and its
//    activation offsets are lane constants.  A wave covers R = 64/L row
//    segments, and each lane carries P rows (P independent accumulators),
//    so one activation read from LDS feeds P rows.
//  * x[M, K] is staged in LDS once per workgroup (with the sum of every
//    16-value group, which the Q4_K/Q4_0 min/offset terms need).  The first
//    piece's weight loads are issued before staging, and every iteration
//    issues the next piece's loads before computing the current one (two
//    register sets used alternately), so HBM requests stay in flight.
//  * Rows are reduced across their L lanes with xor butterflies.
//
// Numerics: f32 FMA accumulation; the reduction order differs from the
// reference's sequential dot_row (quant_q4k.cpp:489-522, mat.cpp:310-314),
// so results agree to f32 rounding, not bit-for-bit.
#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

// x[M*K] into LDS; then sums of each 16-value group (M*K/16 of them).
template <int M, bool SUMS>
__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ X, int K) {
    const int n4 = M * K / 4;
    for (int i = threadIdx.x; i < n4; i += kBlock)
        reinterpret_cast<f32x4*>(xs)[i] = reinterpret_cast<const f32x4*>(X)[i];
    __syncthreads();
    if constexpr (SUMS) {
        float* xsum = xs + M * K;
        const int ng = M * K / 16;
        for (int i = threadIdx.x; i < ng; i += kBlock) {
            const float* p = xs + 16 * i;
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) s += p[j];
            xsum[i] = s;
        }
        __syncthreads();
    }
}

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    // Order-preserving map of f32 to u32 (with -0 folded onto +0), index in
    // the low half inverted so the lowest index wins ties under max.
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<uint64_t>(u) << 32) | (0xffffffffu - idx);
}

// ---------------------------------------------------------------- Q4_K --

template <int P>
struct Q4kRegs {
    u32x4 q[P];
    u32x4 h[P];
};

template <int L, int P, int M>
__global__ __launch_bounds__(kBlock) void k_gemv_q4k(const uint8_t* __restrict__ W,
                                                     const float* __restrict__ X,
                                                     float* __restrict__ Y, int N, int K) {
    extern __shared__ float lds[];
    constexpr int R = kWave / L;
    constexpr int RG = R * P;
    const int lane = threadIdx.x & (kWave - 1);
    const int li = lane & (L - 1);
    const int seg = lane / L;
    const int nb = K >> 8;
    const int S = (nb * 8) / L;
    const int G = (N + RG - 1) / RG;
    const int nwaves = gridDim.x * kWavesPerBlock;
    int g = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);

    // Lane constants: piece p of every block it visits (L is a multiple of 8).
    const int p = li & 7, c = p >> 1, h = p & 1;
    const size_t row_bytes = static_cast<size_t>(nb) * kQ4kBlockBytes;
    const uint8_t* Wl = W + static_cast<size_t>(li >> 3) * kQ4kBlockBytes;
    const size_t t_stride = static_cast<size_t>(L / 8) * kQ4kBlockBytes;
    const int qoff = 16 + 16 * p;

    auto issue = [&](int gg, int tt, Q4kRegs<P>& r) {
        const uint8_t* base = Wl + static_cast<size_t>(tt) * t_stride;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            int row = gg * RG + i * R + seg;
            row = row < N ? row : N - 1;
            const uint8_t* bp = base + static_cast<size_t>(row) * row_bytes;
            r.h[i] = ld16(bp);
            r.q[i] = ld16(bp + qoff);
        }
    };

    Q4kRegs<P> A, B;
    if (g < G) issue(g, 0, A);
    stage_x<M, true>(lds, X, K);
    if (g >= G) return;
    const float* xs = lds;
    const float* xsum = lds + M * K;

    const ScaleSel sel1 = make_scale_sel(2 * c), sel2 = make_scale_sel(2 * c + 1);
    float acc[P][M];
#pragma unroll
    for (int i = 0; i < P; ++i)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[i][m] = 0.0f;

    int t = 0;
    // One piece: compute from `cur`, prefetch into `nxt`.  Returns false when
    // the wave has no further piece.
    auto step = [&](Q4kRegs<P>& cur, Q4kRegs<P>& nxt) -> bool {
        int gn = g, tn = t + 1;
        if (tn == S) {
            tn = 0;
            gn = g + nwaves;
        }
        const bool more = gn < G;
        if (more) issue(gn, tn, nxt);

        float s1[P], n1[P], s2[P], n2[P];
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const float d = f16_bits_to_f32(cur.h[i][0] & 0xffffu);
            const float dm = f16_bits_to_f32(cur.h[i][0] >> 16);
            uint32_t sv1, mv1, sv2, mv2;
            decode_scale_min(sel1, cur.h[i][1], cur.h[i][2], cur.h[i][3], sv1, mv1);
            decode_scale_min(sel2, cur.h[i][1], cur.h[i][2], cur.h[i][3], sv2, mv2);
            s1[i] = d * static_cast<float>(sv1);
            n1[i] = dm * static_cast<float>(mv1);
            // High nibbles are converted as 16*q (mask 0xF0): fold the exact
            // 1/16 into the scale.
            s2[i] = (d * static_cast<float>(sv2)) * 0.0625f;
            n2[i] = dm * static_cast<float>(mv2);
        }
        const int b = (li >> 3) + (L / 8) * t;
        const int xo = b * 256 + c * 64 + h * 16;
        const int go = xo >> 4;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float* xm = xs + m * K + xo;
            f32x4 xl[4], xh[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xl[j] = reinterpret_cast<const f32x4*>(xm)[j];
                xh[j] = reinterpret_cast<const f32x4*>(xm + 32)[j];
            }
            const float sl = xsum[m * (K >> 4) + go];
            const float sh = xsum[m * (K >> 4) + go + 2];
#pragma unroll
            for (int i = 0; i < P; ++i) {
                float dl = 0.0f, dh = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t wl = cur.q[i][j] & 0x0f0f0f0fu;
                    const uint32_t wh = cur.q[i][j] & 0xf0f0f0f0u;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dl = __builtin_fmaf(ubyte_f32(wl, e), xl[j][e], dl);
                        dh = __builtin_fmaf(ubyte_f32(wh, e), xh[j][e], dh);
                    }
                }
                float a = acc[i][m];
                a = __builtin_fmaf(s1[i], dl, a);
                a = __builtin_fmaf(-n1[i], sl, a);
                a = __builtin_fmaf(s2[i], dh, a);
                a = __builtin_fmaf(-n2[i], sh, a);
                acc[i][m] = a;
            }
        }
        if (tn == 0) {
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int row = g * RG + i * R + seg;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float v = segment_sum<L>(acc[i][m]);
                    if (li == 0 && row < N) Y[static_cast<size_t>(m) * N + row] = v;
                    acc[i][m] = 0.0f;
                }
            }
        }
        g = gn;
        t = tn;
        return more;
    };

    for (;;) {
        if (!step(A, B)) break;
        if (!step(B, A)) break;
    }
}

// ---------------------------------------------------------------- BF16 --

template <int P>
struct Bf16Regs {
    u32x4 w[P];
};

template <int L, int P, int M, bool ARGMAX>
__global__ __launch_bounds__(kBlock) void k_gemv_bf16(const uint16_t* __restrict__ W,
                                                      const float* __restrict__ X,
                                                      float* __restrict__ Y, int N, int K,
                                                      uint64_t* __restrict__ key_out) {
    extern __shared__ float lds[];
    constexpr int R = kWave / L;
    constexpr int RG = R * P;
    const int lane = threadIdx.x & (kWave - 1);
    const int li = lane & (L - 1);
    const int seg = lane / L;
    const int S = (K / 8) / L;
    const int G = (N + RG - 1) / RG;
    const int nwaves = gridDim.x * kWavesPerBlock;
    int g = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const uint16_t* Wl = W + 8 * li;

    auto issue = [&](int gg, int tt, Bf16Regs<P>& r) {
        const uint16_t* base = Wl + static_cast<size_t>(tt) * (8 * L);
#pragma unroll
        for (int i = 0; i < P; ++i) {
            int row = gg * RG + i * R + seg;
            row = row < N ? row : N - 1;
            r.w[i] = ld16(base + static_cast<size_t>(row) * K);
        }
    };

    Bf16Regs<P> A, B;
    if (g < G) issue(g, 0, A);
    stage_x<M, false>(lds, X, K);
    uint64_t best = 0;
    if (g < G) {
        const float* xs = lds;
        float acc[P][M];
#pragma unroll
        for (int i = 0; i < P; ++i)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[i][m] = 0.0f;
        int t = 0;
        auto step = [&](Bf16Regs<P>& cur, Bf16Regs<P>& nxt) -> bool {
            int gn = g, tn = t + 1;
            if (tn == S) {
                tn = 0;
                gn = g + nwaves;
            }
            const bool more = gn < G;
            if (more) issue(gn, tn, nxt);
            const int xo = 8 * (li + L * t);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const f32x4 x0 = reinterpret_cast<const f32x4*>(xs + m * K + xo)[0];
                const f32x4 x1 = reinterpret_cast<const f32x4*>(xs + m * K + xo)[1];
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    float a = acc[i][m];
                    a = __builtin_fmaf(bf16_lo_to_f32(cur.w[i][0]), x0[0], a);
                    a = __builtin_fmaf(bf16_hi_to_f32(cur.w[i][0]), x0[1], a);
                    a = __builtin_fmaf(bf16_lo_to_f32(cur.w[i][1]), x0[2], a);
                    a = __builtin_fmaf(bf16_hi_to_f32(cur.w[i][1]), x0[3], a);
                    a = __builtin_fmaf(bf16_lo_to_f32(cur.w[i][2]), x1[0], a);
                    a = __builtin_fmaf(bf16_hi_to_f32(cur.w[i][2]), x1[1], a);
                    a = __builtin_fmaf(bf16_lo_to_f32(cur.w[i][3]), x1[2], a);
                    a = __builtin_fmaf(bf16_hi_to_f32(cur.w[i][3]), x1[3], a);
                    acc[i][m] = a;
                }
            }
            if (tn == 0) {
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    const int row = g * RG + i * R + seg;
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const float v = segment_sum<L>(acc[i][m]);
                        if (li == 0 && row < N) {
                            Y[static_cast<size_t>(m) * N + row] = v;
                            if constexpr (ARGMAX) {
                                if (v == v) {
                                    const uint64_t kk = argmax_key(v, static_cast<uint32_t>(row));
                                    best = kk > best ? kk : best;
                                }
                            }
                        }
                        acc[i][m] = 0.0f;
                    }
                }
            }
            g = gn;
            t = tn;
            return more;
        };
        for (;;) {
            if (!step(A, B)) break;
            if (!step(B, A)) break;
        }
    }
    if constexpr (ARGMAX) {
#pragma unroll
        for (int off = kWave / 2; off >= 1; off >>= 1) {
            const uint64_t o = __shfl_xor(best, off, kWave);
            best = o > best ? o : best;
        }
        if (lane == 0 && best != 0) atomicMax(reinterpret_cast<unsigned long long*>(key_out),
                                              static_cast<unsigned long long>(best));
    }
}

// ---------------------------------------------------------------- Q4_0 --
// Piece = 8 GGUF blocks = 144 bytes = 256 values, loaded as 9 x 16 bytes.

template <int P>
struct Q40Regs {
    u32x4 w[P][9];
};

template <int L, int P, int M>
__global__ __launch_bounds__(kBlock) void k_gemv_q4_0(const uint8_t* __restrict__ W,
                                                      const float* __restrict__ X,
                                                      float* __restrict__ Y, int N, int K) {
    extern __shared__ float lds[];
    constexpr int R = kWave / L;
    constexpr int RG = R * P;
    const int lane = threadIdx.x & (kWave - 1);
    const int li = lane & (L - 1);
    const int seg = lane / L;
    const int nb = K >> 8;  // pieces per row
    const int S = nb / L;
    const int G = (N + RG - 1) / RG;
    const int nwaves = gridDim.x * kWavesPerBlock;
    int g = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const size_t row_bytes = static_cast<size_t>(nb) * 144;
    const uint8_t* Wl = W + static_cast<size_t>(li) * 144;

    auto issue = [&](int gg, int tt, Q40Regs<P>& r) {
        const uint8_t* base = Wl + static_cast<size_t>(tt) * (144 * L);
#pragma unroll
        for (int i = 0; i < P; ++i) {
            int row = gg * RG + i * R + seg;
            row = row < N ? row : N - 1;
            const uint8_t* bp = base + static_cast<size_t>(row) * row_bytes;
#pragma unroll
            for (int j = 0; j < 9; ++j) r.w[i][j] = ld16(bp + 16 * j);
        }
    };

    Q40Regs<P> A, B;
    if (g < G) issue(g, 0, A);
    stage_x<M, true>(lds, X, K);
    if (g >= G) return;
    const float* xs = lds;
    const float* xsum = lds + M * K;
    float acc[P][M];
#pragma unroll
    for (int i = 0; i < P; ++i)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[i][m] = 0.0f;
    int t = 0;

    auto dw = [](const Q40Regs<P>& r, int i, int d) -> uint32_t { return r.w[i][d >> 2][d & 3]; };

    auto step = [&](Q40Regs<P>& cur, Q40Regs<P>& nxt) -> bool {
        int gn = g, tn = t + 1;
        if (tn == S) {
            tn = 0;
            gn = g + nwaves;
        }
        const bool more = gn < G;
        if (more) issue(gn, tn, nxt);
        const int kb = 256 * (li + L * t);
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) {
            // Block blk: d at byte 18*blk, qs at byte 18*blk + 2.
            const int ob = 18 * blk;
            float d[P];
            uint32_t q[P][4];
#pragma unroll
            for (int i = 0; i < P; ++i) {
                d[i] = f16_bits_to_f32((dw(cur, i, ob >> 2) >> (8 * (ob & 3))) & 0xffffu);
                const int oq = ob + 2;
                if ((oq & 3) == 0) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) q[i][j] = dw(cur, i, (oq >> 2) + j);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        q[i][j] = __builtin_amdgcn_alignbyte(dw(cur, i, (oq >> 2) + j + 1),
                                                             dw(cur, i, (oq >> 2) + j), 2);
                }
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float* xm = xs + m * K + kb + 32 * blk;
                f32x4 xl[4], xh[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    xl[j] = reinterpret_cast<const f32x4*>(xm)[j];
                    xh[j] = reinterpret_cast<const f32x4*>(xm + 16)[j];
                }
                const int go = m * (K >> 4) + ((kb + 32 * blk) >> 4);
                const float s32 = xsum[go] + xsum[go + 1];
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    float dot = 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t wl = q[i][j] & 0x0f0f0f0fu;
                        const uint32_t wh = (q[i][j] >> 4) & 0x0f0f0f0fu;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            dot = __builtin_fmaf(ubyte_f32(wl, e), xl[j][e], dot);
                            dot = __builtin_fmaf(ubyte_f32(wh, e), xh[j][e], dot);
                        }
                    }
                    // w = (q - 8) * d  =>  sum w*x = d * (sum q*x - 8 * sum x)
                    acc[i][m] = __builtin_fmaf(d[i], __builtin_fmaf(-8.0f, s32, dot), acc[i][m]);
                }
            }
        }
        if (tn == 0) {
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int row = g * RG + i * R + seg;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float v = segment_sum<L>(acc[i][m]);
                    if (li == 0 && row < N) Y[static_cast<size_t>(m) * N + row] = v;
                    acc[i][m] = 0.0f;
                }
            }
        }
        g = gn;
        t = tn;
        return more;
    };
    for (;;) {
        if (!step(A, B)) break;
        if (!step(B, A)) break;
    }
}

// ------------------------------------------------------------ launchers --

int lowbit_pow2_capped(int64_t v, int cap) {
    int l = 1;
    while (l < cap && (v % (2 * l)) == 0) l *= 2;
    return l;
}

int pick_p(int64_t n, int R, int cus, int pmax) {
    const int64_t target = static_cast<int64_t>(cus) * 8;
    if (pmax >= 4 && (n + 4 * R - 1) / (4 * R) >= target) return 4;
    if (pmax >= 2 && (n + 2 * R - 1) / (2 * R) >= target) return 2;
    return 1;
}

dim3 grid_for(int64_t n, int rows_per_wave, int cus) {
    const int64_t waves = (n + rows_per_wave - 1) / rows_per_wave;
    int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
    const int64_t cap = static_cast<int64_t>(cus) * 8;
    if (blocks > cap) blocks = cap;
    return dim3(static_cast<unsigned>(blocks));
}

template <int L, int P, int M>
hipError_t run_q4k(const void* w, const float* x, float* y, int64_t n, int64_t k, hipStream_t s) {
    const size_t lds = gemv_lds_bytes(RT_HIP_Q4K, M, k);
    const dim3 grid = grid_for(n, (kWave / L) * P, device_info().cus);
    hipLaunchKernelGGL((k_gemv_q4k<L, P, M>), grid, dim3(kBlock), lds, s,
                       static_cast<const uint8_t*>(w), x, y, static_cast<int>(n),
                       static_cast<int>(k));
    return hipGetLastError();
}

template <int L, int P, int M, bool AM>
hipError_t run_bf16(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                    uint64_t* key, hipStream_t s) {
    const size_t lds = gemv_lds_bytes(RT_HIP_BF16, M, k);
    const dim3 grid = grid_for(n, (kWave / L) * P, device_info().cus);
    hipLaunchKernelGGL((k_gemv_bf16<L, P, M, AM>), grid, dim3(kBlock), lds, s, w, x, y,
                       static_cast<int>(n), static_cast<int>(k), key);
    return hipGetLastError();
}

template <int L, int P, int M>
hipError_t run_q40(const void* w, const float* x, float* y, int64_t n, int64_t k, hipStream_t s) {
    const size_t lds = gemv_lds_bytes(RT_HIP_Q4_0, M, k);
    const dim3 grid = grid_for(n, (kWave / L) * P, device_info().cus);
    hipLaunchKernelGGL((k_gemv_q4_0<L, P, M>), grid, dim3(kBlock), lds, s,
                       static_cast<const uint8_t*>(w), x, y, static_cast<int>(n),
                       static_cast<int>(k));
    return hipGetLastError();
}

template <int L>
hipError_t q4k_for_l(const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                     hipStream_t s) {
    if (m == 1) {
        const int p = pick_p(n, kWave / L, device_info().cus, 4);
        if (p == 4) return run_q4k<L, 4, 1>(w, x, y, n, k, s);
        if (p == 2) return run_q4k<L, 2, 1>(w, x, y, n, k, s);
        return run_q4k<L, 1, 1>(w, x, y, n, k, s);
    }
    switch (m) {
        case 2: return run_q4k<L, 1, 2>(w, x, y, n, k, s);
        case 3: return run_q4k<L, 1, 3>(w, x, y, n, k, s);
        case 4: return run_q4k<L, 1, 4>(w, x, y, n, k, s);
        case 5: return run_q4k<L, 1, 5>(w, x, y, n, k, s);
        case 6: return run_q4k<L, 1, 6>(w, x, y, n, k, s);
        case 7: return run_q4k<L, 1, 7>(w, x, y, n, k, s);
        case 8: return run_q4k<L, 1, 8>(w, x, y, n, k, s);
        default: return hipErrorInvalidValue;
    }
}

template <int L>
hipError_t bf16_for_l(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k, int m,
                      uint64_t* key, hipStream_t s) {
    if (m == 1) {
        const int p = pick_p(n, kWave / L, device_info().cus, 4);
        if (key) {
            if (p == 4) return run_bf16<L, 4, 1, true>(w, x, y, n, k, key, s);
            if (p == 2) return run_bf16<L, 2, 1, true>(w, x, y, n, k, key, s);
            return run_bf16<L, 1, 1, true>(w, x, y, n, k, key, s);
        }
        if (p == 4) return run_bf16<L, 4, 1, false>(w, x, y, n, k, nullptr, s);
        if (p == 2) return run_bf16<L, 2, 1, false>(w, x, y, n, k, nullptr, s);
        return run_bf16<L, 1, 1, false>(w, x, y, n, k, nullptr, s);
    }
    switch (m) {
        case 2: return run_bf16<L, 1, 2, false>(w, x, y, n, k, nullptr, s);
        case 3: return run_bf16<L, 1, 3, false>(w, x, y, n, k, nullptr, s);
        case 4: return run_bf16<L, 1, 4, false>(w, x, y, n, k, nullptr, s);
        case 5: return run_bf16<L, 1, 5, false>(w, x, y, n, k, nullptr, s);
        case 6: return run_bf16<L, 1, 6, false>(w, x, y, n, k, nullptr, s);
        case 7: return run_bf16<L, 1, 7, false>(w, x, y, n, k, nullptr, s);
        case 8: return run_bf16<L, 1, 8, false>(w, x, y, n, k, nullptr, s);
        default: return hipErrorInvalidValue;
    }
}

template <int L>
hipError_t q40_for_l(const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                     hipStream_t s) {
    if (m == 1) {
        const int p = pick_p(n, kWave / L, device_info().cus, 2);
        if (p >= 2) return run_q40<L, 2, 1>(w, x, y, n, k, s);
        return run_q40<L, 1, 1>(w, x, y, n, k, s);
    }
    switch (m) {
        case 2: return run_q40<L, 1, 2>(w, x, y, n, k, s);
        case 3: return run_q40<L, 1, 3>(w, x, y, n, k, s);
        case 4: return run_q40<L, 1, 4>(w, x, y, n, k, s);
        case 5: return run_q40<L, 1, 5>(w, x, y, n, k, s);
        case 6: return run_q40<L, 1, 6>(w, x, y, n, k, s);
        case 7: return run_q40<L, 1, 7>(w, x, y, n, k, s);
        case 8: return run_q40<L, 1, 8>(w, x, y, n, k, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

size_t gemv_lds_bytes(int fmt, int m, int64_t k) {
    const size_t xs = static_cast<size_t>(m) * static_cast<size_t>(k) * 4;
    return fmt == RT_HIP_BF16 ? xs : xs + xs / 16;
}

hipError_t launch_gemv_q4k(const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                           hipStream_t s) {
    const int l = lowbit_pow2_capped((k / 256) * 8, kWave);
    switch (l) {
        case 8: return q4k_for_l<8>(w, x, y, n, k, m, s);
        case 16: return q4k_for_l<16>(w, x, y, n, k, m, s);
        case 32: return q4k_for_l<32>(w, x, y, n, k, m, s);
        default: return q4k_for_l<64>(w, x, y, n, k, m, s);
    }
}

hipError_t launch_gemv_bf16(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                            int m, uint64_t* key, hipStream_t s) {
    const int l = lowbit_pow2_capped(k / 8, kWave);
    switch (l) {
        case 1: return bf16_for_l<1>(w, x, y, n, k, m, key, s);
        case 2: return bf16_for_l<2>(w, x, y, n, k, m, key, s);
        case 4: return bf16_for_l<4>(w, x, y, n, k, m, key, s);
        case 8: return bf16_for_l<8>(w, x, y, n, k, m, key, s);
        case 16: return bf16_for_l<16>(w, x, y, n, k, m, key, s);
        case 32: return bf16_for_l<32>(w, x, y, n, k, m, key, s);
        default: return bf16_for_l<64>(w, x, y, n, k, m, key, s);
    }
}

hipError_t launch_gemv_q4_0(const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                            hipStream_t s) {
    const int l = lowbit_pow2_capped(k / 256, kWave);
    switch (l) {
        case 1: return q40_for_l<1>(w, x, y, n, k, m, s);
        case 2: return q40_for_l<2>(w, x, y, n, k, m, s);
        case 4: return q40_for_l<4>(w, x, y, n, k, m, s);
        case 8: return q40_for_l<8>(w, x, y, n, k, m, s);
        case 16: return q40_for_l<16>(w, x, y, n, k, m, s);
        case 32: return q40_for_l<32>(w, x, y, n, k, m, s);
        default: return q40_for_l<64>(w, x, y, n, k, m, s);
    }
}

}  // namespace rt_hip
