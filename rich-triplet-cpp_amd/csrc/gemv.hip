// gemv.hip -- decode GEMV (M <= 8 activation rows) for Q4_K, GGUF Q4_0 and
// BF16 weights on gfx950.
//
// y[m, n] = sum_k x[m, k] * W[n, k]
//
// Work decomposition (all three formats share one pipelined driver):
//  * A "piece" is what one lane loads per weight row per step: 16 bytes of
//    Q4_K qs (32 nibbles) plus the 16-byte header of its super-block, 144
//    bytes of GGUF Q4_0 (8 blocks, 256 values), or 16 bytes of BF16 (8
//    values).
//  * A row is split over L lanes (L = the largest power of two <= 64 that
//    divides the row's piece count), so each lane owns fixed piece
//    positions for the whole kernel: its Q4_K sub-block selector and its
//    activation offsets are lane constants.  A wave covers R = 64/L row
//    segments and each lane carries P rows, so one activation read from LDS
//    feeds P rows.  A "row group" is the R*P rows a wave computes together.
//  * Software pipeline: a ring of D register slots, each holding one piece
//    for P rows.  The loads for the first D pieces are issued before x is
//    staged, and every computed slot is immediately refilled with the piece
//    D steps ahead (walking row groups g = wave, wave + nwaves, ...), so each
//    wave keeps D*P pieces of HBM traffic in flight at all times.
//  * x[M, K] is staged in LDS once per workgroup, with the sum of every
//    16-value group (the Q4_K min term and the Q4_0 offset term need it).
//  * Rows are reduced across their L lanes with xor butterflies.
//
// Numerics: f32 FMA accumulation; the order differs from the reference's
// sequential dot_row (quant_q4k.cpp:489-522, mat.cpp:310-314), so results
// agree to f32 rounding, not bit-for-bit.
#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

// ------------------------------------------------------------ formats --

// Q4_K: piece = (block b, 16-byte qs half-chunk p); regs = {header, qs}.
struct Q4kFmt {
    static constexpr int kRegs = 2;
    __host__ __device__ static int pieces_per_row(int K) { return (K >> 8) * 8; }
    __host__ __device__ static size_t row_bytes(int K) {
        return static_cast<size_t>(K >> 8) * kQ4kBlockBytes;
    }
    struct Lane {
        int p, c, h;
        ScaleSel s1, s2;
    };
    __device__ static Lane lane(int li) {
        Lane ln;
        ln.p = li & 7;
        ln.c = ln.p >> 1;
        ln.h = ln.p & 1;
        ln.s1 = make_scale_sel(2 * ln.c);
        ln.s2 = make_scale_sel(2 * ln.c + 1);
        return ln;
    }
    // LDS layout, piece-major so that consecutive lanes read consecutive
    // 16-byte chunks (no bank conflicts): piece s = 8*b + 2*c + h covers the
    // low-nibble values b*256 + 64c + 16h + [0,16) and the high-nibble
    // values 32 later; f32x4 number j (0-3 low, 4-7 high) of piece s of
    // activation row m sits at xs4[(m*8 + j)*NP + s], NP = K/32 pieces.
    // The two 16-value sums of piece s sit at sums2[m*NP + s].
    __host__ __device__ static size_t lds_floats(int M, int K) {
        return static_cast<size_t>(M) * K + static_cast<size_t>(M) * (K / 16);
    }
    template <int M>
    __device__ static void stage(float* lds, const float* __restrict__ X, int K, int tid, int nthr) {
        const int np = K >> 5;
        f32x4* xs4 = reinterpret_cast<f32x4*>(lds);
        for (int f = tid; f < M * K / 4; f += nthr) {
            const int m = f / (K >> 2), k = 4 * (f - m * (K >> 2));
            const int b = k >> 8, w = k & 255, c = w >> 6, r = w & 63;
            const int hi = r >> 5, h = (r >> 4) & 1, q = (r & 15) >> 2;
            xs4[(m * 8 + 4 * hi + q) * np + 8 * b + 2 * c + h] =
                reinterpret_cast<const f32x4*>(X)[f];
        }
        __syncthreads();
        f32x2* sums = reinterpret_cast<f32x2*>(lds + static_cast<size_t>(M) * K);
        for (int e = tid; e < M * np; e += nthr) {
            const int m = e / np, sp = e - m * np;
            float lo = 0.0f, hi = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 a = xs4[(m * 8 + j) * np + sp];
                const f32x4 b = xs4[(m * 8 + 4 + j) * np + sp];
                lo += a[0]; lo += a[1]; lo += a[2]; lo += a[3];
                hi += b[0]; hi += b[1]; hi += b[2]; hi += b[3];
            }
            sums[e] = f32x2{lo, hi};
        }
        __syncthreads();
    }
    template <int L>
    __device__ static int block_of(int li, int t) { return (li >> 3) + (L / 8) * t; }
    template <int L>
    __device__ static void load(const uint8_t* row, int li, int t, const Lane& ln, u32x4* r) {
        const uint8_t* bp = row + static_cast<size_t>(block_of<L>(li, t)) * kQ4kBlockBytes;
        r[0] = ld16(bp);
        r[1] = ld16(bp + 16 + 16 * ln.p);
    }
    template <int L, int P, int M>
    __device__ static void compute(const u32x4 (&v)[P][kRegs], int li, int t, const Lane& ln,
                                   const float* xs, const float* xsum, int K, float (&acc)[P][M]) {
        float s1[P], n1[P], s2[P], n2[P];
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const u32x4 hd = v[i][0];
            const float d = f16_bits_to_f32(hd[0] & 0xffffu);
            const float dm = f16_bits_to_f32(hd[0] >> 16);
            uint32_t sv1, mv1, sv2, mv2;
            decode_scale_min(ln.s1, hd[1], hd[2], hd[3], sv1, mv1);
            decode_scale_min(ln.s2, hd[1], hd[2], hd[3], sv2, mv2);
            s1[i] = d * static_cast<float>(sv1);
            n1[i] = dm * static_cast<float>(mv1);
            // High nibbles are converted as 16*q (mask 0xF0): fold the exact
            // 1/16 into the scale.
            s2[i] = (d * static_cast<float>(sv2)) * 0.0625f;
            n2[i] = dm * static_cast<float>(mv2);
        }
        const int np = K >> 5;
        const int sp = li + L * t;  // this lane's piece index within the row
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const f32x4* xm = reinterpret_cast<const f32x4*>(xs) + m * 8 * np + sp;
            f32x4 xl[4], xh[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xl[j] = xm[j * np];
                xh[j] = xm[(j + 4) * np];
            }
            const f32x2 ss = reinterpret_cast<const f32x2*>(xsum)[m * np + sp];
            const float sl = ss[0], sh = ss[1];
#pragma unroll
            for (int i = 0; i < P; ++i) {
                float dl = 0.0f, dh = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t wl = v[i][1][j] & 0x0f0f0f0fu;
                    const uint32_t wh = v[i][1][j] & 0xf0f0f0f0u;
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
    }
};

// BF16: piece = 8 consecutive values.
struct Bf16Fmt {
    static constexpr int kRegs = 1;
    __host__ __device__ static int pieces_per_row(int K) { return K / 8; }
    __host__ __device__ static size_t row_bytes(int K) { return static_cast<size_t>(K) * 2; }
    // LDS layout: piece s (values 8s..8s+7) of activation row m as two
    // f32x4 at xs4[(m*2 + j)*NP + s], NP = K/8 (consecutive lanes read
    // consecutive 16-byte chunks).
    __host__ __device__ static size_t lds_floats(int M, int K) { return static_cast<size_t>(M) * K; }
    template <int M>
    __device__ static void stage(float* lds, const float* __restrict__ X, int K, int tid, int nthr) {
        const int np = K >> 3;
        f32x4* xs4 = reinterpret_cast<f32x4*>(lds);
        for (int f = tid; f < M * K / 4; f += nthr) {
            const int m = f / (K >> 2), k4 = f - m * (K >> 2);
            xs4[(m * 2 + (k4 & 1)) * np + (k4 >> 1)] = reinterpret_cast<const f32x4*>(X)[f];
        }
        __syncthreads();
    }
    struct Lane {};
    __device__ static Lane lane(int) { return Lane{}; }
    template <int L>
    __device__ static void load(const uint8_t* row, int li, int t, const Lane&, u32x4* r) {
        r[0] = ld16(row + 16 * static_cast<size_t>(li + L * t));
    }
    template <int L, int P, int M>
    __device__ static void compute(const u32x4 (&v)[P][kRegs], int li, int t, const Lane&,
                                   const float* xs, const float*, int K, float (&acc)[P][M]) {
        const int np = K >> 3;
        const int sp = li + L * t;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const f32x4* xm = reinterpret_cast<const f32x4*>(xs) + m * 2 * np + sp;
            const f32x4 x0 = xm[0];
            const f32x4 x1 = xm[np];
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const u32x4 w = v[i][0];
                float a = acc[i][m];
                a = __builtin_fmaf(bf16_lo_to_f32(w[0]), x0[0], a);
                a = __builtin_fmaf(bf16_hi_to_f32(w[0]), x0[1], a);
                a = __builtin_fmaf(bf16_lo_to_f32(w[1]), x0[2], a);
                a = __builtin_fmaf(bf16_hi_to_f32(w[1]), x0[3], a);
                a = __builtin_fmaf(bf16_lo_to_f32(w[2]), x1[0], a);
                a = __builtin_fmaf(bf16_hi_to_f32(w[2]), x1[1], a);
                a = __builtin_fmaf(bf16_lo_to_f32(w[3]), x1[2], a);
                a = __builtin_fmaf(bf16_hi_to_f32(w[3]), x1[3], a);
                acc[i][m] = a;
            }
        }
    }
};

// GGUF Q4_0: piece = 8 blocks = 144 bytes = 256 values, 9 x 16-byte loads.
struct Q40Fmt {
    static constexpr int kRegs = 9;
    __host__ __device__ static int pieces_per_row(int K) { return K >> 8; }
    __host__ __device__ static size_t row_bytes(int K) { return static_cast<size_t>(K >> 8) * 144; }
    // LDS layout: piece s (values 256s..256s+255) of activation row m as 64
    // f32x4 at xs4[(m*64 + j)*NP + s], NP = K/256; the sum of each 32-value
    // block blk of piece s at sums[(m*8 + blk)*NP + s].
    __host__ __device__ static size_t lds_floats(int M, int K) { return static_cast<size_t>(M) * K * 33 / 32; }
    template <int M>
    __device__ static void stage(float* lds, const float* __restrict__ X, int K, int tid, int nthr) {
        const int np = K >> 8;
        f32x4* xs4 = reinterpret_cast<f32x4*>(lds);
        for (int f = tid; f < M * K / 4; f += nthr) {
            const int m = f / (K >> 2), k4 = f - m * (K >> 2);
            xs4[(m * 64 + (k4 & 63)) * np + (k4 >> 6)] = reinterpret_cast<const f32x4*>(X)[f];
        }
        __syncthreads();
        float* sums = lds + static_cast<size_t>(M) * K;
        for (int e = tid; e < M * 8 * np; e += nthr) {
            const int m = e / (8 * np), r = e - m * 8 * np, blk = r / np, sp = r - blk * np;
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const f32x4 a = xs4[(m * 64 + 8 * blk + j) * np + sp];
                acc += a[0]; acc += a[1]; acc += a[2]; acc += a[3];
            }
            sums[e] = acc;
        }
        __syncthreads();
    }
    struct Lane {};
    __device__ static Lane lane(int) { return Lane{}; }
    template <int L>
    __device__ static void load(const uint8_t* row, int li, int t, const Lane&, u32x4* r) {
        const uint8_t* bp = row + 144 * static_cast<size_t>(li + L * t);
#pragma unroll
        for (int j = 0; j < 9; ++j) r[j] = ld16(bp + 16 * j);
    }
    template <int P>
    __device__ static uint32_t dw(const u32x4 (&v)[P][kRegs], int i, int d) {
        return v[i][d >> 2][d & 3];
    }
    template <int L, int P, int M>
    __device__ static void compute(const u32x4 (&v)[P][kRegs], int li, int t, const Lane&,
                                   const float* xs, const float* xsum, int K, float (&acc)[P][M]) {
        const int np = K >> 8;
        const int sp = li + L * t;
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) {
            // Block blk: d (f16) at byte 18*blk, qs[16] at byte 18*blk + 2.
            const int ob = 18 * blk;
            const int oq = ob + 2;
            float d[P];
            uint32_t q[P][4];
#pragma unroll
            for (int i = 0; i < P; ++i) {
                d[i] = f16_bits_to_f32((dw<P>(v, i, ob >> 2) >> (8 * (ob & 3))) & 0xffffu);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if ((oq & 3) == 0)
                        q[i][j] = dw<P>(v, i, (oq >> 2) + j);
                    else
                        q[i][j] = __builtin_amdgcn_alignbyte(dw<P>(v, i, (oq >> 2) + j + 1),
                                                             dw<P>(v, i, (oq >> 2) + j), 2);
                }
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const f32x4* xm = reinterpret_cast<const f32x4*>(xs) + (m * 64 + 8 * blk) * np + sp;
                f32x4 xl[4], xh[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    xl[j] = xm[j * np];
                    xh[j] = xm[(j + 4) * np];
                }
                const float s32 = xsum[(m * 8 + blk) * np + sp];
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
    }
};

// ------------------------------------------------------------- driver --

// Row groups a wave may own: its row sums (RG rows x M) wait in a 256-float
// LDS area per wave until the loop is over, because an output store among
// the ring's loads makes the compiler wait for every load in flight.
template <int RG, int M>
struct ResArea {
    static constexpr int kGroups = 256 / (RG * M) > 0 ? 256 / (RG * M) : 1;
};
constexpr int kResFloatsPerWave = 256;

template <class F, int L, int P, int M, int D, bool ARGMAX>
__global__ __launch_bounds__(kBlock) void k_gemv(const uint8_t* __restrict__ W,
                                                 const float* __restrict__ X,
                                                 float* __restrict__ Y, int N, int K,
                                                 uint64_t* __restrict__ key_out) {
    extern __shared__ float lds[];
    constexpr int R = kWave / L;
    constexpr int RG = R * P;
    const int lane = threadIdx.x & (kWave - 1);
    const int li = lane & (L - 1);
    const int seg = lane / L;
    const int S = F::pieces_per_row(K) / L;
    const int G = (N + RG - 1) / RG;
    const int nwaves = gridDim.x * kWavesPerBlock;
    const int wave = threadIdx.x >> 6;
    const int g0 = blockIdx.x * kWavesPerBlock + wave;
    const size_t rb = F::row_bytes(K);
    const typename F::Lane ln = F::lane(li);
    // This wave's row groups g0, g0 + nwaves, ... (at most
    // ResArea::kGroups: the launcher sizes the grid) and their pieces, as
    // one sequence the ring streams without a break between groups.
    const int Gw = g0 < G ? (G - 1 - g0) / nwaves + 1 : 0;
    const int Ltot = Gw * S;

    u32x4 ring[D][P][F::kRegs];

    // Issue cursor: the next (row group, piece) whose loads go out.  Loads
    // are unconditional (past the wave's groups they re-read row N-1, in
    // bounds): a conditional load would make the compiler merge register
    // versions and drain the pipeline.
    int ig = g0, it = 0;
    auto issue = [&](u32x4 (&slot)[P][F::kRegs]) {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            int row = ig * RG + i * R + seg;
            row = row < N ? row : N - 1;
            F::template load<L>(W + static_cast<size_t>(row) * rb, li, it, ln, slot[i]);
        }
        const bool wrap = it == S - 1;
        it = __builtin_amdgcn_readfirstlane(wrap ? 0 : it + 1);
        ig = __builtin_amdgcn_readfirstlane(wrap ? ig + nwaves : ig);
    };

#pragma unroll
    for (int j = 0; j < D; ++j) {
        issue(ring[j]);
        __builtin_amdgcn_sched_barrier(0);
    }
    F::template stage<M>(lds, X, K, threadIdx.x, kBlock);

    const float* xs = lds;
    const float* xsum = lds + static_cast<size_t>(M) * K;
    float* const res = lds + F::lds_floats(M, K) + wave * kResFloatsPerWave;
    uint64_t best = 0;
    float acc[P][M];
#pragma unroll
    for (int i = 0; i < P; ++i)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[i][m] = 0.0f;
    int ct = 0, cj = 0;  // consume cursor: piece ct of the wave's group cj
    // After a group's last piece: reduce its rows over their L lanes and
    // park the sums in the wave's LDS area.
    auto finish = [&]() {
        if (ct == S - 1 && cj < Gw) {
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int r = i * R + seg;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float val = segment_sum<L>(acc[i][m]);
                    acc[i][m] = 0.0f;
                    if (li == 0) res[(cj * RG + r) * M + m] = val;
                    if constexpr (ARGMAX) {
                        const int row = (g0 + cj * nwaves) * RG + r;
                        if (val == val && row < N) {
                            const uint64_t kk = argmax_key(val, static_cast<uint32_t>(row));
                            best = kk > best ? kk : best;
                        }
                    }
                }
            }
        }
        const bool wrap = ct == S - 1;
        ct = __builtin_amdgcn_readfirstlane(wrap ? 0 : ct + 1);
        cj = __builtin_amdgcn_readfirstlane(wrap ? cj + 1 : cj);
    };

    // Straight-line rounds: compute slot j, refill it D pieces ahead.  The
    // last round may run past the wave's pieces: those computes land in a
    // group the wave does not own and finish() drops them, and the loads
    // re-read row N-1 -- cheaper than a tail, which the compiler would
    // specialise into a second copy of the body with its own registers.
    for (int i0 = 0; i0 < Ltot; i0 += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            F::template compute<L, P, M>(ring[j], li, ct, ln, xs, xsum, K, acc);
            __builtin_amdgcn_sched_barrier(0);
            issue(ring[j]);
            finish();
        }
    }

    // The wave's sums, written out by all its lanes.
    for (int idx = lane; idx < Gw * RG * M; idx += kWave) {
        const int j = idx / (RG * M), rem = idx - j * (RG * M);
        const int r = rem / M, m = rem - r * M;
        const int row = (g0 + j * nwaves) * RG + r;
        if (row < N) Y[static_cast<size_t>(m) * N + row] = res[idx];
    }
    if constexpr (ARGMAX) {
#pragma unroll
        for (int off = kWave / 2; off >= 1; off >>= 1) {
            const uint64_t o = __shfl_xor(best, off, kWave);
            best = o > best ? o : best;
        }
        if (lane == 0 && best != 0)
            atomicMax(reinterpret_cast<unsigned long long*>(key_out),
                      static_cast<unsigned long long>(best));
    }
}

// ------------------------------------------------------------ launchers --

int lowbit_pow2_capped(int64_t v, int cap) {
    int l = 1;
    while (l < cap && (v % (2 * l)) == 0) l *= 2;
    return l;
}

// Rows per lane: more rows per lane shares activation reads and deepens the
// pipeline, but needs enough row groups to occupy every SIMD.
int pick_p(int64_t n, int R, int cus, int pmax) {
    const int64_t target = static_cast<int64_t>(cus) * 8;
    if (pmax >= 4 && (n + 4 * R - 1) / (4 * R) >= target) return 4;
    if (pmax >= 2 && (n + 2 * R - 1) / (2 * R) >= target) return 2;
    return 1;
}

template <class F, int L, int P, int M, int D, bool AM>
hipError_t run(const void* w, const float* x, float* y, int64_t n, int64_t k, uint64_t* key,
               hipStream_t s, int fmt) {
    constexpr int RG = (kWave / L) * P;
    const size_t lds = gemv_lds_bytes(fmt, M, k);
    const int64_t groups = (n + RG - 1) / RG;
    int64_t blocks = (groups + kWavesPerBlock - 1) / kWavesPerBlock;
    const int64_t cap = static_cast<int64_t>(device_info().cus) * 4;
    if (blocks > cap) blocks = cap;
    // No wave may own more row groups than its result area holds.
    constexpr int64_t gpw = ResArea<RG, M>::kGroups;
    const int64_t need = (groups + gpw * kWavesPerBlock - 1) / (gpw * kWavesPerBlock);
    if (blocks < need) blocks = need;
    hipLaunchKernelGGL((k_gemv<F, L, P, M, D, AM>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kBlock), lds, s, static_cast<const uint8_t*>(w), x, y,
                       static_cast<int>(n), static_cast<int>(k), key);
    return hipGetLastError();
}

// Per-format pipeline depth (pieces in flight per slot ring) for M == 1.
template <class F> struct Depth;
template <> struct Depth<Q4kFmt> { static constexpr int D = 4; };
template <> struct Depth<Bf16Fmt> { static constexpr int D = 8; };
template <> struct Depth<Q40Fmt> { static constexpr int D = 2; };

template <class F, int L, bool AM>
hipError_t for_l(const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                 uint64_t* key, hipStream_t s, int fmt) {
    constexpr int D = Depth<F>::D;
    constexpr int DB = D > 2 ? D / 2 : D;  // batched rows carry M accumulators
    constexpr int PMAX = F::kRegs > 2 ? 1 : (F::kRegs == 2 ? 2 : 4);
    if (m == 1) {
        const int p = pick_p(n, kWave / L, device_info().cus, PMAX);
        if constexpr (AM) {
            if (key) {
                if (p == 4) return run<F, L, 4, 1, D, true>(w, x, y, n, k, key, s, fmt);
                if (p == 2) return run<F, L, 2, 1, D, true>(w, x, y, n, k, key, s, fmt);
                return run<F, L, 1, 1, D, true>(w, x, y, n, k, key, s, fmt);
            }
        }
        if constexpr (PMAX >= 4)
            if (p == 4) return run<F, L, 4, 1, D, false>(w, x, y, n, k, key, s, fmt);
        if constexpr (PMAX >= 2)
            if (p == 2) return run<F, L, 2, 1, D, false>(w, x, y, n, k, key, s, fmt);
        return run<F, L, 1, 1, D, false>(w, x, y, n, k, key, s, fmt);
    }
    switch (m) {
        case 2: return run<F, L, 1, 2, DB, false>(w, x, y, n, k, nullptr, s, fmt);
        case 3: return run<F, L, 1, 3, DB, false>(w, x, y, n, k, nullptr, s, fmt);
        case 4: return run<F, L, 1, 4, DB, false>(w, x, y, n, k, nullptr, s, fmt);
        case 5: return run<F, L, 1, 5, DB, false>(w, x, y, n, k, nullptr, s, fmt);
        case 6: return run<F, L, 1, 6, DB, false>(w, x, y, n, k, nullptr, s, fmt);
        case 7: return run<F, L, 1, 7, DB, false>(w, x, y, n, k, nullptr, s, fmt);
        case 8: return run<F, L, 1, 8, DB, false>(w, x, y, n, k, nullptr, s, fmt);
        default: return hipErrorInvalidValue;
    }
}

template <class F, int LMIN, bool AM>
hipError_t dispatch(const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                    uint64_t* key, hipStream_t s, int fmt) {
    switch (lowbit_pow2_capped(F::pieces_per_row(static_cast<int>(k)), kWave)) {
        case 1: if constexpr (LMIN <= 1) return for_l<F, 1, AM>(w, x, y, n, k, m, key, s, fmt); break;
        case 2: if constexpr (LMIN <= 2) return for_l<F, 2, AM>(w, x, y, n, k, m, key, s, fmt); break;
        case 4: if constexpr (LMIN <= 4) return for_l<F, 4, AM>(w, x, y, n, k, m, key, s, fmt); break;
        case 8: return for_l<F, 8, AM>(w, x, y, n, k, m, key, s, fmt);
        case 16: return for_l<F, 16, AM>(w, x, y, n, k, m, key, s, fmt);
        case 32: return for_l<F, 32, AM>(w, x, y, n, k, m, key, s, fmt);
        default: return for_l<F, 64, AM>(w, x, y, n, k, m, key, s, fmt);
    }
    return hipErrorInvalidValue;
}

}  // namespace

size_t gemv_lds_bytes(int fmt, int m, int64_t k) {
    const int kk = static_cast<int>(k);
    const size_t res = 4 * static_cast<size_t>(kWavesPerBlock) * kResFloatsPerWave;
    switch (fmt) {
        case RT_HIP_Q4K: return 4 * Q4kFmt::lds_floats(m, kk) + res;
        case RT_HIP_BF16: return 4 * Bf16Fmt::lds_floats(m, kk) + res;
        default: return 4 * Q40Fmt::lds_floats(m, kk) + res;
    }
}

hipError_t launch_gemv_q4k(const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                           hipStream_t s) {
    // M == 1 (decode) runs on int8 MFMA; small batches on the VALU kernel.
    if (m == 1 && q4k_m1_lds_bytes(k) <= lds_cap()) return launch_gemv_q4k_mfma(w, x, y, n, k, s);
    // Q4_K pieces per row = 8 * K/256, so L >= 8 always.
    return dispatch<Q4kFmt, 8, false>(w, x, y, n, k, m, nullptr, s, RT_HIP_Q4K);
}

hipError_t launch_gemv_bf16(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                            int m, uint64_t* key, hipStream_t s) {
    // M == 1 (decode, and the fused-argmax lm_head) has its own kernel.
    if (m == 1 && bf16_m1_lds_bytes(k) <= lds_cap()) return launch_gemv_bf16_m1(w, x, y, n, k, key, s);
    return dispatch<Bf16Fmt, 1, true>(w, x, y, n, k, m, key, s, RT_HIP_BF16);
}

hipError_t launch_gemv_q4_0(const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                            hipStream_t s) {
    // M == 1 (decode): whole blocks per lane, rows streamed (gemv_q40.hip).
    if (m == 1 && q40_m1_lds_bytes(k) <= lds_cap() && n <= 64ll * 0x7fffffff / 4)
        return launch_gemv_q4_0_m1(w, x, y, n, k, s);
    return dispatch<Q40Fmt, 1, false>(w, x, y, n, k, m, nullptr, s, RT_HIP_Q4_0);
}

}  // namespace rt_hip
