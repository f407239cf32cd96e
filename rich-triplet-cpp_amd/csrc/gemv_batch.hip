// gemv_batch.hip -- batched GEMV, M = 2..8 activation rows (speculative
// verify): Y[m][n] = sum_k X[m][k] * W[n][k] on MFMA, every weight byte read
// once for all M rows (decode_gemma3.msl:416-518, MAX_BATCH 8).
//
// One MFMA step covers 32 values of K for a 16-row weight tile and up to four
// activation rows t of a group q (Q = ceil(M / 4) groups, one MFMA each):
//  * B is the weight tile: lane l = (n = l%16, g = l/16) supplies the 8
//    weights of row n at k-slots 8g..8g+7 of the step.
//  * A row i = 4t + lambda (lambda < 3; row 4t + 3 is zero) is limb lambda of
//    activation row 4q + t over the same k-slots.
//  * The output lane (n, g) holds C[4g + r][n], r = 0..3: the three limb
//    dots of activation row 4q + g for weight row n, combined in the lane.
//
// Exact activation limbs, so that the MFMA products are exact:
//  * BF16 weights (v_mfma_f32_16x16x32_bf16): three bf16 limbs with
//    h + m + l == x exactly -- h = bf16(x), m = bf16(x - h), l = x - h - m
//    (each difference is exact in f32, the last has at most 8 significant
//    bits).  Products of bf16 values are exact in f32, so only the f32
//    accumulation rounds, as in an f32 dot product.
//  * Q4_K weights (v_mfma_i32_16x16x32_i8): the step is one 32-value
//    sub-block, and x carries the int8 limbs of the M = 1 kernel
//    (q4k_mfma.hpp): per sub-block a power-of-two s and A0 + A1/256 + A2/65536
//    == x / s to 2.5e-7 * absmax.  Each limb dot against the nibbles is an
//    exact int32, and per sub-block j (quant_q4k.cpp:482-523)
//        sum x * w = (d*sv_j) * (s*C0 + s/256*C1 + s/65536*C2) - (dmin*mv_j) * sum(x).
//    Sub-block j's values k = 32j + t sit in byte 32*(j/2) + t of qs, low
//    nibble for even j and high for odd (quant_q4k.cpp:280-317).
//
// Work split.  A workgroup of kWaves waves stages one K-slice of all M rows
// as limbs in LDS and each wave runs one 16-row tile over that slice, its
// weights streamed through a ring of D slots.  LDS bounds the slice, and
// short outputs need several slices to occupy the CUs.  With one slice the
// workgroup writes Y.  With more, every workgroup writes its partial
// products to a workspace and counts its arrival for its tile group; the
// last to arrive adds the group's partials in slice order (so the result
// does not depend on arrival order) and resets the counter.  A slice is
// padded with zero activation steps to whole ring rounds, so the loop has
// no tail: padded steps add exact zeros, and weight loads past the slice's
// real slots get an empty buffer range (zeros, no memory traffic).
#include "q4k_mfma.hpp"
#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kZeroBytes = 16;

// ---- formats -------------------------------------------------------------
// A slot is the unit the ring loads: kSteps 32-value steps of one tile.
// LDS per (step, group): kLimb bytes of A limbs ([g][t][lambda] x kFrag)
// and kCst bytes of per-row constants.

struct BBf16 {
    static constexpr int kSteps = 4;  // 128 values
    static constexpr int kSlotCost = 1;  // one slot's time, in units of one slice's reduction
    static constexpr int kFrag = 16;  // 8 bf16
    static constexpr int kLimb = 48 * kFrag;
    static constexpr int kCst = 0;
    struct Slot { u32x4 v[4]; };
    // The tile's rows start at `tile` (row-major, rb bytes apart); the slot
    // covers values [k, k + 128).  Lane (n, g) reads 16 bytes of row n per
    // step; pieces past K (K % 8 == 0: all or nothing) read zeros.
    __device__ static void load(const uint8_t* tile, int64_t left, int64_t rb, int k, int K, int lane,
                                Slot& s) {
        const BufRsrc rs = make_rsrc(tile + 2 * static_cast<int64_t>(k), left - 2 * static_cast<int64_t>(k));
        const uint32_t roff = static_cast<uint32_t>((lane & 15) * rb);
        const int g = lane >> 4;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const bool in = k + 32 * st + 8 * g < K;
            s.v[st] = ld16(rs, in ? roff + static_cast<uint32_t>(64 * st + 16 * g) : 0xfffffff0u);
        }
    }
};

struct BQ4k {
    static constexpr int kSteps = 8;  // one super-block
    static constexpr int kSlotCost = 2;  // one slot's time, in units of one slice's reduction
    static constexpr int kFrag = 8;   // 8 int8
    static constexpr int kLimb = 48 * kFrag;
    static constexpr int kCst = 64;   // 4 rows x {s, s/256, s/65536, sum}
    struct Slot {
        u32x4 h;      // d | dmin << 16, scales[12]
        u32x2 p[4];   // qs[32c + 8g, +8), c = 0..3
    };
    __device__ static void load(const uint8_t* tile, int64_t left, int64_t rb, int k, int, int lane, Slot& s) {
        const int64_t o = static_cast<int64_t>(k >> 8) * kQ4kBlockBytes;
        const BufRsrc rs = make_rsrc(tile + o, left - o);
        const uint32_t roff = static_cast<uint32_t>((lane & 15) * rb);
        const uint32_t g8 = static_cast<uint32_t>(lane >> 4) * 8u;
        s.h = ld16(rs, roff);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            s.p[c] = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, static_cast<int>(roff + 16u + 32u * c + g8), 0, 0));
    }
};

template <class F>
__host__ __device__ inline size_t batch_lds_bytes(int steps, int q) {
    return static_cast<size_t>(steps) * q * (F::kLimb + F::kCst) + kZeroBytes;
}

// Sum and max over the aligned quad of lanes (every lane gets the same bits).
__device__ __forceinline__ float quad_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false));
    return v;
}
__device__ __forceinline__ float quad_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false)));
    return v;
}

// Partials are stored and reloaded with agent-scope (device-coherent)
// accesses: they bypass the per-XCD L2, so the workgroup that reduces them
// sees every other XCD's stores once those have completed.
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store((__attribute__((address_space(1))) float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load((const __attribute__((address_space(1))) float*)p, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup (blockIdx.x, blockIdx.y) = (group of kWaves tiles, K-slice).
// The slice is `slots` ring slots from slot slice * slots (the last slice may
// hold fewer real ones); `psteps` = slots padded to whole rounds of D, in
// steps, is what LDS holds.  Y is [M][N]; with gridDim.y > 1 slices, P holds
// the partials ([slice][M][N]) and counters[blockIdx.x] the arrivals.
template <class F, int Q, int D, int XP>
__global__ __launch_bounds__(kThreads) void k_gemv_batch(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                         float* __restrict__ Y, float* __restrict__ P,
                                                         uint32_t* __restrict__ counters, int N, int K, int M,
                                                         int slots, int psteps) {
    constexpr bool kQ4 = F::kSteps == 8;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slice = blockIdx.y;
    const int k0 = slice * slots * F::kSteps * 32;          // first value of the slice
    const int kend = min(K, k0 + slots * F::kSteps * 32);  // end of its real values
    const int tile = blockIdx.x * kWaves + wave;
    const int row0 = 16 * tile;
    const int64_t rb = kQ4 ? static_cast<int64_t>(K >> 8) * kQ4kBlockBytes : 2 * static_cast<int64_t>(K);
    const uint8_t* const tbase = W + static_cast<int64_t>(row0) * rb;
    const int64_t tleft = static_cast<int64_t>(N - row0) * rb;  // <= 0 past the last tile: zeros
    // Real slots of this slice; loads of later ones (the padding and the
    // ring's last refills) get an empty range, so no wave reads a byte of
    // the next slice.
    const int nreal = min(slots, (K + F::kSteps * 32 - 1) / (F::kSteps * 32) - slice * slots);
    auto load = [&](int sl, typename F::Slot& dst) {
        F::load(tbase, sl < nreal ? tleft : 0, rb, k0 + sl * F::kSteps * 32, K, lane, dst);
    };

    // x of the slice first, into registers: unit u = (step s, row m, g) is
    // the 8 values k0 + 32 s + 8 g .. + 8 of row m (zero past the slice).
    const int units = psteps * M * 4;
    f32x4 xa[XP], xb[XP];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int u = tid + kThreads * i;
        const int g = u & 3, sm = u >> 2;
        const int s = sm / M, m = sm - s * M;
        const int kk = k0 + 32 * s + 8 * g;
        const bool in = u < units && kk < kend;
        const f32x4* src = reinterpret_cast<const f32x4*>(X + static_cast<int64_t>(in ? m : 0) * K + (in ? kk : 0));
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        xa[i] = in ? src[0] : z;
        xb[i] = in ? src[1] : z;
    }
    __builtin_amdgcn_sched_barrier(0);

    typename F::Slot ring[D];
#pragma unroll
    for (int j = 0; j < D; ++j) {
        load(j, ring[j]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Limbs (and, for Q4_K, the per-row sub-block constants) into LDS.
    const uint32_t zoff = static_cast<uint32_t>(psteps * Q * F::kLimb);
    uint8_t* const cst = lds + zoff + kZeroBytes;
    if (tid == 0) *reinterpret_cast<u32x4*>(lds + zoff) = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int u = tid + kThreads * i;
        const int g = u & 3, sm = u >> 2;
        const int s = sm / M, m = sm - s * M;
        const int q = m >> 2, t = m & 3;
        uint8_t* const dst = lds + (static_cast<size_t>(s) * Q + q) * F::kLimb + ((g * 4 + t) * 3) * F::kFrag;
        if constexpr (kQ4) {
            // Sub-block (s, m) is the quad of units g = 0..3.
            float amax = fmaxf(fmaxf(fmaxf(fabsf(xa[i][0]), fabsf(xa[i][1])), fmaxf(fabsf(xa[i][2]), fabsf(xa[i][3]))),
                               fmaxf(fmaxf(fabsf(xb[i][0]), fabsf(xb[i][1])), fmaxf(fabsf(xb[i][2]), fabsf(xb[i][3]))));
            float sum = ((xa[i][0] + xa[i][1]) + (xa[i][2] + xa[i][3])) + ((xb[i][0] + xb[i][1]) + (xb[i][2] + xb[i][3]));
            amax = quad_max(amax);
            sum = quad_sum(sum);
            float sc, inv;
            q4k_mfma::sub_block_scale(amax, sc, inv);
            uint32_t a0, a1, a2, b0, b1, b2;
            q4k_mfma::limb_words(xa[i], inv, a0, a1, a2);
            q4k_mfma::limb_words(xb[i], inv, b0, b1, b2);
            if (u < units) {
                *reinterpret_cast<u32x2*>(dst) = u32x2{a0, b0};
                *reinterpret_cast<u32x2*>(dst + 8) = u32x2{a1, b1};
                *reinterpret_cast<u32x2*>(dst + 16) = u32x2{a2, b2};
                if (g == 0)
                    *reinterpret_cast<f32x4*>(cst + ((static_cast<size_t>(s) * Q + q) * 4 + t) * 16) =
                        f32x4{sc, sc * (1.0f / 256.0f), sc * (1.0f / 65536.0f), sum};
            }
        } else {
            u32x2 ha, ma, la, hb, mb, lb;
            bf16_limbs4(xa[i], ha, ma, la);
            bf16_limbs4(xb[i], hb, mb, lb);
            if (u < units) {
                u32x4* d4 = reinterpret_cast<u32x4*>(dst);
                d4[0] = u32x4{ha[0], ha[1], hb[0], hb[1]};
                d4[1] = u32x4{ma[0], ma[1], mb[0], mb[1]};
                d4[2] = u32x4{la[0], la[1], lb[0], lb[1]};
            }
        }
    }
    lds_barrier();

    // This lane's A rows: (t, lambda) = ((l % 16) / 4, l % 4) of group q; a
    // zero row (lambda == 3, or a row past M) reads the zero line.
    const int ai = lane & 15, g = lane >> 4;
    const int at = ai >> 2, al = ai & 3;
    uint32_t abase[Q], amask[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const bool live = al < 3 && 4 * q + at < M;
        abase[q] = live ? static_cast<uint32_t>(q * F::kLimb + ((g * 4 + at) * 3 + al) * F::kFrag) : zoff;
        amask[q] = live ? 0xffffffffu : 0u;
    }
    auto a_off = [&](int s, int q) {
        return abase[q] + ((static_cast<uint32_t>(s) * (Q * F::kLimb)) & amask[q]);
    };

    f32x4 C[Q];
    float acc[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        C[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        acc[q] = 0.0f;
    }

    // Steady rounds (straight-line; slots past the slice load zeros and
    // compute against zero limbs).
    const int rounds = psteps / (F::kSteps * D);
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const int slot = r * D + j;
            const int s0 = slot * F::kSteps;
            if constexpr (!kQ4) {
                bf16x8 B[4];
#pragma unroll
                for (int st = 0; st < 4; ++st) B[st] = __builtin_bit_cast(bf16x8, ring[j].v[st]);
                __builtin_amdgcn_sched_barrier(0);
                load(slot + D, ring[j]);
#pragma unroll
                for (int st = 0; st < 4; ++st)
#pragma unroll
                    for (int q = 0; q < Q; ++q) {
                        const bf16x8 A = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lds + a_off(s0 + st, q)));
                        C[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B[st], C[q], 0, 0, 0);
                    }
            } else {
                const u32x4 h = ring[j].h;
                u32x2 p[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) p[c] = ring[j].p[c];
                __builtin_amdgcn_sched_barrier(0);
                load(slot + D, ring[j]);
                const float d = f16_bits_to_f32(h[0] & 0xffffu);
                const float dmin = f16_bits_to_f32(h[0] >> 16);
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    uint32_t sv, mv;
                    decode_scale_min(make_scale_sel(jj), h[1], h[2], h[3], sv, mv);
                    const float a = d * static_cast<float>(sv);
                    const float dm = dmin * static_cast<float>(mv);
                    const u32x2 pc = p[jj >> 1];
                    const uint32_t n0 = (jj & 1) ? (pc[0] >> 4) & 0x0f0f0f0fu : pc[0] & 0x0f0f0f0fu;
                    const uint32_t n1 = (jj & 1) ? (pc[1] >> 4) & 0x0f0f0f0fu : pc[1] & 0x0f0f0f0fu;
                    const long B = static_cast<long>((static_cast<uint64_t>(n1) << 32) | n0);
                    const int s = s0 + jj;
#pragma unroll
                    for (int q = 0; q < Q; ++q) {
                        const long A = *reinterpret_cast<const long*>(lds + a_off(s, q));
                        const i32x4 z = {0, 0, 0, 0};
                        const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, z, 0, 0, 0);
                        const f32x4 k4 = *reinterpret_cast<const f32x4*>(
                            cst + ((static_cast<uint32_t>(s) * Q + q) * 4 + g) * 16);
                        float dot = static_cast<float>(c[0]) * k4[0];
                        dot = __builtin_fmaf(static_cast<float>(c[1]), k4[1], dot);
                        dot = __builtin_fmaf(static_cast<float>(c[2]), k4[2], dot);
                        acc[q] = __builtin_fmaf(a, dot, acc[q]);
                        acc[q] = __builtin_fmaf(-dm, k4[3], acc[q]);
                    }
                }
            }
        }
    }

    // Row n of the tile, activation row 4q + g.
    const int row = row0 + (lane & 15);
    const int nslices = gridDim.y;
    const int64_t total = static_cast<int64_t>(M) * N;
    bool keep[Q];
    int64_t idx[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int m = 4 * q + g;
        keep[q] = m < M && row < N;
        idx[q] = static_cast<int64_t>(m) * N + row;
        const float v = kQ4 ? acc[q] : (C[q][0] + C[q][1]) + C[q][2];
        if (nslices == 1) {
            if (keep[q]) Y[idx[q]] = v;
        } else if (keep[q]) {
            st_dev(P + slice * total + idx[q], v);
        }
    }
    if (nslices == 1) return;

    // Every wave's partials have completed, then one arrival per workgroup.
    // The limbs are dead: LDS dword 0 carries the arrival number.
    // The ordering rests on the accesses themselves rather than on fences:
    // the partials are agent-scope atomic stores (written through past the
    // XCD's L2) whose completion every wave has waited for (vmcnt(0)) before
    // the barrier and the arrival, and the merging workgroup reads them with
    // agent-scope atomic loads (not served from its L2), issued only once
    // the arrival's result is known.  A release/acquire on the arrival would
    // also write back and invalidate the whole L2 of the XCD in every
    // workgroup (buffer_wbl2 / buffer_inv): measured 15.8 against 10.2 us
    // for Q4_K 8192 x 3072 at M = 8.
    wait_vmcnt<0>();
    lds_barrier();
    uint32_t* const flag = reinterpret_cast<uint32_t*>(lds);
    if (tid == 0)
        *flag = __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds_barrier();
    if (*flag != static_cast<uint32_t>(nslices - 1)) return;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        if (!keep[q]) continue;
        float sum = ld_dev(P + idx[q]);
        for (int j = 1; j < nslices; ++j) sum += ld_dev(P + j * total + idx[q]);
        Y[idx[q]] = sum;
    }
    if (tid == 0) __hip_atomic_store(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class F, int Q, int D, int XP>
hipError_t run(const void* w, const float* x, float* y, float* p, uint32_t* counters, int64_t n, int64_t k, int m,
               int slots, int slices, int psteps, hipStream_t s) {
    const int64_t tiles = (n + 15) / 16;
    const dim3 grid(static_cast<unsigned>((tiles + kWaves - 1) / kWaves), static_cast<unsigned>(slices));
    hipLaunchKernelGGL((k_gemv_batch<F, Q, D, XP>), grid, dim3(kThreads), batch_lds_bytes<F>(psteps, Q), s,
                       static_cast<const uint8_t*>(w), x, y, p, counters, static_cast<int>(n), static_cast<int>(k), m,
                       slots, psteps);
    return hipGetLastError();
}

template <class F, int Q, int D>
hipError_t run_d(const void* w, const float* x, float* y, float* p, uint32_t* counters, int64_t n, int64_t k, int m,
                 int per, int slices, hipStream_t s) {
    const int psteps = per * F::kSteps;
    const int xp = static_cast<int>((static_cast<int64_t>(psteps) * m * 4 + kThreads - 1) / kThreads);
    if (xp <= 1) return run<F, Q, D, 1>(w, x, y, p, counters, n, k, m, per, slices, psteps, s);
    if (xp <= 2) return run<F, Q, D, 2>(w, x, y, p, counters, n, k, m, per, slices, psteps, s);
    return run<F, Q, D, 4>(w, x, y, p, counters, n, k, m, per, slices, psteps, s);
}

template <class F, int Q>
hipError_t run_q(const void* w, const float* x, float* y, float* p, uint32_t* counters, int64_t n, int64_t k, int m,
                 int per, int slices, hipStream_t s) {
    const int dmax = tune_param("BATCH_DMAX", 1);
    if (per % 4 == 0 && dmax >= 4) return run_d<F, Q, 4>(w, x, y, p, counters, n, k, m, per, slices, s);
    if (per % 2 == 0 && dmax >= 2) return run_d<F, Q, 2>(w, x, y, p, counters, n, k, m, per, slices, s);
    return run_d<F, Q, 1>(w, x, y, p, counters, n, k, m, per, slices, s);
}

// Slots per slice: what the LDS budget holds and XP <= 4 registers of x per
// thread cover; among those, the least estimated time
//     rounds of workgroups over the CUs * kSlotCost * slots per slice
//     + slices (the last workgroup's reduction reads one partial per slice),
// ties to the longer slice.  Candidates are the shortest slice for each
// slice count.  (Fitted to times measured at N x K = 3072x3072, 8192x3072,
// 3072x8192 (Q4_K), 3072x8192 and 1024x3072 (BF16), M = 2 and 8.)
// The ring depth: one slot.  Deeper rings (2, 4 slots, selectable for
// measurement) measured slower at those shapes -- their registers cost
// resident workgroups, and other waves hide a slot's load better.
template <class F>
bool plan(int64_t n, int64_t k, int m, int64_t* per_out, int64_t* slices_out) {
    const int q = (m + 3) / 4;
    const int64_t total_slots = (k + F::kSteps * 32 - 1) / (F::kSteps * 32);
    const int64_t groups = ((n + 15) / 16 + kWaves - 1) / kWaves;
    const int64_t cus = device_info().cus;
    const size_t budget = static_cast<size_t>(tune_param("BATCH_LDS", 65536));
    auto fits = [&](int64_t per) {
        const int64_t ps = per * F::kSteps;
        return batch_lds_bytes<F>(static_cast<int>(ps), q) <= budget && ps * m * 4 <= 4 * static_cast<int64_t>(kThreads);
    };
    if (!fits(1)) return false;
    int64_t per = 1, best = -1, prev = 0;
    for (int64_t sl = 1; sl <= total_slots; ++sl) {
        const int64_t c = (total_slots + sl - 1) / sl;
        if (c == prev || !fits(c)) continue;
        prev = c;
        const int64_t cost = (groups * sl + cus - 1) / cus * F::kSlotCost * c + sl;
        if (best < 0 || cost < best) {
            best = cost;
            per = c;
        }
    }
    const int forced = tune_param("BATCH_SLOTS", 0);
    if (forced > 0 && fits(forced)) per = forced;
    *per_out = per;
    *slices_out = (total_slots + per - 1) / per;
    return true;
}

template <class F>
hipError_t dispatch(const void* w, const float* x, float* y, int64_t n, int64_t k, int m, hipStream_t s) {
    const int q = (m + 3) / 4;
    const int64_t groups = ((n + 15) / 16 + kWaves - 1) / kWaves;
    int64_t per = 0, slices = 0;
    if (!plan<F>(n, k, m, &per, &slices)) return hipErrorInvalidValue;

    float* part = nullptr;
    uint32_t* counters = nullptr;
    if (slices > 1) {
        if (groups > static_cast<int64_t>(kArrivalCounters)) return hipErrorInvalidValue;
        hipError_t e;
        counters = arrival_counters(s, &e);
        if (!counters) return e;
        part = static_cast<float*>(workspace(static_cast<size_t>(slices) * m * n * sizeof(float), s, &e));
        if (!part) return e;
    }
    const int sl = static_cast<int>(per), nsl = static_cast<int>(slices);
    if (q == 1) return run_q<F, 1>(w, x, y, part, counters, n, k, m, sl, nsl, s);
    return run_q<F, 2>(w, x, y, part, counters, n, k, m, sl, nsl, s);
}

}  // namespace

size_t gemv_batch_workspace_bytes(int fmt, int64_t n, int64_t k, int m) {
    if (m < 2 || m > 8) return 0;
    int64_t per = 0, slices = 0;
    const bool ok = fmt == RT_HIP_Q4K ? plan<BQ4k>(n, k, m, &per, &slices)
                                      : (fmt == RT_HIP_BF16 ? plan<BBf16>(n, k, m, &per, &slices) : false);
    return ok && slices > 1 ? static_cast<size_t>(slices) * m * n * sizeof(float) : 0;
}

hipError_t launch_gemv_batch(int fmt, const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                             hipStream_t s) {
    if (m < 2 || m > 8) return hipErrorInvalidValue;
    if (fmt == RT_HIP_Q4K) return dispatch<BQ4k>(w, x, y, n, k, m, s);
    if (fmt == RT_HIP_BF16) return dispatch<BBf16>(w, x, y, n, k, m, s);
    return hipErrorInvalidValue;
}

}  // namespace rt_hip
