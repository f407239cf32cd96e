// gemv_mfma.hip -- M = 1 Q4_K GEMV on int8 MFMA (the decode hot path).
//
// y[n] = sum_k x[k] * W[n, k], W in Q4_K blocks (K % 256 == 0).  One launch
// can carry up to four such products that share x and K (a layer's q/k/v, or
// gate/up): their 16-row tiles are numbered consecutively and each wave looks
// its tile up in the job table.
//
// A wave owns one 16-row tile (q4k_mfma.hpp: lane = (row n, chunk g)), or
// 1/KS of its super-blocks: the KS waves of a tile combine their partial rows
// through LDS.  A workgroup holds max(4, KS) waves, i.e. 4/KS tiles for
// KS <= 4 and one tile of KS waves beyond, so short outputs still put enough
// loads in flight per CU.
// Each wave keeps a ring of D super-blocks of its tile loaded ahead of the
// one it computes, so D * 16 rows * 144 bytes stay in flight per wave.
// The activation is staged once per workgroup as int8 limbs in LDS; its
// global loads are issued before the weight prologue so that waiting for
// them does not drain the weight loads (vmcnt completes in order).
#include <type_traits>

#include "gemv_bf16.hpp"
#include "q4k_mfma.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

using namespace q4k_mfma;

constexpr int kMaxThreads = 768;  // up to 12 waves per workgroup
constexpr int kMaxJobs = 4;

// Job table passed by value: job j owns tiles [tile0[j], tile0[j + 1]), the
// last one up to `total`; unused entries hold `total`.
// y last: the output pointers are read after the weight prologue, and next
// to the weight pointers of jobs 2 and 3 (read before it, by the waves of
// those jobs only) the compiler merged both into one scalar load issued
// ahead of the job lookup, which every wave then waited for.
struct Jobs {
    const uint8_t* w[kMaxJobs];
    int n[kMaxJobs];
    int tile0[kMaxJobs];
    int total;
    int count;
    float* y[kMaxJobs];
};

// Rotary position embedding on the outputs of the jobs in `jobs` (a bit
// mask), in the interleaved pairing of GGUF's llama weights (rows 2i and
// 2i + 1 of a head, llama_rope in transformer5.cpp:95-125):
//     out_2i   = x_2i * cos(a) - x_2i+1 * sin(a)
//     out_2i+1 = x_2i * sin(a) + x_2i+1 * cos(a),   a = pos * inv_freq[i]
// with i the pair within the head.  Rows 2i and 2i + 1 of a 16-row tile are
// lanes n and n ^ 1 of the wave that stores them, so the pair meets in one
// lane swap.
// What the epilogue does with a finished row: store it, rotate it first
// (RoPE, below), or add it to what y holds (the residual add of
// LlamaBlock::forward_cached, transformer5.cpp:205-212: x = x + attn(...),
// x = x + mlp(...)).
// kEpiArgmax: store the row and fold it into its tile's greedy-argmax key
// (the first index of the strict maximum, NaN never chosen:
// transformer5.cpp:382-391), one key per 16-row tile in Rope::keys; a
// second launch folds those (launch_argmax_reduce).
enum Epi { kEpiNone = 0, kEpiRope = 1, kEpiAdd = 2, kEpiArgmax = 3 };

struct Rope {
    const float* inv_freq = nullptr;  // [head_dim / 2], device
    const int32_t* pos_dev = nullptr;  // position in device memory (else pos)
    int64_t cache_row = 0;             // with pos_dev: jobs in cache_jobs store at y + position * cache_row
    int pos = 0;
    int head_dim = 0;
    int jobs = 0;
    int half = 0;  // half-split pairing: rows of rotated jobs tiled interleaved
    int cache_jobs = 0;
    uint64_t* keys = nullptr;  // kEpiArgmax: one key per tile

    // A scalar load: the position does not change during a launch.  (As a
    // vector load, uniform, its value would go through readfirstlane, which
    // waits for every load in flight, the weight ring's too.)
    __device__ __forceinline__ int position() const {
        return pos_dev ? ((const __attribute__((address_space(4))) int32_t*)pos_dev)[0] : pos;
    }
    // Where output set j (a job, or kRopeCacheBf16Bit for the BF16 rows) starts.
    __device__ __forceinline__ float* dest(float* y, int j) const { return dest_at(y, j, position()); }
    // The same with the position already read (p == position()).
    __device__ __forceinline__ float* dest_at(float* y, int j, int p) const {
        return pos_dev && ((cache_jobs >> j) & 1) ? y + static_cast<int64_t>(p) * cache_row : y;
    }
};

// Job-table fields read into scalar registers through readfirstlane, and
// picked with scalar selects: read straight from the kernel arguments (or
// from an array), a job lookup becomes an indexed load and a wait.
template <typename T>
struct Four {
    T a, b, c, d;
    __device__ __forceinline__ T operator[](int j) const { return j == 3 ? d : (j == 2 ? c : (j == 1 ? b : a)); }
};

__device__ __forceinline__ int sreg(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint64_t sreg(const void* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// The K-split of a launch and its job count, packed by the host into one
// preloaded argument so that no wave divides: bits 0-3 KS (waves per tile),
// 4-7 TPW (tiles per workgroup), 8-15 super-blocks per wave, 16-28
// ceil(4096 / KS), with which wave / KS = (wave * m) >> 12 exactly for
// wave < 16 and KS <= 12 (the rounding adds < 16/4096, below the gap 1/KS
// to the next integer), 29-31 the job count (1..4).
__host__ __device__ inline uint32_t pack_split(int ks, int tpw, int bpw, int count) {
    return static_cast<uint32_t>(ks) | (static_cast<uint32_t>(tpw) << 4) | (static_cast<uint32_t>(bpw) << 8) |
           (static_cast<uint32_t>((4096 + ks - 1) / ks) << 16) | (static_cast<uint32_t>(count) << 29);
}

// The x operations (XOp) are declared with the BF16 body (gemv_bf16.hpp).

// LDS byte offset of the RMSNorm partial sums (one float per wave, after
// the limb planes and the K-split partial rows).
__host__ __device__ inline size_t norm_offset(int K, int waves) {
    return lds_bytes(K) + static_cast<size_t>(waves) * 16 * sizeof(float);
}

// Whether an instantiation can see x longer than its register batch: only
// the widest batch (16 f32x4 per thread, 8 with an x operation), which the
// host picks when nothing narrower covers K.  The narrower ones carry no
// loop (its registers and code cost the short launches measurably).
// kXPostNorm1 needs all of b before any x exists, so it never has a rest:
// the host runs it only where the batch covers K.
template <int XP, int XOP>
constexpr bool kHasRest = XP >= (XOP == kXNone ? 16 : 8) && XOP != kXPostNorm1;

// kXPostNorm1's operands: x = X + RMSNorm(b) * (1 + g2), stored to out.
// Its own kernel takes them (k_gemv_q4k_postnorm), so the other x-op
// kernels' arguments do not grow.
struct PostNorm {
    const float* b = nullptr;
    const float* g2 = nullptr;
    float* out = nullptr;
};

// x operations that end in an RMSNorm, and those whose gamma applies as 1 + g
template <int XOP>
constexpr bool kNormOp = XOP == kXRmsNorm || XOP == kXRmsNorm1 || XOP == kXPostNorm1;
template <int XOP>
constexpr bool kOnePlus = XOP == kXRmsNorm1 || XOP == kXPostNorm1;

// The part of x past a staging batch held in registers (K beyond what XP
// f32x4 per thread cover, up to the LDS bound): f32x4 f = first, first +
// step, ..., loaded, transformed by the x operation and written as limbs;
// returns the sum of squares of the raw values (the RMSNorm partial).
// first and step are multiples of 64 plus the lane, and K / 4 is a multiple
// of 64, so every wave runs whole iterations (the 8-lane limb reductions
// need the whole group).
template <int XOP>
__device__ __forceinline__ float stage_rest(const float* __restrict__ X, const float* __restrict__ aux, int K,
                                            int first, int step, uint8_t* lds) {
    const int nx = K >> 2;
    const f32x4* const X4 = reinterpret_cast<const f32x4*>(X);
    const f32x4* const A4 = reinterpret_cast<const f32x4*>(aux);
    float sq = 0.0f;
    for (int f = first; f < nx; f += step) {
        f32x4 v = X4[f];
        if constexpr (XOP == kXRmsNorm || XOP == kXRmsNorm1) {
            const f32x4 a = A4[f];
            sq += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] *= XOP == kXRmsNorm1 ? 1.0f + a[e] : a[e];
        } else if constexpr (XOP == kXSwiGlu) {
            const f32x4 a = A4[f];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = swiglu1(v[e], a[e]);
        } else if constexpr (XOP == kXGelu) {
            const f32x4 a = A4[f];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu1(v[e], a[e]);
        }
        limbs_of(v, lds, K, f, true);
    }
    return sq;
}

// x staged by the converter waves of a warp-specialized workgroup (CW > 0
// below): thread c of the cthreads converter threads loads x[4f .. 4f+3] for
// f = c + cthreads * i (XP of them), applies the x operation, writes the
// limb planes and, for RMSNorm, its wave's partial sum of squares into
// slot `nslot` of the norm partials.  The weight waves of the workgroup
// issue their loads meanwhile; nothing here waits for them.
// kXPostNorm1 (cthreads * XP * 4 >= K, checked by the host): X is the
// residual a, and x = a + (b * rms_inv(b)) * (1 + g2) is formed first, in
// the separate norm's order (k_rmsnorm_rows); the sum of squares of b goes
// through one more barrier (the weight waves take part in it), its wave
// partials in the K-split rows' LDS, which are not used before the staging
// barrier.  `store_x` (one workgroup) stores x to pn.out.
template <int XP, int XOP>
__device__ __forceinline__ void convert_x(const float* __restrict__ X, const float* __restrict__ aux, int K, int c,
                                          int cthreads, int lane, int nslot, float* norm_part, uint8_t* lds,
                                          float eps, const PostNorm& pn, bool store_x) {
    const int nx = K >> 2;
    const f32x4* const X4 = reinterpret_cast<const f32x4*>(X);
    constexpr int XPN = XOP == kXPostNorm1 ? XP : 1;
    f32x4 xv[XP], av[XP], bv[XPN], gv[XPN];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int f = c + cthreads * i;
        xv[i] = X4[f < nx ? f : 0];
    }
    if constexpr (XOP != kXNone) {
        const f32x4* const A4 = reinterpret_cast<const f32x4*>(aux);
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int f = c + cthreads * i;
            av[i] = A4[f < nx ? f : 0];
        }
    }
    if constexpr (XOP == kXPostNorm1) {
        const f32x4* const B4 = reinterpret_cast<const f32x4*>(pn.b);
        const f32x4* const G4 = reinterpret_cast<const f32x4*>(pn.g2);
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int f = c + cthreads * i;
            bv[i] = B4[f < nx ? f : 0];
        }
        // x, the next gamma and b come from preloaded pointers; g2's comes
        // from the argument segment: its loads go last, so that waiting for
        // that pointer holds up no other load
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int f = c + cthreads * i;
            gv[i] = G4[f < nx ? f : 0];
        }
        float sb = 0.0f;
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const f32x4 v = c + cthreads * i < nx ? bv[i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            sb += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
        }
        sb = bf16_gemv::wave_sum(sb, lane);
        float* const bpart = reinterpret_cast<float*>(lds + lds_bytes(K));
        if (lane == 0) bpart[nslot] = sb;
        lds_barrier();
        float tb = 0.0f;
        for (int w = 0; w < (cthreads >> 6); ++w) tb += bpart[w];
        const float rb = 1.0f / __builtin_sqrtf(tb * (1.0f / static_cast<float>(K)) + eps);
#pragma unroll
        for (int i = 0; i < XP; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[i][e] = xv[i][e] + (bv[i][e] * rb) * (1.0f + gv[i][e]);
        if (store_x) {
            f32x4* const O4 = reinterpret_cast<f32x4*>(pn.out);
#pragma unroll
            for (int i = 0; i < XP; ++i) {
                const int f = c + cthreads * i;
                if (f < nx) O4[f] = xv[i];
            }
        }
    }
    float rest_sq = 0.0f;
    if constexpr (kHasRest<XP, XOP>) rest_sq = stage_rest<XOP>(X, aux, K, c + cthreads * XP, cthreads, lds);
    if constexpr (kNormOp<XOP>) {
        float sq = rest_sq;
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const f32x4 v = c + cthreads * i < nx ? xv[i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            sq += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
        }
        sq = bf16_gemv::wave_sum(sq, lane);
        if (lane == 0) norm_part[nslot] = sq;
#pragma unroll
        for (int i = 0; i < XP; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[i][e] *= kOnePlus<XOP> ? 1.0f + av[i][e] : av[i][e];
    } else if constexpr (XOP == kXSwiGlu) {
#pragma unroll
        for (int i = 0; i < XP; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[i][e] = swiglu1(xv[i][e], av[i][e]);
    } else if constexpr (XOP == kXGelu) {
#pragma unroll
        for (int i = 0; i < XP; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[i][e] = gelu1(xv[i][e], av[i][e]);
    }
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int f = c + cthreads * i;
        limbs_of(xv[i], lds, K, f, f < nx);
    }
    if (c < 4) reinterpret_cast<u32x4*>(lds + 3 * static_cast<size_t>(K))[c] = u32x4{0u, 0u, 0u, 0u};
}

// KS waves split a tile's super-blocks; a workgroup of blockDim.x / 64 waves
// holds TPW = waves / KS tiles.
// The arguments every wave needs before its first load come first, as
// scalars: they are preloaded into SGPRs at wave launch (the library builds
// with -amdgpu-kernarg-preload-count), so x and the weight prologue issue
// without waiting for a kernel-argument load.  Jobs 2 and 3 (and every
// output pointer) come from the table.
// The body of workgroup `blk` (the kernel below, and the Q4_K workgroups of
// the fused q/k/v launch); `lds` holds mfma_gemv_lds_bytes(K, waves).
//
// CW > 0 (warp-specialized): the workgroup is KS * TPW weight waves and CW
// converter waves after them (nthreads counts both).  The converter waves
// stage x (XP f32x4 per converter thread) and leave at the staging barrier;
// the weight waves issue their ring at once and load no x, so nothing of x
// sits ahead of the weights in their in-order load counters.
template <int D, int XP, bool TILED, bool J34, int XOP = kXNone, int EPI = kEpiNone, int CW = 0>
__device__ __forceinline__ void q4k_tiles(int blk, const float* __restrict__ X, int K, uint32_t split, int nthreads,
                                          const uint8_t* w0, const uint8_t* w1, int n0, int n1, int tile1,
                                          const Jobs& jobs, uint8_t* lds, const float* __restrict__ aux = nullptr,
                                          float eps = 0.0f, const Rope& rope = Rope{},
                                          const PostNorm& pn = PostNorm{}) {
    static_assert(XOP != kXPostNorm1 || CW > 0, "the post-norm residual step runs in converter waves");
    const int count = static_cast<int>(split >> 29);
    const int wwaves = (nthreads >> 6) - CW;  // weight waves
    if constexpr (CW > 0) {
        const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
        if (w >= wwaves) {
            const int c = static_cast<int>(threadIdx.x) - wwaves * kWave;
            float* const np = reinterpret_cast<float*>(lds + norm_offset(K, wwaves));
            convert_x<XP, XOP>(X, aux, K, c, CW * kWave, static_cast<int>(threadIdx.x) & 63, w - wwaves, np, lds,
                               eps, pn, blk == 0);
            lds_barrier();
            return;
        }
    }
    // nthreads == blockDim.x, passed as a preloaded argument: blockDim
    // itself is a kernel-argument load that the first x loads would wait for.
    const int KS = static_cast<int>(split & 15u), TPW = static_cast<int>((split >> 4) & 15u);
    const int bpw = static_cast<int>((split >> 8) & 255u);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = K >> 8;
    const int tslot = (wave * static_cast<int>((split >> 16) & 0x1fffu)) >> 12;
    const int ks = wave - tslot * KS;
    const int b0 = ks * bpw;
    const int nbw = min(nb, b0 + bpw) - b0;  // >= 1: the host picks KS so every split is non-empty
    const Lane ln = make_lane(lane, K);
    const int64_t rb = static_cast<int64_t>(nb) * kQ4kBlockBytes;
    const uint32_t roff = static_cast<uint32_t>(ln.n * rb);
    const int nx = K >> 2;

    // x first, straight into registers: XP f32x4 per thread, thread tid
    // holding x[4f .. 4f+3] for f = tid + nthreads * i, so each aligned
    // 8-lane group holds one 32-value sub-block.  The scheduling barrier
    // keeps these loads ahead of the weight prologue; vmcnt counts them in
    // order, so waiting for them is partial.
    const f32x4* const X4 = reinterpret_cast<const f32x4*>(X);
    constexpr int XPW = CW > 0 ? 1 : XP;  // the weight waves of a specialized workgroup load no x
    f32x4 xv[XPW], av[XPW];
    if constexpr (CW == 0) {
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int f = tid + nthreads * i;
            xv[i] = X4[f < nx ? f : 0];
        }
        if constexpr (XOP != kXNone) {
            const f32x4* const A4 = reinterpret_cast<const f32x4*>(aux);
#pragma unroll
            for (int i = 0; i < XP; ++i) {
                const int f = tid + nthreads * i;
                av[i] = A4[f < nx ? f : 0];
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // This wave's tile: job and first row (wave-uniform).  A tile slot past
    // the last tile belongs to the last job with rows past its end, so its
    // loads read zeros and it stores nothing.
    const int t = blk * TPW + tslot;
    int job, tile_base, n_job;
    const uint8_t* wj;
    job = (count > 1 && t >= tile1) ? 1 : 0;
    tile_base = job ? tile1 : 0;
    n_job = job ? n1 : n0;
    wj = job ? w1 : w0;
    if (J34 && count > 2) {
        // jobs 2 and 3 (a layer's k/v after q): from the table.  A separate
        // instantiation, so that launches of one or two jobs never wait for
        // a table load before their first weight load.  Job 2 starts after
        // the tiles of jobs 0 and 1, which follow from the preloaded row
        // counts, so the waves of jobs 0 and 1 read no table at all; the
        // others read all they may need from it unconditionally, one batch
        // of scalar loads and one latency.  (Looked up one field after
        // another, the job-2 start, then the chosen job's row count and
        // weights behind a branch, every wave waited for two or three scalar
        // loads in series before its weight prologue.  Headline token on one
        // box 698.2-700.9 against 699.9-702.3 us: the v tiles still wait for
        // one.)
        const int t2 = tile1 + ((n1 + 15) >> 4);
        if (t >= t2) {  // wave-uniform
            const int t3 = sreg(jobs.tile0[3]);
            const int n2 = sreg(jobs.n[2]), n3 = sreg(jobs.n[3]);
            const uint64_t w2 = sreg(jobs.w[2]), w3 = sreg(jobs.w[3]);
            const bool j3 = count > 3 && t >= t3;
            job = j3 ? 3 : 2;
            tile_base = j3 ? t3 : t2;
            n_job = j3 ? n3 : n2;
            wj = reinterpret_cast<const uint8_t*>(j3 ? w3 : w2);
        }
    }
    const int row0 = 16 * (t - tile_base);
    // Row-major blocks: the tile's rows are rb apart and block b sits at
    // b * 144 in its row.  Tiled: the tile's block b is 2304 contiguous bytes
    // at (tile * nb + b) * 2304, rows past N stored as zeros.
    constexpr int64_t kStride = TILED ? kTiledBlockBytes : kQ4kBlockBytes;
    const int64_t off0 = TILED ? (static_cast<int64_t>(row0 >> 4) * nb + b0) * kTiledBlockBytes
                               : static_cast<int64_t>(row0) * rb + static_cast<int64_t>(b0) * kQ4kBlockBytes;
    const int64_t job_bytes = TILED ? static_cast<int64_t>((n_job + 15) >> 4) * 16 * rb
                                    : static_cast<int64_t>(n_job) * rb;
    const uint8_t* const tbase = wj + off0;
    const int64_t tleft = job_bytes - off0;
    const TLane tl = make_tlane(lane);

    // Block i of the wave's range through a resource based at that block of
    // the tile; past the range (or past the job) the resource is empty:
    // zeros, no memory traffic.
    using B = typename std::conditional<TILED, BlkT, Blk>::type;
    // 32-bit bounds: the clamp is done once per wave, not per slot.
    const uint32_t tl32 = rsrc_bytes(tleft);
    auto issue = [&](B& slot, int i) {
        const uint32_t o = static_cast<uint32_t>(i) * static_cast<uint32_t>(kStride);
        // readfirstlane: the compiler may compute the (uniform) size on the
        // VALU, and a resource in VGPRs becomes a waterfall loop per load.
        const uint32_t left = static_cast<uint32_t>(
            __builtin_amdgcn_readfirstlane(static_cast<int>(i < nbw && o < tl32 ? tl32 - o : 0u)));
        const BufRsrc rs = make_rsrc_n(tbase + o, left);
        if constexpr (TILED)
            load_blk_t(rs, static_cast<uint32_t>(lane), slot);
        else
            load_blk(rs, roff, ln, slot);
    };
    auto dec = [&](const B& slot) {
        if constexpr (TILED)
            return decode_t(slot, tl);
        else
            return decode(slot, ln);
    };

    // The scheduling barriers keep the ring's loads in slot order, so that
    // slot j's data is always the oldest in flight when it is consumed and
    // the waits stay partial (s_waitcnt vmcnt(3*(D-1))); in the main loop
    // the barrier sits between decoding a slot and refilling it.
    B ring[D];
#pragma unroll
    for (int j = 0; j < D; ++j) {
        issue(ring[j], j);
        __builtin_amdgcn_sched_barrier(0);
    }

    // The epilogue's own operands, loaded right behind the prologue so that
    // their latency passes while the weights stream rather than after the
    // last product: the value a row adds to (kEpiAdd), the position and the
    // row's rotation frequency (kEpiRope).  Lanes past 16 and tile slots past
    // the last tile read a row of the job that exists, unused.
    const int row = row0 + ln.n;
    const Four<uint64_t> ys = {sreg(jobs.y[0]), sreg(jobs.y[1]), sreg(jobs.y[2]), sreg(jobs.y[3])};
    float* yj = reinterpret_cast<float*>(ys[job]);
    // Global (not flat) loads: a flat load also counts in lgkmcnt, and the
    // staging barrier's LDS wait would then wait for it.
    using GF = const __attribute__((address_space(1))) float;
    float y_old = 0.0f;
    if constexpr (EPI == kEpiAdd) y_old = ((GF*)yj)[min(row, n_job - 1)];
    int rpos = 0;
    float rfreq = 0.0f;
    if constexpr (EPI == kEpiRope) {
        rpos = rope.position();
        if ((rope.jobs >> job) & 1)  // wave-uniform
            rfreq = ((GF*)rope.inv_freq)[(row % rope.head_dim) >> 1];
    }
    __builtin_amdgcn_sched_barrier(0);

    // The x loads are older than the 3*D prologue loads: wait for them
    // alone (XP * nthreads >= K/4, checked by the host), then convert.
    // (The residual load above is younger still: this wait leaves it.)
    if constexpr (CW == 0) {
    wait_vmcnt<3 * D + (EPI == kEpiAdd ? 1 : 0)>();
    // x past the register batch (K above XP * nthreads * 4): loaded after
    // the weight prologue, so its waits are full ones; large K only.
    float rest_sq = 0.0f;
    if constexpr (kHasRest<XP, XOP>) rest_sq = stage_rest<XOP>(X, aux, K, tid + nthreads * XP, nthreads, lds);
    if constexpr (XOP == kXRmsNorm || XOP == kXRmsNorm1) {
        // RMSNorm(x) * g = rms_inv * (x * g) with one scalar rms_inv per
        // launch, so the staged activation is x * g and rms_inv multiplies
        // the finished dot product: equal in exact arithmetic, and the sum
        // of squares then needs no barrier of its own.  Per thread, then
        // over the wave (DPP and permlane); each wave's partial goes to LDS
        // before the limb barrier below and is summed after it.
        float sq = rest_sq;
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const f32x4 v = tid + nthreads * i < nx ? xv[i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            sq += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
        }
        sq = bf16_gemv::wave_sum(sq, lane);
        if (lane == 0) reinterpret_cast<float*>(lds + norm_offset(K, nthreads >> 6))[wave] = sq;
#pragma unroll
        for (int i = 0; i < XP; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[i][e] *= XOP == kXRmsNorm1 ? 1.0f + av[i][e] : av[i][e];
    } else if constexpr (XOP == kXSwiGlu) {
        // The sigmoid from the hardware exp2 and reciprocal (v_exp_f32,
        // v_rcp_f32, about 1 ulp each) rather than the correctly rounded
        // library expf and division, which cost ~30 VALU per value on the
        // down projection's 8192 inputs.  Then silu = g * sigmoid and times
        // up, in the reference's order.  Tails: exp overflows to inf for
        // g < -88 and the sigmoid is 0, as the reference's is.
#pragma unroll
        for (int i = 0; i < XP; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[i][e] = swiglu1(xv[i][e], av[i][e]);
    } else if constexpr (XOP == kXGelu) {
#pragma unroll
        for (int i = 0; i < XP; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[i][e] = gelu1(xv[i][e], av[i][e]);
    }
    // Every lane converts its values (past the end: a dummy that is not
    // stored; the 8-lane reductions need the whole group).  No branch may
    // skip a round: the compiler would sink that round's x load below the
    // weight prologue.  The host picks the smallest XP that covers x.
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int f = tid + nthreads * i;
        limbs_of(xv[i], lds, K, f, f < nx);
    }
    if (tid < 4) reinterpret_cast<u32x4*>(lds + 3 * static_cast<size_t>(K))[tid] = u32x4{0u, 0u, 0u, 0u};
    }
    // the converter waves' first barrier (their sum of squares of b)
    if constexpr (XOP == kXPostNorm1) __builtin_amdgcn_s_barrier();
    lds_barrier();
    // rms_inv = 1 / sqrt(sum(x^2) * (1/K) + eps), as the reference forms it
    // (the sum itself is reduced in a tree).
    float out_scale = 1.0f;
    if constexpr (kNormOp<XOP>) {
        const int parts = CW > 0 ? CW : (nthreads >> 6);
        const float* part = reinterpret_cast<const float*>(lds + norm_offset(K, CW > 0 ? wwaves : (nthreads >> 6)));
        float tot = 0.0f;
        for (int w = 0; w < parts; ++w) tot += part[w];
        out_scale = 1.0f / __builtin_sqrtf(tot * (1.0f / static_cast<float>(K)) + eps);
    }

    // Steady rounds: straight-line, no branch around the ring's loads (a
    // branch there makes the compiler merge register versions and drain
    // the pipeline).  Decode slot j, refill it with block i + D + j, then
    // compute: once decoded its registers are free, so the refill needs no
    // copy.  The tail consumes the last <= D blocks and issues nothing.
    float acc = 0.0f;
    int i = 0;
    for (; i + D < nbw; i += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const Dec dc = dec(ring[j]);
            __builtin_amdgcn_sched_barrier(0);
            issue(ring[j], i + D + j);
            acc = dot(dc, b0 + i + j, ln, lds, acc);
        }
    }
#pragma unroll
    for (int j = 0; j < D; ++j)
        if (i + j < nbw) acc = dot(dec(ring[j]), b0 + i + j, ln, lds, acc);

    // Row n's partial: sum the four chunk lanes g.
    float v = acc;
    v += __shfl_xor(v, 16, kWave);
    v += __shfl_xor(v, 32, kWave);
    const bool keep = row < n_job;  // false for tile slots past the last tile
    if constexpr (EPI == kEpiRope) yj = rope.dest_at(yj, job, rpos);
    // Where the row is stored: with the half-split pairing the rows of a
    // rotated job were tiled interleaved (row 2j of a head holds element j,
    // row 2j + 1 element j + head_dim / 2), and go back to their places here.
    int drow = row;
    if constexpr (EPI == kEpiRope) {
        if (rope.half && ((rope.jobs >> job) & 1)) {
            const int r = row % rope.head_dim;
            drow = row - r + (r >> 1) + ((r & 1) ? rope.head_dim / 2 : 0);
        }
    }
    // The row's final value, computed by every lane of the storing wave (the
    // RoPE partner exchange needs the whole wave).
    auto finish = [&](float val) {
        if constexpr (kNormOp<XOP>) val *= out_scale;
        if constexpr (EPI == kEpiRope) {
            const float other = __shfl_xor(val, 1, kWave);
            if ((rope.jobs >> job) & 1) {  // wave-uniform
                const int j = row % rope.head_dim;
                const float ang = static_cast<float>(rpos) * rfreq;
                const float c = cosf(ang), sn = sinf(ang);
                val = (j & 1) ? other * sn + val * c : val * c - other * sn;
            }
        }
        return val;
    };
    uint64_t key = 0;  // kEpiArgmax: this lane's row (0: none)
    auto keep_key = [&](float out) {
        if constexpr (EPI == kEpiArgmax)
            if (lane < 16 && keep && out == out) key = argmax_key(out, static_cast<uint32_t>(row));
    };
    if (KS == 1) {
        const float out = finish(v);
        if (lane < 16 && keep) yj[drow] = EPI == kEpiAdd ? y_old + out : out;
        keep_key(out);
    } else {
        float* red = reinterpret_cast<float*>(lds + lds_bytes(K));  // [TPW][KS][16]
        float* rp = red + tslot * KS * 16;
        if (lane < 16) rp[ks * 16 + lane] = v;
        lds_barrier();
        if (ks == 0) {  // the whole wave: lanes past 16 repeat rows, unstored
            float s = rp[lane & 15];
#pragma unroll
            for (int q = 1; q < KS; ++q) s += rp[q * 16 + (lane & 15)];
            const float out = finish(s);
            if (lane < 16 && keep) yj[drow] = EPI == kEpiAdd ? y_old + out : out;
            keep_key(out);
        }
    }
    if constexpr (EPI == kEpiArgmax) {
        // One wave finishes each tile (KS == 1: every wave; else the ks == 0
        // one): its largest key goes to the tile's slot, with no barrier.
        if (KS == 1 || ks == 0) {
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const uint64_t o = __shfl_xor(key, off, kWave);
                key = o > key ? o : key;
            }
            if (lane == 0 && t < jobs.total) rope.keys[t] = key;
        }
    }
}

template <int D, int XP, bool TILED, bool J34, int CW>
__global__ __launch_bounds__(CW > 0 ? 1024 : kMaxThreads) void k_gemv_q4k_mfma(
    const float* __restrict__ X, int K, uint32_t split, int nthreads, const uint8_t* w0, const uint8_t* w1,
    int n0, int n1, int tile1, const Jobs jobs) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    q4k_tiles<D, XP, TILED, J34, kXNone, kEpiNone, CW>(static_cast<int>(blockIdx.x), X, K, split, nthreads, w0, w1,
                                                       n0, n1, tile1, jobs, lds);
}

// The same with a layer operation applied to x while it is staged (XOp).
// Pointers first, then the 32-bit arguments: no padding, so all fourteen
// leading dwords (aux, gamma or up, included) are preloaded.
template <int XP, bool J34, int XOP, int EPI, int CW>
__global__ __launch_bounds__(CW > 0 ? 1024 : kMaxThreads) void k_gemv_q4k_xop(
    const float* __restrict__ X, const float* __restrict__ aux, const uint8_t* w0, const uint8_t* w1, int K,
    uint32_t split, int nthreads, int n0, int n1, int tile1, const Jobs jobs, float eps, const Rope rope) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    q4k_tiles<4, XP, true, J34, XOP, EPI, CW>(static_cast<int>(blockIdx.x), X, K, split, nthreads, w0, w1, n0, n1,
                                               tile1, jobs, lds, aux, eps, rope);
}

// kXPostNorm1 (one shape: converter waves, two f32x4 per converter thread).
// The arguments the first loads need fill the fourteen preloaded dwords: x,
// b and the next norm's gamma for the converter waves, the weights, K, the
// split word and the row counts for the weight waves; the block size and
// the first tile of job 1 follow from the split word and n0.  (With the
// PostNorm struct read from the argument segment first, Gemma-3-4B tokens
// measured 1549-1557 against 1538-1546 us.)
template <bool J34>
__global__ __launch_bounds__(1024) void k_gemv_q4k_postnorm(
    const float* __restrict__ X, const float* __restrict__ b, const float* __restrict__ aux, const uint8_t* w0,
    const uint8_t* w1, int K, uint32_t split, int n0, int n1, const Jobs jobs, float eps, const PostNorm pn_rest) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int nthreads = (static_cast<int>(split & 15u) * static_cast<int>((split >> 4) & 15u) + 8) * kWave;
    const int tile1 = (n0 + 15) >> 4;
    PostNorm pn = pn_rest;
    pn.b = b;
    q4k_tiles<4, 2, true, J34, kXPostNorm1, kEpiNone, 8>(static_cast<int>(blockIdx.x), X, K, split, nthreads, w0,
                                                         w1, n0, n1, tile1, jobs, lds, aux, eps, Rope{}, pn);
}

// A layer's q/k/v when v is BF16 (Q6_K widened): the first q4k_wgs
// workgroups run the tiled Q4_K GEMVs, the rest the BF16 rows, all on the
// same x.  One launch instead of two dependent ones; each workgroup's work is
// exactly that of the separate kernels (4 waves per workgroup on both sides).
// Pointers first, then the 32-bit arguments, so the fourteen preloaded
// dwords hold everything a Q4_K workgroup needs before its first loads
// (the block size is the compile-time bf16_gemv::kThreads).
template <int XPQ, bool J34, int XPB, int XOP = kXNone, int EPI = kEpiNone>
__global__ __launch_bounds__(bf16_gemv::kThreads) void k_gemv_q4k_bf16(
    const float* __restrict__ X, const float* __restrict__ aux, const uint8_t* w0, const uint8_t* w1, int K,
    uint32_t split, int q4k_wgs, int n0, int n1, int tile1, const uint16_t* __restrict__ wb, float* __restrict__ yb,
    int nb_rows, const Jobs jobs, float eps, const Rope rope) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int blk = static_cast<int>(blockIdx.x);
    if (blk < q4k_wgs)
        q4k_tiles<4, XPQ, true, J34, XOP, EPI>(blk, X, K, split, bf16_gemv::kThreads, w0, w1, n0, n1, tile1, jobs,
                                               lds, aux, eps, rope);
    else
        bf16_gemv::rows<8, XPB, false, bf16_gemv::kThreads, XOP>(
            blk - q4k_wgs, (nb_rows + 3) / 4, wb, X, EPI == kEpiRope ? rope.dest(yb, kRopeCacheBf16Bit) : yb,
            nb_rows, K, nullptr, lds, aux, eps);
}

// The x operation, its second vector and eps (XOp).
struct XArgs {
    const float* aux = nullptr;
    float eps = 0.0f;
    Rope rope;
    PostNorm pn;
};

// `waves` weight waves plus CW converter waves per workgroup.
template <int D, int XP, bool TILED, bool J34, int XOP, int EPI, int CW>
hipError_t run(const Jobs& jobs, const float* x, const XArgs& xa, int64_t k, int ks, int waves, hipStream_t s) {
    const int tpw = waves / ks;
    const int64_t wgs = (static_cast<int64_t>(jobs.total) + tpw - 1) / tpw;
    const int all = waves + CW;
    const size_t lds = mfma_gemv_lds_bytes(k, all);
    const uint32_t split = pack_split(ks, tpw, static_cast<int>((k / 256 + ks - 1) / ks), jobs.count);
    const dim3 g(static_cast<unsigned>(wgs)), b(static_cast<unsigned>(all * kWave));
    if constexpr (XOP == kXNone && EPI == kEpiNone) {
        hipLaunchKernelGGL((k_gemv_q4k_mfma<D, XP, TILED, J34, CW>), g, b, lds, s, x, static_cast<int>(k), split,
                           all * kWave, jobs.w[0], jobs.w[1], jobs.n[0], jobs.n[1], jobs.tile0[1], jobs);
    } else if constexpr (XOP == kXPostNorm1) {
        static_assert(D == 4 && XP == 2 && TILED && EPI == kEpiNone && CW == 8, "the post-norm kernel's one shape");
        hipLaunchKernelGGL((k_gemv_q4k_postnorm<J34>), g, b, lds, s, x, xa.pn.b, xa.aux, jobs.w[0], jobs.w[1],
                           static_cast<int>(k), split, jobs.n[0], jobs.n[1], jobs, xa.eps, xa.pn);
    } else {
        static_assert(D == 4 && TILED, "x operations and RoPE run on the tiled layout, ring depth 4");
        hipLaunchKernelGGL((k_gemv_q4k_xop<XP, J34, XOP, EPI, CW>), g, b, lds, s, x, xa.aux, jobs.w[0], jobs.w[1],
                           static_cast<int>(k), split, all * kWave, jobs.n[0], jobs.n[1], jobs.tile0[1], jobs,
                           xa.eps, xa.rope);
    }
    return hipGetLastError();
}

// x prefetch depth: enough f32x4 per thread for all of x (up to K = 8192 at
// 256 threads) before the weight prologue; with CW converter waves, per
// converter thread.
template <int D, bool TILED, int XOP, int EPI, int CW = 0>
hipError_t run_xp(const Jobs& jobs, const float* x, const XArgs& xa, int64_t k, int ks, int waves,
                  hipStream_t s) {
    const int xthreads = (CW > 0 ? CW : waves) * kWave;
    const int64_t per = (k / 4 + xthreads - 1) / xthreads;
    // At most 16 float4 per thread in registers, 8 with an x operation (its
    // second vector doubles the registers); the rest of a longer x is
    // staged by a loop after them.
    constexpr bool kPlain = XOP == kXNone && EPI == kEpiNone;
    if (jobs.count > 2) {
        if (per <= 2) return run<D, 2, TILED, true, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
        if (per <= 3) return run<D, 3, TILED, true, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
        if (per <= 4) return run<D, 4, TILED, true, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
        if (per <= 8 || !kPlain) return run<D, 8, TILED, true, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
        if constexpr (kPlain) return run<D, 16, TILED, true, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
    }
    if (per <= 2) return run<D, 2, TILED, false, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
    if (per <= 3) return run<D, 3, TILED, false, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
    if (per <= 4) return run<D, 4, TILED, false, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
    if (per <= 8 || !kPlain) return run<D, 8, TILED, false, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
    if constexpr (kPlain) return run<D, 16, TILED, false, XOP, EPI, CW>(jobs, x, xa, k, ks, waves, s);
    return hipErrorInvalidValue;
}

// K-split per tile.  One round of workgroups (at most one per CU) is what
// matters for the short outputs of a decode step: a launch whose last few
// CUs get a second workgroup takes twice as long.  Among the splits of
// {1, 2, 3, 4, 6, 8, 10, 12} that divide the super-block count, leave every
// wave at least two super-blocks and fit one workgroup per CU, the one with
// the fewest rounds of x conversion per SIMD (every wave converts its share
// of x before it uses any weight: waves per SIMD x f32x4 per thread, the
// latter as the register batch the launch instantiates, 2, 3, 4 or 8, and
// past 8 counted twice, since the rest is converted after the weight
// prologue with full waits), and among those the largest (more loads in
// flight).  Measured: o 3072 x 3072 3.84 us at KS = 4 (3 rounds) against
// 4.41 us at KS = 6 (4 rounds); down 3072 x 8192 best at KS = 8; the
// Gemma-3-4B down 2560 x 10240 (GELU gating) at KS = 10 (4 f32x4 per
// thread, 12 rounds) rather than 8 (5, batched as 8: 16 rounds), engine
// token 1609-1613 against 1633-1641 us (KS = 4: 1672-1678, 5: 1669).
// Outputs too long for one round even at KS = 1 use KS = 4 (the lm_head:
// 38.0 us against 40.9 us at KS = 2).
// KS = 1, 2, 4 run 4 waves per workgroup (4/KS tiles); other splits one
// tile per workgroup of KS waves.
struct Shape {
    int ks = 1;     // waves per tile
    int waves = 4;  // weight waves per workgroup
    int cw = 0;     // converter waves per workgroup
};

template <bool TILED>
bool shape_for(int64_t tiles, int64_t k, Shape& sh) {
    const int64_t nb = k / 256;
    const int64_t cus = device_info().cus;
    static const int kSplits[] = {1, 2, 3, 4, 6, 8, 10, 12};
    auto waves_for = [](int c) { return c <= 4 ? (4 / c) * c : c; };
    auto wgs_for = [&](int c) { return (tiles + waves_for(c) / c - 1) / (waves_for(c) / c); };
    auto rounds = [&](int c) {
        const int64_t w = waves_for(c), per = (k / 4 + 64 * w - 1) / (64 * w);
        const int64_t batch = per <= 2 ? 2 : (per <= 4 ? per : (per <= 8 ? 8 : 2 * per - 8));
        return (w + 3) / 4 * batch;
    };
    auto usable = [&](int c) { return nb % c == 0 && (c == 1 || 2 * c <= nb); };
    int ks = 1;
    for (int c : kSplits)
        if (usable(c) && wgs_for(c) <= cus && rounds(c) <= rounds(ks)) ks = c;
    // (Swept on the headline step's lm_head, 8016 tiles: KS 4 with one tile
    // per workgroup 701-702 us against 703-705 for KS 4 x 2 tiles, 2 x 2,
    // 2 x 4, 1 x 4 and 1 x 8.)
    const bool many = wgs_for(1) > cus;
    if (many) ks = tune_param("Q4K_MANY_KS", usable(4) ? 4 : (usable(2) ? 2 : 1));
    if (const int forced = tune_param("Q4K_KS", 0)) ks = (nb % forced == 0 && forced <= 12) ? forced : ks;
    // a whole number of tiles per workgroup: 4 waves for KS = 1, 2, 4;
    // exactly KS waves (one tile) otherwise
    int waves = ks <= 4 ? (4 / ks) * ks : ks;
    if (many) waves = ks * tune_param("Q4K_MANY_TPW", waves / ks);
    // More tiles than one round of those workgroups holds, but no more than
    // 8 per CU: one round at KS = 1 with one weight wave per tile (and the
    // converter waves beside them).  Gemma-3-4B's gate+up, 1280 tiles at
    // K = 2560: 256 workgroups of 5 tiles instead of 640 of 2.
    if (TILED && (tiles + waves / ks - 1) / (waves / ks) > cus && (tiles + cus - 1) / cus <= 8 && k <= 4096 &&
        tune_param("Q4K_ONE_ROUND", 1)) {
        ks = 1;
        waves = static_cast<int>((tiles + cus - 1) / cus);
    }
    if (const int tpw = tune_param("Q4K_TPW", 0)) waves = ks * tpw;
    if (waves % ks != 0 || waves > kMaxThreads / kWave) return false;
    // Converter waves (tiled layout): measured per launch shape on the
    // headline token, 8 of them beside the weight waves take o 3072 x 3072
    // from 3.85 to 3.62-3.67 us, the q/k/v launch from 4.86 to 4.57-4.60 and
    // gate+up from 7.29-7.33 to 7.18-7.26, but the K = 8192 down projection
    // from 5.90 to 6.66-6.73 and the lm_head (31 rounds of workgroups) from
    // 37.4 to 43.9: so one round of workgroups and K <= 4096 only.
    const int64_t wgs_now = (tiles + waves / ks - 1) / (waves / ks);
    int cw = tune_param("Q4K_CONV", TILED && wgs_now <= cus && k <= 4096 && waves + 8 <= 16 ? 8 : 0);
    if (!(TILED && cw == 8 && waves + 8 <= 16)) cw = 0;
    sh.ks = ks;
    sh.waves = waves;
    sh.cw = cw;
    return true;
}

template <bool TILED, int XOP = kXNone, int EPI = kEpiNone>
hipError_t dispatch(const Jobs& jobs, const float* x, int64_t k, hipStream_t s, const XArgs& xa = XArgs{}) {
    Shape sh;
    if (!shape_for<TILED>(jobs.total, k, sh)) return hipErrorInvalidValue;
    const int ks = sh.ks, waves = sh.waves;
    if constexpr (XOP == kXPostNorm1) {
        // converter waves only (K <= 4096), two f32x4 per converter thread
        // covering K
        if (sh.cw != 8 || k > 2 * 4 * 8 * kWave) return hipErrorNotSupported;
        return jobs.count > 2 ? run<4, 2, TILED, true, XOP, EPI, 8>(jobs, x, xa, k, ks, waves, s)
                              : run<4, 2, TILED, false, XOP, EPI, 8>(jobs, x, xa, k, ks, waves, s);
    } else {
        if (sh.cw == 8) return run_xp<4, TILED, XOP, EPI, 8>(jobs, x, xa, k, ks, waves, s);
        if constexpr (XOP != kXNone || EPI != kEpiNone) {
            return run_xp<4, TILED, XOP, EPI>(jobs, x, xa, k, ks, waves, s);
        } else {
            const int d = tune_param("Q4K_RING", 4);
            return d == 8 ? run_xp<8, TILED, XOP, EPI>(jobs, x, xa, k, ks, waves, s)
                          : run_xp<4, TILED, XOP, EPI>(jobs, x, xa, k, ks, waves, s);
        }
    }
}

}  // namespace

size_t mfma_gemv_lds_bytes(int64_t k, int waves) {
    // limb planes, the K-split partial rows, then one float per wave for
    // the RMSNorm partial sums
    return norm_offset(static_cast<int>(k), waves) + 16 * sizeof(float);
}

size_t q4k_m1_lds_bytes(int64_t k) { return mfma_gemv_lds_bytes(k, kMaxThreads / kWave); }

namespace {

// The job table of `count` (1..4) products; unused entries repeat job 0
// with no tiles.
Jobs make_jobs(int count, const void* const* w, float* const* y, const int64_t* n) {
    Jobs jobs{};
    jobs.count = count;
    int64_t tiles = 0;
    for (int j = 0; j < count; ++j) {
        jobs.w[j] = static_cast<const uint8_t*>(w[j]);
        jobs.y[j] = y[j];
        jobs.n[j] = static_cast<int>(n[j]);
        jobs.tile0[j] = static_cast<int>(tiles);
        tiles += (n[j] + 15) / 16;
    }
    for (int j = count; j < kMaxJobs; ++j) {
        jobs.w[j] = jobs.w[0];
        jobs.y[j] = jobs.y[0];
        jobs.n[j] = jobs.n[0];
        jobs.tile0[j] = static_cast<int>(tiles);
    }
    jobs.total = static_cast<int>(tiles);
    return jobs;
}

}  // namespace

hipError_t launch_gemv_q4k_xop(int xop, int count, const void* const* w, float* const* y, const int64_t* n,
                              const float* x, const float* aux, float eps, int64_t k, hipStream_t s,
                              const float* inv_freq, int pos, int head_dim, int rope_jobs, bool add,
                              const RopeCache& cache, uint64_t* argmax_keys) {
    if (count < 1 || count > kMaxJobs || (aux == nullptr && xop != kXNone)) return hipErrorInvalidValue;
    const Jobs jobs = make_jobs(count, w, y, n);
    XArgs xa;
    xa.aux = aux;
    xa.eps = eps;
    if (argmax_keys) {
        // the lm_head: the final norm while staging, the argmax after the rows
        if (rope_jobs || add) return hipErrorInvalidValue;
        xa.rope.keys = argmax_keys;
        switch (xop) {
            case kXRmsNorm: return dispatch<true, kXRmsNorm, kEpiArgmax>(jobs, x, k, s, xa);
            case kXRmsNorm1: return dispatch<true, kXRmsNorm1, kEpiArgmax>(jobs, x, k, s, xa);
            default: return hipErrorInvalidValue;
        }
    }
    if (rope_jobs) {
        xa.rope.inv_freq = inv_freq;
        xa.rope.pos = pos;
        xa.rope.head_dim = head_dim;
        xa.rope.jobs = rope_jobs & 0xff;
        xa.rope.half = (rope_jobs >> 8) & 1;
        xa.rope.pos_dev = cache.pos;
        xa.rope.cache_row = cache.row;
        xa.rope.cache_jobs = cache.jobs;
        switch (xop) {
            case kXRmsNorm: return dispatch<true, kXRmsNorm, kEpiRope>(jobs, x, k, s, xa);
            case kXRmsNorm1: return dispatch<true, kXRmsNorm1, kEpiRope>(jobs, x, k, s, xa);
            default: return hipErrorInvalidValue;
        }
    }
    if (add) {
        switch (xop) {
            case kXNone: return dispatch<true, kXNone, kEpiAdd>(jobs, x, k, s, xa);
            case kXSwiGlu: return dispatch<true, kXSwiGlu, kEpiAdd>(jobs, x, k, s, xa);
            default: return hipErrorInvalidValue;
        }
    }
    switch (xop) {
        case kXRmsNorm: return dispatch<true, kXRmsNorm>(jobs, x, k, s, xa);
        case kXRmsNorm1: return dispatch<true, kXRmsNorm1>(jobs, x, k, s, xa);
        case kXSwiGlu: return dispatch<true, kXSwiGlu>(jobs, x, k, s, xa);
        case kXGelu: return dispatch<true, kXGelu>(jobs, x, k, s, xa);
        default: return hipErrorInvalidValue;
    }
}

bool q4k_postnorm_fits(int count, const int64_t* n, int64_t k) {
    if (count < 1 || count > kMaxJobs || k % 256 != 0) return false;
    int64_t tiles = 0;
    for (int j = 0; j < count; ++j) tiles += (n[j] + 15) / 16;
    Shape sh;
    return shape_for<true>(tiles, k, sh) && sh.cw == 8 && k <= 2 * 4 * 8 * kWave;
}

hipError_t launch_gemv_q4k_postnorm(int count, const void* const* w, float* const* y, const int64_t* n,
                                    const float* a, const float* b, const float* g2, const float* gamma, float eps,
                                    int64_t k, float* x_out, hipStream_t s) {
    if (count < 1 || count > kMaxJobs || !a || !b || !g2 || !gamma || !x_out) return hipErrorInvalidValue;
    if (!q4k_postnorm_fits(count, n, k)) return hipErrorNotSupported;
    const Jobs jobs = make_jobs(count, w, y, n);
    XArgs xa;
    xa.aux = gamma;
    xa.eps = eps;
    xa.pn.b = b;
    xa.pn.g2 = g2;
    xa.pn.out = x_out;
    return dispatch<true, kXPostNorm1>(jobs, a, k, s, xa);
}

hipError_t launch_gemv_q4k_mfma_multi(int count, const void* const* w, float* const* y,
                                      const int64_t* n, const float* x, int64_t k, hipStream_t s,
                                      bool tiled) {
    if (count < 1 || count > kMaxJobs) return hipErrorInvalidValue;
    const Jobs jobs = make_jobs(count, w, y, n);
    return tiled ? dispatch<true>(jobs, x, k, s) : dispatch<false>(jobs, x, k, s);
}

namespace {

template <int XPQ, bool J34, int XPB, int XOP, int EPI>
hipError_t run_fused(const Jobs& jobs, int ks, int q4k_wgs, const uint16_t* wb, float* yb, int64_t nb_rows,
                     const float* x, const XArgs& xa, int64_t k, size_t lds, hipStream_t s) {
    const int64_t bwgs = (nb_rows + 3) / 4;  // one row per wave, 4 waves
    hipLaunchKernelGGL((k_gemv_q4k_bf16<XPQ, J34, XPB, XOP, EPI>), dim3(static_cast<unsigned>(q4k_wgs + bwgs)),
                       dim3(bf16_gemv::kThreads), lds, s, x, xa.aux, jobs.w[0], jobs.w[1], static_cast<int>(k),
                       pack_split(ks, 4 / ks, static_cast<int>((k / 256 + ks - 1) / ks), jobs.count), q4k_wgs,
                       jobs.n[0], jobs.n[1], jobs.tile0[1], wb, yb, static_cast<int>(nb_rows), jobs, xa.eps,
                       xa.rope);
    return hipGetLastError();
}

template <int XOP, int EPI>
hipError_t fused_xp(const Jobs& jobs, int ks, int q4k_wgs, const uint16_t* wb, float* yb, int64_t nb_rows,
                    const float* x, const XArgs& xa, int64_t k, size_t lds, hipStream_t s) {
    const bool j34 = jobs.count > 2;
    const int64_t per = (k / 4 + 255) / 256;  // f32x4 of x per thread
    if (k <= 4096) {
        if (per <= 2)
            return j34 ? run_fused<2, true, 4, XOP, EPI>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s)
                       : run_fused<2, false, 4, XOP, EPI>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s);
        if (per <= 3)
            return j34 ? run_fused<3, true, 4, XOP, EPI>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s)
                       : run_fused<3, false, 4, XOP, EPI>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s);
        return j34 ? run_fused<4, true, 4, XOP, EPI>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s)
                   : run_fused<4, false, 4, XOP, EPI>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s);
    }
    if (per <= 8)
        return j34 ? run_fused<8, true, 8, XOP, EPI>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s)
                   : run_fused<8, false, 8, XOP, EPI>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s);
    return hipErrorInvalidValue;
}

}  // namespace

size_t q4k_bf16_fused_lds_bytes(int64_t k) {
    const size_t a = mfma_gemv_lds_bytes(k, 4), b = bf16_gemv::lds_bytes(k);
    return a > b ? a : b;
}

hipError_t launch_gemv_q4k_bf16_fused(int count, const void* const* w, float* const* y, const int64_t* n,
                                      const uint16_t* wb, float* yb, int64_t nb_rows, const float* x,
                                      int64_t k, hipStream_t s, int xop, const float* aux, float eps,
                                      const float* inv_freq, int pos, int head_dim, int rope_jobs,
                                      const RopeCache& cache) {
    if (count < 1 || count > kMaxJobs || k > 8192) return hipErrorInvalidValue;
    const Jobs jobs = make_jobs(count, w, y, n);
    // Four waves per workgroup on both sides, so the Q4_K split is 4, 2 or 1
    // waves per tile: the largest that divides the super-blocks, leaves two
    // per wave and keeps the Q4_K part to one workgroup per CU.
    const int64_t nb = k / 256, cus = device_info().cus;
    int ks = 1;
    for (int c : {4, 2})
        if (nb % c == 0 && 2 * c <= nb && (jobs.total + (4 / c) - 1) / (4 / c) <= cus) {
            ks = c;
            break;
        }
    const int tpw = 4 / ks;
    const int q4k_wgs = (jobs.total + tpw - 1) / tpw;
    const size_t lds = q4k_bf16_fused_lds_bytes(k);
    XArgs xa;
    xa.aux = aux;
    xa.eps = eps;
    if (rope_jobs) {
        xa.rope.inv_freq = inv_freq;
        xa.rope.pos = pos;
        xa.rope.head_dim = head_dim;
        xa.rope.jobs = rope_jobs & 0xff;
        xa.rope.half = (rope_jobs >> 8) & 1;
        xa.rope.pos_dev = cache.pos;
        xa.rope.cache_row = cache.row;
        xa.rope.cache_jobs = cache.jobs;
        switch (xop) {
            case kXRmsNorm: return fused_xp<kXRmsNorm, kEpiRope>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s);
            case kXRmsNorm1:
                return fused_xp<kXRmsNorm1, kEpiRope>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s);
            default: return hipErrorInvalidValue;
        }
    }
    switch (xop) {
        case kXNone: return fused_xp<kXNone, kEpiNone>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s);
        case kXRmsNorm: return fused_xp<kXRmsNorm, kEpiNone>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s);
        case kXRmsNorm1: return fused_xp<kXRmsNorm1, kEpiNone>(jobs, ks, q4k_wgs, wb, yb, nb_rows, x, xa, k, lds, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_q4k_mfma(const void* w, const float* x, float* y, int64_t n, int64_t k,
                                hipStream_t s) {
    return launch_gemv_q4k_mfma_multi(1, &w, &y, &n, x, k, s, false);
}

}  // namespace rt_hip
