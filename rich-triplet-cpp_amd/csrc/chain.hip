// chain.hip -- a decode step's dependent Q4_K GEMVs in one persistent launch.
//
// A decode step is a chain of GEMV stages: each stage's activation is
// produced by the stages before it (q/k/v -> attention -> o -> norm ->
// gate/up -> SwiGLU -> down -> next layer).  Launched one kernel per stage,
// every stage pays the launch gap, the kernel-argument fetch and the
// first-load latency of HBM before any weight byte arrives, so a 3B model's
// 113 stages spend more time starting than streaming.
//
// Here one workgroup per CU stays resident for the whole chain.  Every wave
// owns a fixed share of each stage (a 16-row tile, or 1/KS of one).  Weights
// never depend on the chain, so a wave may issue P of its share's first D
// weight loads for stage s+1 before stage s is complete on the other CUs;
// only the activation waits: after a stage barrier the workgroup copies x
// into LDS (coherent loads), converts it to int8 limbs (q4k_mfma.hpp) and
// computes.
//
// Measured on MI355X (Llama-3.2-3B shapes, pure Q4_K, 113 stages): the stage
// handoff -- coherent output stores and their acknowledgement, the two-level
// flag barrier, the coherent copy of x -- costs about as much as a kernel
// boundary, and loads issued before the barrier queue in the CU's memory
// pipeline ahead of the barrier's polls (P = 0: 877 us per step, P = 4:
// 937 us, one launch per stage: 743 us).  The default is P = 0.
//
// Stage barrier: each workgroup publishes "stage s done" in its own flag
// (one 64-byte line); the first workgroup of every group of 32 polls its
// members' flags and publishes a group flag in 32 replicas; every workgroup
// polls one replica set.  Flags only grow: a run's targets are the
// workgroup's own flag value at kernel start plus the stage number, so
// repeated runs (and hipGraph replays) need no reset.  Every poll is bounded;
// a poll that runs out sets the chain's error word, and every later poll of
// the run gives up at once, so the grid always drains.
//
// Coherence: outputs are stored with agent-scope (sc1, write-through)
// stores, each storing wave waits for its stores before the workgroup's flag
// is published, and activations are read with sc1 loads, so a stage may
// read any earlier stage's output without an L2 writeback or invalidate.
//
// Numerics: each tile is computed exactly as by k_gemv_q4k_mfma with the
// same K split (int8 MFMA on exact limbs, f32 epilogue); the KS partial rows
// are summed in part order.
#include "q4k_mfma.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

using namespace q4k_mfma;

constexpr int kWaves = 16;  // waves per workgroup (one workgroup per CU)
constexpr int kThreads = kWaves * kWave;
constexpr int kJobs = 4;
constexpr int kGroup = 32;       // workgroups per first-level flag group
constexpr int kReplicas = 32;    // copies of each group flag
constexpr int kFlagDw = 16;      // dwords between flags: one 64-byte line each
constexpr int kReplicaDw = 1024; // dwords between replica sets (4 KB)
constexpr int kMaxGroups = kReplicaDw / kFlagDw;
constexpr int kSpinLimit = 1 << 20;
constexpr int kMaxK = 8192;      // x staging: two f32x4 per thread

// One stage in device memory (read with scalar loads).  Job j owns tiles
// [tile0[j], tile0[j + 1]); unused entries hold `tiles`.
struct Stage {
    const float* x;
    const uint8_t* w[kJobs];
    float* y[kJobs];
    int n[kJobs];
    int tile0[kJobs];
    int k, ks, tiles, rounds;
};

// Device-side state: per-workgroup flags, replicated group flags, error word.
struct Sync {
    uint32_t* flags;
    uint32_t* gflags;
    uint32_t* err;
};

__device__ __forceinline__ uint32_t ld_coherent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Through a global-address-space pointer: a flat store (the default for a
// pointer read from memory) also counts as a possible LDS access, and the
// compiler then waits for every load in flight before the next LDS read.
__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store((__attribute__((address_space(1))) float*)p, v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int sreg(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <typename T>
__device__ __forceinline__ T* sreg(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
    return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}
// Pick entry j of four scalars.  Every field is read into an SGPR first:
// a select over loaded values would otherwise become one load from a
// selected address, issued as a vector load in the middle of the ring's.
template <typename T>
__device__ __forceinline__ T pick4(int j, T a, T b, T c, T d) {
    return j == 3 ? d : (j == 2 ? c : (j == 1 ? b : a));
}

// A wave's share of one stage round: blocks [b0, b0 + nbw) of one tile.
struct Unit {
    const uint8_t* base;  // block b0 of the tile (tiled layout)
    int64_t left;         // readable bytes from base; 0 = no tile (loads read zeros)
    float* y;             // output of the tile's row 0
    int rows;             // rows to store (0 = none)
    int b0, nbw;
};

__device__ __forceinline__ Unit make_unit(const Stage* __restrict__ st, int s, int r, int wg, int G,
                                          int wave) {
    const Stage& S = st[s];
    const int ks = sreg(S.ks), nb = sreg(S.k) >> 8, tiles = sreg(S.tiles);
    const int bpw = nb / ks;  // the host picks ks | nb
    const int tpw = kWaves / ks;
    const int tslot = wave / ks, part = wave - tslot * ks;
    const int t = (r * tpw + tslot) * G + wg;
    const int t1 = sreg(S.tile0[1]), t2 = sreg(S.tile0[2]), t3 = sreg(S.tile0[3]);
    const int j = (t >= t1 ? 1 : 0) + (t >= t2 ? 1 : 0) + (t >= t3 ? 1 : 0);
    const uint8_t* w = pick4(j, sreg(S.w[0]), sreg(S.w[1]), sreg(S.w[2]), sreg(S.w[3]));
    float* y = pick4(j, sreg(S.y[0]), sreg(S.y[1]), sreg(S.y[2]), sreg(S.y[3]));
    const int n = pick4(j, sreg(S.n[0]), sreg(S.n[1]), sreg(S.n[2]), sreg(S.n[3]));
    const int t0 = pick4(j, 0, t1, t2, t3);
    const bool valid = t < tiles;
    const int lt = t - t0;
    const int64_t job_bytes = static_cast<int64_t>((n + 15) >> 4) * nb * kTiledBlockBytes;
    const int64_t off = (static_cast<int64_t>(lt) * nb + part * bpw) * kTiledBlockBytes;
    Unit u;
    u.base = w + (valid ? off : 0);
    u.left = valid ? job_bytes - off : 0;
    u.y = y + (valid ? 16 * lt : 0);
    const int rows = n - 16 * lt;
    u.rows = (valid && part == 0) ? (rows < 16 ? rows : 16) : 0;
    u.b0 = part * bpw;
    u.nbw = bpw;
    return u;
}

// Wave 0 waits until every workgroup has published `want`; the other waves
// wait at the barrier that follows.
__device__ __forceinline__ void stage_wait(const Sync& sy, uint32_t want, int wg, int G, int lane) {
    if (ld_coherent(sy.err) != 0) return;  // an earlier poll gave up: drain
    const int g = wg / kGroup, ng = (G + kGroup - 1) / kGroup;
    int it = 0;
    bool ok = true;
    if (wg % kGroup == 0) {
        const int m = g * kGroup + lane;
        for (;;) {
            const uint32_t v = (lane < kGroup && m < G) ? ld_coherent(&sy.flags[m * kFlagDw]) : want;
            if (__all(static_cast<int32_t>(v - want) >= 0)) break;
            if (++it > kSpinLimit) {
                ok = false;
                break;
            }
        }
        if (ok && lane < kReplicas) st_coherent(&sy.gflags[lane * kReplicaDw + g * kFlagDw], want);
    }
    const int rep = wg % kReplicas;
    while (ok) {
        const uint32_t v = lane < ng ? ld_coherent(&sy.gflags[rep * kReplicaDw + lane * kFlagDw]) : want;
        if (__all(static_cast<int32_t>(v - want) >= 0)) break;
        if (++it > kSpinLimit) ok = false;
        if ((it & 1023) == 0 && ld_coherent(sy.err) != 0) break;
    }
    if (!ok && lane == 0) st_coherent(sy.err, 1u);
}

// D: ring depth (super-blocks in flight per wave).  P <= D of them are
// loaded for stage s+1 before the stage barrier; the rest after x is staged.
// Everything issued before the barrier sits in the CU's memory queue ahead
// of the barrier's polls and the activation copies, so P trades weight
// prefetch against handoff latency.
template <int D, int P>
__global__ __launch_bounds__(kThreads) void k_chain(const Stage* __restrict__ st, int nst, Sync sy) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = sreg(tid >> 6);
    const int wg = blockIdx.x, G = gridDim.x;
    const TLane tl = make_tlane(lane);
    float* const red = reinterpret_cast<float*>(lds + stage_bytes(kMaxK));  // [tile slot][part][16]

    // Run epoch: this workgroup's own flag (all flags advance together).
    const uint32_t e0 = static_cast<uint32_t>(sreg(static_cast<int>(ld_coherent(&sy.flags[wg * kFlagDw]))));

    BlkT ring[D];
    auto issue = [&](BlkT& slot, const Unit& u, int i) {
        const int64_t o = static_cast<int64_t>(i) * kTiledBlockBytes;
        load_blk_t(make_rsrc(u.base + o, i < u.nbw ? u.left - o : 0), static_cast<uint32_t>(lane), slot);
    };
    auto prologue = [&](const Unit& u, int lo, int hi) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if (j >= lo && j < hi) {
                issue(ring[j], u, j);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    Unit u = make_unit(st, 0, 0, wg, G, wave);
    prologue(u, 0, P);

    for (int s = 0; s < nst; ++s) {
        const int K = st[s].k, ks = st[s].ks, R = st[s].rounds;
        if (s > 0) {
            if (wave == 0) stage_wait(sy, e0 + static_cast<uint32_t>(s), wg, G, lane);
            lds_barrier();
        }
        // x -> LDS (raw f32, coherent copies), then limb planes in place.
        const float* X = st[s].x;
        for (int c = wave; c < (K >> 8); c += kWaves)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(X + c * 256 + lane * 4),
                                             (__attribute__((address_space(3))) void*)(lds + c * 1024), 16, 0,
                                             16 /* sc1 */);
        wait_vmcnt<0>();
        lds_barrier();
        const int nx = K >> 2;
        f32x4 xv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int f = tid + kThreads * i;
            xv[i] = *reinterpret_cast<const f32x4*>(lds + 16 * (f < nx ? f : 0));
        }
        lds_barrier();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int f = tid + kThreads * i;
            limbs_of(xv[i], lds, K, f, f < nx);
        }
        if (tid < 4) reinterpret_cast<u32x4*>(lds + 3 * static_cast<size_t>(K))[tid] = u32x4{0u, 0u, 0u, 0u};
        lds_barrier();
        prologue(u, P, D);

        const Lane ln = make_lane(lane, K);
        const int tslot = wave / ks, part = wave - tslot * ks;
        for (int r = 0; r < R; ++r) {
            // The ring holds u's first D blocks.  Straight-line steady
            // rounds, then a tail that issues nothing (as k_gemv_q4k_mfma).
            const int nbw = u.nbw;
            float acc = 0.0f;
            int i = 0;
            for (; i + D < nbw; i += D) {
#pragma unroll
                for (int j = 0; j < D; ++j) {
                    const Dec dc = decode_t(ring[j], tl);
                    __builtin_amdgcn_sched_barrier(0);
                    issue(ring[j], u, i + D + j);
                    acc = dot(dc, u.b0 + i + j, ln, lds, acc);
                }
            }
#pragma unroll
            for (int j = 0; j < D; ++j)
                if (i + j < nbw) acc = dot(decode_t(ring[j], tl), u.b0 + i + j, ln, lds, acc);

            float v = acc;
            v += __shfl_xor(v, 16, kWave);
            v += __shfl_xor(v, 32, kWave);
            if (ks > 1) {
                float* rp = red + tslot * ks * 16;
                if (lane < 16) rp[part * 16 + lane] = v;
                lds_barrier();
                if (part == 0) {
                    float sum = rp[lane & 15];
                    for (int q = 1; q < ks; ++q) sum += rp[q * 16 + (lane & 15)];
                    v = sum;
                }
            }
            if (u.rows > 0) {
                if (lane < u.rows) st_coherent(u.y + lane, v);
                wait_vmcnt<0>();  // stored before this workgroup publishes
            }
            // Next share: the stage's next round, else the next stage's first.
            // Stores (outputs, the flag) are complete before the next loads
            // are issued: vmcnt counts both, and with a store pending among
            // the ring's loads the compiler can only wait for zero.
            const bool more = r + 1 < R;
            const int ns = more ? s : s + 1;
            if (!more && ns < nst) {
                lds_barrier();  // every wave's outputs are stored
                if (tid == 0) st_coherent(&sy.flags[wg * kFlagDw], e0 + static_cast<uint32_t>(s + 1));
                wait_vmcnt<0>();
            }
            if (ns < nst) {
                u = make_unit(st, ns, more ? r + 1 : 0, wg, G, wave);
                prologue(u, 0, more ? D : P);
            }
            if (ks > 1 && more) lds_barrier();  // partial rows are read before reuse
        }
    }
}

}  // namespace

size_t chain_lds_bytes() { return stage_bytes(kMaxK) + static_cast<size_t>(kWaves) * 16 * sizeof(float); }

int chain_threads() { return kThreads; }

int chain_max_k() { return kMaxK; }

size_t chain_err_word(int grid) {
    return static_cast<size_t>(grid) * kFlagDw + static_cast<size_t>(kReplicas) * kReplicaDw;
}

size_t chain_sync_words(int grid) { return chain_err_word(grid) + kFlagDw; }

int chain_max_grid() { return kMaxGroups * kGroup; }

// Stage table layout for the host (mirrors Stage).
size_t chain_stage_bytes() { return sizeof(Stage); }

void chain_fill_stage(void* dst, const float* x, int count, const void* const* w, float* const* y,
                      const int64_t* n, int64_t k, int ks, int tiles, int rounds, const int* tile0) {
    Stage S{};
    S.x = x;
    for (int j = 0; j < kJobs; ++j) {
        const int jj = j < count ? j : 0;
        S.w[j] = static_cast<const uint8_t*>(w[jj]);
        S.y[j] = y[jj];
        S.n[j] = static_cast<int>(n[jj]);
        S.tile0[j] = j < count ? tile0[j] : tiles;
    }
    S.k = static_cast<int>(k);
    S.ks = ks;
    S.tiles = tiles;
    S.rounds = rounds;
    *static_cast<Stage*>(dst) = S;
}

int chain_waves_per_wg() { return kWaves; }

hipError_t chain_occupancy(int* blocks_per_cu) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_chain<4, 4>, kThreads, chain_lds_bytes());
}

hipError_t launch_chain(const void* stages, int nst, uint32_t* sync_words, int grid, hipStream_t s) {
    Sync sy;
    sy.flags = sync_words;
    sy.gflags = sync_words + static_cast<size_t>(grid) * kFlagDw;
    sy.err = sync_words + chain_err_word(grid);
    const Stage* st = static_cast<const Stage*>(stages);
    const int pre = tune_param("CHAIN_PREFETCH", 0);
    const dim3 g(static_cast<unsigned>(grid)), b(kThreads);
    const size_t lds = chain_lds_bytes();
    if (pre <= 0)
        hipLaunchKernelGGL((k_chain<4, 0>), g, b, lds, s, st, nst, sy);
    else if (pre == 1)
        hipLaunchKernelGGL((k_chain<4, 1>), g, b, lds, s, st, nst, sy);
    else if (pre == 2)
        hipLaunchKernelGGL((k_chain<4, 2>), g, b, lds, s, st, nst, sy);
    else
        hipLaunchKernelGGL((k_chain<4, 4>), g, b, lds, s, st, nst, sy);
    return hipGetLastError();
}

}  // namespace rt_hip
