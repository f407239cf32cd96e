// flow.hip -- a chain of dependent decode GEMV stages in one persistent launch.
//
// A decode token's linear work is a chain: q/k/v read RMSNorm(h), o reads
// the attention output, gate/up read RMSNorm(h + o), down reads
// silu(gate) * up, and the next layer reads h + down.  Launched one kernel
// per stage, every stage pays a kernel boundary plus the first-load latency
// of its weights.  Here one workgroup per CU stays resident for the whole
// chain and each stage hands its output to the next through memory:
//
//  * Outputs are tagged: every element is stored as one 64-bit word
//    {f32 bits, run tag} with an agent-scope atomic store, so a consumer
//    polls the data itself -- no flag, no barrier, no second hop.  The tag
//    is the run counter + 1 (SyncD::epoch, advanced by the run's last
//    workgroup), so a replayed launch never needs a reset.
//  * Weights never depend on the chain.  Every wave issues its input loads,
//    then at once the first weight loads of its share of the stage, so the
//    weights stream while the input is still being produced; the input
//    loads are the older ones, so waiting for them never waits for weights
//    (loads complete in order).  A stale input slot is read again until it
//    carries the run's tag.  The input lands in LDS as the Q4_K GEMV's int8
//    limbs (q4k_mfma.hpp) or the BF16 GEMV's piece layout (gemv_bf16.hpp),
//    with RMSNorm's gamma applied (its scale multiplies the finished dots).
//  * A stage runs on its first `wgs` workgroups (the host sizes it to the
//    stage's weight bytes: every taking part reads the whole input, so a
//    small stage spread over every CU would move more input than weight).
//  * Q4_K stages: 16-row tiles in the tiled layout; tile t of a round goes
//    to workgroup t mod wgs, split over KS waves by super-block (the host
//    picks KS so the stage uses every wave); partial rows are summed in LDS
//    in wave order.  A gate/up stage may pair its two jobs tile by tile
//    in one workgroup and also store silu(gate) * up, the down projection's
//    input.  BF16 stages: whole rows per wave, as the BF16 GEMV does.
//    Numerics are those of the stand-alone GEMVs.
//
// Every wait is bounded: a wait that runs out records 1 + its stage in the
// error word and the waits after it give up at once, so the grid always
// drains (the results of such a run are undefined; the host reports it).
// All G workgroups must be resident at once (the host launches one per CU).
#include "flow.hpp"
#include "gemv_bf16.hpp"
#include "q4k_mfma.hpp"

namespace rt_hip {
namespace flow {
namespace {

using namespace q4k_mfma;

constexpr int kXI = kMaxK / 4 / kThreads;  // input groups of 4 elements per thread, at most
constexpr int kD = 4;                      // Q4_K super-blocks in flight per wave
constexpr int kDB = 8;                     // BF16 pieces (1 KB of a row) in flight per wave
constexpr uint32_t kSpinLimit = 1u << 21;

// LDS: the staged input, the per-wave RMSNorm sums of squares, the Q4_K
// K-split partial rows, and two stage descriptors (the current stage's and
// the next one's, fetched during the current stage).
constexpr int kXOff = 0;
constexpr int kNormOff = 4 * kMaxK;
constexpr int kRedOff = kNormOff + 64;
constexpr int kDescOff = kRedOff + kMaxRounds * kWaves * 16 * 4;
constexpr int kDescBytes = static_cast<int>(sizeof(StageD));
constexpr int kLdsBytes = kDescOff + 2 * kDescBytes;
static_assert(kDescBytes == 256 && kDescBytes / 4 == kWave, "one dword of a descriptor per lane");

typedef __attribute__((address_space(1))) uint64_t g_u64;
typedef __attribute__((address_space(1))) uint32_t g_u32;
typedef __attribute__((address_space(1))) float g_f32;
typedef __attribute__((address_space(1))) const f32x4 g_f32x4;

// Global loads and stores through address-space-1 pointers: a pointer read
// from a descriptor is generic, and a flat access also counts against the
// LDS wait counter, so every LDS barrier would wait for it.
__device__ __forceinline__ f32x4 ld4(const float* p, int f) { return ((g_f32x4*)p)[f]; }
__device__ __forceinline__ float ld1(const float* p, int i) { return ((const g_f32*)p)[i]; }
__device__ __forceinline__ void st1(float* p, int i, float v) { ((g_f32*)p)[i] = v; }

// Tagged slots are read first through the XCD's L2 (workgroup scope: the
// line may be stale, which the tag shows), then, while stale, at agent scope
// (coherent across XCDs).  An agent-scope read also refreshes the L2 line,
// so the other CUs of the XCD then find the fresh value there.
__device__ __forceinline__ uint64_t ld_slot_l2(const uint64_t* p) {
    return __hip_atomic_load((g_u64*)const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint64_t ld_slot(const uint64_t* p) {
    return __hip_atomic_load((g_u64*)const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_slot(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store((g_u64*)p, (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_word(uint32_t* p) {
    return __hip_atomic_load((g_u32*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_word(uint32_t* p, uint32_t v) {
    __hip_atomic_store((g_u32*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool fresh(uint64_t v, uint32_t tag) { return static_cast<uint32_t>(v >> 32) == tag; }
__device__ __forceinline__ float value(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }
__device__ __forceinline__ int sreg(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float sreg(float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); }
// Descriptor fields live in LDS; read into scalar registers (a pointer in
// vector registers would turn every buffer load into a loop over lanes).
template <typename T>
__device__ __forceinline__ T* sreg(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
    return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// A wave's bounded wait: true to poll again, false once it gives up (its
// own limit, recorded in the error word, or another wait's).  Uniform.
__device__ __forceinline__ bool keep_waiting(uint32_t& spins, SyncD* sync, int stage, bool& ok, bool sleep = true) {
    if (!ok) return false;
    ++spins;
    if (spins > kSpinLimit) {
        st_word(&sync->err, 1u + static_cast<uint32_t>(stage));
        ok = false;
        return false;
    }
    if ((spins & 255u) == 0 && sreg(static_cast<int>(ld_word(&sync->err))) != 0) {
        ok = false;
        return false;
    }
    if (sleep) __builtin_amdgcn_s_sleep(1);
    return true;
}

// One lane's wait for a tagged element already read once into r.
__device__ __forceinline__ uint64_t wait_slot(const uint64_t* p, uint64_t r, uint32_t tag, SyncD* sync, int stage) {
    uint32_t spins = 0;
    while (!fresh(r, tag)) {
        if (++spins > kSpinLimit || ((spins & 255u) == 0 && ld_word(&sync->err) != 0)) {
            st_word(&sync->err, 1u + static_cast<uint32_t>(stage));
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        r = ld_slot(p);
    }
    return r;
}


// One thread's share of a stage's input: groups f = tid + kThreads * i of
// four consecutive elements (an aligned 8-lane group then holds one
// 32-element sub-block, as the limb conversion needs): tagged slots, or the
// values of an external input; and their gamma.  Loaded values are only
// used after the waits, so no load is waited for early.
struct XIn {
    uint64_t s[kXI][4];
    f32x4 e[kXI];
    f32x4 g[kXI];
};

// Issue the input loads (no wait).  Groups past the input (f >= nx) are
// zeros.
__device__ __forceinline__ void x_issue(XIn& X, const uint64_t* in_s, const float* in_e, const float* gamma,
                                        bool norm, int nx, int tid, uint32_t tag) {
    const uint64_t done = static_cast<uint64_t>(tag) << 32;
#pragma unroll
    for (int i = 0; i < kXI; ++i) {
        const int f = tid + kThreads * i;
        const bool live = f < nx;
        if (in_e) {
            X.e[i] = ld4(in_e, live ? f : 0);  // past the input: group 0, discarded
#pragma unroll
            for (int e = 0; e < 4; ++e) X.s[i][e] = done;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) X.s[i][e] = live ? ld_slot(in_s + 4 * f + e) : done;
        }
        if (norm) X.g[i] = ld4(gamma, live ? f : 0);
    }
}

// Wait until every slot of the wave carries the run's tag (bounded).  While
// slots are stale the wave polls one of them (every lane loads the same
// word: one request), then reads the stale ones again, so a wait costs the
// memory system a word per poll, not the whole input.
__device__ __forceinline__ void x_wait(XIn& X, const uint64_t* in_s, const float* in_e, int nx, int tid, int lane,
                                       uint32_t tag, SyncD* sync, int stage, bool& ok) {
    if (in_e) return;
    uint32_t spins = 0;
    for (;;) {
        int first = -1;  // this lane's first stale slot, as 4 * group + element
#pragma unroll
        for (int i = kXI - 1; i >= 0; --i)
#pragma unroll
            for (int e = 3; e >= 0; --e)
                if (!fresh(X.s[i][e], tag)) first = 4 * i + e;
        const uint64_t mask = __builtin_amdgcn_ballot_w64(first >= 0);
        if (mask == 0 || !ok) return;
        const int l0 = __builtin_ctzll(mask);
        const int m0 = __builtin_amdgcn_readlane(first, l0);
        const uint64_t* rep = in_s + 4 * (tid - lane + l0 + kThreads * (m0 >> 2)) + (m0 & 3);
        while (!fresh(ld_slot(rep), tag))
            if (!keep_waiting(spins, sync, stage, ok, false)) return;
#pragma unroll
        for (int i = 0; i < kXI; ++i) {
            const int f = tid + kThreads * i;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (f < nx && !fresh(X.s[i][e], tag)) X.s[i][e] = ld_slot(in_s + 4 * f + e);
        }
    }
}

// Group i of the input with gamma applied; the square sum accumulates the
// raw values (RMSNorm(x) * g = rms_inv * (x * g): the scale multiplies the
// finished dot products).
__device__ __forceinline__ f32x4 x_value(const XIn& X, int i, bool live, bool ext, int xop, float& sq) {
    f32x4 v = ext ? X.e[i] : f32x4{value(X.s[i][0]), value(X.s[i][1]), value(X.s[i][2]), value(X.s[i][3])};
    if (!live) v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (xop == kXRmsNorm || xop == kXRmsNorm1) {
        sq += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] *= xop == kXRmsNorm1 ? 1.0f + X.g[i][e] : X.g[i][e];
    }
    return v;
}

// The per-wave square sums to LDS (before the staging barrier) and, after
// it, the RMSNorm output scale 1 / sqrt(sum(x^2) / K + eps).
__device__ __forceinline__ void norm_part(uint8_t* lds, float sq, int lane, int wave) {
    sq = bf16_gemv::wave_sum(sq, lane);
    if (lane == 0) reinterpret_cast<float*>(lds + kNormOff)[wave] = sq;
}
__device__ __forceinline__ float norm_scale(const uint8_t* lds, int K, float eps) {
    const float* part = reinterpret_cast<const float*>(lds + kNormOff);
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += part[w];
    return 1.0f / __builtin_sqrtf(tot * (1.0f / static_cast<float>(K)) + eps);
}

// ---- Q4_K stage --------------------------------------------------------------
// Units are tiles of the stage's jobs in order or, for a paired stage
// (act >= 0: jobs 0 and 1 of equal length), unit 2p + q is tile p of job q.
// A workgroup's round r holds `per` tiles (paired: `per` pairs, tile slots
// 2m and 2m + 1 holding pair m).
__device__ __forceinline__ void run_q4k(const StageD& S, SyncD* sync, uint8_t* lds,
                                        uint32_t tag, int stage, bool& ok, int G, int blk, int tid, int lane,
                                        int wave) {
    const int K = sreg(S.k), nb = K >> 8, nx = K >> 2, units = sreg(S.units), KS = sreg(S.ks);
    const int xop = sreg(S.xop);
    const bool norm = xop == kXRmsNorm || xop == kXRmsNorm1;
    uint64_t* const act = sreg(S.act);
    const bool paired = act != nullptr;
    const int TPW = kWaves / KS;
    const int slot = wave / KS, kp = wave - slot * KS;
    const int bpw = (nb + KS - 1) / KS, b0 = kp * bpw;
    const int nbw = slot < TPW ? max(0, min(nb, b0 + bpw) - b0) : 0;
    const int per = paired ? TPW >> 1 : TPW;
    const int groups = paired ? units >> 1 : units;
    const int R = (groups + G * per - 1) / (G * per);
    const int L = R * nbw;
    const Lane ln = make_lane(lane, K);
    const TLane tl = make_tlane(lane);
    uint8_t* const limbs = lds + kXOff;
    float* const red = reinterpret_cast<float*>(lds + kRedOff);

    auto unit_of = [&](int r, int sl) {
        return paired ? 2 * ((r * per + (sl >> 1)) * G + blk) + (sl & 1) : (r * per + sl) * G + blk;
    };
    auto job_of = [&](int u) {
        int j = 0;
        if (paired) {
            j = u & 1;
        } else {
#pragma unroll
            for (int q = 1; q < kMaxJobs; ++q)
                if (u >= sreg(S.job[q].unit0)) j = q;
        }
        return j;
    };

    // 1. the input loads
    XIn X;
    const uint64_t* const in_s = sreg(S.in_s);
    const float* const in_e = sreg(S.in_e);
    x_issue(X, in_s, in_e, sreg(S.gamma), norm, nx, tid, tag);
    __builtin_amdgcn_sched_barrier(0);

    // 2. the weight prologue.  Issue cursor: round ir, block ip of the
    // round's tile, whose first block is at tb (rounds past the stage's
    // tiles read nothing).
    auto tile_ptr = [&](int r, uint32_t& bytes) -> const uint8_t* {
        const int u = unit_of(r, slot);
        const int j = job_of(u);
        const int tile = paired ? (u >> 1) : u - sreg(S.job[j].unit0);
        bytes = u < units ? static_cast<uint32_t>(kTiledBlockBytes) : 0u;
        return sreg(S.job[j].w) + (static_cast<int64_t>(tile) * nb + b0) * kTiledBlockBytes;
    };
    BlkT ring[kD];
    int ir = 0, ip = 0;
    uint32_t tbytes = 0;
    const uint8_t* tb = tile_ptr(0, tbytes);
    auto issue = [&](BlkT& r) {
        load_blk_t(make_rsrc_n(tb + ip * kTiledBlockBytes, tbytes), static_cast<uint32_t>(lane), r);
        if (ip == nbw - 1) {
            ip = 0;
            ++ir;
            tb = tile_ptr(ir, tbytes);
        } else {
            ++ip;
        }
    };
#pragma unroll
    for (int j = 0; j < kD; ++j) {
        if (j < L) issue(ring[j]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // 3. the residuals of this thread's rows (two store elements at most:
    // R * per * 16 <= 1024), read now so that the stores never wait.  The
    // jobs are visited in turn (their fields are scalars); each element
    // belongs to one of them.
    const int per_rows = per * 16;
    const int cnt = R * per_rows;
    uint64_t res[2] = {0, 0};      // tagged residuals
    float rese[2] = {0.0f, 0.0f};  // external ones
    const int njobs = sreg(S.njobs);
    if (!paired) {
        for (int j = 0; j < kMaxJobs; ++j) {
            if (j >= njobs) break;
            const JobD& J = S.job[j];
            const uint64_t* const as = sreg(J.add_s);
            const float* const ae = sreg(J.add_e);
            if (!as && !ae) continue;
            const int u0 = sreg(J.unit0), n = sreg(J.n), u1 = j + 1 < njobs ? sreg(S.job[j + 1].unit0) : units;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int e = tid + kThreads * q;
                const int r = e / per_rows, rem = e - r * per_rows;
                const int u = unit_of(r, rem >> 4);
                const int row = (u - u0) * 16 + (rem & 15);
                const bool mine = e < cnt && u >= u0 && u < u1 && row < n;
                if (ae) rese[q] = mine ? ld1(ae, row) : rese[q];
                else if (mine) res[q] = ld_slot_l2(as + row);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 4. wait for the input, stage it as limbs
    x_wait(X, in_s, in_e, nx, tid, lane, tag, sync, stage, ok);
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < kXI; ++i) {
        if (kThreads * i < nx) {  // uniform: the 8-lane reductions need whole groups
            const bool live = tid + kThreads * i < nx;
            limbs_of(x_value(X, i, live, in_e != nullptr, xop, sq), limbs, K, tid + kThreads * i, live);
        }
    }
    if (tid < 4) reinterpret_cast<u32x4*>(limbs + 3 * static_cast<size_t>(K))[tid] = u32x4{0u, 0u, 0u, 0u};
    if (norm) norm_part(lds, sq, lane, wave);
    lds_barrier();
    const float scale = norm ? norm_scale(lds, K, sreg(S.eps)) : 1.0f;

    // 5. stream the share
    float acc = 0.0f;
    int cr = 0, cp = 0;
    auto consume = [&](const Dec& dc) {
        acc = dot(dc, b0 + cp, ln, limbs, acc);
        if (cp == nbw - 1) {
            float v = acc;
            v += __shfl_xor(v, 16, kWave);
            v += __shfl_xor(v, 32, kWave);
            if (lane < 16) red[(cr * kWaves + wave) * 16 + lane] = v;
            acc = 0.0f;
        }
        const bool wrap = cp == nbw - 1;
        cp = sreg(wrap ? 0 : cp + 1);
        cr = sreg(wrap ? cr + 1 : cr);
    };
    int i = 0;
    for (; i + kD < L; i += kD) {
#pragma unroll
        for (int j = 0; j < kD; ++j) {
            const Dec dc = decode_t(ring[j], tl);
            __builtin_amdgcn_sched_barrier(0);
            issue(ring[j]);
            consume(dc);
        }
    }
#pragma unroll
    for (int j = 0; j < kD; ++j)
        if (i + j < L) consume(decode_t(ring[j], tl));
    lds_barrier();

    // 6. rows: the KS partials in wave order, the norm scale, the residual,
    // the tagged store (and the plain copy); paired: gate, up and
    // silu(gate) * up.
    auto partial = [&](int r, int sl, int n) {
        float sum = 0.0f;
        for (int q = 0; q < KS; ++q) sum += red[(r * kWaves + sl * KS + q) * 16 + n];
        return sum * scale;
    };
    if (paired) {
        uint64_t* const og = sreg(S.job[0].out);
        uint64_t* const ou = sreg(S.job[1].out);
        float* const pg = sreg(S.job[0].plain);
        float* const pu = sreg(S.job[1].plain);
        const int n = sreg(S.job[0].n);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int e = tid + kThreads * q;
            const int r = e / per_rows, rem = e - r * per_rows;
            const int sl = rem >> 4;
            const int u = unit_of(r, 2 * sl);  // the pair's gate tile
            const int row = (u >> 1) * 16 + (rem & 15);
            if (e < cnt && u < units && row < n) {
                const float gv = partial(r, 2 * sl, rem & 15), uv = partial(r, 2 * sl + 1, rem & 15);
                st_slot(og + row, gv, tag);
                st_slot(ou + row, uv, tag);
                st_slot(act + row, swiglu1(gv, uv), tag);
                if (pg) st1(pg, row, gv);
                if (pu) st1(pu, row, uv);
            }
        }
    } else {
        for (int j = 0; j < kMaxJobs; ++j) {
            if (j >= njobs) break;
            const JobD& J = S.job[j];
            uint64_t* const out = sreg(J.out);
            const uint64_t* const as = sreg(J.add_s);
            const float* const ae = sreg(J.add_e);
            float* const pl = sreg(J.plain);
            const int u0 = sreg(J.unit0), n = sreg(J.n), u1 = j + 1 < njobs ? sreg(S.job[j + 1].unit0) : units;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int e = tid + kThreads * q;
                const int r = e / per_rows, rem = e - r * per_rows;
                const int sl = rem >> 4;
                const int u = unit_of(r, sl);
                const int row = (u - u0) * 16 + (rem & 15);
                if (e < cnt && u >= u0 && u < u1 && row < n) {
                    float val = partial(r, sl, rem & 15);
                    if (ae) val = rese[q] + val;
                    else if (as) val = value(wait_slot(as + row, res[q], tag, sync, stage)) + val;
                    st_slot(out + row, val, tag);
                    if (pl) st1(pl, row, val);
                }
            }
        }
    }
}

// ---- BF16 stage --------------------------------------------------------------
__device__ __forceinline__ void run_bf16(const StageD& S, SyncD* sync, uint8_t* lds,
                                         uint32_t tag, int stage, bool& ok, int G, int blk, int tid, int lane,
                                         int wave) {
    const int K = sreg(S.k), N = sreg(S.job[0].n), nx = K >> 2;
    const int xop = sreg(S.xop);
    const bool norm = xop == kXRmsNorm || xop == kXRmsNorm1;
    const int P = (K + bf16_gemv::kPiece - 1) / bf16_gemv::kPiece;
    const int nx4 = P * (bf16_gemv::kPiece / 4);
    const int NW = G * kWaves, gw = blk * kWaves + wave;
    const int Rw = gw < N ? (N - 1 - gw) / NW + 1 : 0;
    const int L = Rw * P;
    const int64_t rowb = static_cast<int64_t>(K) * 2;
    const int64_t stride = static_cast<int64_t>(NW) * rowb;
    const uint8_t* const wb = sreg(S.job[0].w) + static_cast<int64_t>(gw) * rowb;
    const uint32_t loff = static_cast<uint32_t>(lane) * 16u;
    const JobD& J = S.job[0];

    XIn X;
    const uint64_t* const in_s = sreg(S.in_s);
    const float* const in_e = sreg(S.in_e);
    x_issue(X, in_s, in_e, sreg(S.gamma), norm, nx, tid, tag);
    __builtin_amdgcn_sched_barrier(0);

    u32x4 ring[kDB];
    int ir = 0, ip = 0;
    auto issue = [&](u32x4& r) {
        const int64_t o = static_cast<int64_t>(ip) * (bf16_gemv::kPiece * 2);
        r = ld16(make_rsrc(wb + ir * stride + o, ir < Rw ? rowb - o : 0), loff);
        const bool wrap = ip == P - 1;
        ip = sreg(wrap ? 0 : ip + 1);
        ir = sreg(wrap ? ir + 1 : ir);
    };
#pragma unroll
    for (int j = 0; j < kDB; ++j) {
        if (j < L) issue(ring[j]);
        __builtin_amdgcn_sched_barrier(0);
    }

    const uint64_t* const as = sreg(J.add_s);
    const float* const ae = sreg(J.add_e);
    uint64_t res = 0;
    float rese = 0.0f;
    const int rrow = lane < Rw ? gw + lane * NW : 0;
    if (ae) rese = ld1(ae, rrow);
    else if (as && lane < Rw) res = ld_slot_l2(as + rrow);
    __builtin_amdgcn_sched_barrier(0);

    x_wait(X, in_s, in_e, nx, tid, lane, tag, sync, stage, ok);
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < kXI; ++i) {
        const int f = tid + kThreads * i;
        if (f < nx4) {
            const f32x4 v = x_value(X, i, f < nx, in_e != nullptr, xop, sq);
            *reinterpret_cast<f32x4*>(lds + kXOff + bf16_gemv::x_off(f)) = v;
        }
    }
    if (norm) norm_part(lds, sq, lane, wave);
    lds_barrier();
    const float scale = norm ? norm_scale(lds, K, sreg(S.eps)) : 1.0f;

    const uint8_t* const xs = lds + kXOff;
    float acc = 0.0f, rsum = 0.0f;
    int cr = 0, cp = 0;
    auto consume = [&](const u32x4 w) {
        const f32x4 xa = *reinterpret_cast<const f32x4*>(xs + ((((cp << 1) + 0) << 6) + lane) * 16);
        const f32x4 xb = *reinterpret_cast<const f32x4*>(xs + ((((cp << 1) + 1) << 6) + lane) * 16);
        float a = acc;
        a = __builtin_fmaf(bf16_lo_to_f32(w[0]), xa[0], a);
        a = __builtin_fmaf(bf16_hi_to_f32(w[0]), xa[1], a);
        a = __builtin_fmaf(bf16_lo_to_f32(w[1]), xa[2], a);
        a = __builtin_fmaf(bf16_hi_to_f32(w[1]), xa[3], a);
        a = __builtin_fmaf(bf16_lo_to_f32(w[2]), xb[0], a);
        a = __builtin_fmaf(bf16_hi_to_f32(w[2]), xb[1], a);
        a = __builtin_fmaf(bf16_lo_to_f32(w[3]), xb[2], a);
        a = __builtin_fmaf(bf16_hi_to_f32(w[3]), xb[3], a);
        acc = a;
        if (cp == P - 1) {
            const float v = bf16_gemv::wave_sum(acc, lane);
            rsum = lane == cr ? v : rsum;
            acc = 0.0f;
        }
        const bool wrap = cp == P - 1;
        cp = sreg(wrap ? 0 : cp + 1);
        cr = sreg(wrap ? cr + 1 : cr);
    };
    int i = 0;
    for (; i + kDB < L; i += kDB) {
#pragma unroll
        for (int j = 0; j < kDB; ++j) {
            const u32x4 w = ring[j];
            __builtin_amdgcn_sched_barrier(0);
            issue(ring[j]);
            consume(w);
        }
    }
#pragma unroll
    for (int j = 0; j < kDB; ++j)
        if (i + j < L) consume(ring[j]);
    // Every wave is past its last read of the staged input before the next
    // stage overwrites it.
    lds_barrier();

    if (lane < Rw) {
        const int row = gw + lane * NW;
        float val = rsum * scale;
        if (ae) val = rese + val;
        else if (as) val = value(wait_slot(as + row, res, tag, sync, stage)) + val;
        st_slot(sreg(J.out) + row, val, tag);
        float* const pl = sreg(J.plain);
        if (pl) st1(pl, row, val);
    }
}

// Whether workgroup blk has rows in stage S (uniform over the workgroup).
__device__ __forceinline__ bool has_work(const StageD& S, int blk) {
    const int units = sreg(S.units);
    if (blk >= sreg(S.wgs)) return false;
    if (sreg(S.kind) != kQ4K) return blk * kWaves < units;
    return blk < (sreg(S.act) ? units >> 1 : units);
}

__global__ __launch_bounds__(kThreads) void k_flow(const StageD* __restrict__ st, int nst,
                                                   SyncD* __restrict__ sync) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int G = static_cast<int>(gridDim.x), blk = static_cast<int>(blockIdx.x);
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = sreg(tid >> 6);
    const uint32_t tag = static_cast<uint32_t>(sreg(static_cast<int>(ld_word(&sync->epoch)))) + 1u;
    uint32_t* const desc = reinterpret_cast<uint32_t*>(lds + kDescOff);
    if (wave == 0) desc[lane] = reinterpret_cast<const uint32_t*>(st)[lane];
    lds_barrier();
    bool ok = true;
    for (int s = 0; s < nst; ++s) {
        const StageD& S = *reinterpret_cast<const StageD*>(desc + (s & 1) * kWave);
        // the next stage's descriptor: loaded first (the oldest load of the
        // stage), landed in the other LDS slot at the end of this one
        uint32_t next = 0;
        if (wave == 0 && s + 1 < nst) next = reinterpret_cast<const uint32_t*>(st + s + 1)[lane];
        if (has_work(S, blk)) {
            const int Gs = sreg(S.wgs);
            if (sreg(S.kind) == kQ4K)
                run_q4k(S, sync, lds, tag, s, ok, Gs, blk, tid, lane, wave);
            else
                run_bf16(S, sync, lds, tag, s, ok, Gs, blk, tid, lane, wave);
        }
        if (wave == 0) desc[((s + 1) & 1) * kWave + lane] = next;
        lds_barrier();
    }
    // The run's last workgroup to arrive advances the run counter; every
    // workgroup read it at its start, before arriving.
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add((g_u32*)&sync->arrive, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        if (old == static_cast<uint32_t>(G - 1)) {
            st_word(&sync->arrive, 0u);
            st_word(&sync->epoch, tag);
        }
    }
}

}  // namespace

size_t lds_bytes() { return kLdsBytes; }

hipError_t launch(const StageD* stages, int nstages, SyncD* sync, int workgroups, hipStream_t stream) {
    hipLaunchKernelGGL(k_flow, dim3(static_cast<unsigned>(workgroups)), dim3(kThreads), kLdsBytes, stream, stages,
                       nstages, sync);
    return hipGetLastError();
}

}  // namespace flow
}  // namespace rt_hip
