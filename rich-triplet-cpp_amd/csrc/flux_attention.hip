// flux_attention.hip -- FLUX's multi-head attention with no mask (every token
// attends to every token), streamed over key tiles with an online softmax:
// the reference's flux_attention (src/shaders/flux.msl:145-331) and the CPU
// attention it replaces (src/flux.cpp:282-323).
//
// q, k, v, out: [T][n_heads * D] f32 rows; D = head_dim, a multiple of 8 up
// to 128 (the reference's limits, metal_flux.mm:443-452).
// out[i][h] = sum_j softmax_j(scale * q_i . k_j) v_j for head h.
//
// A workgroup owns a block of 128 queries of one head (8 waves x 16) and
// streams K and V once for all of them in tiles of 32 keys through a
// two-stage LDS ring (2 x 32 KB at D = 128: two workgroups per CU): the
// tiles are copied straight from memory into LDS by buffer loads (no
// registers), the next tile's copy in flight while the current one is
// used.  The products run in f32 on the matrix cores
// (v_mfma_f32_16x16x4_f32), so every product and partial sum is an f32
// operation, as in the reference:
//  * S^T = K Q^T per 16-key x 16-query tile: lane (g = l/16, n = l%16)
//    supplies K[key n][dim] and Q[query n][dim] for the same dim, so any
//    assignment of dims to (k-step, lane group) is a valid contraction; dims
//    16a + 4g + b over steps 4a + b let each lane read 4 consecutive dims
//    with one 16-byte LDS read.  The result leaves lane (g, n) holding the
//    scores of query n against keys 16t + 4g + r (t over the tile's two
//    16-key halves).
//  * Online softmax per query: the running maximum and denominator; the
//    accumulator is rescaled by exp(m_old - m_new) before the tile is folded
//    in (flux.msl:232-271).
//  * O^T += V^T P^T: lane (g, n) supplies P[query n][key 16t + 4g + r] --
//    exactly the score it holds -- and V[key 16t + 4g + r][dim 16c + n], so
//    V stays key-major in LDS (as the copy writes it) and the result leaves
//    lane (g, n) holding O[query n][dims 16c + 4g .. + 3]: its own query,
//    rescaled by its own factor and stored as one 16-byte write.
// The head is padded to DP in {32, 64, 128} dims with zeros (they add
// nothing to a score and are never stored).  Keys past T are masked to -inf
// (weight 0), their tile rows zero-filled by the copy's range check; query
// rows past T are computed and not stored.  LDS rows are XOR-swizzled
// (K by 16-byte granule, V by 16-dim block) so that the reads above hit
// distinct banks; the copies apply the swizzle on the memory side.
#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kBQ = 16 * kWaves;  // queries per workgroup
constexpr int kBK = 32;           // keys per tile
constexpr int kNT = kBK / 16;     // 16-key MFMA tiles per key tile
constexpr float kLog2e = 1.44269504088896341f;
constexpr uint32_t kNoRead = 0x7ffffff0u;  // past every tile's range: the copy writes zeros

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

template <int DP>
constexpr int stage_floats() {
    return 2 * kBK * DP;  // K tile, then V tile
}
template <int DP>
constexpr size_t flux_lds_bytes() {
    return static_cast<size_t>(2) * stage_floats<DP>() * 4;
}

// float offset of K[key][granule gr] (4 dims): granule slot gr ^ (key & mask)
template <int DP>
__device__ __forceinline__ int k_off(int key, int gr) {
    constexpr int kMask = (DP / 4 < 16 ? DP / 4 : 16) - 1;
    return key * DP + ((gr ^ (key & kMask)) << 2);
}
// V[key][dim] sits at dim ^ v_sw(key): the 16-dim blocks of keys 4j .. 4j + 3
// are exchanged by j (mod DP / 16, at most 4), so the four keys 4g + r
// (g = 0..3) that one PV read touches fall in four different bank groups.
template <int DP>
__device__ __forceinline__ int v_sw(int key) {
    constexpr int kMask = (DP / 16 < 4 ? DP / 16 : 4) - 1;
    return ((key >> 2) & kMask) << 4;
}

// Partial states of a split query block: O [kBQ][DP], then m [kBQ], l [kBQ].
template <int DP>
constexpr int piece_floats() {
    return kBQ * DP + 2 * kBQ;
}

// Stored and reloaded with agent-scope (device-coherent) accesses: they
// bypass the per-XCD L2, so the workgroup that merges sees the other
// workgroup's stores once those have completed.
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store((__attribute__((address_space(1))) float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load((const __attribute__((address_space(1))) float*)p, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Work: item i = (head i / nqb, query block i % nqb) over key tiles
// [0, ntile).  Without `part` workgroup (head, block) = (blockIdx.x,
// blockIdx.y) does one whole item.  With it (more items than workgroup
// slots) the flat sequence of (item, tile) units is cut into gridDim.x equal
// ranges of `per` >= ntile units, one per workgroup, so every workgroup does
// the same work and no partial round is left at the end.  An item cut by
// the boundary between workgroups w and w + 1 has two pieces: each stores
// its state (o, m, l) in part[w][piece] and counts its arrival in cnt[w];
// the second to arrive merges the two states and stores the output.
// Two workgroups per CU (4 waves per SIMD): at most 128 VGPRs.
template <int DP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_flux_attn(
    const float* __restrict__ Q, const float* __restrict__ K,
                                                        const float* __restrict__ V, float* __restrict__ O, int T,
                                                        int n_heads, int D, float scale, float* __restrict__ part,
                                                        uint32_t* __restrict__ cnt, int per) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ uint32_t arrival;
    constexpr int NA = DP / 16;
    constexpr int SF = stage_floats<DP>();
    // Copy roles: a tile of one operand is DP / 8 instructions of 1 KB (64
    // lanes x 16 bytes); wave w issues instructions w and w + 8.  Lane l of
    // instruction j fills LDS granule 64 j + l = (key, slot) of the tile with
    // the memory granule the swizzle puts there (offsets relative to the
    // tile's first row, below 2^31 (key * stride * 4 < 32 * 2^26); dims past
    // D read nothing).
    constexpr int NI = DP / 8, CPW = (NI + kWaves - 1) / kWaves;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int64_t stride = static_cast<int64_t>(n_heads) * D;
    const int ntile = (T + kBK - 1) / kBK, nqb = (T + kBQ - 1) / kBQ;

    // the units of this workgroup
    int64_t u, u_end;
    if (part) {
        u = static_cast<int64_t>(blockIdx.x) * per;
        u_end = min(u + per, static_cast<int64_t>(n_heads) * nqb * ntile);
    } else {
        const int64_t item = static_cast<int64_t>(blockIdx.x) * nqb + blockIdx.y;
        u = item * ntile;
        u_end = u + ntile;
    }
    while (u < u_end) {
        const int64_t item = u / ntile;
        const int t0 = static_cast<int>(u % ntile);
        const int t1 = static_cast<int>(min(static_cast<int64_t>(ntile), t0 + (u_end - u)));
        u += t1 - t0;
        const int head = static_cast<int>(item / nqb), q0 = static_cast<int>(item % nqb) * kBQ;
        const float* kb = K + static_cast<int64_t>(head) * D;
        const float* vb = V + static_cast<int64_t>(head) * D;
        auto copy_tile = [&](int tile, float* st) {
            const int base = tile * kBK, rows = min(kBK, T - base);
            const uint32_t bytes = static_cast<uint32_t>(((rows - 1) * stride + D) * 4);
            const BufRsrc rk = make_rsrc_n(kb + base * stride, bytes);
            const BufRsrc rv = make_rsrc_n(vb + base * stride, bytes);
#pragma unroll
            for (int i = 0; i < CPW; ++i) {
                const int j = wave + kWaves * i;
                if (j >= NI) break;  // wave-uniform
                const int G = 64 * j + lane;
                const int key = G / (DP / 4), slot = G % (DP / 4);
                const int kd = 4 * (slot ^ (key & ((DP / 4 < 16 ? DP / 4 : 16) - 1)));
                const int vd = (4 * slot) ^ v_sw<DP>(key);
                const int row = key * static_cast<int>(stride);
                const uint32_t koff = kd < D ? static_cast<uint32_t>((row + kd) * 4) : kNoRead;
                const uint32_t voff = vd < D ? static_cast<uint32_t>((row + vd) * 4) : kNoRead;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rk, (__attribute__((address_space(3))) void*)(st + j * 256), 16, static_cast<int>(koff), 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rv, (__attribute__((address_space(3))) void*)(st + kBK * DP + j * 256), 16,
                    static_cast<int>(voff), 0, 0, 0);
            }
        };

        // this lane's query row (n of the wave's 16): dims 16a + 4g .. + 3
        const int qrow = q0 + wave * 16 + n;
        const float* qb = Q + static_cast<int64_t>(head) * D;
        float qf[4 * NA];
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            f32x4 v4 = {0.0f, 0.0f, 0.0f, 0.0f};
            if (qrow < T && 16 * a + 4 * g < D)
                v4 = *reinterpret_cast<const f32x4*>(qb + qrow * stride + 16 * a + 4 * g);
#pragma unroll
            for (int b = 0; b < 4; ++b) qf[4 * a + b] = v4[b];
        }
        f32x4 o[NA];  // o[c][r]: O[query n][dim 16c + 4g + r]
#pragma unroll
        for (int c = 0; c < NA; ++c) o[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float m_run = -__builtin_inff(), l_run = 0.0f;  // of query n

        // The previous item's last barrier ended every read of the ring.
        copy_tile(t0, lds);
        wait_vmcnt<0>();
        __syncthreads();
        for (int tile = t0; tile < t1; ++tile) {
            const float* ks = lds + ((tile - t0) & 1) * SF;
            const float* vs = ks + kBK * DP;
            // the next tile into the other stage (last read before the previous barrier)
            if (tile + 1 < t1) copy_tile(tile + 1, lds + ((tile + 1 - t0) & 1) * SF);
            const int base = tile * kBK;

            // S^T: the tile's 16-key halves against the wave's 16 queries
            f32x4 st[kNT];
#pragma unroll
            for (int t = 0; t < kNT; ++t) {
                f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int a = 0; a < NA; ++a) {
                    const f32x4 k4 = *reinterpret_cast<const f32x4*>(ks + k_off<DP>(16 * t + n, 4 * a + g));
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        c = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[b], qf[4 * a + b], c, 0, 0, 0);
                }
                st[t] = c;
            }
            // scale, mask, the tile's maximum for query n (8 in lane, 4 lanes)
            float mx = -__builtin_inff();
#pragma unroll
            for (int t = 0; t < kNT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool valid = base + 16 * t + 4 * g + r < T;
                    st[t][r] = valid ? st[t][r] * scale : -__builtin_inff();
                    mx = fmaxf(mx, st[t][r]);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
            mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
            const float m_new = fmaxf(m_run, mx);  // finite: key `base` is valid
            const float alpha = exp_fast(m_run - m_new);  // 0 on the first tile
            float sum = 0.0f;
#pragma unroll
            for (int t = 0; t < kNT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    st[t][r] = exp_fast(st[t][r] - m_new);  // -inf -> 0
                    sum += st[t][r];
                }
            sum += __shfl_xor(sum, 16, kWave);
            sum += __shfl_xor(sum, 32, kWave);
            l_run = l_run * alpha + sum;
            m_run = m_new;
#pragma unroll
            for (int c = 0; c < NA; ++c) o[c] *= alpha;
            // O^T += V^T P^T
#pragma unroll
            for (int t = 0; t < kNT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = 16 * t + 4 * g + r;
                    const float* vrow = vs + key * DP;
                    const int sw = v_sw<DP>(key);
#pragma unroll
                    for (int c = 0; c < NA; ++c)
                        o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[(16 * c + n) ^ sw], st[t][r], o[c], 0, 0, 0);
                }
            // this wave's copy of the next tile has landed; after the barrier
            // every wave's has, and every wave is done with this stage
            wait_vmcnt<0>();
            __syncthreads();
        }

        if (t0 > 0 || t1 < ntile) {
            // One of two pieces of the item: its state, then the arrival.
            const int piece = t0 == 0 ? 0 : 1;
            const int bnd = static_cast<int>(blockIdx.x) - piece;  // the boundary that cut the item
            float* mine = part + (static_cast<int64_t>(bnd) * 2 + piece) * piece_floats<DP>();
            const int ql = wave * 16 + n;
#pragma unroll
            for (int c = 0; c < NA; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) st_dev(mine + ql * DP + 16 * c + 4 * g + r, o[c][r]);
            if (g == 0) {
                st_dev(mine + kBQ * DP + ql, m_run);
                st_dev(mine + kBQ * DP + kBQ + ql, l_run);
            }
            wait_vmcnt<0>();
            __syncthreads();
            // acq_rel at agent scope: the release orders this piece's state
            // stores before the arrival, and the acquire orders the merging
            // piece's loads of the other state after it.
            if (tid == 0) arrival = __hip_atomic_fetch_add(cnt + bnd, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            if (arrival == 0) continue;  // the other piece merges
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            // Merge: m = max, each side scaled by exp(m_side - m).  Two terms,
            // so the result does not depend on which piece merges.
            const float* other = part + (static_cast<int64_t>(bnd) * 2 + (1 - piece)) * piece_floats<DP>();
            const float mo = ld_dev(other + kBQ * DP + ql), lo = ld_dev(other + kBQ * DP + kBQ + ql);
            const float m = fmaxf(m_run, mo);
            const float am = exp_fast(m_run - m), ao = exp_fast(mo - m);
            l_run = l_run * am + lo * ao;
#pragma unroll
            for (int c = 0; c < NA; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[c][r] = o[c][r] * am + ld_dev(other + ql * DP + 16 * c + 4 * g + r) * ao;
            if (tid == 0) __hip_atomic_store(cnt + bnd, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // out[query n][dims 16c + 4g ..]: divide by the denominator
        if (qrow < T) {
            float* dst = O + qrow * stride + static_cast<int64_t>(head) * D;
            const float inv = 1.0f / l_run;
#pragma unroll
            for (int c = 0; c < NA; ++c)
                if (16 * c + 4 * g < D) *reinterpret_cast<f32x4*>(dst + 16 * c + 4 * g) = o[c] * inv;
        }
    }
}

template <int DP>
hipError_t run(const float* q, const float* k, const float* v, float* out, int64_t t, int n_heads, int d, float scale,
               float* part, uint32_t* cnt, int slots, hipStream_t s) {
    const int64_t nqb = (t + kBQ - 1) / kBQ, ntile = (t + kBK - 1) / kBK, items = n_heads * nqb;
    if (!part) {
        const dim3 grid(static_cast<unsigned>(n_heads), static_cast<unsigned>(nqb));
        hipLaunchKernelGGL(k_flux_attn<DP>, grid, dim3(kThreads), flux_lds_bytes<DP>(), s, q, k, v, out,
                           static_cast<int>(t), n_heads, d, scale, nullptr, nullptr, 0);
    } else {
        const int64_t per = (items * ntile + slots - 1) / slots;  // >= ntile: more items than slots
        hipLaunchKernelGGL(k_flux_attn<DP>, dim3(static_cast<unsigned>(slots)), dim3(kThreads), flux_lds_bytes<DP>(),
                           s, q, k, v, out, static_cast<int>(t), n_heads, d, scale, part, cnt, static_cast<int>(per));
    }
    return hipGetLastError();
}

// Workgroup slots: two per CU (64 KB of LDS and 4 waves per SIMD each).
int flux_slots() { return 2 * static_cast<int>(device_info().cus); }

int padded_dims(int head_dim) { return head_dim <= 32 ? 32 : (head_dim <= 64 ? 64 : 128); }

}  // namespace

size_t flux_attention_workspace(int64_t t, int n_heads, int head_dim) {
    const int64_t items = n_heads * ((t + kBQ - 1) / kBQ);
    const int slots = flux_slots();
    if (items <= slots) return 0;
    const int dp = padded_dims(head_dim);
    return static_cast<size_t>(slots) * 2 * (kBQ * dp + 2 * kBQ) * sizeof(float);
}

hipError_t launch_flux_attention(const float* q, const float* k, const float* v, float* out, int64_t t, int n_heads,
                                 int head_dim, float scale, float* part, uint32_t* counters, hipStream_t s) {
    const int slots = flux_slots();
    if (part && (!counters || static_cast<size_t>(slots) > kArrivalCounters)) return hipErrorInvalidValue;
    switch (padded_dims(head_dim)) {
        case 32: return run<32>(q, k, v, out, t, n_heads, head_dim, scale, part, counters, slots, s);
        case 64: return run<64>(q, k, v, out, t, n_heads, head_dim, scale, part, counters, slots, s);
        default: return run<128>(q, k, v, out, t, n_heads, head_dim, scale, part, counters, slots, s);
    }
}

}  // namespace rt_hip
