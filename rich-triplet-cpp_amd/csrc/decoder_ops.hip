// decoder_ops.hip -- the operations of a decode step between the GEMVs, for the
// decode engine (decoder.cpp): the embedding lookup, standalone RMSNorm and
// the norm-then-residual-add of Gemma 3, the q/k preparation (per-head
// RMSNorm, RoPE in either pairing and either angle form, and the KV-cache
// append in f32 or f16), grouped-query attention over the cache with a
// sliding window at head_dim 64/128/256, and the GELU-tanh gating.
//
// Every operation that depends on the token or its position reads them from
// device memory (`tokens`, `pos`), so a captured graph of the step is replayed
// for every token without being captured again.
//
// The references are the Metal decode engine's kernels
// (src/shaders/decode_gemma3.msl) as src/metal_decode.mm:436-482 sequences
// them, and the Llama layer's operations (src/transformer5.cpp:95-212).
#include <math.h>

#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

constexpr float kLog2e = 1.44269504088896341f;

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// Sum over a workgroup of T threads (result in every thread).
template <int T>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = segment_sum<kWave>(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (T > kWave) {
        if (lane == 0) red[wave] = v;
        __syncthreads();
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < T / kWave; ++w) t += red[w];
        __syncthreads();
        return t;
    }
    return v;
}

// ---- embedding (decode_gemma3.msl:202-233; the Llama lookup is scale 1) ----
template <bool BF16>
__global__ __launch_bounds__(256) void k_embed(const void* __restrict__ table, const int32_t* __restrict__ tokens,
                                               float scale, float* __restrict__ out, int H) {
    const int m = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= H) return;
    const int64_t row = static_cast<int64_t>(tokens[m]) * H;
    float w;
    if constexpr (BF16) {
        w = bf16_lo_to_f32(static_cast<const uint16_t*>(table)[row + i]);
    } else {
        w = static_cast<const float*>(table)[row + i];
    }
    out[static_cast<int64_t>(m) * H + i] = w * scale;
}

// ---- RMSNorm rows, and the Gemma 3 post-norm residual add -----------------
// rms_inv = 1 / sqrt(sum(x^2) * (1/D) + eps); out = (x * rms_inv) * g with
// g = gamma or 1 + gamma (TensorNode::rms_norm / rms_norm_gemma3,
// tensor_node.cpp:320-344, 383-387; rms_norm_gemma3, decode_gemma3.msl:7-53).
// ADD: out = resid + that (metal_decode.mm:468-469, 479-481).  out may be resid.
// D % 4 == 0 and D <= 1024 V: each thread loads its V groups of 4 (x, gamma,
// resid) at once, before the reduction, so the row costs one memory latency
// instead of one per group.
template <bool ADD, int V>
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float* __restrict__ x, const float* __restrict__ gamma,
                                                      const float* resid, float* out, int D, float eps,
                                                      int gemma) {
    __shared__ float red[4];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * D;
    const int n4 = D >> 2, tid = threadIdx.x;
    const f32x4* x4 = reinterpret_cast<const f32x4*>(x + base);
    const f32x4* g4 = reinterpret_cast<const f32x4*>(gamma);
    const f32x4* r4 = reinterpret_cast<const f32x4*>(resid + (ADD ? base : 0));
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 xv[V], gv[V], rv[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int i = tid + 256 * v;
        xv[v] = i < n4 ? x4[i] : z;
        gv[v] = i < n4 ? g4[i] : z;
        if constexpr (ADD) rv[v] = i < n4 ? r4[i] : z;
    }
    float sq = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
        for (int e = 0; e < 4; ++e) sq = __builtin_fmaf(xv[v][e], xv[v][e], sq);
    sq = block_sum<256>(sq, red);
    const float rms_inv = 1.0f / sqrtf(sq * (1.0f / static_cast<float>(D)) + eps);
    f32x4* o4 = reinterpret_cast<f32x4*>(out + base);
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int i = tid + 256 * v;
        if (i >= n4) break;
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float g = gemma ? 1.0f + gv[v][e] : gv[v][e];
            const float t = (xv[v][e] * rms_inv) * g;
            o[e] = ADD ? rv[v][e] + t : t;
        }
        o4[i] = o;
    }
}

// ---- q/k preparation ---------------------------------------------------------
// Workgroup (head slot, row m): slots [0, nq) are query heads, [nq, nq+nkv)
// key heads, [nq+nkv, nq+2nkv) value heads.  Query and key heads take the
// optional per-head RMSNorm (x * rms_inv * (1 + gamma), rms_norm_per_head,
// decode_gemma3.msl:63-97) and RoPE at position pos[0] + m; keys and values
// are appended to the cache row of that position (kv_cache_append,
// decode_gemma3.msl:174-187: half() in f16, RNE; LlamaLayerKvCache::append,
// transformer5.cpp:59-68, f32).
// RoPE angle: mode 0, pos * tab[i] (llama_rope with Config5::inv_freq,
// transformer5.cpp:95-125); mode 1, (pos * freq_scale) / tab[i] with tab the
// pow(theta, 2i/d) denominators (rope_neox, decode_gemma3.msl:99-126).
// Pairing: half-split (i, i + d/2), or interleaved (2i, 2i + 1).
struct PrepArgs {
    const float* q;
    const float* k;
    const float* v;
    float* q_out;
    void* kc;
    void* vc;
    const int32_t* pos;
    const float* qg;
    const float* kg;
    const float* tab;
    float freq_scale, eps;
    int nq, nkv, d, half, mode, f16;
    int64_t q_stride, kv_stride;  // row strides of the M inputs (floats)
    int64_t cache_row;            // floats (or halves) per cache row: nkv * d
};

__global__ __launch_bounds__(128) void k_qk_prep(const PrepArgs a) {
    __shared__ float red[2];
    const int slot = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const int d = a.d, hd = d / 2;
    const int p = a.pos[0] + m;
    const bool is_q = slot < a.nq, is_k = !is_q && slot < a.nq + a.nkv;
    const int head = is_q ? slot : (is_k ? slot - a.nq : slot - a.nq - a.nkv);
    const float* src = is_q ? a.q + m * a.q_stride + static_cast<int64_t>(head) * d
                            : (is_k ? a.k : a.v) + m * a.kv_stride + static_cast<int64_t>(head) * d;
    // thread t owns the pair (i0, i1)
    const bool active = t < hd;
    const int i0 = a.half ? t : 2 * t, i1 = a.half ? t + hd : 2 * t + 1;
    float x0 = active ? src[i0] : 0.0f, x1 = active ? src[i1] : 0.0f;
    if (!(is_q || is_k)) {  // value head: append only
        const int64_t o = static_cast<int64_t>(p) * a.cache_row + static_cast<int64_t>(head) * d;
        if (active) {
            if (a.f16) {
                _Float16* vc = static_cast<_Float16*>(a.vc);
                vc[o + i0] = static_cast<_Float16>(x0);
                vc[o + i1] = static_cast<_Float16>(x1);
            } else {
                float* vc = static_cast<float*>(a.vc);
                vc[o + i0] = x0;
                vc[o + i1] = x1;
            }
        }
        return;
    }
    const float* g = is_q ? a.qg : a.kg;
    if (g) {
        float sq = x0 * x0;
        sq = __builtin_fmaf(x1, x1, sq);
        sq = block_sum<128>(sq, red);
        const float rms_inv = 1.0f / sqrtf(sq / static_cast<float>(d) + a.eps);
        if (active) {
            x0 = x0 * rms_inv * (1.0f + g[i0]);
            x1 = x1 * rms_inv * (1.0f + g[i1]);
        }
    }
    if (!active) return;
    const float ang = a.mode == 0 ? static_cast<float>(p) * a.tab[t]
                                  : (static_cast<float>(p) * a.freq_scale) / a.tab[t];
    const float c = cosf(ang), s = sinf(ang);
    const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
    if (is_q) {
        float* dst = a.q_out + m * a.q_stride + static_cast<int64_t>(head) * d;
        dst[i0] = y0;
        dst[i1] = y1;
    } else {
        const int64_t o = static_cast<int64_t>(p) * a.cache_row + static_cast<int64_t>(head) * d;
        if (a.f16) {
            _Float16* kc = static_cast<_Float16*>(a.kc);
            kc[o + i0] = static_cast<_Float16>(y0);
            kc[o + i1] = static_cast<_Float16>(y1);
        } else {
            float* kc = static_cast<float*>(a.kc);
            kc[o + i0] = y0;
            kc[o + i1] = y1;
        }
    }
}

// ---- attention over the cache --------------------------------------------------
// Flash decoding as attention.hip, generalized: head_dim HD (64, 128, 256),
// an f32 or f16 cache, up to M query rows (row m at position pos[0] + m, or
// at k_end_host - 1 when pos is null), and a sliding window (0 = none): row
// m attends over [k_start, k_end) with k_end = its position + 1 and
// k_start = max(0, k_end - window) (attention_window, metal_decode.mm:
// 404-411).  Workgroup (kv head, split, row) streams its share of the range
// once for the G query heads of the group; lanes per position LP = HD / 8,
// 8 values each.  Each workgroup stores its (max, denominator, weighted sum)
// state per query head; the last of the S workgroups of a (row, kv head) to
// arrive merges the S states in split order into out, so one launch does
// the whole attention and the result does not depend on arrival order.
constexpr int kAT = 256;  // 4 waves
constexpr int kAU = 4;    // positions per group loaded ahead

template <int HD>
struct AttnGeom {
    static constexpr int LP = HD / 8;            // lanes per position
    static constexpr int GPW = kWave / LP;       // position groups per wave
    static constexpr int NG = (kAT / kWave) * GPW;  // groups per workgroup
    static constexpr int BATCH = NG * kAU;       // positions per round
    static constexpr int PART = 4 + HD;          // floats per partial state
};

// AttnGeom<hd>::BATCH for the host (head_dim 64, 128 or 256).
constexpr int attn_round_positions(int hd) { return (kAT / kWave) * (kWave / (hd / 8)) * kAU; }
static_assert(attn_round_positions(64) == AttnGeom<64>::BATCH && attn_round_positions(128) == AttnGeom<128>::BATCH &&
                  attn_round_positions(256) == AttnGeom<256>::BATCH,
              "host and kernel agree on the positions per round");

struct AttnArgs {
    const float* q;      // [M][n_q * HD]
    const void* kc;
    const void* vc;
    float* part;         // [M][n_q][S][PART]
    const int32_t* pos;  // device start position (or null)
    int k_end_host;      // used when pos is null (row m then ends at k_end_host + m)
    int window;
    int n_kv;
    float scale;
    int64_t row;         // cache row stride (elements)
    float* out;          // [M][n_q * HD]
    uint32_t* cnt;       // [M][n_kv] arrival counters, zero between launches
    // > 0: the cache's row count, when no row ever has a window and S
    // splits of one round cover it (so split s starts at s * BATCH whatever
    // the position): the first round's loads are then issued before the
    // position is read, rows clamped below this count.  0: after it.
    int early_rows;
};

// Partials are stored and reloaded with agent-scope (device-coherent)
// accesses: they bypass the per-XCD L2, so the workgroup that merges them
// sees every other XCD's stores once those have completed.
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store((__attribute__((address_space(1))) float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load((const __attribute__((address_space(1))) float*)p, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Fold the S split states of P (row, query head, dimension d) pairs in split
// order (so the result does not depend on which workgroup merges): running
// (M, L, O), rescaled between batches of up to kCB splits whose loads, for
// all P pairs, are issued before any is used (indices past S repeat split
// S - 1, in bounds, with weight 0): one memory latency per batch instead of
// one per split and pair.
constexpr int kCB = 16;  // splits per batch of loads

// The running (M, L, O) of splits [s_begin, s_end) (none: -inf, 0, 0).
// Plain-stored partials (!COH) are read after the launch that wrote them, so
// a split's (M, L) pair, the same for the whole wave when ph and s_begin are,
// is one scalar load through the constant address space: the wave's vector
// loads are then only the O values (a third of them), which the memory
// pipeline takes in fewer issue slots.
typedef const __attribute__((address_space(4))) f32x2 ConstF2;
template <int PART, int P, bool COH, int CB = kCB>
__device__ __forceinline__ void fold_state(const float* const (&ph)[P], const int (&d)[P], int s_begin, int s_end,
                                           float (&M)[P], float (&L)[P], float (&O)[P]) {
    auto ld = [](const float* p) { return COH ? ld_dev(p) : *p; };
#pragma unroll
    for (int p = 0; p < P; ++p) {
        M[p] = -__builtin_inff();
        L[p] = 0.0f;
        O[p] = 0.0f;
    }
    const int S = s_end;
    for (int s0 = s_begin; s0 < S; s0 += CB) {
        // every load of the batch, for all of this thread's P pairs, first
        float ms[P][CB], ls[P][CB], os[P][CB];
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int j = 0; j < CB; ++j) {
                const float* ps = ph[p] + min(s0 + j, S - 1) * PART;
                if constexpr (COH) {
                    ms[p][j] = ld(ps);
                    ls[p][j] = ld(ps + 1);
                } else {
                    const f32x2 ml = *((ConstF2*)(ps));  // PART even: 8-byte aligned
                    ms[p][j] = ml[0];
                    ls[p][j] = ml[1];
                }
                os[p][j] = ld(ps + 4 + d[p]);
            }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < P; ++p) {
            float Mb = M[p];
#pragma unroll
            for (int j = 0; j < CB; ++j) Mb = s0 + j < S ? fmaxf(Mb, ms[p][j]) : Mb;
            // No state yet (Mb = -inf, so M = -inf, L = O = 0): every weight
            // is 0 and nothing changes.  Selects, not a branch: behind a
            // branch the compiler issues the O loads only once the M loads
            // have arrived, two memory latencies instead of one.
            const bool any = Mb != -__builtin_inff();
            const float r = M[p] == -__builtin_inff() ? 0.0f : exp_fast(M[p] - Mb);
            L[p] *= r;
            O[p] *= r;
#pragma unroll
            for (int j = 0; j < CB; ++j) {
                const float w = s0 + j < S && any ? exp_fast(ms[p][j] - Mb) : 0.0f;
                L[p] += ls[p][j] * w;
                O[p] += os[p][j] * w;
            }
            M[p] = Mb;
        }
    }
}

template <int PART, int P, bool COH, int CB = kCB>
__device__ __forceinline__ void fold_splits(const float* const (&ph)[P], const int (&d)[P], int S, float (&res)[P]) {
    float M[P], L[P], O[P];
    fold_state<PART, P, COH, CB>(ph, d, 0, S, M, L, O);
#pragma unroll
    for (int p = 0; p < P; ++p) res[p] = L[p] > 0.0f ? O[p] / L[p] : 0.0f;
}

// Eight f16 values (their bits in w) widened to f32.
__device__ __forceinline__ void widen8(const u32x4 w, f32x4& a, f32x4& b) {
    auto h2 = [](uint32_t u) { return f32x2{f16_bits_to_f32(u & 0xffffu), f16_bits_to_f32(u >> 16)}; };
    const f32x2 p0 = h2(w[0]), p1 = h2(w[1]), p2 = h2(w[2]), p3 = h2(w[3]);
    a = f32x4{p0[0], p0[1], p1[0], p1[1]};
    b = f32x4{p2[0], p2[1], p3[0], p3[1]};
}

template <bool F16>
__device__ __forceinline__ void load8(const void* base, int64_t off, f32x4& a, f32x4& b) {
    if constexpr (F16) {
        widen8(*reinterpret_cast<const u32x4*>(static_cast<const _Float16*>(base) + off), a, b);
    } else {
        const float* p = static_cast<const float*>(base) + off;
        a = *reinterpret_cast<const f32x4*>(p);
        b = *reinterpret_cast<const f32x4*>(p + 4);
    }
}

__device__ __forceinline__ void attn_range(const AttnArgs& a, int m, int& k0, int& k1) {
    k1 = (a.pos ? a.pos[0] + 1 : a.k_end_host) + m;
    k0 = a.window > 0 && k1 > a.window ? k1 - a.window : 0;
}

// Sum over aligned groups of L lanes (8, 16 or 32), every lane of a group
// ending with the same bits: DPP within a 16-lane row (lane ^ 1, lane ^ 2,
// the half-row mirror, the row mirror), one cross-row shuffle for 32.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

template <int L>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(L == 8 || L == 16 || L == 32, "8, 16 or 32 lanes");
    v += dpp_f<0xb1>(v);
    v += dpp_f<0x4e>(v);
    v += dpp_f<0x141>(v);
    if constexpr (L >= 16) v += dpp_f<0x140>(v);
    if constexpr (L == 32) v += __shfl_xor(v, 16, kWave);
    return v;
}

// Positions per split: whole rounds of BATCH.
template <int BATCH>
__device__ __forceinline__ int attn_chunk(int len, int S) {
    const int chunk = (len + S - 1) / S;
    return (chunk + BATCH - 1) / BATCH * BATCH;
}

// k_qk_prep's operations on NH heads held as 8 values per lane each (dims
// 8 sub .. 8 sub + 7) by the LP lanes of a position group: the optional
// per-head RMSNorm (norm[h]), x * rms_inv * (1 + g) with rms_inv = 1 /
// sqrt(sum(x^2) / d + eps), then RoPE with cs / sn the cosine and sine of
// each dim's pair angle.  Half-split pairs (j, j + d/2) meet across lanes
// sub and sub ^ (LP / 2); interleaved pairs (2i, 2i + 1) sit in one lane.
// All heads go through each step together, with one uniform branch per
// step rather than per head, so their sums, exchanges and products
// overlap instead of running head after head.
template <int HD, int NH>
__device__ __forceinline__ void prep_heads(f32x4 (&xa)[NH], f32x4 (&xb)[NH], const bool (&norm)[NH],
                                           const float* const (&g)[NH], const float (&cs)[8],
                                           const float (&sn)[8], bool half, float eps, int sub) {
    constexpr int LP = HD / 8;
    float x[NH][8];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[h][e] = xa[h][e];
            x[h][e + 4] = xb[h][e];
        }
    bool any = false;
#pragma unroll
    for (int h = 0; h < NH; ++h) any = any || norm[h];
    if (any) {  // uniform
        float sq[NH];
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            sq[h] = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) sq[h] += x[h][e] * x[h][e];
        }
#pragma unroll
        for (int h = 0; h < NH; ++h) sq[h] = group_sum<LP>(sq[h]);
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const float rms_inv = 1.0f / sqrtf(sq[h] / static_cast<float>(HD) + eps);
#pragma unroll
            for (int e = 0; e < 8; ++e) x[h][e] = norm[h] ? x[h][e] * rms_inv * (1.0f + g[h][e]) : x[h][e];
        }
    }
    if (half) {  // uniform
        const bool lower = sub < LP / 2;
        float y[NH][8];
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) y[h][e] = __shfl_xor(x[h][e], LP / 2, kWave);
        // the pair's lower dim: x0 * c - x1 * s; its upper dim: x0 * s + x1 * c
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                x[h][e] = lower ? x[h][e] * cs[e] - y[h][e] * sn[e] : y[h][e] * sn[e] + x[h][e] * cs[e];
    } else {
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float x0 = x[h][e], x1 = x[h][e + 1];
                x[h][e] = x0 * cs[e] - x1 * sn[e];
                x[h][e + 1] = x0 * sn[e] + x1 * cs[e];
            }
    }
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            xa[h][e] = x[h][e];
            xb[h][e] = x[h][e + 4];
        }
}

// MERGE: the last split of a (row, kv head) to arrive merges in this launch
// (partials stored device-coherent); otherwise partials are plain stores
// and k_attn2_combine merges them in a second launch.
// PREP (one row, device position): k_qk_prep's work is done here.  Every
// workgroup normalizes and rotates its query heads from the raw q, and the
// new token's key and value from the raw k and v (rounded as the cache
// stores them); the position group that meets the new position uses those
// instead of the cache row, and the workgroup whose split holds it appends
// them to the cache for the next tokens.  No other workgroup reads that row,
// so the separate launch before the attention is gone.
template <int HD, int G, bool F16, bool MERGE, bool PREP>
__device__ __forceinline__ void attn2_partial(const AttnArgs& a, const PrepArgs& pp) {
    static_assert(!(PREP && MERGE), "the fused prep runs in the two-launch form");
    using Geo = AttnGeom<HD>;
    constexpr int LP = Geo::LP, NG = Geo::NG;
    __shared__ float sm[NG][G][2];
    __shared__ f32x4 so[NG][G][HD / 4];
    const int kvh = blockIdx.x, sp = blockIdx.y, S = gridDim.y, m = blockIdx.z;
    const int n_q = a.n_kv * G;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = wave * Geo::GPW + lane / LP, sub = lane % LP;
    // q first: its loads do not wait for the device-side position
    f32x4 qa[G], qb[G], oa[G], ob[G];
    float mx[G], l[G];
    const float* const qsrc = PREP ? pp.q : a.q;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float* qp = qsrc + static_cast<int64_t>(m) * n_q * HD + (static_cast<int64_t>(kvh) * G + h) * HD + sub * 8;
        qa[h] = *reinterpret_cast<const f32x4*>(qp);
        qb[h] = *reinterpret_cast<const f32x4*>(qp + 4);
        oa[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        ob[h] = oa[h];
        mx[h] = -__builtin_inff();
        l[h] = 0.0f;
    }
    // PREP: the new token's raw key and value, the norm gammas and, for
    // thread t < d/2, pair t's rotation-table entry, also before the position
    // (Unconditional loads: behind a branch each would be waited for on its
    // own; an absent gamma reads the raw k instead, unused.)
    f32x4 kna, knb, vna, vnb;
    float qg[8], kg[8], tv = 1.0f;
    if constexpr (PREP) {
        const int64_t o = static_cast<int64_t>(kvh) * HD + sub * 8;
        kna = *reinterpret_cast<const f32x4*>(pp.k + o);
        knb = *reinterpret_cast<const f32x4*>(pp.k + o + 4);
        vna = *reinterpret_cast<const f32x4*>(pp.v + o);
        vnb = *reinterpret_cast<const f32x4*>(pp.v + o + 4);
        const float* const qgp = (pp.qg ? pp.qg : pp.k) + sub * 8;
        const float* const kgp = (pp.kg ? pp.kg : pp.k) + sub * 8;
        const f32x4 qg0 = *reinterpret_cast<const f32x4*>(qgp), qg1 = *reinterpret_cast<const f32x4*>(qgp + 4);
        const f32x4 kg0 = *reinterpret_cast<const f32x4*>(kgp), kg1 = *reinterpret_cast<const f32x4*>(kgp + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            qg[e] = qg0[e];
            qg[e + 4] = qg1[e];
            kg[e] = kg0[e];
            kg[e + 4] = kg1[e];
        }
        tv = pp.tab[tid < HD / 2 ? tid : 0];
    }
    // The range [k0, k1) of row m and this split's share [p0, p1) of it
    // (pcur: PREP's new position), once the position has been read.
    int k0 = 0, k1 = 0, len = 0, chunk = 0, p0 = 0, p1 = 0, pcur = 0;
    auto set_range = [&]() {
        attn_range(a, m, k0, k1);
        len = k1 - k0;
        chunk = attn_chunk<Geo::BATCH>(len, S);
        p0 = k0 + sp * chunk;
        p1 = min(k1, p0 + chunk);
        pcur = k1 - 1;
    };
    // early_rows > 0: split sp's first round is positions sp * BATCH + [0,
    // BATCH) for every position (no window, chunk = BATCH), so its loads go
    // out before the position's own load has returned.
    const bool early = a.early_rows > 0;  // uniform

    // One round: the K and V of positions pb, pb + NG, ... (kAU of them)
    // issued, then their scores and the running state.  Every load is
    // issued with no branch around it (a position past the range reads row
    // k0, which exists, and `land` replaces it with zeros): loads behind
    // branches leave the compiler unsure how many are in flight, so a later
    // wait for an older load becomes a wait for all of them.  An f16
    // cache's bits are loaded into ka / va as they are and widened in
    // `land`, after the round's loads are all issued.  Issued before the
    // range is known (`before`), a row is clamped to the cache instead.
    auto issue = [&](int pb, f32x4 (&ka)[kAU], f32x4 (&kb)[kAU], f32x4 (&va)[kAU], f32x4 (&vb)[kAU],
                     bool before = false) {
#pragma unroll
        for (int u = 0; u < kAU; ++u) {
            const int p = pb + u * NG;
            const int r = before ? min(p, a.early_rows - 1) : (p < p1 ? p : k0);
            const int64_t off = static_cast<int64_t>(r) * a.row + static_cast<int64_t>(kvh) * HD + sub * 8;
            if constexpr (F16) {
                ka[u] = __builtin_bit_cast(f32x4,
                                           *reinterpret_cast<const u32x4*>(static_cast<const _Float16*>(a.kc) + off));
                va[u] = __builtin_bit_cast(f32x4,
                                           *reinterpret_cast<const u32x4*>(static_cast<const _Float16*>(a.vc) + off));
            } else {
                load8<false>(a.kc, off, ka[u], kb[u]);
                load8<false>(a.vc, off, va[u], vb[u]);
            }
        }
        // every load of the round before any use (else the compiler
        // interleaves the first products and waits between the loads)
        __builtin_amdgcn_sched_barrier(0);
    };
    auto land = [&](int pb, f32x4 (&ka)[kAU], f32x4 (&kb)[kAU], f32x4 (&va)[kAU], f32x4 (&vb)[kAU]) {
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < kAU; ++u) {
            if constexpr (F16) {
                widen8(__builtin_bit_cast(u32x4, ka[u]), ka[u], kb[u]);
                widen8(__builtin_bit_cast(u32x4, va[u]), va[u], vb[u]);
            }
            const bool in = pb + u * NG < p1;  // uniform per position group
            ka[u] = in ? ka[u] : z;
            kb[u] = in ? kb[u] : z;
            va[u] = in ? va[u] : z;
            vb[u] = in ? vb[u] : z;
        }
    };
    auto consume = [&](int pb, const f32x4 (&ka)[kAU], const f32x4 (&kb)[kAU], const f32x4 (&va)[kAU],
                       const f32x4 (&vb)[kAU]) {
        // The round's kAU scores do not depend on each other: all of them
        // first (their cross-lane sums overlap), then one running-maximum
        // update and one rescale per round instead of one per position.
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float sc[kAU];
            float mn = mx[h];
#pragma unroll
            for (int u = 0; u < kAU; ++u) {
                float dd = (qa[h][0] * ka[u][0] + qa[h][1] * ka[u][1]) + (qa[h][2] * ka[u][2] + qa[h][3] * ka[u][3]);
                dd += (qb[h][0] * kb[u][0] + qb[h][1] * kb[u][1]) + (qb[h][2] * kb[u][2] + qb[h][3] * kb[u][3]);
                const float v = group_sum<LP>(dd) * a.scale;
                sc[u] = pb + u * NG < p1 ? v : -__builtin_inff();  // uniform per position group
                mn = fmaxf(mn, sc[u]);
            }
            // No position of this group yet (mn = -inf, so mx = -inf and l, o
            // are 0): a finite reference makes every weight 0 and changes
            // nothing.  A select, not a branch, so the G heads' chains
            // interleave.
            const float mref = mn == -__builtin_inff() ? 0.0f : mn;
            const float al = exp_fast(mx[h] - mref);  // 0 while mx is -inf
            l[h] *= al;
            oa[h] *= al;
            ob[h] *= al;
#pragma unroll
            for (int u = 0; u < kAU; ++u) {
                const float be = exp_fast(sc[u] - mref);  // 0 for positions past the range
                l[h] += be;
                oa[h] += va[u] * be;
                ob[h] += vb[u] * be;
            }
            mx[h] = mn;
        }
    };

    // PREP: the new position's key and value are this launch's own, not the
    // cache row (in whichever round of its split the position falls)
    auto own_row = [&](int pb, f32x4 (&ka)[kAU], f32x4 (&kb)[kAU], f32x4 (&va)[kAU], f32x4 (&vb)[kAU]) {
#pragma unroll
        for (int u = 0; u < kAU; ++u) {
            if (pb + u * NG == pcur) {  // uniform per position group
                ka[u] = kna;
                kb[u] = knb;
                va[u] = vna;
                vb[u] = vnb;
            }
        }
    };

    // The first round by every group, with no branch around its loads (a
    // group with no position left reads row k0, replaced by zeros, and
    // scores -inf).  With `early` its loads go out before the position is
    // read.  PREP: the loads are in flight while the new token is
    // prepared: the workgroup's threads share the d/2 rotation angles of
    // k_qk_prep (pos * tab[i], or (pos * freq_scale) / tab[i]) through LDS,
    // one cosine and sine each.
    if (!early) set_range();  // uniform; a scalar load, so no vector wait is lost
    int pb = (early ? sp * Geo::BATCH : p0) + grp;
    {
        f32x4 ka[kAU], kb[kAU], va[kAU], vb[kAU];
        issue(pb, ka, kb, va, vb, early);
        if (early) set_range();
        if constexpr (PREP) {
            __shared__ float tcs[HD / 2], tsn[HD / 2];
            if (tid < HD / 2) {
                const float ang = pp.mode == 0 ? static_cast<float>(pcur) * tv
                                               : (static_cast<float>(pcur) * pp.freq_scale) / tv;
                tcs[tid] = cosf(ang);
                tsn[tid] = sinf(ang);
            }
            __syncthreads();
            float cs[8], sn[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // the pair of dim j: j mod d/2 (half-split) or j / 2
                const int i = pp.half ? (sub * 8 + e) % (HD / 2) : (sub * 8 + e) >> 1;
                cs[e] = tcs[i];
                sn[e] = tsn[i];
            }
            // the G query heads and the new key, together
            f32x4 ha[G + 1], hb[G + 1];
            bool hn[G + 1];
            const float* hg[G + 1];
#pragma unroll
            for (int h = 0; h < G; ++h) {
                ha[h] = qa[h];
                hb[h] = qb[h];
                hn[h] = pp.qg != nullptr;
                hg[h] = qg;
            }
            ha[G] = kna;
            hb[G] = knb;
            hn[G] = pp.kg != nullptr;
            hg[G] = kg;
            prep_heads<HD, G + 1>(ha, hb, hn, hg, cs, sn, pp.half, pp.eps, sub);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                qa[h] = ha[h];
                qb[h] = hb[h];
            }
            kna = ha[G];
            knb = hb[G];
            const int64_t o = static_cast<int64_t>(pcur) * pp.cache_row + static_cast<int64_t>(kvh) * HD + sub * 8;
            const bool store = grp == 0 && pcur >= p0 && pcur < p1;  // one group of one workgroup per kv head
            if constexpr (F16) {
                // the cache's rounding (RNE), kept for this launch's own use
                _Float16 hk[8], hv[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    hk[e] = static_cast<_Float16>(kna[e]);
                    hk[e + 4] = static_cast<_Float16>(knb[e]);
                    hv[e] = static_cast<_Float16>(vna[e]);
                    hv[e + 4] = static_cast<_Float16>(vnb[e]);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    kna[e] = static_cast<float>(hk[e]);
                    knb[e] = static_cast<float>(hk[e + 4]);
                    vna[e] = static_cast<float>(hv[e]);
                    vnb[e] = static_cast<float>(hv[e + 4]);
                }
                if (store) {
                    _Float16* kc = static_cast<_Float16*>(pp.kc) + o;
                    _Float16* vc = static_cast<_Float16*>(pp.vc) + o;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        kc[e] = hk[e];
                        vc[e] = hv[e];
                    }
                }
            } else if (store) {
                float* kc = static_cast<float*>(pp.kc) + o;
                float* vc = static_cast<float*>(pp.vc) + o;
                *reinterpret_cast<f32x4*>(kc) = kna;
                *reinterpret_cast<f32x4*>(kc + 4) = knb;
                *reinterpret_cast<f32x4*>(vc) = vna;
                *reinterpret_cast<f32x4*>(vc + 4) = vnb;
            }
        }
        land(pb, ka, kb, va, vb);
        if constexpr (PREP) own_row(pb, ka, kb, va, vb);
        consume(pb, ka, kb, va, vb);
        pb += NG * kAU;
    }
    for (; pb < p1; pb += NG * kAU) {
        f32x4 ka[kAU], kb[kAU], va[kAU], vb[kAU];
        issue(pb, ka, kb, va, vb);
        land(pb, ka, kb, va, vb);
        if constexpr (PREP) own_row(pb, ka, kb, va, vb);
        consume(pb, ka, kb, va, vb);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        if (sub == 0) {
            sm[grp][h][0] = mx[h];
            sm[grp][h][1] = l[h];
        }
        so[grp][h][sub * 2] = oa[h];
        so[grp][h][sub * 2 + 1] = ob[h];
    }
    __syncthreads();
    for (int t = tid; t < G * (HD / 4); t += kAT) {
        const int h = t / (HD / 4), d4 = t % (HD / 4);
        float M = -__builtin_inff();
        for (int g = 0; g < NG; ++g) M = fmaxf(M, sm[g][h][0]);
        float L = 0.0f;
        f32x4 O = {0.0f, 0.0f, 0.0f, 0.0f};
        if (M != -__builtin_inff()) {
            for (int g = 0; g < NG; ++g) {
                const float w = exp_fast(sm[g][h][0] - M);
                L += sm[g][h][1] * w;
                O += so[g][h][d4] * w;
            }
        }
        float* dst = a.part + ((static_cast<int64_t>(m) * n_q + kvh * G + h) * S + sp) * Geo::PART;
        if constexpr (MERGE) {
            if (d4 == 0) {
                st_dev(dst, M);
                st_dev(dst + 1, L);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) st_dev(dst + 4 + d4 * 4 + e, O[e]);
        } else {
            if (d4 == 0) {
                dst[0] = M;
                dst[1] = L;
            }
            *reinterpret_cast<f32x4*>(dst + 4 + d4 * 4) = O;  // PART = 4 + HD: 16-byte aligned
        }
    }
    if constexpr (!MERGE) return;
    // Every thread's partial stores have completed, then one arrival per
    // workgroup; the last of the S splits of (row, kv head) merges them and
    // resets the counter for the next launch.
    wait_vmcnt<0>();
    __syncthreads();
    __shared__ uint32_t arrival;
    uint32_t* const cnt = a.cnt + static_cast<int64_t>(m) * a.n_kv + kvh;
    // acq_rel at agent scope: the release orders this split's partial
    // stores before the arrival, the acquire the last arriver's loads of the
    // other splits' partials after it.
    if (tid == 0) arrival = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrival != static_cast<uint32_t>(S - 1)) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // this thread's (query head, dim) pairs t = tid, tid + kAT, ..., all
    // merged together
    constexpr int P = (G * HD + kAT - 1) / kAT;
    const float* ph[P];
    int dd[P];
    float res[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int t = tid + kAT * p < G * HD ? tid + kAT * p : tid;  // past the pairs: a repeat, not stored
        dd[p] = t % HD;
        ph[p] = a.part + (static_cast<int64_t>(m) * n_q + kvh * G + t / HD) * S * Geo::PART;
    }
    // splits past the range (chunk * busy >= len) hold empty states: skip them
    const int busy = min(S, (len + chunk - 1) / chunk);
    fold_splits<Geo::PART, P, true>(ph, dd, busy, res);
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int t = tid + kAT * p;
        if (t < G * HD) a.out[(static_cast<int64_t>(m) * n_q + kvh * G + t / HD) * HD + t % HD] = res[p];
    }
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The partial kernel takes the fields its first loads need as scalar
// arguments ahead of the struct: the first 14 argument dwords arrive
// preloaded in SGPRs (-amdgpu-kernarg-preload-count), while a struct
// argument is read from the argument segment with scalar loads whose latency
// the first vector loads would wait for.  Measured in a timing copy
// (Llama-3.2-3B geometry, 17 splits, 64 launches in a hipGraph): partial
// and merge 9.08 against 8.14 us per layer, the same bits.  The fused-prep
// kernel keeps its two structs: its first loads need the gammas and the
// rotation table as well, which one batch of scalar loads brings together
// (with the 14 hottest pointers preloaded and the rest loaded, Gemma-3-4B
// tokens measured 1561-1576 against 1537-1554 us).
template <int HD, int G, bool F16, bool MERGE>
__global__ __launch_bounds__(kAT) void k_attn2_partial(const float* q, const void* kc, const void* vc,
                                                       const int32_t* pos, int row, int early_rows, int window,
                                                       int k_end_host, float scale, int n_kv, const AttnArgs rest) {
    AttnArgs a = rest;
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.pos = pos;
    a.row = row;
    a.early_rows = early_rows;
    a.window = window;
    a.k_end_host = k_end_host;
    a.scale = scale;
    a.n_kv = n_kv;
    attn2_partial<HD, G, F16, MERGE, false>(a, PrepArgs{});
}

template <int HD, int G, bool F16>
__global__ __launch_bounds__(kAT) void k_attn2_partial_prep(const AttnArgs a, const PrepArgs p) {
    attn2_partial<HD, G, F16, false, true>(a, p);
}

// Second launch of the two-launch form: workgroup (query head, row), one
// thread per dimension and part.  Part r folds the plain-stored partials of
// its contiguous share of the S splits in split order, with no read of the
// position, so its loads issue at once (a split past the cached range holds
// M = -inf, L = O = 0 and changes nothing); with R parts of at most kCB
// splits that is one memory latency.  Part 0 then folds the R states in
// order: the result is the same for every run.
template <int HD, int R, int CB = kCB>
__global__ __launch_bounds__(HD * R) void k_attn2_combine(const float* part, float* out_all, int S) {
    using Geo = AttnGeom<HD>;
    const int h = blockIdx.x, m = blockIdx.y, d = static_cast<int>(threadIdx.x) % HD;
    // the part: the same for a whole wave (HD >= 64), said so to the compiler
    // so that the (M, L) loads are scalar
    const int r = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / HD);
    const int n_q = gridDim.x;
    const float* ph[1] = {part + (static_cast<int64_t>(m) * n_q + h) * S * Geo::PART};
    const int dd[1] = {d};
    float* const out = out_all + (static_cast<int64_t>(m) * n_q + h) * HD + d;
    if constexpr (R == 1) {
        float res[1];
        fold_splits<Geo::PART, 1, false, CB>(ph, dd, S, res);
        *out = res[0];
    } else {
        float M[1], L[1], O[1];
        fold_state<Geo::PART, 1, false>(ph, dd, (S * r) / R, (S * (r + 1)) / R, M, L, O);
        __shared__ float sm[R], sl[R], so[R][HD];
        if (d == 0) {
            sm[r] = M[0];
            sl[r] = L[0];
        }
        so[r][d] = O[0];
        __syncthreads();
        if (r != 0) return;
        float mx = sm[0];
#pragma unroll
        for (int q = 1; q < R; ++q) mx = fmaxf(mx, sm[q]);
        float lt = 0.0f, ot = 0.0f;
#pragma unroll
        for (int q = 0; q < R; ++q) {
            const float w = sm[q] == -__builtin_inff() ? 0.0f : exp_fast(sm[q] - mx);
            lt += sl[q] * w;
            ot += so[q][d] * w;
        }
        *out = lt > 0.0f ? ot / lt : 0.0f;
    }
}

// The combine launch: ceil(S / kCB) parts (at most 4), so each part is one
// batch of loads.  Measured (engine tokens at 1024 positions, vector loads
// for every value): Llama-3.2-3B, 17 splits, 1120-1123 us with two parts
// against 1129-1136 with one and 1136-1142 with four; Gemma-3-4B (head_dim
// 256, 32 and 34 splits) one part 1649-1659 against 1663-1669 with two.
// With the (M, L) pairs as scalar loads, timed alone in a hipGraph: 17
// splits at head_dim 128 in two parts 2.47 against 2.66 us, 33 splits at
// head_dim 256 in two parts 3.60 against 4.00 for one part with vector loads.
template <int HD>
void launch_combine(const AttnArgs& a, int n_q, int S, int M, hipStream_t s) {
    int parts = tune_param("ATTN_COMBINE_PARTS", (S + kCB - 1) / kCB);
    parts = parts < 1 ? 1 : (parts > 4 ? 4 : parts);
    const dim3 g(static_cast<unsigned>(n_q), static_cast<unsigned>(M));
    switch (parts) {
        case 1: hipLaunchKernelGGL((k_attn2_combine<HD, 1>), g, dim3(HD), 0, s, a.part, a.out, S); break;
        case 2: hipLaunchKernelGGL((k_attn2_combine<HD, 2>), g, dim3(HD * 2), 0, s, a.part, a.out, S); break;
        case 3: hipLaunchKernelGGL((k_attn2_combine<HD, 3>), g, dim3(HD * 3), 0, s, a.part, a.out, S); break;
        default: hipLaunchKernelGGL((k_attn2_combine<HD, 4>), g, dim3(HD * 4), 0, s, a.part, a.out, S); break;
    }
}

template <int HD, int G, bool F16>
hipError_t run_attn(const AttnArgs& a, int S, int M, hipStream_t s, const PrepArgs* prep) {
    const dim3 grid(static_cast<unsigned>(a.n_kv), static_cast<unsigned>(S), static_cast<unsigned>(M));
    if (prep) {
        hipLaunchKernelGGL((k_attn2_partial_prep<HD, G, F16>), grid, dim3(kAT), 0, s, a, *prep);
        launch_combine<HD>(a, a.n_kv * G, S, M, s);
        return hipGetLastError();
    }
    // Two launches by default.  Measured at 1024 cached positions: the
    // Llama-3.2-3B engine token 1162 us against 1201 us with the merge in
    // the last-arriving workgroup (Gemma-3-4B shapes 1989 against 1982 us);
    // 28 layers of attention alone 289 against 322 us.  The in-launch
    // merge's device-coherent partial stores, arrival atomic and coherent
    // reloads are three memory round trips in series, more than a kernel
    // boundary costs.
    if (tune_param("ATTN_MERGE_IN_LAUNCH", 0)) {
        hipLaunchKernelGGL((k_attn2_partial<HD, G, F16, true>), grid, dim3(kAT), 0, s, a.q, a.kc, a.vc, a.pos,
                           static_cast<int>(a.row), a.early_rows, a.window, a.k_end_host, a.scale, a.n_kv, a);
    } else {
        hipLaunchKernelGGL((k_attn2_partial<HD, G, F16, false>), grid, dim3(kAT), 0, s, a.q, a.kc, a.vc, a.pos,
                           static_cast<int>(a.row), a.early_rows, a.window, a.k_end_host, a.scale, a.n_kv, a);
        // Measured (engine tokens, Llama-3.2-3B / Gemma-3-4B shapes, 1024
        // positions, 17 splits): 1120 / 1951 us against 1125-1130 / 1949-1963
        // folding only the busy splits after reading the position; batches
        // of 32 splits (one latency for all 17) 1137-1150 / 2002-2044.
        launch_combine<HD>(a, a.n_kv * G, S, M, s);
    }
    return hipGetLastError();
}

template <int HD, bool F16>
hipError_t attn_g(const AttnArgs& a, int G, int S, int M, hipStream_t s, const PrepArgs* prep) {
    switch (G) {
        case 1: return run_attn<HD, 1, F16>(a, S, M, s, prep);
        case 2: return run_attn<HD, 2, F16>(a, S, M, s, prep);
        case 3: return run_attn<HD, 3, F16>(a, S, M, s, prep);
        case 4: return run_attn<HD, 4, F16>(a, S, M, s, prep);
        default: return hipErrorInvalidValue;
    }
}

// ---- GELU-tanh gating (gelu_tanh_kernel + elem_mul, decode_gemma3.msl:128-158) --
__global__ __launch_bounds__(256) void k_gelu_mul(const float* __restrict__ gate, const float* __restrict__ up,
                                                  float* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = gate[i];
    const float v3 = v * v * v;
    float inner = 0.7978845608f * (v + 0.044715f * v3);
    inner = fminf(fmaxf(inner, -10.0f), 10.0f);
    out[i] = (0.5f * v * (1.0f + tanhf(inner))) * up[i];
}

}  // namespace

// ---- launchers -------------------------------------------------------------------

hipError_t launch_embed(const void* table, bool bf16, const int32_t* tokens, float scale, float* out, int64_t h,
                        int m, hipStream_t s) {
    const dim3 g(static_cast<unsigned>((h + 255) / 256), static_cast<unsigned>(m));
    if (bf16)
        hipLaunchKernelGGL(k_embed<true>, g, dim3(256), 0, s, table, tokens, scale, out, static_cast<int>(h));
    else
        hipLaunchKernelGGL(k_embed<false>, g, dim3(256), 0, s, table, tokens, scale, out, static_cast<int>(h));
    return hipGetLastError();
}

template <int V>
hipError_t rmsnorm_v(const float* x, const float* gamma, const float* resid, float* out, int64_t d, int rows,
                     float eps, bool gemma, hipStream_t s) {
    if (resid)
        hipLaunchKernelGGL((k_rmsnorm_rows<true, V>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, x, gamma,
                           resid, out, static_cast<int>(d), eps, gemma ? 1 : 0);
    else
        hipLaunchKernelGGL((k_rmsnorm_rows<false, V>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, x, gamma,
                           resid, out, static_cast<int>(d), eps, gemma ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const float* x, const float* gamma, const float* resid, float* out, int64_t d,
                               int rows, float eps, bool gemma, hipStream_t s) {
    if (d % 4 != 0 || d > 16384) return hipErrorInvalidValue;
    if (d <= 4096) return rmsnorm_v<4>(x, gamma, resid, out, d, rows, eps, gemma, s);
    if (d <= 8192) return rmsnorm_v<8>(x, gamma, resid, out, d, rows, eps, gemma, s);
    return rmsnorm_v<16>(x, gamma, resid, out, d, rows, eps, gemma, s);
}

static PrepArgs prep_args(const QkPrep& p) {
    PrepArgs a;
    a.q = p.q;
    a.k = p.k;
    a.v = p.v;
    a.q_out = p.q_out;
    a.kc = p.k_cache;
    a.vc = p.v_cache;
    a.pos = p.pos;
    a.qg = p.q_gamma;
    a.kg = p.k_gamma;
    a.tab = p.rope_tab;
    a.freq_scale = p.freq_scale;
    a.eps = p.eps;
    a.nq = p.n_q;
    a.nkv = p.n_kv;
    a.d = p.head_dim;
    a.half = p.half_split ? 1 : 0;
    a.mode = p.pow_angle ? 1 : 0;
    a.f16 = p.f16 ? 1 : 0;
    a.q_stride = static_cast<int64_t>(p.n_q) * p.head_dim;
    a.kv_stride = static_cast<int64_t>(p.n_kv) * p.head_dim;
    a.cache_row = static_cast<int64_t>(p.n_kv) * p.head_dim;
    return a;
}

hipError_t launch_qk_prep(const QkPrep& p, hipStream_t s) {
    if (p.head_dim < 2 || p.head_dim > 256 || p.head_dim % 2) return hipErrorInvalidValue;
    const PrepArgs a = prep_args(p);
    hipLaunchKernelGGL(k_qk_prep, dim3(static_cast<unsigned>(p.n_q + 2 * p.n_kv), static_cast<unsigned>(p.m)),
                       dim3(128), 0, s, a);
    return hipGetLastError();
}

// Enough (kv head, split, row) workgroups for every CU, at least one round
// of the partial kernel's positions per split (64 at head_dim 128, 32 at
// 256): each workgroup then loads its positions in one round, one memory
// latency.  Measured at 1024 positions: Llama-3.2-3B engine, 17 splits 6.44
// us per partial launch, 32 splits of 32 positions (2 loaded ahead per
// group) 6.88 us; Gemma-3-4B engine (head_dim 256) 1889-1903 us/token at 64
// positions per split (two rounds), 1796-1799 at 32, 1847 at 16.
int attention2_splits(int n_kv, int m, int64_t max_len, int head_dim) {
    const int64_t cus = device_info().cus;
    int64_t want = (cus + n_kv * m - 1) / (n_kv * m);
    const int64_t per = tune_param("ATTN_SPLIT_POS", attn_round_positions(head_dim));
    const int64_t by_len = (max_len + per - 1) / per;
    want = want < by_len ? want : by_len;
    return static_cast<int>(want < 1 ? 1 : want);
}

size_t attention2_workspace(int n_q, int head_dim, int splits, int m) {
    return static_cast<size_t>(m) * n_q * splits * (4 + head_dim) * sizeof(float);
}

hipError_t launch_attention2(const Attn2& p, float* part, uint32_t* counters, hipStream_t s) {
    if (!counters || p.splits < 1) return hipErrorInvalidValue;
    AttnArgs a;
    a.q = p.q;
    a.kc = p.k_cache;
    a.vc = p.v_cache;
    a.part = part;
    a.pos = p.pos;
    a.k_end_host = p.k_end;
    a.window = p.window;
    a.n_kv = p.n_kv;
    a.scale = p.scale;
    a.row = static_cast<int64_t>(p.n_kv) * p.head_dim;
    if (a.row > 0x7fffffff) return hipErrorInvalidValue;  // passed to the kernels as an int
    a.out = p.out;
    a.cnt = counters;
    const int64_t round = attn_round_positions(p.head_dim);
    a.early_rows = p.cache_rows > 0 && p.window == 0 && static_cast<int64_t>(p.splits) * round >= p.cache_rows
                       ? p.cache_rows
                       : 0;
    const int G = p.n_q / p.n_kv;
    PrepArgs pa{};
    if (p.prep) {
        // the fused form: one row at a device position, the same geometry
        const QkPrep& q = *p.prep;
        if (p.m != 1 || q.m != 1 || !p.pos || q.pos != p.pos || q.n_q != p.n_q || q.n_kv != p.n_kv ||
            q.head_dim != p.head_dim || q.f16 != p.f16 || !q.rope_tab || q.k_cache != p.k_cache ||
            q.v_cache != p.v_cache)
            return hipErrorInvalidValue;
        pa = prep_args(q);
    }
    const PrepArgs* pp = p.prep ? &pa : nullptr;
    switch (p.head_dim) {
        case 64: return p.f16 ? attn_g<64, true>(a, G, p.splits, p.m, s, pp)
                              : attn_g<64, false>(a, G, p.splits, p.m, s, pp);
        case 128: return p.f16 ? attn_g<128, true>(a, G, p.splits, p.m, s, pp)
                               : attn_g<128, false>(a, G, p.splits, p.m, s, pp);
        case 256: return p.f16 ? attn_g<256, true>(a, G, p.splits, p.m, s, pp)
                               : attn_g<256, false>(a, G, p.splits, p.m, s, pp);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gelu_mul(const float* gate, const float* up, float* out, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_gelu_mul, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, gate, up, out, n);
    return hipGetLastError();
}

}  // namespace rt_hip

namespace rt_hip {
namespace {

// out = a + b (n elements; out may alias a).
__global__ __launch_bounds__(256) void k_add(const float* a, const float* __restrict__ b, float* out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

// out = silu(gate) * up with the sigmoid first (TensorNode::silu,
// tensor_node.cpp:391-402; LlamaMlp::forward, transformer5.cpp:186-190).
__global__ __launch_bounds__(256) void k_swiglu(const float* __restrict__ gate, const float* __restrict__ up,
                                                float* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const float g = gate[i];
    const float sig = 1.0f / (1.0f + expf(-g));
    out[i] = (g * sig) * up[i];
}

}  // namespace

hipError_t launch_add(const float* a, const float* b, float* out, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_add, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, a, b, out, n);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* gate, const float* up, float* out, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_swiglu, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, gate, up, out, n);
    return hipGetLastError();
}

}  // namespace rt_hip
