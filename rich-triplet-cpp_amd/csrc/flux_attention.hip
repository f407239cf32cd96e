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
// streams K and V once for all of them in tiles of 32 keys through LDS (K as
// [key][dim], V transposed to [dim][key], 32 KB at D = 128: two workgroups
// per CU at 125 VGPRs).  The products run in f32 on the
// matrix cores (v_mfma_f32_16x16x4_f32), so every product and partial sum
// is an f32 operation, as in the reference:
//  * S^T = K Q^T per 16-key x 16-query tile: lane (g = l/16, n = l%16)
//    supplies K[key n][dim] and Q[query n][dim] for the same dim, so any
//    assignment of dims to (k-step, lane group) is a valid contraction; dims
//    16a + 4g + b over steps 4a + b let each lane read 4 consecutive dims
//    with one 16-byte LDS read.  The result leaves lane (g, n) holding the
//    scores of query n against keys 16t + 4g + r (t over the tile's two
//    16-key halves).
//  * Online softmax per query: the running maximum and denominator; the
//    accumulator rows are rescaled by exp(m_old - m_new) before the tile is
//    folded in (flux.msl:232-271).
//  * O += P V: lane (g, n) supplies P[query n][key 16t + 4g + r] -- exactly
//    the scores it holds -- and V[key 16t + 4g + r][dim 16c + n], one 16-byte
//    read of the transposed tile for the four r.
// The head is padded to DP in {32, 64, 128} dims with zeros (they add
// nothing to a score and are never stored).  Keys past T are masked to -inf
// (weight 0), their tile rows zero-filled; query rows past T are computed and
// not stored.  LDS rows are XOR-swizzled by 16-byte granule so that the
// 16-lane reads above hit distinct banks without padding.
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

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

template <int DP>
constexpr size_t flux_lds_bytes() {
    return static_cast<size_t>(kBK) * DP * 4 * 2;  // K tile + V^T tile
}

// float offset of K[key][granule gr] (4 dims) and of V^T[dim][key]
template <int DP>
__device__ __forceinline__ int k_off(int key, int gr) {
    constexpr int kMask = (DP / 4 < 16 ? DP / 4 : 16) - 1;
    return key * DP + ((gr ^ (key & kMask)) << 2);
}
__device__ __forceinline__ int vt_off(int dim, int key) {
    constexpr int kMask = kBK / 4 - 1;  // granules per V^T row, minus one
    return dim * kBK + ((((key >> 2) ^ (dim & kMask))) << 2) + (key & 3);
}

template <int DP>
__global__ __launch_bounds__(kThreads) void k_flux_attn(const float* __restrict__ Q, const float* __restrict__ K,
                                                        const float* __restrict__ V, float* __restrict__ O, int T,
                                                        int n_heads, int D, float scale) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float* const ks = lds;                                  // [kBK][DP], swizzled granules
    float* const vt = lds + static_cast<size_t>(kBK) * DP;  // [DP][kBK], swizzled granules
    constexpr int NA = DP / 16;
    const int head = blockIdx.x, q0 = blockIdx.y * kBQ;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int64_t stride = static_cast<int64_t>(n_heads) * D;
    const float* qb = Q + static_cast<int64_t>(head) * D;
    const float* kb = K + static_cast<int64_t>(head) * D;
    const float* vb = V + static_cast<int64_t>(head) * D;

    // this lane's query row (n of the wave's 16): dims 16a + 4g .. + 3
    const int qrow = q0 + wave * 16 + n;
    float qf[4 * NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) {
        f32x4 v4 = {0.0f, 0.0f, 0.0f, 0.0f};
        if (qrow < T && 16 * a + 4 * g < D) v4 = *reinterpret_cast<const f32x4*>(qb + qrow * stride + 16 * a + 4 * g);
#pragma unroll
        for (int b = 0; b < 4; ++b) qf[4 * a + b] = v4[b];
    }
    f32x4 o[NA];
#pragma unroll
    for (int c = 0; c < NA; ++c) o[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -__builtin_inff(), l_run = 0.0f;  // of query n

    for (int base = 0; base < T; base += kBK) {
        // K tile: a row's granules over consecutive lanes (coalesced reads)
#pragma unroll
        for (int f = tid; f < kBK * DP / 4; f += kThreads) {
            const int key = f / (DP / 4), gr = f % (DP / 4);
            f32x4 kv = {0.0f, 0.0f, 0.0f, 0.0f};
            if (base + key < T && 4 * gr < D) kv = *reinterpret_cast<const f32x4*>(kb + (base + key) * stride + 4 * gr);
            *reinterpret_cast<f32x4*>(ks + k_off<DP>(key, gr)) = kv;
        }
        // V tile, transposed: consecutive lanes take consecutive keys, so
        // each scalar LDS store of a wave fills one row of V^T
#pragma unroll
        for (int f = tid; f < kBK * DP / 4; f += kThreads) {
            const int key = f % kBK, d4 = (f / kBK) * 4;
            f32x4 vv = {0.0f, 0.0f, 0.0f, 0.0f};
            if (base + key < T && d4 < D) vv = *reinterpret_cast<const f32x4*>(vb + (base + key) * stride + d4);
#pragma unroll
            for (int i = 0; i < 4; ++i) vt[vt_off(d4 + i, key)] = vv[i];
        }
        __syncthreads();

        // S^T: the tile's 16-key halves against the wave's 16 queries
        f32x4 st[kNT];
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int a = 0; a < NA; ++a) {
                const f32x4 k4 = *reinterpret_cast<const f32x4*>(ks + k_off<DP>(16 * t + n, 4 * a + g));
#pragma unroll
                for (int b = 0; b < 4; ++b) c = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[b], qf[4 * a + b], c, 0, 0, 0);
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
        // rescale accumulator rows 4g + r by their queries' alpha
        float ar[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r, kWave);
#pragma unroll
        for (int c = 0; c < NA; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[c][r] *= ar[r];
        // O += P V
#pragma unroll
        for (int t = 0; t < kNT; ++t)
#pragma unroll
            for (int c = 0; c < NA; ++c) {
                const f32x4 v4 = *reinterpret_cast<const f32x4*>(vt + vt_off(16 * c + n, 16 * t + 4 * g));
#pragma unroll
                for (int r = 0; r < 4; ++r) o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[t][r], v4[r], o[c], 0, 0, 0);
            }
        __syncthreads();
    }
    // out rows 4g + r of the wave's queries: divide by their denominators
    float lr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) lr[r] = __shfl(l_run, 4 * g + r, kWave);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = q0 + wave * 16 + 4 * g + r;
        if (row < T) {
            float* dst = O + row * stride + static_cast<int64_t>(head) * D;
            const float inv = 1.0f / lr[r];
#pragma unroll
            for (int c = 0; c < NA; ++c)
                if (16 * c + n < D) dst[16 * c + n] = o[c][r] * inv;
        }
    }
}

template <int DP>
hipError_t run(const float* q, const float* k, const float* v, float* out, int64_t t, int n_heads, int d, float scale,
               hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(n_heads), static_cast<unsigned>((t + kBQ - 1) / kBQ));
    hipLaunchKernelGGL(k_flux_attn<DP>, grid, dim3(kThreads), flux_lds_bytes<DP>(), s, q, k, v, out,
                       static_cast<int>(t), n_heads, d, scale);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_flux_attention(const float* q, const float* k, const float* v, float* out, int64_t t, int n_heads,
                                 int head_dim, float scale, hipStream_t s) {
    if (head_dim <= 32) return run<32>(q, k, v, out, t, n_heads, head_dim, scale, s);
    if (head_dim <= 64) return run<64>(q, k, v, out, t, n_heads, head_dim, scale, s);
    return run<128>(q, k, v, out, t, n_heads, head_dim, scale, s);
}

}  // namespace rt_hip
