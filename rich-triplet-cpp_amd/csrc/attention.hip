// attention.hip -- decode attention over a KV cache: one query token, grouped
// query heads (gqa_attention_cached's decode path, transformer4.cpp:379-432).
//
// For each query head h (KV head h / group): s_c = (q_h . k_c) * scale over
// the cached positions c < seq_len, p = softmax(s), out_h = sum_c p_c v_c.
// The cache is f32 rows of n_kv * head_dim (LlamaLayerKvCache), head_dim 128,
// up to 4 query heads per KV head (the partial states of a workgroup live in
// static LDS: 16 groups x 4 heads x 528 bytes).
//
// Split over positions (flash decoding): workgroup (kv head, split) streams
// its chunk of positions once for all the query heads of its group and keeps
// an online softmax per head -- running max m, sum l = sum exp(s - m) and
// o = sum exp(s - m) v.  A position is read by 16 lanes, 8 values each, so
// a wave covers 4 positions per step and a 16-lane DPP reduction finishes
// each dot.  The workgroup's 16 partial states merge through LDS into one
// (m, l, o[128]) per head and split; a second launch merges the splits in
// split order and divides: out = o / l.  The order of every sum is fixed,
// so results are deterministic.  exp is the hardware exp2 on a log2(e)
// scaled argument (about 1 ulp).
#include <mutex>

#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

constexpr int kHd = 128;      // head_dim
constexpr int kT = 256;       // threads per partial workgroup
constexpr int kGroups = 16;   // 4 waves x 4 sixteen-lane position groups
constexpr int kU = 4;         // positions per group loaded ahead
constexpr float kLog2e = 1.44269504088896341f;

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the aligned 16-lane row; every lane of the row ends with the same bits.
__device__ __forceinline__ float row16_sum(float v) {
    v += dppf<0xb1>(v);   // lane ^ 1
    v += dppf<0x4e>(v);   // lane ^ 2
    v += dppf<0x141>(v);  // half-row mirror
    v += dppf<0x140>(v);  // row mirror
    return v;
}

// Partial state of one (query head, split): m, l, two pad floats, then
// o[128]; 528 bytes, so every state and its o vector are 16-byte aligned.
constexpr int kPO = 4;
constexpr int kPart = kPO + kHd;

template <int G>
__global__ __launch_bounds__(kT) void k_attn_partial(const float* __restrict__ q, const float* __restrict__ kc,
                                                     const float* __restrict__ vc, float* __restrict__ part,
                                                     int n_kv, int seq_len, int chunk, float scale) {
    __shared__ float sm[kGroups][G][2];
    __shared__ f32x4 so[kGroups][G][kHd / 4];
    const int kvh = blockIdx.x, sp = blockIdx.y, S = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = wave * 4 + (lane >> 4), sub = lane & 15;
    const int p0 = sp * chunk, p1 = min(seq_len, p0 + chunk);
    const int64_t row = static_cast<int64_t>(n_kv) * kHd;

    f32x4 qa[G], qb[G], oa[G], ob[G];
    float m[G], l[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float* qp = q + (static_cast<int64_t>(kvh) * G + h) * kHd + sub * 8;
        qa[h] = *reinterpret_cast<const f32x4*>(qp);
        qb[h] = *reinterpret_cast<const f32x4*>(qp + 4);
        oa[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        ob[h] = oa[h];
        m[h] = -__builtin_inff();
        l[h] = 0.0f;
    }
    // Positions p0 + grp + 16 j: the bound is uniform per 16-lane group, and
    // the DPP reductions stay inside the group.  kU positions per group are
    // loaded before any is used, so each batch costs one memory latency.
    for (int pb = p0 + grp; pb < p1; pb += kGroups * kU) {
        // Every load issued with no branch around it (a position past the
        // split reads row p0, which exists, and is replaced by zeros once
        // the batch's loads are all issued): behind branches the compiler
        // cannot count the loads in flight and waits for all of them.
        f32x4 ka[kU], kb[kU], va[kU], vb[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int p = pb + u * kGroups;
            const int pr = p < p1 ? p : p0;
            const float* kp = kc + pr * row + kvh * kHd + sub * 8;
            const float* vp = vc + pr * row + kvh * kHd + sub * 8;
            ka[u] = *reinterpret_cast<const f32x4*>(kp);
            kb[u] = *reinterpret_cast<const f32x4*>(kp + 4);
            va[u] = *reinterpret_cast<const f32x4*>(vp);
            vb[u] = *reinterpret_cast<const f32x4*>(vp + 4);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            const bool in = pb + u * kGroups < p1;  // uniform per group
            ka[u] = in ? ka[u] : z;
            kb[u] = in ? kb[u] : z;
            va[u] = in ? va[u] : z;
            vb[u] = in ? vb[u] : z;
        }
        // The batch's kU scores do not depend on each other: all of them
        // first (their cross-lane sums overlap), then one running-maximum
        // update and one rescale per batch instead of one per position.
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float sc[kU];
            float mn = m[h];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                float d = (qa[h][0] * ka[u][0] + qa[h][1] * ka[u][1]) + (qa[h][2] * ka[u][2] + qa[h][3] * ka[u][3]);
                d += (qb[h][0] * kb[u][0] + qb[h][1] * kb[u][1]) + (qb[h][2] * kb[u][2] + qb[h][3] * kb[u][3]);
                const float v = row16_sum(d) * scale;
                sc[u] = pb + u * kGroups < p1 ? v : -__builtin_inff();  // uniform per group
                mn = fmaxf(mn, sc[u]);
            }
            if (mn == -__builtin_inff()) continue;  // no position of this group yet
            const float a = exp_fast(m[h] - mn);    // 0 while m is -inf
            l[h] *= a;
            oa[h] *= a;
            ob[h] *= a;
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const float b = exp_fast(sc[u] - mn);  // 0 for positions past the range
                l[h] += b;
                oa[h] += va[u] * b;
                ob[h] += vb[u] * b;
            }
            m[h] = mn;
        }
    }
    // Merge the 16 group states: every group writes, then thread (h, d4)
    // folds them in group order.
#pragma unroll
    for (int h = 0; h < G; ++h) {
        if (sub == 0) {
            sm[grp][h][0] = m[h];
            sm[grp][h][1] = l[h];
        }
        so[grp][h][sub * 2] = oa[h];
        so[grp][h][sub * 2 + 1] = ob[h];
    }
    __syncthreads();
    for (int t = tid; t < G * (kHd / 4); t += kT) {
        const int h = t / (kHd / 4), d4 = t % (kHd / 4);
        float M = -__builtin_inff();
        for (int g = 0; g < kGroups; ++g) M = fmaxf(M, sm[g][h][0]);
        float L = 0.0f;
        f32x4 O = {0.0f, 0.0f, 0.0f, 0.0f};
        if (M != -__builtin_inff()) {
            for (int g = 0; g < kGroups; ++g) {
                const float w = exp_fast(sm[g][h][0] - M);
                L += sm[g][h][1] * w;
                O += so[g][h][d4] * w;
            }
        }
        float* dst = part + (static_cast<int64_t>(kvh * G + h) * S + sp) * kPart;
        if (d4 == 0) {
            dst[0] = M;
            dst[1] = L;
        }
        *reinterpret_cast<f32x4*>(dst + kPO + d4 * 4) = O;
    }
}

// One workgroup of 128 threads per query head: fold the splits in order.
// Up to kBatch splits load in one batch (indices past S repeat split S - 1,
// in bounds, and get weight 0), so the merge costs one memory latency.
constexpr int kBatch = 32;

__global__ __launch_bounds__(kHd) void k_attn_combine(const float* __restrict__ part, float* __restrict__ out,
                                                      int S) {
    const int h = blockIdx.x, d = threadIdx.x;
    const float* ph = part + static_cast<int64_t>(h) * S * kPart;
    float M = -__builtin_inff(), L = 0.0f, O = 0.0f;
    if (S <= kBatch) {
        float ms[kBatch], ls[kBatch], os[kBatch];
#pragma unroll
        for (int s = 0; s < kBatch; ++s) {
            const float* ps = ph + min(s, S - 1) * kPart;
            ms[s] = ps[0];
            ls[s] = ps[1];
            os[s] = ps[kPO + d];
        }
#pragma unroll
        for (int s = 0; s < kBatch; ++s) M = fmaxf(M, ms[s]);
        if (M != -__builtin_inff()) {
#pragma unroll
            for (int s = 0; s < kBatch; ++s) {
                const float w = s < S ? exp_fast(ms[s] - M) : 0.0f;
                L += ls[s] * w;
                O += os[s] * w;
            }
        }
    } else {
#pragma unroll 8
        for (int s = 0; s < S; ++s) M = fmaxf(M, ph[s * kPart]);
        if (M != -__builtin_inff()) {
#pragma unroll 8
            for (int s = 0; s < S; ++s) {
                const float w = exp_fast(ph[s * kPart] - M);
                L += ph[s * kPart + 1] * w;
                O += ph[s * kPart + kPO + d] * w;
            }
        }
    }
    out[static_cast<int64_t>(h) * kHd + d] = L > 0.0f ? O / L : 0.0f;
}

template <int G>
hipError_t run(const float* q, const float* kc, const float* vc, float* out, float* part, int n_kv, int seq_len,
               int S, int chunk, float scale, hipStream_t s) {
    hipLaunchKernelGGL(k_attn_partial<G>, dim3(static_cast<unsigned>(n_kv), static_cast<unsigned>(S)), dim3(kT), 0,
                       s, q, kc, vc, part, n_kv, seq_len, chunk, scale);
    hipLaunchKernelGGL(k_attn_combine, dim3(static_cast<unsigned>(n_kv * G)), dim3(kHd), 0, s, part, out, S);
    return hipGetLastError();
}

}  // namespace

void attention_decode_shape(int64_t n_kv, int64_t seq_len, int* splits, int* chunk) {
    // About one workgroup per CU, and whole batches: at least one batch of
    // kU positions per group (64 positions) per split.
    const int64_t cus = device_info().cus;
    const int64_t want = (cus + n_kv - 1) / n_kv;
    const int64_t batch = kGroups * kU;
    int64_t c = (seq_len + want - 1) / want;
    c = (c + batch - 1) / batch * batch;
    const int64_t S = (seq_len + c - 1) / c;
    *splits = static_cast<int>(S < 1 ? 1 : S);
    *chunk = static_cast<int>(c);
}

// Scratch of rt_hip_attention_decode_noalloc: the split partials of one
// call in a file-scope device array, so that entry point allocates nothing.
// Each device holds its own copy at its own address; in host code the
// array's name is only a stand-in, so its device address is looked up once
// per device (attention_scratch_setup, with that device current) and that
// pointer is what kernels receive.  Every call on a device shares the array
// and leaves the last call's partials in it; the partial kernel writes every
// state the merge reads, so nothing needs clearing.  Calls that overlap on
// one device race.
constexpr size_t kNoallocScratchBytes = size_t{1} << 20;
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};
}  // namespace

size_t attention_scratch_bytes() { return kNoallocScratchBytes; }

hipError_t attention_scratch_setup(int dev, void** out) {
    if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = p;
    }
    if (out) *out = g_scratch_ptr[dev];
    return hipSuccess;
}

size_t attention_decode_workspace(int64_t n_q, int64_t n_kv, int64_t seq_len) {
    int S, c;
    attention_decode_shape(n_kv, seq_len, &S, &c);
    return static_cast<size_t>(n_q) * S * kPart * sizeof(float);
}

hipError_t launch_attention_decode(const float* q, const float* kc, const float* vc, float* out, float* part,
                                   int64_t n_q, int64_t n_kv, int64_t seq_len, float scale, hipStream_t s) {
    int S, chunk;
    attention_decode_shape(n_kv, seq_len, &S, &chunk);
    const int G = static_cast<int>(n_q / n_kv), nk = static_cast<int>(n_kv), L = static_cast<int>(seq_len);
    switch (G) {
        case 1: return run<1>(q, kc, vc, out, part, nk, L, S, chunk, scale, s);
        case 2: return run<2>(q, kc, vc, out, part, nk, L, S, chunk, scale, s);
        case 3: return run<3>(q, kc, vc, out, part, nk, L, S, chunk, scale, s);
        case 4: return run<4>(q, kc, vc, out, part, nk, L, S, chunk, scale, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rt_hip
