// gemv_mfma.hip -- M = 1 Q4_K GEMV on int8 MFMA (the decode hot path).
//
// y[n] = sum_k x[k] * W[n, k], W in Q4_K blocks (K % 256 == 0).  One launch
// can carry up to four such products that share x and K (a layer's q/k/v, or
// gate/up): their 16-row tiles are numbered consecutively and each wave looks
// its tile up in the job table.
//
// A wave owns 16-row tiles (q4k_mfma.hpp: lane = (row n, chunk g)); a
// workgroup of 4 waves works on 4/KS tiles at a time, the KS waves of a tile
// splitting its super-blocks and combining their partial rows through LDS.
// Each wave keeps a ring of D super-blocks of its tile loaded ahead of the
// one it computes, so D * 16 rows * 144 bytes stay in flight per wave.
// The activation is staged once per workgroup as int8 limbs in LDS; its
// global loads are issued before the weight prologue so that waiting for
// them does not drain the weight loads (vmcnt completes in order).
#include "q4k_mfma.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

using namespace q4k_mfma;

constexpr int kThreads = 256;
constexpr int kMaxJobs = 4;
constexpr int kXPre = 4;  // f32x4 of x per thread loaded before the weight prologue

// LDS-only workgroup barrier: waits for this wave's LDS traffic, not for its
// global loads, so the weight pipeline keeps running across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Job table passed by value: job j owns tiles [tile0[j], tile0[j + 1]).
struct Jobs {
    const uint8_t* w[kMaxJobs];
    float* y[kMaxJobs];
    int n[kMaxJobs];
    int tile0[kMaxJobs + 1];
    int count;
};

template <int D, int KS>
__global__ __launch_bounds__(kThreads) void k_gemv_q4k_mfma(const Jobs jobs,
                                                            const float* __restrict__ X, int K) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int TPW = 4 / KS;  // tiles per workgroup pass
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nb = K >> 8;
    const int T = jobs.tile0[jobs.count];
    const int ks = wave % KS, tslot = wave / KS;
    const int bpw = (nb + KS - 1) / KS;
    const int b0 = ks * bpw;
    const int nbw = min(nb, b0 + bpw) - b0;  // >= 1: the host picks KS so every split is non-empty
    const int passes = (T + TPW * static_cast<int>(gridDim.x) - 1) / (TPW * static_cast<int>(gridDim.x));
    const Lane ln = make_lane(lane, K);
    const size_t rb = static_cast<size_t>(nb) * kQ4kBlockBytes;
    const int nx = K >> 2;
    const f32x4* X4 = reinterpret_cast<const f32x4*>(X);

    f32x4 xv[kXPre];
#pragma unroll
    for (int i = 0; i < kXPre; ++i) {
        const int f = tid + kThreads * i;
        xv[i] = X4[f < nx ? f : 0];
    }

    // Tile t -> (job, first row); tiles past the end repeat the last one, so
    // that the pipeline's look-ahead loads stay in bounds.
    auto locate = [&](int pass, int& job, int& row0) {
        int t = (static_cast<int>(blockIdx.x) + pass * static_cast<int>(gridDim.x)) * TPW + tslot;
        t = t < T ? t : T - 1;
        job = 0;
#pragma unroll
        for (int j = 1; j < kMaxJobs; ++j) job += (j < jobs.count && t >= jobs.tile0[j]) ? 1 : 0;
        row0 = 16 * (t - jobs.tile0[job]);
    };
    auto row_ptr = [&](int pass) {
        int job, row0;
        locate(pass, job, row0);
        int row = row0 + ln.n;
        row = row < jobs.n[job] ? row : jobs.n[job] - 1;
        return jobs.w[job] + static_cast<size_t>(row) * rb;
    };
    int ip = 0, ib = 0;  // issue cursor: pass, block within this wave's range
    const uint8_t* iw = row_ptr(0);
    auto issue = [&](Blk& slot) {
        load_blk(iw, b0 + ib, ln, slot);
        if (++ib == nbw) {
            ib = 0;
            iw = row_ptr(++ip);
        }
    };

    // The scheduling barriers keep the ring's loads in slot order, so that
    // slot j's data is always the oldest in flight when it is consumed and
    // the waits stay partial (s_waitcnt vmcnt(3*(D-1))).
    Blk ring[D];
#pragma unroll
    for (int j = 0; j < D; ++j) {
        issue(ring[j]);
        __builtin_amdgcn_sched_barrier(0);
    }

#pragma unroll
    for (int i = 0; i < kXPre; ++i) {
        const int f = tid + kThreads * i;
        if (f < nx) limbs_of(xv[i], lds, K, f);
    }
    for (int f = tid + kThreads * kXPre; f < nx; f += kThreads) limbs_of(X4[f], lds, K, f);
    if (tid < 4) reinterpret_cast<u32x4*>(lds + 3 * static_cast<size_t>(K))[tid] = u32x4{0u, 0u, 0u, 0u};
    float* red = reinterpret_cast<float*>(lds + lds_bytes(K));  // [2][TPW][KS][16]
    lds_barrier();

    float acc = 0.0f;
    int pc = 0, bc = 0;  // compute cursor
    for (;;) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            acc = block_dot(ring[j], b0 + bc, ln, lds, acc);
            issue(ring[j]);
            __builtin_amdgcn_sched_barrier(0);
            if (++bc == nbw) {
                // Row n's partial: sum the four chunk lanes g.
                float v = acc;
                v += __shfl_xor(v, 16, kWave);
                v += __shfl_xor(v, 32, kWave);
                acc = 0.0f;
                const int t = (static_cast<int>(blockIdx.x) + pc * static_cast<int>(gridDim.x)) * TPW + tslot;
                int job, row0;
                locate(pc, job, row0);
                const int row = row0 + ln.n;
                const bool keep = t < T && row < jobs.n[job];
                if constexpr (KS == 1) {
                    if (lane < 16 && keep) jobs.y[job][row] = v;
                } else {
                    float* rp = red + ((pc & 1) * TPW + tslot) * KS * 16;
                    if (lane < 16) rp[ks * 16 + lane] = v;
                    lds_barrier();
                    if (ks == 0 && lane < 16 && keep) {
                        float s = rp[lane];
#pragma unroll
                        for (int q = 1; q < KS; ++q) s += rp[q * 16 + lane];
                        jobs.y[job][row] = s;
                    }
                }
                bc = 0;
                if (++pc == passes) goto done;
            }
        }
    }
done:
    return;
}

template <int D, int KS>
hipError_t run(const Jobs& jobs, const float* x, int64_t k, hipStream_t s) {
    constexpr int TPW = 4 / KS;
    const int64_t tiles = jobs.tile0[jobs.count];
    int64_t wgs = (tiles + TPW - 1) / TPW;
    const int64_t cap = static_cast<int64_t>(device_info().cus) * tune_param("Q4K_WGS_PER_CU", 8);
    if (wgs > cap) wgs = cap;
    const size_t lds = lds_bytes(static_cast<int>(k)) + 2 * TPW * KS * 16 * sizeof(float);
    hipLaunchKernelGGL((k_gemv_q4k_mfma<D, KS>), dim3(static_cast<unsigned>(wgs)), dim3(kThreads),
                       lds, s, jobs, x, static_cast<int>(k));
    return hipGetLastError();
}

}  // namespace

// K-split per tile: enough waves to cover the chip for short outputs, whole
// rows per wave for long ones.
hipError_t launch_gemv_q4k_mfma_multi(int count, const void* const* w, float* const* y,
                                      const int64_t* n, const float* x, int64_t k, hipStream_t s) {
    if (count < 1 || count > kMaxJobs) return hipErrorInvalidValue;
    Jobs jobs{};
    jobs.count = count;
    jobs.tile0[0] = 0;
    for (int j = 0; j < count; ++j) {
        jobs.w[j] = static_cast<const uint8_t*>(w[j]);
        jobs.y[j] = y[j];
        jobs.n[j] = static_cast<int>(n[j]);
        jobs.tile0[j + 1] = jobs.tile0[j] + static_cast<int>((n[j] + 15) / 16);
    }
    for (int j = count; j < kMaxJobs; ++j) jobs.tile0[j + 1] = jobs.tile0[count];
    const int64_t tiles = jobs.tile0[count];
    const int64_t nb = k / 256;
    const int64_t want = static_cast<int64_t>(device_info().cus) * tune_param("Q4K_WANT_WAVES_PER_CU", 8);
    // every wave of a split must own at least one super-block
    auto splits_ok = [&](int64_t ks) { return (ks - 1) * ((nb + ks - 1) / ks) < nb; };
    const int d = tune_param("Q4K_RING", 4);
    if (tiles >= want || !splits_ok(2))
        return d == 8 ? run<8, 1>(jobs, x, k, s) : run<4, 1>(jobs, x, k, s);
    if (tiles * 2 >= want || !splits_ok(4))
        return d == 8 ? run<8, 2>(jobs, x, k, s) : run<4, 2>(jobs, x, k, s);
    return d == 8 ? run<8, 4>(jobs, x, k, s) : run<4, 4>(jobs, x, k, s);
}

hipError_t launch_gemv_q4k_mfma(const void* w, const float* x, float* y, int64_t n, int64_t k,
                                hipStream_t s) {
    return launch_gemv_q4k_mfma_multi(1, &w, &y, &n, x, k, s);
}

}  // namespace rt_hip
