// gemv_q40.hip -- M = 1 GEMV on GGUF Q4_0 blocks (decode): y[n] = sum_k x[k] * W[n, k].
//
// GGUF Q4_0 (gguf.cpp:495-529): 18-byte blocks of 32 values, d f16 then
// qs[16]; value j < 16 is (qs[j] & 15) - 8, value 16 + j is (qs[j] >> 4) - 8,
// both times d.  Rows are K/32 blocks; with K % 256 == 0 a row is a multiple
// of 144 bytes, so rows (and runs of 64 blocks) start 16-byte aligned.
//
// A lane owns whole blocks: lane l reads block 64 p + l of a row as the five
// dwords covering bytes [18 l, 18 l + 18) of the 64-block run, one 16-byte
// and one 4-byte load (18 l is 0 or 2 mod 4; an odd lane's d sits in the
// high half of its first dword and its qs are its next four dwords, an even
// lane's qs straddle dwords and are rebuilt with funnel shifts).  The activation is staged in LDS chunk-major
// -- 16-byte chunk c of block b at (c * NB + b) * 16 -- so the 8 lanes an
// LDS read serves together (consecutive blocks) hit consecutive chunks, and
// each block's sum of x is precomputed for the -8 offset:
//     block dot = d * (sum_j lo_j x_j + hi_j x_{16+j} - 8 * sum(x)).
// A wave streams its rows' blocks through one ring of D slots (one block per
// lane per slot) that runs on from row to row, as the BF16 row loop
// (gemv_bf16.hpp), and keeps row r's sum in lane r.
//
// Numerics: f32, factorized and reordered against the reference's
// sequential dequant-and-dot (quant_q4.cpp:92-114); agreement to f32
// rounding (normwise 1e-5 in the tests).
#include "gemv_bf16.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

constexpr int kBlockBytes = 18;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

struct Slot {
    uint32_t w0, w1, w2, w3, w4;
};

template <int D, int XP, int kT>
__global__ __launch_bounds__(kT) void k_gemv_q40(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                 float* __restrict__ Y, int N, int K) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int NB = K >> 5;              // blocks per row
    const int SP = (NB + 63) >> 6;      // slots (64-block runs) per row
    const int nx4 = K >> 2;
    const f32x4* X4 = reinterpret_cast<const f32x4*>(X);
    f32x4* const xs = reinterpret_cast<f32x4*>(lds);             // [8][NB]
    float* const sums = reinterpret_cast<float*>(lds + 16 * nx4);  // [NB]

    f32x4 xv[XP];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int f = tid + kT * i;
        xv[i] = X4[f < nx4 ? f : 0];
    }
    __builtin_amdgcn_sched_barrier(0);

    // Rows of this wave: gw, gw + NW, ... (at most 64: the launcher sizes
    // the grid).
    const int NW = static_cast<int>(gridDim.x) * (kT / kWave);
    const int gw = static_cast<int>(blockIdx.x) * (kT / kWave) + wave;
    const int R = gw < N ? (N - 1 - gw) / NW + 1 : 0;
    const int L = R * SP;
    const int64_t rowb = static_cast<int64_t>(NB) * kBlockBytes;
    const int64_t stride = static_cast<int64_t>(NW) * rowb;
    const uint8_t* const wb = W + static_cast<int64_t>(gw) * rowb;
    const uint32_t loff = static_cast<uint32_t>(lane * kBlockBytes) & ~3u;
    const bool odd = (lane & 1) != 0;

    int ir = 0, ip = 0, cr = 0, cp = 0;
    Slot ring[D];
    auto issue = [&](Slot& sl) {
        const int64_t o = static_cast<int64_t>(ip) * (64 * kBlockBytes);
        const BufRsrc rs = make_rsrc(wb + ir * stride + o, ir < R ? rowb - o : 0);
        // a 16-byte load at a 4-byte aligned offset (buffer loads need only
        // dword alignment), then the fifth dword: two instructions, not five
        const u32x4 v = ld16(rs, loff);
        sl.w0 = v[0];
        sl.w1 = v[1];
        sl.w2 = v[2];
        sl.w3 = v[3];
        sl.w4 = __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(loff + 16), 0, 0);
        const bool wrap = ip == SP - 1;
        ip = __builtin_amdgcn_readfirstlane(wrap ? 0 : ip + 1);
        ir = __builtin_amdgcn_readfirstlane(wrap ? ir + 1 : ir);
    };
#pragma unroll
    for (int j = 0; j < D; ++j) {
        issue(ring[j]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Stage x chunk-major, with the per-block sums: a block's 8 chunks sit in
    // 8 consecutive lanes (f = tid + kT * i), summed by DPP within the group
    // (every lane of the group ends with the same bits); its first lane
    // stores the sum.
    auto stage = [&](const f32x4 v, int f) {
        float sm = (v[0] + v[1]) + (v[2] + v[3]);
        sm += dpp_f<0xb1>(sm);   // lane ^ 1
        sm += dpp_f<0x4e>(sm);   // lane ^ 2
        sm += dpp_f<0x141>(sm);  // half-row mirror: lane i <-> 7 - i
        if (f < nx4) {
            xs[(f & 7) * NB + (f >> 3)] = v;
            if ((f & 7) == 0) sums[f >> 3] = sm;
        }
    };
#pragma unroll
    for (int i = 0; i < XP; ++i) stage(xv[i], tid + kT * i);
    for (int f0 = kT * XP; f0 < nx4; f0 += kT) {
        const int f = f0 + tid;
        stage(X4[f < nx4 ? f : 0], f);
    }
    lds_barrier();

    float acc = 0.0f, res = 0.0f;
    auto consume = [&](const Slot& sl) {
        const int b = cp * 64 + lane;  // this lane's block (past NB: zeros, never read)
        const int bb = b < NB ? b : 0;
        // qs dwords and d: an odd lane's block starts 2 bytes into w0.
        const uint32_t q0 = odd ? sl.w1 : __builtin_amdgcn_alignbyte(sl.w1, sl.w0, 2);
        const uint32_t q1 = odd ? sl.w2 : __builtin_amdgcn_alignbyte(sl.w2, sl.w1, 2);
        const uint32_t q2 = odd ? sl.w3 : __builtin_amdgcn_alignbyte(sl.w3, sl.w2, 2);
        const uint32_t q3 = odd ? sl.w4 : __builtin_amdgcn_alignbyte(sl.w4, sl.w3, 2);
        const float d = f16_bits_to_f32(odd ? (sl.w0 >> 16) : (sl.w0 & 0xffffu));
        const uint32_t q[4] = {q0, q1, q2, q3};
        // Four independent chains (one per qs dword): one wave per SIMD
        // leaves a single chain latency-bound.
        float dc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const f32x4 lo = xs[c * NB + bb], hi = xs[(c + 4) * NB + bb];
            const uint32_t v = q[c];
            float t = ubyte_f32(v & 0x0f0f0f0fu, 0) * lo[0];
            t = __builtin_fmaf(ubyte_f32(v & 0x0f0f0f0fu, 1), lo[1], t);
            t = __builtin_fmaf(ubyte_f32(v & 0x0f0f0f0fu, 2), lo[2], t);
            t = __builtin_fmaf(ubyte_f32(v & 0x0f0f0f0fu, 3), lo[3], t);
            const uint32_t h = (v >> 4) & 0x0f0f0f0fu;
            t = __builtin_fmaf(ubyte_f32(h, 0), hi[0], t);
            t = __builtin_fmaf(ubyte_f32(h, 1), hi[1], t);
            t = __builtin_fmaf(ubyte_f32(h, 2), hi[2], t);
            t = __builtin_fmaf(ubyte_f32(h, 3), hi[3], t);
            dc[c] = t;
        }
        const float dot = (dc[0] + dc[1]) + (dc[2] + dc[3]);
        const float blk = d * __builtin_fmaf(-8.0f, sums[bb], dot);
        acc += b < NB ? blk : 0.0f;
        if (cp == SP - 1) {
            const float v = bf16_gemv::wave_sum(acc, lane);
            res = lane == cr ? v : res;
            acc = 0.0f;
        }
        const bool cwrap = cp == SP - 1;
        cp = __builtin_amdgcn_readfirstlane(cwrap ? 0 : cp + 1);
        cr = __builtin_amdgcn_readfirstlane(cwrap ? cr + 1 : cr);
    };

    int i = 0;
    for (; i + D < L; i += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            consume(ring[j]);
            __builtin_amdgcn_sched_barrier(0);
            issue(ring[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < D; ++j)
        if (i + j < L) consume(ring[j]);

    auto* const Yg = (__attribute__((address_space(1))) float*)Y;
    if (lane < R) Yg[gw + lane * NW] = res;
}

}  // namespace

size_t q40_m1_lds_bytes(int64_t k) { return static_cast<size_t>(k) * 4 + static_cast<size_t>(k / 32) * 4; }

hipError_t launch_gemv_q4_0_m1(const void* w, const float* x, float* y, int64_t n, int64_t k, hipStream_t s) {
    // Rows per wave: four 64-block runs per wave, at most 64 rows (row sums
    // stay in lanes).  Measured at 4096 x 4096 (two runs per row): 2 rows
    // per wave 5.65 us, 4 rows (a full ring of 8) 5.92 us, 1 row 6.26 us --
    // more waves per CU hide more latency than a fuller ring.  8 waves per
    // workgroup where that is one round of workgroups (x staged once per CU
    // instead of twice): 5.51-5.53 us against 5.69-5.76 with 4 (1 row per
    // wave at 8: 6.13; 4 rows: 7.04).
    const int64_t runs = (k / 32 + 63) / 64;
    int64_t rpw = tune_param("Q40_ROWS_PER_WAVE", static_cast<int>((4 + runs - 1) / runs));
    rpw = rpw < 1 ? 1 : (rpw > 64 ? 64 : rpw);
    const int T = tune_param("Q40_THREADS", (n + 8 * rpw - 1) / (8 * rpw) <= device_info().cus ? 512 : 256) == 512
                      ? 512
                      : 256;
    const int64_t waves = T / kWave;
    const int64_t wgs = (n + waves * rpw - 1) / (waves * rpw);
    const int64_t per = (k / 4 + T - 1) / T;
    const size_t lds = q40_m1_lds_bytes(k);
    const dim3 g(static_cast<unsigned>(wgs)), b(T);
    const auto* wb = static_cast<const uint8_t*>(w);
    const int in = static_cast<int>(n), ik = static_cast<int>(k);
    if (T == 512) {
        if (per <= 4)
            hipLaunchKernelGGL((k_gemv_q40<8, 4, 512>), g, b, lds, s, wb, x, y, in, ik);
        else
            hipLaunchKernelGGL((k_gemv_q40<8, 8, 512>), g, b, lds, s, wb, x, y, in, ik);
    } else if (per <= 4) {
        hipLaunchKernelGGL((k_gemv_q40<8, 4, 256>), g, b, lds, s, wb, x, y, in, ik);
    } else {
        hipLaunchKernelGGL((k_gemv_q40<8, 8, 256>), g, b, lds, s, wb, x, y, in, ik);
    }
    return hipGetLastError();
}

}  // namespace rt_hip
