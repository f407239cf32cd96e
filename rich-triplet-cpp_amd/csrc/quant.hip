// quant.hip -- Q4_K dequantization (to f32 or bf16) and quantization.
//
// Dequant: one lane per 8 (bf16) or 4 (f32) consecutive outputs, so every
// store instruction writes 1 KB of contiguous output; bit-exact with
// Q4KMat::dequantize_row_into (quant_q4k.cpp:280-317) because both products
// are exact and only the subtraction rounds.  The bf16 variant rounds that
// f32 value to nearest-even, as flux_dequant_q4k's bfloat() conversion does
// (shaders/flux.msl:78-79).
//
// Quantize: one wave per 256-value super-block, lane l holding values
// 4l..4l+3 (sub-block l/8).  Every arithmetic step is the reference's
// (quant_q4k.cpp:71-158) in the same order with the same rounding: min/max
// are exact whatever the reduction order, the per-sub-block and per-block
// scalars are computed identically by every lane, IEEE division and
// reciprocal (hipcc's default correctly-rounded f32 divide), no
// contraction (the library builds with -ffp-contract=off), and the f16
// header conversion is the reference's truncating one restated on bits.
#include "q4k_mfma.hpp"
#include "rt_common.hpp"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

// One lane per kPer consecutive outputs of a super-block: 8 for bf16 (32
// lanes per block), 4 for f32 (64 lanes); either way a wave's store covers
// 1 KB of contiguous output.  Sub-block sb's 32 values are the low (even
// sb) or high nibbles of qs chunk sb/2, so a lane reads kPer qs bytes and
// the 16-byte header.  w = (d*sv)*q - dmin*mv: the product is exact in f32,
// so the fma rounds only the subtraction, as the reference does.  bf16 is
// v_cvt_pk_bf16_f32, round-to-nearest-even with NaN quieting: identical to
// the reference's f32 -> bf16 (bf16.hpp:50-60) on every f32, NaNs included
// (checked on the device against the bit rule).
template <bool BF16>
__device__ __forceinline__ void dequant_unit(const uint8_t* __restrict__ W, void* __restrict__ out, int64_t u) {
    constexpr int kPer = BF16 ? 8 : 4;
    constexpr int kLanesPerSub = 32 / kPer;
    constexpr int kLanesPerBlk = 8 * kLanesPerSub;
    const int64_t blk = u / kLanesPerBlk;
    const int l = static_cast<int>(u % kLanesPerBlk);
    const int sb = l / kLanesPerSub, part = l % kLanesPerSub;
    const uint8_t* bp = W + blk * kQ4kBlockBytes;
    const u32x4 hd = ld16(bp);
    const uint8_t* qp = bp + 16 + (sb >> 1) * 32 + part * kPer;
    uint32_t q[2];
    if constexpr (BF16) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(qp);
        q[0] = v[0];
        q[1] = v[1];
    } else {
        q[0] = *reinterpret_cast<const uint32_t*>(qp);
        q[1] = 0;
    }
    uint32_t sv, mv;
    decode_scale_min(make_scale_sel(sb), hd[1], hd[2], hd[3], sv, mv);
    const float sc = f16_bits_to_f32(hd[0] & 0xffffu) * static_cast<float>(sv);
    const float mn = f16_bits_to_f32(hd[0] >> 16) * static_cast<float>(mv);
    const uint32_t sh = static_cast<uint32_t>(sb & 1) * 4u;
    float w[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e)
        w[e] = __builtin_fmaf(sc, static_cast<float>((q[e >> 2] >> (8 * (e & 3) + sh)) & 15u), -mn);
    const int64_t o = blk * kQ4kBlockElems + sb * 32 + part * kPer;
    if constexpr (BF16) {
        *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + o) =
            u32x4{bf16_pair(w[0], w[1]), bf16_pair(w[2], w[3]), bf16_pair(w[4], w[5]), bf16_pair(w[6], w[7])};
    } else {
        *reinterpret_cast<f32x4*>(static_cast<float*>(out) + o) = f32x4{w[0], w[1], w[2], w[3]};
    }
}

// Grid-stride over units, kUnroll per lane per round so that several loads
// are in flight per wave; one lane per unit made 52 K short waves for a
// 8192 x 3072 weight, and wave launch, not HBM, set the time.
constexpr int kUnroll = 4;

template <bool BF16>
__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t* __restrict__ W, void* __restrict__ out,
                                                     int64_t units) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t u0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; u0 < units; u0 += stride * kUnroll) {
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) {
            const int64_t u = u0 + j * stride;
            if (u < units) dequant_unit<BF16>(W, out, u);
        }
    }
}

// A GEMM's two input conversions in one launch: units [0, wunits)
// dequantize W to bf16, the next aunits convert 8 f32 activations each to
// bf16 (the same rounding).
__global__ __launch_bounds__(256) void k_dequant_q4k_cvt(const uint8_t* __restrict__ W, uint16_t* __restrict__ wout,
                                                         int64_t wunits, const float* __restrict__ A,
                                                         uint16_t* __restrict__ aout, int64_t aunits) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256, total = wunits + aunits;
    for (int64_t u0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; u0 < total; u0 += stride * kUnroll) {
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) {
            const int64_t u = u0 + j * stride;
            if (u < wunits) {
                dequant_unit<true>(W, wout, u);
            } else if (u < total) {
                const int64_t i = u - wunits;
                const f32x4 a = reinterpret_cast<const f32x4*>(A)[2 * i];
                const f32x4 b = reinterpret_cast<const f32x4*>(A)[2 * i + 1];
                reinterpret_cast<u32x4*>(aout)[i] = u32x4{bf16_pair(a[0], a[1]), bf16_pair(a[2], a[3]),
                                                          bf16_pair(b[0], b[1]), bf16_pair(b[2], b[3])};
            }
        }
    }
}

// --- quantizer -------------------------------------------------------------

// Rust-style saturating f32 -> u8 (quant_q4k.cpp:27-35).
__device__ __forceinline__ uint32_t sat_u8(float v) {
    if (!(v > 0.0f)) return 0;
    if (v >= 255.0f) return 255;
    return static_cast<uint32_t>(v);
}

// Truncating f32 -> f16 bits (bf16.hpp:101-126).
__device__ __forceinline__ uint32_t f32_to_f16_trunc(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int32_t exp = static_cast<int32_t>((bits >> 23) & 0xffu);
    const uint32_t mant = bits & 0x7fffffu;
    if (exp == 0xff) return sign | 0x7c00u | (mant >> 13);
    const int32_t e16 = exp - 127 + 15;
    if (e16 >= 0x1f) return sign | 0x7c00u;
    if (e16 <= 0) {
        if (e16 < -10) return sign;
        const uint32_t m = mant | 0x800000u;
        return sign | (m >> (static_cast<uint32_t>(1 - e16) + 13u));
    }
    return sign | (static_cast<uint32_t>(e16) << 10) | (mant >> 13);
}

// std::min / std::max argument order of the reference (first wins on ties).
__device__ __forceinline__ float ref_min(float a, float b) { return b < a ? b : a; }
__device__ __forceinline__ float ref_max(float a, float b) { return a < b ? b : a; }

__global__ __launch_bounds__(256) void k_quantize_q4k(const float* __restrict__ w,
                                                      uint8_t* __restrict__ out, int64_t rows,
                                                      int64_t cols) {
    const int64_t nb = cols >> 8;
    const int64_t blk = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (blk >= rows * nb) return;
    const int lane = threadIdx.x & 63;
    const int64_t row = blk / nb, b = blk % nb;
    const float* src = w + row * cols + b * 256 + 4 * lane;
    const f32x4 v = *reinterpret_cast<const f32x4*>(src);

    // Step 1: sub-block (8 lanes) min / max, seeded with +-inf as the
    // reference's loop is, so a NaN input is skipped exactly as there.
    float smin = __builtin_inff(), smax = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        smin = ref_min(smin, v[e]);
        smax = ref_max(smax, v[e]);
    }
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) {
        smin = ref_min(smin, __shfl_xor(smin, off, 64));
        smax = ref_max(smax, __shfl_xor(smax, off, 64));
    }
    float sub_min, sub_scale;
    if (smin >= 0.0f) {
        sub_min = 0.0f;
        sub_scale = smax > 0.0f ? smax / 15.0f : 0.0f;
    } else {
        sub_min = smin;
        sub_scale = smax > smin ? (smax - smin) / 15.0f : 0.0f;
    }
    // Step 2: block maxima over the 8 sub-blocks.
    float max_scale = ref_max(0.0f, sub_scale), max_min = ref_max(0.0f, -sub_min);
#pragma unroll
    for (int off = 8; off <= 32; off <<= 1) {
        max_scale = ref_max(max_scale, __shfl_xor(max_scale, off, 64));
        max_min = ref_max(max_min, __shfl_xor(max_min, off, 64));
    }
    const float d = max_scale > 0.0f ? max_scale / 63.0f : 0.0f;
    const float dmin = max_min > 0.0f ? max_min / 63.0f : 0.0f;
    // Step 3: 6-bit scale and min of this lane's sub-block.
    uint32_t sv = 0, mv = 0;
    if (d > 0.0f) {
        const float inv = 1.0f / d;
        sv = min(63u, sat_u8(sub_scale * inv + 0.5f));
    }
    if (dmin > 0.0f) {
        const float inv = 1.0f / dmin;
        mv = min(63u, sat_u8(-sub_min * inv + 0.5f));
    }
    // Step 4: f16 header (truncating).
    const uint32_t d16 = f32_to_f16_trunc(d), m16 = f32_to_f16_trunc(dmin);
    const float dv = f16_bits_to_f32(d16), mvv = f16_bits_to_f32(m16);
    // Step 6: nibbles with the f16-rounded scales.
    const float sc = dv * static_cast<float>(sv), mn = mvv * static_cast<float>(mv);
    uint32_t qn = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t q = sc > 0.0f ? min(15u, sat_u8((v[e] + mn) / sc + 0.5f)) : 0u;
        qn |= q << (8 * e);
    }
    uint8_t* ob = out + blk * kQ4kBlockBytes;
    // Value 4*lane+e sits in chunk c = lane/16; lanes with (lane%16) < 8 hold
    // low nibbles, lane+8 the matching high nibbles.
    const uint32_t partner = __shfl_xor(qn, 8, 64);
    if ((lane & 15) < 8) {
        const int c = lane >> 4;
        const uint32_t word = qn | (partner << 4);
        *reinterpret_cast<uint32_t*>(ob + 16 + 32 * c + 4 * (lane & 7)) = word;
    }
    // Step 5: pack the 12 scale bytes (pack_scales, quant_q4k.cpp:43-55).
    uint32_t svs[8], mvs[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        svs[j] = __shfl(sv, 8 * j, 64);
        mvs[j] = __shfl(mv, 8 * j, 64);
    }
    if (lane == 0) {
        uint32_t s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s0 |= ((svs[j] & 0x3fu) | ((svs[j + 4] & 0x30u) << 2)) << (8 * j);
            s1 |= ((mvs[j] & 0x3fu) | ((mvs[j + 4] & 0x30u) << 2)) << (8 * j);
            s2 |= ((svs[j + 4] & 0x0fu) | ((mvs[j + 4] & 0x0fu) << 4)) << (8 * j);
        }
        *reinterpret_cast<u32x4*>(ob) = u32x4{d16 | (m16 << 16), s0, s1, s2};
    }
}

// Reference row-major Q4_K blocks -> tiled layout (q4k_mfma.hpp): one thread
// per (tile, super-block, lane) writes that lane's header dword and its two
// 16-byte halves of qs; rows past N are written as zeros.  With hd > 0 the
// rows of each head of hd rows are interleaved on the way: tiled row 2j of a
// head takes source row j, row 2j + 1 takes source row j + hd / 2 (the
// half-split RoPE pairs become adjacent rows).
__global__ __launch_bounds__(256) void k_q4k_tile(const uint8_t* __restrict__ src,
                                                  uint8_t* __restrict__ dst, int64_t n, int nb,
                                                  int64_t threads, int hd) {
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (gid >= threads) return;
    const int l = static_cast<int>(gid & 63);
    const int64_t tb = gid >> 6;  // tile * nb + b
    const int b = static_cast<int>(tb % nb);
    const int64_t t = tb / nb;
    const int g = l >> 4;
    const int64_t row = t * 16 + (l & 15);
    uint8_t* out = dst + tb * q4k_mfma::kTiledBlockBytes;
    uint32_t hdr = 0;
    u32x4 qa = {0u, 0u, 0u, 0u}, qb = {0u, 0u, 0u, 0u};
    if (row < n) {
        int64_t srow = row;
        if (hd > 0) {
            const int64_t r = row % hd;
            srow = row - r + (r >> 1) + ((r & 1) ? hd / 2 : 0);
        }
        const uint8_t* blk = src + (srow * nb + b) * kQ4kBlockBytes;
        const u32x4 h = ld16(blk);
        uint32_t sv0, mv0, sv1, mv1;
        decode_scale_min(make_scale_sel(2 * g), h[1], h[2], h[3], sv0, mv0);
        decode_scale_min(make_scale_sel(2 * g + 1), h[1], h[2], h[3], sv1, mv1);
        const uint32_t dbyte = (h[0] >> (8 * g)) & 0xffu;
        hdr = sv0 | (sv1 << 6) | (mv0 << 12) | (mv1 << 18) | (dbyte << 24);
        qa = ld16(blk + 16 + 32 * g);
        qb = ld16(blk + 32 + 32 * g);
    }
    reinterpret_cast<uint32_t*>(out)[l] = hdr;
    reinterpret_cast<u32x4*>(out + q4k_mfma::kTiledQa)[l] = qa;
    reinterpret_cast<u32x4*>(out + q4k_mfma::kTiledQb)[l] = qb;
}

}  // namespace

// Grid for `units` lanes of work: one round of kUnroll units per lane, at
// most 8 workgroups per CU.
static dim3 unit_grid(int64_t units) {
    const int64_t want = (units + 256 * kUnroll - 1) / (256 * kUnroll), cap = 8 * device_info().cus;
    return dim3(static_cast<unsigned>(want < cap ? (want < 1 ? 1 : want) : cap));
}

hipError_t launch_dequant_q4k(const void* w, void* out, bool bf16, int64_t n, int64_t k,
                              hipStream_t s) {
    const int64_t units = n * k / (bf16 ? 8 : 4);
    if (bf16)
        hipLaunchKernelGGL(k_dequant_q4k<true>, unit_grid(units), dim3(256), 0, s, static_cast<const uint8_t*>(w),
                           out, units);
    else
        hipLaunchKernelGGL(k_dequant_q4k<false>, unit_grid(units), dim3(256), 0, s, static_cast<const uint8_t*>(w),
                           out, units);
    return hipGetLastError();
}

hipError_t launch_dequant_q4k_cvt(const void* w, uint16_t* wout, int64_t n, int64_t k, const float* a,
                                  uint16_t* aout, int64_t a_elems, hipStream_t s) {
    const int64_t wunits = n * k / 8, aunits = a_elems / 8;
    hipLaunchKernelGGL(k_dequant_q4k_cvt, unit_grid(wunits + aunits), dim3(256), 0, s,
                       static_cast<const uint8_t*>(w), wout, wunits, a, aout, aunits);
    return hipGetLastError();
}

hipError_t launch_quantize_q4k(const float* w, void* blocks, int64_t n, int64_t k,
                               hipStream_t s) {
    const int64_t nblk = n * (k / 256);
    const unsigned grid = static_cast<unsigned>((nblk + 3) / 4);
    hipLaunchKernelGGL(k_quantize_q4k, dim3(grid), dim3(256), 0, s, w,
                       static_cast<uint8_t*>(blocks), n, k);
    return hipGetLastError();
}

hipError_t launch_q4k_tile(const void* blocks, void* tiled, int64_t n, int64_t k, hipStream_t s, int head_dim) {
    const int nb = static_cast<int>(k / 256);
    const int64_t threads = (n + 15) / 16 * nb * 64;
    const int64_t grid = (threads + 255) / 256;
    hipLaunchKernelGGL(k_q4k_tile, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s,
                       static_cast<const uint8_t*>(blocks), static_cast<uint8_t*>(tiled), n, nb,
                       threads, head_dim);
    return hipGetLastError();
}

}  // namespace rt_hip
