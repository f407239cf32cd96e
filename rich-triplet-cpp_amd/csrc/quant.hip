// quant.hip -- Q4_K dequantization (to f32 or bf16) and quantization.
//
// Dequant: one lane per 16-byte piece of qs (32 values), as the GEMV reads
// them; bit-exact with Q4KMat::dequantize_row_into (quant_q4k.cpp:280-317)
// because both products are exact and only the subtraction rounds.  The
// bf16 variant rounds that f32 value to nearest-even, as flux_dequant_q4k's
// bfloat() conversion does (shaders/flux.msl:78-79).
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

__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t* __restrict__ W,
                                                     void* __restrict__ out, int64_t pieces,
                                                     bool bf16) {
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (gid >= pieces) return;
    const int64_t blk = gid >> 3;
    const int p = static_cast<int>(gid & 7), c = p >> 1, h = p & 1;
    const uint8_t* bp = W + blk * kQ4kBlockBytes;
    const u32x4 hd = ld16(bp);
    const u32x4 q = ld16(bp + 16 + 16 * p);
    const float d = f16_bits_to_f32(hd[0] & 0xffffu);
    const float dm = f16_bits_to_f32(hd[0] >> 16);
    uint32_t sv1, mv1, sv2, mv2;
    decode_scale_min(make_scale_sel(2 * c), hd[1], hd[2], hd[3], sv1, mv1);
    decode_scale_min(make_scale_sel(2 * c + 1), hd[1], hd[2], hd[3], sv2, mv2);
    const float s1 = d * static_cast<float>(sv1), n1 = dm * static_cast<float>(mv1);
    const float s2 = d * static_cast<float>(sv2), n2 = dm * static_cast<float>(mv2);
    float lo[16], hi[16];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t byte = (q[j] >> (8 * e)) & 0xffu;
            lo[4 * j + e] = s1 * static_cast<float>(byte & 0x0fu) - n1;
            hi[4 * j + e] = s2 * static_cast<float>(byte >> 4) - n2;
        }
    const int64_t o = blk * kQ4kBlockElems + c * 64 + h * 16;
    if (!bf16) {
        float* dst = static_cast<float*>(out) + o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            reinterpret_cast<f32x4*>(dst)[j] = f32x4{lo[4 * j], lo[4 * j + 1], lo[4 * j + 2], lo[4 * j + 3]};
            reinterpret_cast<f32x4*>(dst + 32)[j] =
                f32x4{hi[4 * j], hi[4 * j + 1], hi[4 * j + 2], hi[4 * j + 3]};
        }
    } else {
        uint16_t* dst = static_cast<uint16_t*>(out) + o;
        u32x4 a, b;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a[j] = f32_to_bf16_rne(lo[2 * j]) | (static_cast<uint32_t>(f32_to_bf16_rne(lo[2 * j + 1])) << 16);
            b[j] = f32_to_bf16_rne(lo[8 + 2 * j]) |
                   (static_cast<uint32_t>(f32_to_bf16_rne(lo[8 + 2 * j + 1])) << 16);
        }
        reinterpret_cast<u32x4*>(dst)[0] = a;
        reinterpret_cast<u32x4*>(dst)[1] = b;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a[j] = f32_to_bf16_rne(hi[2 * j]) | (static_cast<uint32_t>(f32_to_bf16_rne(hi[2 * j + 1])) << 16);
            b[j] = f32_to_bf16_rne(hi[8 + 2 * j]) |
                   (static_cast<uint32_t>(f32_to_bf16_rne(hi[8 + 2 * j + 1])) << 16);
        }
        reinterpret_cast<u32x4*>(dst + 32)[0] = a;
        reinterpret_cast<u32x4*>(dst + 32)[1] = b;
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
// 16-byte halves of qs; rows past N are written as zeros.
__global__ __launch_bounds__(256) void k_q4k_tile(const uint8_t* __restrict__ src,
                                                  uint8_t* __restrict__ dst, int64_t n, int nb,
                                                  int64_t threads) {
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
        const uint8_t* blk = src + (row * nb + b) * kQ4kBlockBytes;
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

hipError_t launch_dequant_q4k(const void* w, void* out, bool bf16, int64_t n, int64_t k,
                              hipStream_t s) {
    const int64_t pieces = n * (k / 256) * 8;
    const unsigned blocks = static_cast<unsigned>((pieces + 255) / 256);
    hipLaunchKernelGGL(k_dequant_q4k, dim3(blocks), dim3(256), 0, s,
                       static_cast<const uint8_t*>(w), out, pieces, bf16);
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

hipError_t launch_q4k_tile(const void* blocks, void* tiled, int64_t n, int64_t k, hipStream_t s) {
    const int nb = static_cast<int>(k / 256);
    const int64_t threads = (n + 15) / 16 * nb * 64;
    const int64_t grid = (threads + 255) / 256;
    hipLaunchKernelGGL(k_q4k_tile, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s,
                       static_cast<const uint8_t*>(blocks), static_cast<uint8_t*>(tiled), n, nb,
                       threads);
    return hipGetLastError();
}

}  // namespace rt_hip
