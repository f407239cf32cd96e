// rt_common.hpp -- device helpers shared by the gfx950 kernels.
//
// Numeric contracts (these are what make the kernels bit-exact where the
// reference is exact):
//  * f16 -> f32 is exact (v_cvt_f32_f16; f16 denormals are kept, the
//    kernels never change the MODE register).  include/rt/bf16.hpp:66-93.
//  * bf16 -> f32 is a 16-bit shift.  bf16.hpp:42-44.
//  * Q4_K dequant w = (d*sv)*q - dmin*mv: both products are exact in f32
//    (at most 11+6+4 significant bits), so only the subtraction rounds and
//    the value cannot depend on FMA contraction.  quant_q4k.cpp:301-312.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rt_hip {

constexpr int kWave = 64;
constexpr int kQ4kBlockBytes = 144;
constexpr int kQ4kBlockElems = 256;
constexpr int kQ40BlockBytes = 18;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two f32 -> one dword of bf16 (a in the low half): v_cvt_pk_bf16_f32,
// round-to-nearest-even with NaN quieting, identical to f32_to_bf16_rne
// below on every f32, NaNs included (checked on the device against the bit
// rule over 4 M values).
__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

__device__ __forceinline__ float bf16_lo_to_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi_to_f32(uint32_t w) {
    return __uint_as_float(w & 0xffff0000u);
}

// Byte k (0..3) of a dword as f32: v_cvt_f32_ubyte{k}.
__device__ __forceinline__ float ubyte_f32(uint32_t w, int k) {
    return static_cast<float>((w >> (8 * k)) & 0xffu);
}

// 16-byte load through the vector memory path.
__device__ __forceinline__ u32x4 ld16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// Raw buffer resource over [base, base + bytes): loads at byte offsets
// >= bytes return zeros without touching memory.  Word 3 is the gfx9-family
// raw-buffer format (stride 0, no swizzle).  The range check covers the
// per-lane offset and the instruction offset, not soffset, so callers move
// the base rather than pass soffset.
typedef __amdgpu_buffer_rsrc_t BufRsrc;
__device__ __forceinline__ BufRsrc make_rsrc_n(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}
// `bytes` clamped to [0, 2^32 - 1].
__device__ __forceinline__ uint32_t rsrc_bytes(int64_t bytes) {
    return bytes <= 0 ? 0u : (bytes >= 0xffffffffll ? 0xffffffffu : static_cast<uint32_t>(bytes));
}
__device__ __forceinline__ BufRsrc make_rsrc(const void* base, int64_t bytes) {
    return make_rsrc_n(base, rsrc_bytes(bytes));
}
__device__ __forceinline__ u32x4 ld16(BufRsrc r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0));
}

// LDS-only workgroup barrier: waits for this wave's LDS traffic, not for its
// global loads, so a weight pipeline keeps running across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// s_waitcnt vmcnt(N) alone (gfx9 encoding: vmcnt bits [3:0] and [15:14],
// expcnt [6:4] and lgkmcnt [11:8] left at their no-wait maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Non-temporal 16-byte load for weights that are streamed exactly once.
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Argmax key of (value, index): an order-preserving map of the f32 (-0
// folded onto +0) in the high half and (0xffffffff - index) in the low half,
// so the maximum key is the largest value with the lowest index.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<uint64_t>(u) << 32) | (0xffffffffu - idx);
}

// bf16 limbs of four activations (one f32x4): three 8-byte bf16 quads with
// h + m + l == x exactly for every finite x (each residual is exact in f32);
// an infinite x keeps its infinity in h and zero low limbs.  Each limb is one
// v_cvt_pk_bf16_f32 per pair (bf16_pair): the same bits as f32_to_bf16_rne at
// a fifth of the VALU.
__device__ __forceinline__ void bf16_limbs4(const f32x4 v, u32x2& h, u32x2& m, u32x2& l) {
    const uint32_t h01 = bf16_pair(v[0], v[1]), h23 = bf16_pair(v[2], v[3]);
    const float hf[4] = {__uint_as_float(h01 << 16), __uint_as_float(h01 & 0xffff0000u), __uint_as_float(h23 << 16),
                         __uint_as_float(h23 & 0xffff0000u)};
    float r1[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r1[e] = __builtin_isinf(hf[e]) ? 0.0f : v[e] - hf[e];
    const uint32_t m01 = bf16_pair(r1[0], r1[1]), m23 = bf16_pair(r1[2], r1[3]);
    const float r2[4] = {r1[0] - __uint_as_float(m01 << 16), r1[1] - __uint_as_float(m01 & 0xffff0000u),
                         r1[2] - __uint_as_float(m23 << 16), r1[3] - __uint_as_float(m23 & 0xffff0000u)};
    h = u32x2{h01, h23};
    m = u32x2{m01, m23};
    l = u32x2{bf16_pair(r2[0], r2[1]), bf16_pair(r2[2], r2[3])};
}

// f32 -> bf16 round-to-nearest-even with NaN quieting (bf16.hpp:50-60).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float v) {
    const uint32_t bits = __float_as_uint(v);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((bits >> 16) | 0x40u);
    return static_cast<uint16_t>((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

// Sum over the `L` lanes of an aligned lane segment (L = 8..64), by xor
// butterflies; every lane of the segment ends with the same value.
template <int L>
__device__ __forceinline__ float segment_sum(float v) {
#pragma unroll
    for (int off = L / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Q4_K 6-bit scale/min of sub-block j of a super-block, from the three
// scale dwords s0 = sc[0..3], s1 = sc[4..7], s2 = sc[8..11]
// (Q4KMat::scale_min, quant_q4k.cpp:58-69):
//   j < 4 : sv = sc[j] & 63,            mv = sc[j+4] & 63
//   j >= 4: sv = (sc[j+4] & 15) | ((sc[j-4] >> 6) << 4)
//           mv = (sc[j+4] >> 4) | ((sc[j]   >> 6) << 4)
// Lanes carry a per-lane j, so the selection is written branch-free from
// precomputed bit offsets (ScaleSel).
struct ScaleSel {
    uint32_t lo_s_off;  // offset of the low 4 bits of sv
    uint32_t lo_m_off;  // offset of the low 4 bits of mv
    uint32_t hi_off;    // offset of the top 2 bits (sv in s0, mv in s1)
    bool high;          // j >= 4: low bits come from s2
};

__device__ __forceinline__ ScaleSel make_scale_sel(int j) {
    ScaleSel s;
    const uint32_t t = static_cast<uint32_t>(j & 3) * 8u;
    s.high = j >= 4;
    s.lo_s_off = t;
    s.lo_m_off = s.high ? t + 4u : t;
    s.hi_off = s.high ? t + 6u : t + 4u;
    return s;
}

__device__ __forceinline__ void decode_scale_min(const ScaleSel& s, uint32_t s0, uint32_t s1,
                                                 uint32_t s2, uint32_t& sv, uint32_t& mv) {
    const uint32_t src_s = s.high ? s2 : s0;
    const uint32_t src_m = s.high ? s2 : s1;
    sv = __builtin_amdgcn_ubfe(src_s, s.lo_s_off, 4) | (__builtin_amdgcn_ubfe(s0, s.hi_off, 2) << 4);
    mv = __builtin_amdgcn_ubfe(src_m, s.lo_m_off, 4) | (__builtin_amdgcn_ubfe(s1, s.hi_off, 2) << 4);
}

}  // namespace rt_hip
