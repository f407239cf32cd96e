// q4k_mfma.hpp -- Q4_K x f32 dot products on gfx950 int8 MFMA.
//
// The f32 activation is represented exactly enough to stand in for f32: per
// 32-value sub-block (the Q4_K sub-block size), a power-of-two scale s
// (2^(E-5) for the sub-block's absmax exponent E) and three int8 limbs
//     a = s * (A0 + A1/256 + A2/65536) + e,   |A0| <= 64, -128 <= A1,A2 <= 127,
//     |e| <= 0.5 * s / 65536 <= 2.4e-7 * absmax,
// i.e. R = rint(a/s * 2^16) written in signed base-256 digits.  A
// power-of-two s keeps the one-hot case exact: x = e_k gives A0 = 1/s,
// A1 = A2 = 0, and the result is the dequantized weight bit-for-bit.
//
// v_mfma_i32_16x16x64_i8 computes C[16x16] += A[16x64] * B[64x16] exactly in
// int32.  For a 16-row weight tile, lane l = (n = l%16, g = l/16) supplies
// column n of B: 16 nibble bytes of chunk g of row n's super-block (sub-block
// 2g from the low nibbles, 2g+1 from the high ones).  Row m = 4*gm + lambda
// of A is nonzero only in the K-slots of lane group gm, where it holds limb
// lambda of the matching activations.  The hardware leaves lane l holding
// C[4g + r][n], r = 0..3, i.e. exactly the three limb dots of its own
// sub-block for its own row -- no cross-lane traffic before the epilogue.
//
// Exactness of the integer part: |C| <= 32 * 15 * 128 < 2^24, so the int32
// sums and their f32 conversions are exact; the only roundings are the
// epilogue's f32 operations.
#pragma once

#include "rt_common.hpp"

namespace rt_hip {
namespace q4k_mfma {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// LDS layout of one staged activation vector of length K (K % 256 == 0):
//   [0, 3K)            limb planes lambda = 0, 1, 2 (int8, K bytes each)
//   [3K, 3K + 64)      zeros (the A operand of inactive lanes)
//   [3K + 64, ...)     per sub-block f32x4 {s, s/256, s/65536, sum}
__host__ __device__ inline size_t lds_bytes(int K) {
    return 3 * static_cast<size_t>(K) + 64 + static_cast<size_t>(K / 32) * 16;
}
// The decode chain first lands x as raw f32 in the same area, so it needs
// the larger of the two (4K bytes for every K > 128).
__host__ __device__ inline size_t stage_bytes(int K) {
    const size_t raw = 4 * static_cast<size_t>(K), limbs = lds_bytes(K);
    return raw > limbs ? raw : limbs;
}

// DPP lane swizzles within a row of 16 lanes (VALU, no LDS round trip).
constexpr int kDppQuadSwap1 = 0xb1;    // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4e;    // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror: lane i <-> 7 - i in each 8
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum and max over the aligned 8-lane group.  The pairing tree is
// ((l, l^1), (l^2 pair)), (other quad): every lane of the group ends with
// the same bits, since each step adds two values in either order.
__device__ __forceinline__ void group8_sum_max(float& sum, float& amax) {
    sum += dpp<kDppQuadSwap1>(sum);
    amax = fmaxf(amax, dpp<kDppQuadSwap1>(amax));
    sum += dpp<kDppQuadSwap2>(sum);
    amax = fmaxf(amax, dpp<kDppQuadSwap2>(amax));
    sum += dpp<kDppHalfMirror>(sum);
    amax = fmaxf(amax, dpp<kDppHalfMirror>(amax));
}

// Scale of a sub-block from its absmax: s = 2^(E-5), E = unbiased exponent
// of amax, and inv = 1/s; zero (or subnormal-range) sub-blocks get s = 0
// and zero limbs.  An Inf/NaN activation makes s non-finite so the output
// is NaN/Inf, as the reference's f32 arithmetic would make it.  Masks
// rather than conditionals: written as selects, the compiler made branches
// of them, with exec-mask saves around each.
__device__ __forceinline__ void sub_block_scale(float amax, float& s, float& inv) {
    const uint32_t eb = (__float_as_uint(amax) >> 23) & 0xffu;
    const uint32_t live = 0u - static_cast<uint32_t>(eb - 7u < 248u);  // 7 <= eb <= 254
    const uint32_t nonfinite = 0u - static_cast<uint32_t>(eb == 0xffu);
    s = __uint_as_float((((eb - 5u) << 23) & live) | (__float_as_uint(amax) & nonfinite));
    inv = __uint_as_float(((259u - eb) << 23) & live);
}

// The three limb words (planes A0, A1, A2; value e in byte e) of four
// activations of one sub-block, inv = 1/s.  |v * inv| < 64 and the scaling
// is exact, so b = v * inv * 2^16 + 1.5 * 2^23 is rounded once, to the
// nearest integer, and its bits are 0x4B400000 + R with R = rint(v/s * 2^16),
// |R| < 2^22.  The signed base-256 digits of R are then bytes of b:
//     A2 = R mod 256 (as int8)          = byte 0 of b
//     A1 = ((R + 128) >> 8) mod 256     = byte 1 of b + 128
//     A0 = (R + 32896) >> 16            = byte 2 of b + 0x8080 - 0x400000
// (the last subtracts the magic's own 0x40 in bits 16..23), so that
// R = 65536 A0 + 256 A1 + A2 with |A0| <= 64.  v_perm gathers each plane.
__device__ __forceinline__ void limb_words(const f32x4 v, float inv, uint32_t& w0, uint32_t& w1, uint32_t& w2) {
    uint32_t b[4], m[4], h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        b[e] = __float_as_uint(__builtin_fmaf(v[e] * inv, 65536.0f, 12582912.0f));
        m[e] = b[e] + 128u;
        h[e] = b[e] - 4161408u;  // + 0x8080 - 0x400000
    }
    // perm(hi, lo, sel): byte j of the result is byte sel_j of {hi:lo}
    auto gather = [](const uint32_t (&x)[4], uint32_t byte) {
        const uint32_t pair = 0x0c0c0400u | (byte * 0x0101u);
        return __builtin_amdgcn_perm(__builtin_amdgcn_perm(x[3], x[2], pair),
                                     __builtin_amdgcn_perm(x[1], x[0], pair), 0x05040100u);
    };
    w0 = gather(h, 2);
    w1 = gather(m, 1);
    w2 = gather(b, 0);
}

// Limbs of 4 activations (one f32x4) of a sub-block whose 8 holders are the
// aligned 8-lane group of the calling lane.  Writes the limb bytes and, from
// the group's first lane, the sub-block constants; with store == false it
// only takes part in the group reductions (lanes past the end of x).
__device__ __forceinline__ void limbs_of(const f32x4 v, uint8_t* lds, int K, int f, bool store = true) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    float sum = (v[0] + v[1]) + (v[2] + v[3]);
    group8_sum_max(sum, amax);
    float s, inv;
    sub_block_scale(amax, s, inv);
    uint32_t w0, w1, w2;
    limb_words(v, inv, w0, w1, w2);
    if (!store) return;
    uint32_t* l32 = reinterpret_cast<uint32_t*>(lds);
    l32[f] = w0;
    l32[(K >> 2) + f] = w1;
    l32[(K >> 1) + f] = w2;
    if ((f & 7) == 0) {
        f32x4* cst = reinterpret_cast<f32x4*>(lds + 3 * static_cast<size_t>(K) + 64);
        cst[f >> 3] = f32x4{s, s * (1.0f / 256.0f), s * (1.0f / 65536.0f), sum};
    }
}

// Per-lane constants of the tile layout.
struct Lane {
    int n, g;          // weight row within the tile, chunk / C row group
    uint32_t a_base;   // LDS byte offset of this lane's A operand (block 0)
    uint32_t a_mask;   // 0 for inactive A lanes (they read the zero area)
    uint32_t cst_base; // LDS byte offset of the constants of sub-block 2g
    uint32_t hmask;    // ~0 when g >= 2: sub-blocks 4..7 (split 6-bit scale layout)
};

__device__ __forceinline__ Lane make_lane(int lane, int K) {
    Lane ln;
    ln.n = lane & 15;
    ln.g = lane >> 4;
    const int m = lane & 15, gm = m >> 2, lambda = m & 3;
    const bool active = gm == ln.g && lambda < 3;
    ln.a_base = active ? static_cast<uint32_t>(lambda * K + 64 * ln.g) : static_cast<uint32_t>(3 * K);
    ln.a_mask = active ? 0xffffffffu : 0u;
    ln.cst_base = static_cast<uint32_t>(3 * K + 64 + 32 * ln.g);
    ln.hmask = ln.g >= 2 ? 0xffffffffu : 0u;
    return ln;
}

// Registers one lane holds per super-block: its header and its 32-byte chunk.
struct Blk {
    u32x4 h, q0, q1;
};

__device__ __forceinline__ void load_blk(const uint8_t* row, int b, const Lane& ln, Blk& r) {
    const uint8_t* bp = row + static_cast<size_t>(b) * kQ4kBlockBytes;
    r.h = ld16(bp);
    r.q0 = ld16(bp + 16 + 32 * ln.g);
    r.q1 = ld16(bp + 32 + 32 * ln.g);
}

// Same, through a buffer resource whose base is super-block b of the tile's
// first row: `roff` = n * row_bytes, lane's row; rows past the resource's end
// read as zeros.
__device__ __forceinline__ void load_blk(BufRsrc rs, uint32_t roff, const Lane& ln, Blk& r) {
    r.h = ld16(rs, roff);
    r.q0 = ld16(rs, roff + 16 + 32 * ln.g);
    r.q1 = ld16(rs, roff + 32 + 32 * ln.g);
}

// A super-block with its loaded registers already taken apart: the nibble
// planes as MFMA B operands and this lane's two scale and min products.
// Once a block is decoded its load registers are free for the next load.
// The products d*sv and dmin*mv are exact in f32 (11 + 6 significant bits),
// so every layout that yields the same (d, dmin, sv, mv) gives the same bits.
struct Dec {
    i32x4 B0, B1, B2, B3;
    float ds0, ds1;  // d * sv of sub-blocks 2g, 2g+1
    float dm0, dm1;  // dmin * mv of sub-blocks 2g, 2g+1
};

__device__ __forceinline__ void nibble_planes(const u32x4 q0, const u32x4 q1, Dec& o) {
    o.B0 = __builtin_bit_cast(i32x4, q0 & 0x0f0f0f0fu);
    o.B1 = __builtin_bit_cast(i32x4, q1 & 0x0f0f0f0fu);
    o.B2 = __builtin_bit_cast(i32x4, (q0 >> 4) & 0x0f0f0f0fu);
    o.B3 = __builtin_bit_cast(i32x4, (q1 >> 4) & 0x0f0f0f0fu);
}

__device__ __forceinline__ Dec decode(const Blk& r, const Lane& ln) {
    Dec o;
    // Scales: bytes 2g and 2g+1 of the 6-bit scale/min arrays
    // (Q4KMat::scale_min, quant_q4k.cpp:58-69), both decoded at once.
    const uint32_t off = 16u * static_cast<uint32_t>(ln.g & 1);
    const uint32_t a0 = __builtin_amdgcn_ubfe(r.h[1], off, 16);
    const uint32_t a1 = __builtin_amdgcn_ubfe(r.h[2], off, 16);
    const uint32_t a2 = __builtin_amdgcn_ubfe(r.h[3], off, 16);
    // Both layouts computed, then selected with the lane mask (no branch).
    const uint32_t sv_lo = a0 & 0x3f3fu, mv_lo = a1 & 0x3f3fu;
    const uint32_t sv_hi = (a2 & 0x0f0fu) | ((a0 >> 2) & 0x3030u);
    const uint32_t mv_hi = ((a2 >> 4) & 0x0f0fu) | ((a1 >> 2) & 0x3030u);
    const uint32_t svp = sv_lo ^ ((sv_lo ^ sv_hi) & ln.hmask);
    const uint32_t mvp = mv_lo ^ ((mv_lo ^ mv_hi) & ln.hmask);
    const float d = f16_bits_to_f32(r.h[0] & 0xffffu);
    const float dm = f16_bits_to_f32(r.h[0] >> 16);
    o.ds0 = d * ubyte_f32(svp, 0);
    o.ds1 = d * ubyte_f32(svp, 1);
    o.dm0 = dm * ubyte_f32(mvp, 0);
    o.dm1 = dm * ubyte_f32(mvp, 1);
    nibble_planes(r.q0, r.q1, o);
    return o;
}

// ---- tiled layout ---------------------------------------------------------
// A 16-row tile's super-block b is 2304 contiguous bytes in lane order
// (lane l = n + 16 g: row n of the tile, chunk g):
//   [0, 256)      one dword per lane: sv(2g) | sv(2g+1) << 6 | mv(2g) << 12 |
//                 mv(2g+1) << 18 | byte g of (d | dmin << 16) << 24
//   [256, 1280)   16 bytes per lane: qs[32g, 32g+16) of row n
//   [1280, 2304)  16 bytes per lane: qs[32g+16, 32g+32) of row n
// Tiles are stored one after another, each as its nb super-blocks in order,
// so a tile is 16 * row_bytes bytes, the same as its 16 rows; rows past N in
// the last tile are zero.  Every load of the GEMV reads contiguous memory.
constexpr int kTiledHdr = 256;
constexpr int kTiledQa = 256;
constexpr int kTiledQb = 1280;
constexpr int kTiledBlockBytes = 2304;

struct BlkT {
    uint32_t h;
    u32x4 q0, q1;
};

// Lane constants for reassembling (d | dmin << 16) from the byte each of the
// four lanes of a row holds: shift of bytes g, g^1, g^2, g^3.
struct TLane {
    uint32_t s0, s1, s2, s3;
    bool odd_row, high_half;  // 16-lane row g is odd / g >= 2
};

__device__ __forceinline__ TLane make_tlane(int lane) {
    const uint32_t g = static_cast<uint32_t>(lane >> 4);
    return TLane{8u * g, 8u * (g ^ 1u), 8u * (g ^ 2u), 8u * (g ^ 3u), (g & 1u) != 0, g >= 2u};
}

// x from lane l ^ 16 and from lane l ^ 32 (gfx950 permlane swaps: a swap of
// a register with itself exchanges whole 16- or 32-lane groups).
__device__ __forceinline__ uint32_t xor16(uint32_t x, bool odd_row) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return odd_row ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t xor32(uint32_t x, bool high_half) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return high_half ? r[0] : r[1];
}

__device__ __forceinline__ void load_blk_t(BufRsrc rs, uint32_t lane, BlkT& r) {
    r.h = __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(lane * 4u), 0, 0);
    r.q0 = ld16(rs, kTiledQa + lane * 16u);
    r.q1 = ld16(rs, kTiledQb + lane * 16u);
}

__device__ __forceinline__ Dec decode_t(const BlkT& r, const TLane& tl) {
    Dec o;
    const uint32_t b = r.h >> 24;
    const uint32_t b1 = xor16(b, tl.odd_row);
    const uint32_t b2 = xor32(b, tl.high_half);
    const uint32_t b3 = xor32(b1, tl.high_half);
    const uint32_t dd = (b << tl.s0) | (b1 << tl.s1) | (b2 << tl.s2) | (b3 << tl.s3);
    const float d = f16_bits_to_f32(dd & 0xffffu);
    const float dm = f16_bits_to_f32(dd >> 16);
    o.ds0 = d * static_cast<float>(__builtin_amdgcn_ubfe(r.h, 0, 6));
    o.ds1 = d * static_cast<float>(__builtin_amdgcn_ubfe(r.h, 6, 6));
    o.dm0 = dm * static_cast<float>(__builtin_amdgcn_ubfe(r.h, 12, 6));
    o.dm1 = dm * static_cast<float>(__builtin_amdgcn_ubfe(r.h, 18, 6));
    nibble_planes(r.q0, r.q1, o);
    return o;
}

// acc += this lane's share (chunk g of block b) of row n's dot product;
// `lds` is the staged activation (layout above).
__device__ __forceinline__ float dot(const Dec& r, int b, const Lane& ln, const uint8_t* lds,
                                     float acc) {
    auto lds_a = [&](uint32_t off) { return *reinterpret_cast<const i32x4*>(lds + off); };
    auto lds_f4 = [&](uint32_t off) { return *reinterpret_cast<const f32x4*>(lds + off); };
    const uint32_t a_addr = ln.a_base + ((static_cast<uint32_t>(b) << 8) & ln.a_mask);
    const i32x4 A0 = lds_a(a_addr), A1 = lds_a(a_addr + 16), A2 = lds_a(a_addr + 32),
                A3 = lds_a(a_addr + 48);
    const i32x4 z = {0, 0, 0, 0};
    i32x4 clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, r.B0, z, 0, 0, 0);
    clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, r.B1, clo, 0, 0, 0);
    i32x4 chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, r.B2, z, 0, 0, 0);
    chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(A3, r.B3, chi, 0, 0, 0);

    const uint32_t c_addr = ln.cst_base + (static_cast<uint32_t>(b) << 7);
    const f32x4 kl = lds_f4(c_addr), kh = lds_f4(c_addr + 16);
    // dot of the sub-block in activation units: s*C0 + s/256*C1 + s/65536*C2
    float dl = static_cast<float>(clo[0]) * kl[0];
    dl = __builtin_fmaf(static_cast<float>(clo[1]), kl[1], dl);
    dl = __builtin_fmaf(static_cast<float>(clo[2]), kl[2], dl);
    float dh = static_cast<float>(chi[0]) * kh[0];
    dh = __builtin_fmaf(static_cast<float>(chi[1]), kh[1], dh);
    dh = __builtin_fmaf(static_cast<float>(chi[2]), kh[2], dh);
    // sum_w x = (d*sv) * dot - (dmin*mv) * sum(x), per sub-block
    acc = __builtin_fmaf(r.ds0, dl, acc);
    acc = __builtin_fmaf(-r.dm0, kl[3], acc);
    acc = __builtin_fmaf(r.ds1, dh, acc);
    acc = __builtin_fmaf(-r.dm1, kh[3], acc);
    return acc;
}

}  // namespace q4k_mfma
}  // namespace rt_hip
