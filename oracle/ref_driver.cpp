// ref_driver.cpp -- C entry points over the reference's own compiled sources.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's src/quant_q4k.cpp, src/quant_q4.cpp and src/mat.cpp, read in
// place from the reference tree, with the reference's Release flags
// (-O3 -DNDEBUG -ffp-contract=off -fno-fast-math, CMakeLists.txt:17-47) and no
// RT_FEATURE_* macro (the Linux build: no Accelerate, no Metal).  The result,
// oracle/_ref/libref_oracle.so, is used by the tests to pin the C restatement
// in rt_oracle.c bit-for-bit, and optionally as bench.py's CPU baseline.
//
// Every wrapper copies its inputs into the reference's types and calls the
// reference's public method; nothing here computes on its own.
#include <cstdint>
#include <cstring>
#include <memory>
#include <span>
#include <vector>

#include "rt/bf16.hpp"
#include "rt/init_rng.hpp"
#include "rt/mat.hpp"
#include "rt/parallel.hpp"
#include "rt/quant.hpp"

using namespace rt;

namespace {
Mat make_mat(const float* p, std::size_t rows, std::size_t cols) {
    return Mat(std::vector<float>(p, p + rows * cols), rows, cols);
}
Q4KMat make_q4k(const std::uint8_t* blocks, std::size_t rows, std::size_t cols) {
    Q4KMat q;
    q.rows = rows;
    q.cols = cols;
    q.blocks.assign(blocks, blocks + rows * (cols / 256) * 144);
    return q;
}
}  // namespace

extern "C" {

float ref_bf16_to_f32(std::uint16_t b) { return bf16_to_f32(b); }
std::uint16_t ref_f32_to_bf16(float v) { return f32_to_bf16(v); }
float ref_f16_to_f32(std::uint16_t b) { return f16_to_f32(b); }
std::uint16_t ref_f32_to_f16(float v) { return f32_to_f16(v); }

int ref_hardware_threads() { return static_cast<int>(hardware_threads()); }

void ref_q4k_scale_min(const std::uint8_t* sc, std::size_t j, float* s, float* m) {
    Q4KMat::scale_min(sc, j, *s, *m);
}

void ref_q4k_quantize_block(const float* x, std::uint8_t* out) {
    Q4KMat::quantize_block(std::span<const float>(x, 256), std::span<std::uint8_t>(out, 144));
}

// Q4KMat::quantize (quant_q4k.cpp:199-205); out holds rows*(cols/256)*144 bytes.
void ref_q4k_quantize(const float* w, std::size_t rows, std::size_t cols, std::uint8_t* out) {
    const Q4KMat q = Q4KMat::quantize(make_mat(w, rows, cols));
    std::memcpy(out, q.blocks.data(), q.blocks.size());
}

// Q4KMat::quantize_from_bf16 (quant_q4k.cpp:207-218)
void ref_q4k_quantize_from_bf16(const std::uint16_t* w, std::size_t rows, std::size_t cols,
                                std::uint8_t* out) {
    const MatBf16 m(std::vector<std::uint16_t>(w, w + rows * cols), rows, cols);
    const Q4KMat q = Q4KMat::quantize_from_bf16(m);
    std::memcpy(out, q.blocks.data(), q.blocks.size());
}

// Q4KMat::dequantize_row_into (quant_q4k.cpp:280-317)
void ref_q4k_dequant_row(const std::uint8_t* blocks, std::size_t rows, std::size_t cols,
                         std::size_t row, float* out) {
    const Q4KMat q = make_q4k(blocks, rows, cols);
    q.dequantize_row_into(row, std::span<float>(out, cols));
}

// Q4KMat::dot_row (quant_q4k.cpp:482-523)
float ref_q4k_dot_row(const std::uint8_t* blocks, std::size_t rows, std::size_t cols,
                      std::size_t row, const float* a) {
    const Q4KMat q = make_q4k(blocks, rows, cols);
    return q.dot_row(row, std::span<const float>(a, cols));
}

// Q4KMat::matmul_q4k_t (quant_q4k.cpp:602-624): M==1 -> gemv_mt, else scalar
void ref_q4k_matmul_t(const std::uint8_t* blocks, std::size_t rows, std::size_t cols,
                      const float* a, std::size_t m, float* y) {
    const Q4KMat q = make_q4k(blocks, rows, cols);
    const Mat out = q.matmul_q4k_t(make_mat(a, m, cols));
    std::memcpy(y, out.data.data(), m * rows * sizeof(float));
}

// Persistent-weight variant for timing: the handle owns a Q4KMat so a timed
// loop measures only the product, as the reference's callers see it.
void* ref_q4k_new(const std::uint8_t* blocks, std::size_t rows, std::size_t cols) {
    return new Q4KMat(make_q4k(blocks, rows, cols));
}
void ref_q4k_delete(void* h) { delete static_cast<Q4KMat*>(h); }
void ref_q4k_handle_matmul_t(void* h, const float* a, std::size_t m, float* y) {
    const Q4KMat& q = *static_cast<Q4KMat*>(h);
    const Mat out = q.matmul_q4k_t(make_mat(a, m, q.cols));
    std::memcpy(y, out.data.data(), m * q.rows * sizeof(float));
}

// Q4KMat::quantize_activation_q8 (quant_q4k.cpp:525-562)
void ref_q4k_quantize_activation_q8(const float* a, std::size_t k, std::int8_t* q8,
                                    float* scales, float* sums) {
    const Q8Activation r = Q4KMat::quantize_activation_q8(std::span<const float>(a, k));
    std::memcpy(q8, r.q8.data(), r.q8.size());
    std::memcpy(scales, r.scales.data(), r.scales.size() * sizeof(float));
    std::memcpy(sums, r.sums.data(), r.sums.size() * sizeof(float));
}

// MatBf16::matmul_by_t (mat.cpp:351-414): M==1 -> gemv_mt, else scalar rows
void ref_bf16_matmul_t(const std::uint16_t* w, std::size_t rows, std::size_t cols,
                       const float* a, std::size_t m, float* y) {
    const MatBf16 mb(std::vector<std::uint16_t>(w, w + rows * cols), rows, cols);
    const Mat out = mb.matmul_by_t(make_mat(a, m, cols));
    std::memcpy(y, out.data.data(), m * rows * sizeof(float));
}
void* ref_bf16_new(const std::uint16_t* w, std::size_t rows, std::size_t cols) {
    return new MatBf16(std::vector<std::uint16_t>(w, w + rows * cols), rows, cols);
}
void ref_bf16_delete(void* h) { delete static_cast<MatBf16*>(h); }
void ref_bf16_handle_matmul_t(void* h, const float* a, std::size_t m, float* y) {
    const MatBf16& mb = *static_cast<MatBf16*>(h);
    const Mat out = mb.matmul_by_t(make_mat(a, m, mb.cols));
    std::memcpy(y, out.data.data(), m * mb.rows * sizeof(float));
}

// Q4Mat::quantize / dequantize / matmul_q4_t (quant_q4.cpp:17-114)
void ref_q4mat_quantize(const float* w, std::size_t rows, std::size_t cols,
                        std::uint8_t* packed, float* scales) {
    const Q4Mat q = Q4Mat::quantize(make_mat(w, rows, cols));
    std::memcpy(packed, q.packed.data(), q.packed.size());
    std::memcpy(scales, q.scales.data(), q.scales.size() * sizeof(float));
}
void ref_q4mat_matmul_t(const std::uint8_t* packed, const float* scales, std::size_t rows,
                        std::size_t cols, const float* a, std::size_t m, float* y) {
    Q4Mat q;
    q.rows = rows;
    q.cols = cols;
    const std::size_t n = rows * cols;
    q.packed.assign(packed, packed + (n + 1) / 2);
    q.scales.assign(scales, scales + (n + 31) / 32);
    const Mat out = q.matmul_q4_t(make_mat(a, m, cols));
    std::memcpy(y, out.data.data(), m * rows * sizeof(float));
}

// InitRng (init_rng.hpp:14-47)
void ref_initrng_normal(std::uint64_t seed, std::size_t n, float std_dev, float* out) {
    InitRng rng(seed);
    const std::vector<float> v = rng.normal_vec(n, std_dev);
    std::memcpy(out, v.data(), n * sizeof(float));
}

}  // extern "C"
