/*
 * rt_oracle.h -- CPU restatement of rich-triplet's quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product library (librt_hip.so) never links or calls it.
 *
 * Every function restates one reference function; the citation is the
 * reference file:line it follows (paths relative to the reference root).
 * All floating-point code is compiled with -ffp-contract=off -fno-fast-math,
 * the reference's global flags (CMakeLists.txt:33-47), so sequential f32
 * results are bit-identical to the reference's x86 build.
 *
 * Pinning (what checks each function beyond restating it):
 *   conversions ........ special values + exhaustive f16 round trip, and
 *                        bit-equality with oracle/_ref (compiled reference)
 *   q4k scale_min/pack . the reference's pack/unpack vectors
 *                        (tests/test_gguf.cpp:379-404) + _ref
 *   q4k quantize ....... byte-equality with _ref on random and adversarial
 *                        matrices; properties of tests/test_quant.cpp:138-214
 *   q4k dequant ........ hand-built blocks (closed form) + _ref
 *   q4k dot/gemv ....... one-hot activations reproduce dequantized columns
 *                        bit-exactly; fp64 brute force; bit-equality with _ref
 *   bf16 dot/gemv ...... fp64 brute force; bit-equality with _ref
 *   q4mat .............. _ref; tests/test_quant.cpp:25-83 bounds
 *   gguf q4_0 .......... the reference's hand-built block
 *                        (tests/test_gguf.cpp:175-218)
 *   q6_k ............... the reference's mt19937(1234) known block
 *                        (tests/test_gguf.cpp:292-335)
 *   argmax ............. hand-built ties, NaN, -inf
 *   initrng ............ _ref (same libm in the same process)
 *   flux attention ..... closed forms (one key -> v; equal scores -> the
 *                        mean of v; a dominant key -> its v), float64
 *                        softmax attention, key-permutation invariance
 */
#ifndef RT_ORACLE_H
#define RT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* include/rt/bf16.hpp:42-126 */
float orc_bf16_to_f32(uint16_t bits);
uint16_t orc_f32_to_bf16(float v);
float orc_f16_to_f32(uint16_t bits);
uint16_t orc_f32_to_f16(float v);
void orc_f32_to_bf16_n(const float* src, uint16_t* dst, size_t n);

/* src/quant_q4k.cpp:27-35 (Rust-style saturating f32 -> u8) */
uint8_t orc_sat_u8(float v);

/* src/quant_q4k.cpp:58-69 */
void orc_q4k_scale_min(const uint8_t* sc, size_t j, float* scale, float* min);
/* src/quant_q4k.cpp:43-55 */
void orc_q4k_pack_scales(const uint8_t sv[8], const uint8_t mv[8], uint8_t sc[12]);
/* src/quant_q4k.cpp:71-158: 256 f32 -> 144 bytes */
void orc_q4k_quantize_block(const float* x, uint8_t* out);
/* src/quant_q4k.cpp:164-205: rows x cols f32 -> rows * (cols/256) blocks.
 * Release semantics: floor(cols/256) super-blocks per row. */
void orc_q4k_quantize(const float* w, size_t rows, size_t cols, uint8_t* blocks,
                      int n_threads);
/* src/quant_q4k.cpp:207-218 */
void orc_q4k_quantize_from_bf16(const uint16_t* w, size_t rows, size_t cols,
                                uint8_t* blocks, int n_threads);
/* src/quant_q4k.cpp:280-317: writes floor(cols/256)*256 values of row `row` */
void orc_q4k_dequant_row(const uint8_t* blocks, size_t cols, size_t row, float* out);
/* src/quant_q4k.cpp:482-523 (x86 branch) */
float orc_q4k_dot_row(const uint8_t* blocks, size_t cols, size_t row, const float* a);
/* src/quant_q4k.cpp:564-600 (x86 branch): T = max(1, min(n_threads, rows/128)) */
void orc_q4k_gemv_mt(const uint8_t* blocks, size_t rows, size_t cols, const float* a,
                     float* y, int n_threads);
/* src/quant_q4k.cpp:602-624: M == 1 -> gemv_mt, else scalar loop.
 * Rows [r0, r1) only (r0 = 0, r1 = rows for the full product); y is M x rows
 * and only columns [r0, r1) are written. */
void orc_q4k_matmul_t(const uint8_t* blocks, size_t rows, size_t cols, const float* a,
                      size_t m, float* y, int n_threads, size_t r0, size_t r1);
/* src/quant_q4k.cpp:525-562 (portable part of the aarch64 activation path) */
void orc_q4k_quantize_activation_q8(const float* a, size_t k, int8_t* q8, float* scales,
                                    float* sums);
/* src/quant_q4k.cpp:425-478 (dot_row_q8, aarch64): integer chunk dots, then
 * the f32 combination left to right.  Pinned (tests/test_oracle_q8.py) by the
 * integer dots recomputed in int64, activations that Q8 represents exactly
 * (the result then equals the f64 dequantized dot to f32 rounding), the
 * quantization error bound on random activations, one-hot and constant
 * blocks in closed form, and a planted dropped term. */
float orc_q4k_dot_row_q8(const uint8_t* blocks, size_t cols, size_t row, const int8_t* q8,
                         const float* scales, const float* sums);
/* src/quant_q4k.cpp:564-600 (aarch64 branch): quantize once, dot_row_q8 per row */
void orc_q4k_gemv_q8(const uint8_t* blocks, size_t rows, size_t cols, const float* a, float* y);

/* src/mat.cpp:304-316 (x86 branch) */
float orc_bf16_dot_row(const uint16_t* w, size_t cols, size_t row, const float* a);
/* src/mat.cpp:318-349 */
void orc_bf16_gemv_mt(const uint16_t* w, size_t rows, size_t cols, const float* a, float* y,
                      int n_threads);
/* src/mat.cpp:351-414 (non-BLAS branch for M > 1); rows [r0, r1) as above */
void orc_bf16_matmul_t(const uint16_t* w, size_t rows, size_t cols, const float* a, size_t m,
                       float* y, int n_threads, size_t r0, size_t r1);

/* src/quant_q4.cpp:17-54: packed = ceil(n/2) bytes, scales = ceil(n/32) */
void orc_q4mat_quantize(const float* w, size_t n, uint8_t* packed, float* scales);
/* src/quant_q4.cpp:67-74 */
void orc_q4mat_dequant(const uint8_t* packed, const float* scales, size_t n, float* out);
/* src/quant_q4.cpp:92-114 (single-threaded, any M) */
void orc_q4mat_matmul_t(const uint8_t* packed, const float* scales, size_t rows, size_t cols,
                        const float* a, size_t m, float* y);

/* src/gguf.cpp:495-529: GGUF Q4_0 (18-byte blocks) -> f32 */
void orc_q4_0_decode_f32(const uint8_t* blocks, size_t n_elem, float* out);
/* src/gguf.cpp:392-450: GGUF Q4_0 -> Q4Mat */
void orc_q4_0_to_q4mat(const uint8_t* blocks, size_t n_elem, uint8_t* packed, float* scales);
/* tests/test_gguf.cpp:43-54: the reference's only Q4_0 encoder (test helper) */
void orc_q4_0_encode_block(const float* vals, float scale, uint8_t* out18);

/* GGUF Q4_0 bytes for n_elem (multiple of 32) values: scale = absmax/7 per
 * block, stored as truncated f16, nibbles via orc_q4_0_encode_block.  The
 * reference ships no production Q4_0 encoder; this is the test helper's rule
 * applied block by block. */
void orc_q4_0_quantize(const float* w, size_t n_elem, uint8_t* out);

/* src/gguf.cpp:531-580 */
void orc_q6k_decode_f32(const uint8_t* blocks, size_t n_elem, float* out);

/* RMSNorm of one row and SwiGLU, as the reference computes them
 * (tensor_node.cpp:320-344, 383-402; transformer5.cpp:186-190).
 * Pinned by: closed forms (a constant row c gives c / sqrt(c^2 + eps) * g;
 * gemma3 = the plain form with 1 + gamma), the scale invariance
 * rmsnorm(a x) = rmsnorm(x) for eps = 0 and a power of two, silu's fixed
 * points (silu(0) = 0, silu(x) -> x and -> 0 at the tails) and its identity
 * silu(x) - silu(-x) = x, each checked in float64 by tests/test_oracle_layer_ops.py.
 * The reference's own tensor_node.cpp needs its autograd graph (TensorNode,
 * Mat and their sources) and is not built here. */
void orc_rmsnorm(const float* x, const float* gamma, size_t d, float eps, int gemma3, float* out);

/* Config5::inv_freq and llama_rope, interleaved pairing (transformer5.cpp:
 * 36-52, 95-125).  Pinned in tests/test_oracle_layer_ops.py by: pos 0 is the
 * identity bit for bit; each pair keeps its length; the output equals the
 * float64 rotation of the same pairs by the same f32 angles; the pairing is
 * (2i, 2i + 1), not (i, i + head_dim / 2); inv_freq matches the float64
 * formula, divisors included. */
void orc_llama_inv_freq(float theta, size_t head_dim, const float* divisors, size_t n_div, float* out);

/* gqa_attention_cached's decode path (transformer4.cpp:379-432).  Pinned in
 * tests/test_oracle_layer_ops.py by: one cached position gives out = v
 * exactly; equal keys give the mean of the values; the float64 softmax of
 * the same scores; and the GQA head mapping (query head h reads KV head
 * h / group, checked with distinct per-head values). */
void orc_gqa_attention_decode(const float* q, const float* k_cache, const float* v_cache, size_t k_start,
                              size_t k_end, size_t n_q_heads, size_t n_kv_heads, size_t d_head, float scale,
                              float* out);
void orc_llama_rope_half(const float* x, size_t n_heads, size_t head_dim, size_t pos, const float* inv_freq,
                         float* out);
void orc_llama_rope_interleaved(const float* x, size_t n_heads, size_t head_dim, size_t pos, const float* inv_freq,
                                float* out);
void orc_swiglu(const float* gate, const float* up, size_t n, float* out);

/* src/transformer5.cpp:382-391: first index of the strict maximum; NaN never wins */
int64_t orc_argmax_first(const float* v, size_t n);

/* include/rt/init_rng.hpp:14-47 */
void orc_initrng_normal(uint64_t seed, size_t n, float std_dev, float* out);
void orc_initrng_uniform(uint64_t seed, size_t n, float* out);

/* include/rt/parallel.hpp:18-21 */
int orc_hardware_threads(void);

/* ---- Gemma 3 decode operations of the Metal engine
 * (src/shaders/decode_gemma3.msl; sequenced by src/metal_decode.mm:436-482) */
/* decode_gemma3.msl:63-97 */
void orc_rmsnorm_per_head(const float* x, const float* gamma, size_t n_heads, size_t head_dim, float eps,
                          float* out);
/* decode_gemma3.msl:99-126 (NeoX half-split pairing, pow-form angle) */
void orc_rope_neox(const float* x, size_t n_heads, size_t head_dim, float theta, float freq_scale, size_t pos,
                   float* out);
/* decode_gemma3.msl:128-145 */
void orc_gelu_tanh(const float* x, size_t n, float* out);
/* decode_gemma3.msl:174-187: half() of the KV-cache append, IEEE RNE */
uint16_t orc_f32_to_f16_rne(float v);
void orc_f32_to_f16_rne_n(const float* src, uint16_t* dst, size_t n);

/* ---- FLUX attention: src/flux.cpp:282-323 (the CPU path the Metal
 * flux_attention kernel, src/shaders/flux.msl:145-331, stands in for).
 * q, k, v [t][n_heads * head_dim]; out [n_rows][n_heads * head_dim] holds
 * the output rows rows[0..n_rows) (all of them: rows = NULL, n_rows = t),
 * each computed exactly as the reference computes that row. */
void orc_flux_attention(const float* q, const float* k, const float* v, size_t t, size_t n_heads,
                        size_t head_dim, const int64_t* rows, size_t n_rows, float* out);

#ifdef __cplusplus
}
#endif

#endif /* RT_ORACLE_H */
