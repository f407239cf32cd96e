/*
 * rt_hip.h -- C ABI of the MI355X (gfx950) quantized-linear library.
 *
 * Drop-in boundary for rich-triplet's quantized-weight linear path.  Every
 * entry point takes plain device pointers and sizes; nothing here carries a
 * C++ or torch type.  Weights are [N, K] row-major (out_features x
 * in_features), activations [M, K] row-major f32, outputs [M, N] f32:
 * y = x * W^T, exactly the reference's `Mat` / `Q4KMat` / `MatBf16`
 * convention (include/rt/quant.hpp:119-199, include/rt/mat.hpp:157-207).
 * An output may not overlap an input of the same call (x, gamma, up, gate):
 * every workgroup reads its inputs while others store outputs.  Such calls
 * fail with RT_HIP_E_ARG.
 *
 * Errors: every function returns an rt_hip_status; 0 is success.  The
 * message for the last failure on the calling thread is rt_hip_last_error().
 * (The reference aborts in its GPU ops, metal_ops.mm:312-315, and asserts
 * on the CPU; a C ABI reports instead.)  Kernels run asynchronously on the
 * given stream (NULL = the legacy default stream); a status of 0 means the
 * launch was accepted.  Calls on different streams may run concurrently,
 * except calls that use the per-device library workspace -- argmax, GEMM,
 * and GEMV with m > 1 (its K-slice partials and arrival counters): those
 * must not overlap on one device (issue them on one stream, or order the
 * streams).
 *
 * Weight byte formats (verbatim, as the reference holds them in memory):
 *   RT_HIP_Q4K   144-byte GGUF Q4_K super-blocks, K/256 per row
 *                (d:f16 | dmin:f16 | scales[12] | qs[128]); quant.hpp:119-137
 *   RT_HIP_Q4_0  18-byte GGUF Q4_0 blocks, K/32 per row (d:f16 | qs[16]);
 *                gguf.cpp:495-529 -- the form Q4Mat decodes from
 *   RT_HIP_BF16  uint16 bf16 bits; mat.hpp:157-207
 *   RT_HIP_Q4MAT the reference's Q4Mat (quant.hpp:23-75) in one buffer: its
 *                `packed` bytes (flat element r*K + c is the low nibble of
 *                byte (r*K + c)/2 when even, the high nibble when odd; 4-bit
 *                two's complement) at offset 0, then its f32 `scales` (one
 *                per 32 flat elements) at rt_hip_q4mat_scales_offset(n, k);
 *                rt_hip_q4mat_bytes(n, k) in all.  Requires K % 32 == 0.
 */
#ifndef RT_HIP_H
#define RT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* rt_hip_stream; /* a hipStream_t */

typedef enum {
    RT_HIP_OK = 0,
    RT_HIP_E_ARG = 1,          /* null pointer, negative size, bad enum */
    RT_HIP_E_SHAPE = 2,        /* M/N/K outside what the kernel supports */
    RT_HIP_E_ALIGN = 3,        /* K not a multiple of the block size, or a
                                  pointer not 16-byte aligned */
    RT_HIP_E_OOM = 4,          /* device allocation failed */
    RT_HIP_E_HIP = 5,          /* a HIP runtime call failed */
    RT_HIP_E_UNSUPPORTED = 6,  /* no gfx950 device, or format not handled */
    RT_HIP_E_FORMAT = 7        /* a GGUF file that is not one, or is corrupt */
} rt_hip_status;

typedef enum {
    RT_HIP_F32 = 0,
    RT_HIP_BF16 = 1,
    RT_HIP_Q4K = 2,
    RT_HIP_Q4_0 = 3,
    RT_HIP_Q4MAT = 4,
    RT_HIP_Q6K = 5   /* GGUF Q6_K blocks: the decode engine's Llama down projection (rt_hip_decoder_set_tensor) */
} rt_hip_format;

/* Largest activation batch the GEMV kernels take; the reference's
 * speculative-verify batch is MAX_BATCH 8 (shaders/decode_gemma3.msl:418). */
#define RT_HIP_GEMV_MAX_M 8

/* ---- library ----------------------------------------------------------- */

/* Thread-local message of the last failed call ("" if none). */
const char* rt_hip_last_error(void);
/* Library version string. */
const char* rt_hip_version(void);
/* Checks that device `ordinal` exists and is gfx950; makes it current and
 * creates its arrival counters (zeroed u32s the batched GEMV counts K-slice
 * arrivals in).  Call it once per device before any other call on it, and
 * before capturing library calls into a hipGraph. */
int rt_hip_init(int ordinal);

/* ---- workspace ------------------------------------------------------------
 * Some calls take scratch from a per-device library workspace: the GEMM (bf16
 * copies of f32 A and of a Q4_K weight shared by several M tiles, split-K
 * partials), the batched GEMV (K-slice partials), decode attention (split
 * partials) and argmax (8 bytes per row).  It grows on demand (the reference
 * likewise grows its Metal scratch on demand, src/metal_ops.mm:378-423).  A
 * replaced buffer is kept until the process ends, because a hipGraph that
 * captured a call still writes the buffer that call used on every replay.
 * Growth allocates, so it is refused while the stream is being captured
 * (RT_HIP_E_HIP, "... before capture"): reserve what a graph's calls need
 * first.  The *_workspace_bytes functions give one call's need (-1 for
 * invalid sizes); rt_hip_workspace_bytes the current size of the current
 * device's workspace.  Calls that share the workspace must not overlap on a
 * device (one stream, or ordered streams). */
int rt_hip_reserve_workspace(int64_t bytes);
int64_t rt_hip_workspace_bytes(void);
int64_t rt_hip_gemm_workspace_bytes(int32_t format, int32_t a_dtype, int64_t m, int64_t n, int64_t k);
int64_t rt_hip_gemv_workspace_bytes(int32_t format, int64_t n, int64_t k, int32_t m);
int64_t rt_hip_attention_workspace_bytes(int32_t n_q_heads, int32_t n_kv_heads, int64_t seq_len);

/* ---- GEMV: M <= 8 activation rows ---------------------------------------
 * Replace: Q4KMat::matmul_q4k_t / _blas for M == 1 (gemv_mt) and the M > 1
 * scalar loop for small M (src/quant_q4k.cpp:564-634); the Metal
 * metal_gemv_q4k_t (include/rt/metal_ops.hpp:57-62, src/metal_ops.mm:663-669)
 * and the engine kernels gemv_q4k_t / gemv_q4k_t_batch
 * (src/shaders/decode_gemma3.msl:328-470).
 * Requires K % 256 == 0 (the reference's Q4_K precondition, quant.hpp:139,
 * which its Release build does not check -- here it is an error).
 * m == 1 runs the decode GEMV; m = 2..8 one batched launch that reads each
 * weight byte once for all m rows. */
int rt_hip_gemv_q4k(const void* blocks, const float* x, float* y, int64_t n, int64_t k,
                    int32_t m, rt_hip_stream stream);

/* Up to RT_HIP_MULTI_MAX Q4_K GEMVs (M == 1) that read the same x and K, in
 * one launch: y[j] = x * W[j]^T for j < count.  A layer's q/k/v or gate/up.
 * blocks, y and n are host arrays of device pointers / row counts.
 * Replace: the engine's back-to-back dispatch_gemv calls on one activation
 * (src/metal_decode.mm:448-450, 472-473), which the reference issues as
 * separate dispatches inside one command buffer. */
#define RT_HIP_MULTI_MAX 4
int rt_hip_gemv_q4k_multi(int32_t count, const void* const* blocks, float* const* y,
                          const int64_t* n, const float* x, int64_t k, rt_hip_stream stream);

/* Tiled Q4_K layout.  No counterpart in the reference: a one-time,
 * size-preserving rearrangement of Q4KMat's row-major blocks, made once
 * when a weight is uploaded to the GPU (where the reference's GPU path
 * copies the blocks unchanged: upload_linear_detect_type,
 * src/metal_decode.mm:157-175), so that every load of the M == 1 GEMV reads
 * contiguous memory.  Each 16-row tile's super-block becomes 2304 bytes in
 * the GEMV's lane order; the scale/min bytes are re-encoded per lane, the
 * values are not changed, and GEMV results are bit-identical to
 * rt_hip_gemv_q4k on the same blocks.
 * rt_hip_q4k_tiled_bytes: size of the tiled copy (rows rounded up to a
 * multiple of 16), or -1 for invalid n, k (K % 256 == 0 required).
 * rt_hip_q4k_tile: device blocks -> device tiled copy (not in place). */
int64_t rt_hip_q4k_tiled_bytes(int64_t n, int64_t k);
int rt_hip_q4k_tile(const void* blocks, void* tiled, int64_t n, int64_t k, rt_hip_stream stream);
/* rt_hip_q4k_tile_rope_half: rt_hip_q4k_tile for a q or k projection whose
 * output takes RoPE in the half-split pairing (llama_rope,
 * src/transformer5.cpp:95-125, RopePairing::HalfSplit: HuggingFace's
 * weights).  The rows of each head of head_dim rows are interleaved on the
 * way (tiled row 2j <- row j, 2j + 1 <- row j + head_dim / 2), so that each
 * rotated pair is two adjacent rows; rt_hip_gemv_q4k_tiled_rmsnorm_rope with
 * RT_HIP_ROPE_HALF stores them back in place.  n % head_dim == 0, head_dim
 * even.  The values are not changed. */
int rt_hip_q4k_tile_rope_half(const void* blocks, void* tiled, int64_t n, int64_t k, int32_t head_dim,
                              rt_hip_stream stream);

/* M == 1 Q4_K GEMV on a tiled copy: same contract and results as
 * rt_hip_gemv_q4k (m == 1) / rt_hip_gemv_q4k_multi.
 * Replace: as rt_hip_gemv_q4k, for callers that keep weights tiled. */
int rt_hip_gemv_q4k_tiled(const void* tiled, const float* x, float* y, int64_t n, int64_t k,
                          rt_hip_stream stream);
int rt_hip_gemv_q4k_tiled_multi(int32_t count, const void* const* tiled, float* const* y,
                                const int64_t* n, const float* x, int64_t k, rt_hip_stream stream);

/* ---- Q8 activations (the reference's aarch64 GEMV path) -------------------
 * rt_hip_q4k_quantize_activation_q8: a [k] f32 -> q8 [ceil(k/32) * 32] int8
 * (zero-padded), scales and sums [ceil(k/32)] f32, bit for bit as
 * Q4KMat::quantize_activation_q8 (src/quant_q4k.cpp:525-562; struct
 * Q8Activation, include/rt/quant.hpp:108-117): per 32 values scale =
 * absmax / 127, q = clamp(round(a / scale), -128, 127), sum in order.
 * Any k >= 1; a, scales, sums 4-byte aligned; no output may overlap a.
 * rt_hip_gemv_q4k_q8 / rt_hip_gemv_q4k_tiled_q8: M == 1 y = W x with x
 * quantized as above inside the launch, then per row the integer chunk dots
 * and the f32 combination of dot_row_q8 (src/quant_q4k.cpp:425-478), chunks
 * summed in order: bit-identical to the reference's arithmetic (its build
 * does not contract, CMakeLists.txt:17-47).
 * Replace: Q4KMat::gemv_mt's aarch64 branch (src/quant_q4k.cpp:573-576,
 * 590-591), which trades ~0.4% accuracy for integer dot products
 * (include/rt/quant.hpp:160-170).  k % 256 == 0, k <= 16384; row-major
 * blocks or the tiled layout. */
int rt_hip_q4k_quantize_activation_q8(const float* a, int64_t k, int8_t* q8, float* scales, float* sums,
                                      rt_hip_stream stream);
int rt_hip_gemv_q4k_q8(const void* blocks, const float* x, float* y, int64_t n, int64_t k, rt_hip_stream stream);
int rt_hip_gemv_q4k_tiled_q8(const void* tiled, const float* x, float* y, int64_t n, int64_t k,
                             rt_hip_stream stream);

/* A layer's q/k/v when v is BF16 (the Q6_K-widened v of a Q4_K_M model,
 * src/transformer4_load.cpp:141-143): up to four tiled-Q4_K GEMVs and one
 * BF16 GEMV w_bf16 [n_bf16, k] that all read x, in one launch.
 * Replace: the q/k/v projections of one layer (src/transformer5.cpp:152-172,
 * Linear2::fused_linear per weight) and their three decode dispatches
 * (src/metal_decode.mm:436-482).  Outputs equal those of
 * rt_hip_gemv_q4k_tiled_multi (to f32 rounding: the Q4_K K split may differ)
 * and, bit for bit, of rt_hip_gemv_bf16.  k % 256 == 0, k <= 8192. */
int rt_hip_gemv_q4k_tiled_bf16(int32_t count, const void* const* tiled, float* const* y,
                               const int64_t* n, const uint16_t* w_bf16, float* y_bf16,
                               int64_t n_bf16, const float* x, int64_t k, rt_hip_stream stream);

/* ---- layer operations fused into a decode GEMV's activation staging ------
 * The first part of the full-graph decode engine: the operation that feeds a
 * projection runs inside the projection's launch, on the activation as each
 * workgroup stages it, instead of as a launch of its own.
 *
 * rt_hip_gemv_q4k_tiled_rmsnorm_multi: y_j = W_j . RMSNorm(x) for up to four
 * tiled Q4_K weights sharing x (a layer's q/k/v, or gate/up).
 * Replace: RmsNorm2::forward then the projections (include/rt/nn2.hpp:246-257,
 * src/transformer5.cpp:198-203), i.e. TensorNode::rms_norm
 * (src/tensor_node.cpp:320-344, 383): rms_inv = 1 / sqrt(sum(x^2) / k + eps),
 * x_hat = x * rms_inv, then x_hat * gamma; gemma3 != 0 uses (1 + gamma)
 * (TensorNode::rms_norm_gemma3, :387; the Gemma 3 Metal kernel
 * rms_norm_gemma3, shaders/decode_gemma3.msl:7-53).  gamma [k] device f32.
 *
 * rt_hip_gemv_q4k_tiled_swiglu: y = W . (silu(gate) * up), the Llama MLP's
 * down projection on its gate/up outputs.
 * Replace: LlamaMlp::forward's silu, mul_elem_node and down_proj
 * (src/transformer5.cpp:186-190; TensorNode::silu, src/tensor_node.cpp:
 * 391-402, sigmoid first, then the product).
 *
 * Outputs match the separate operations followed by rt_hip_gemv_q4k_tiled_multi
 * to f32 rounding: the sum of squares is reduced in a tree, not in sequence,
 * and the scalar rms_inv multiplies the finished dot product rather than
 * each activation (equal in exact arithmetic).
 * k % 256 == 0; any k whose staged activation (3.5 bytes per value) fits one
 * workgroup's LDS (160 KB on gfx950: k up to about 45 000). */
int rt_hip_gemv_q4k_tiled_rmsnorm_multi(int32_t count, const void* const* tiled, float* const* y,
                                        const int64_t* n, const float* x, const float* gamma, float eps,
                                        int32_t gemma3, int64_t k, rt_hip_stream stream);
int rt_hip_gemv_q4k_tiled_swiglu(const void* tiled, const float* gate, const float* up, float* y, int64_t n,
                                 int64_t k, rt_hip_stream stream);
/* rt_hip_gemv_q4k_tiled_rmsnorm_rope: rt_hip_gemv_q4k_tiled_rmsnorm_multi
 * plus rotary position embedding on the outputs of the jobs in rope_jobs (a
 * bit mask: 0x3 for q and k of a q/k/v launch), at position pos, in the
 * interleaved pairing of GGUF's llama weights.
 * Replace: llama_rope (src/transformer5.cpp:95-125, RopePairing::Interleaved):
 * for the pair (2i, 2i + 1) of each head, a = pos * inv_freq[i],
 * out_2i = x_2i cos a - x_2i+1 sin a, out_2i+1 = x_2i sin a + x_2i+1 cos a.
 * inv_freq [head_dim / 2] is the caller's (Config5::inv_freq,
 * transformer5.cpp:36-52).  Writing k and v through y pointers into the KV
 * cache rows of position pos is LlamaLayerKvCache::append (:59-68).  Each
 * rotated job's n must be a multiple of head_dim (even).
 * rope_jobs | RT_HIP_ROPE_HALF selects RopePairing::HalfSplit instead: pair
 * (i, i + head_dim/2), angle pos * inv_freq[i], with the rotated jobs'
 * weights tiled by rt_hip_q4k_tile_rope_half (the other jobs' by
 * rt_hip_q4k_tile). */
#define RT_HIP_ROPE_HALF 0x100
int rt_hip_gemv_q4k_tiled_rmsnorm_rope(int32_t count, const void* const* tiled, float* const* y, const int64_t* n,
                                       const float* x, const float* gamma, float eps, int32_t gemma3,
                                       const float* inv_freq, int32_t pos, int32_t head_dim, int32_t rope_jobs,
                                       int64_t k, rt_hip_stream stream);

/* The residual adds: resid += W . x (the attention output projection) and
 * resid += W . (silu(gate) * up) (the MLP's down projection, Q4_K or
 * BF16-widened), the finished rows added to resid in the store.
 * Replace: LlamaBlock::forward_cached's `x + attn(...)` and `h + mlp(...)`
 * (src/transformer5.cpp:205-212) with the o / down projections before them.
 * resid [n] is read and written; it must not alias x, gate or up. */
int rt_hip_gemv_q4k_tiled_residual(const void* tiled, const float* x, float* resid, int64_t n, int64_t k,
                                   rt_hip_stream stream);
int rt_hip_gemv_q4k_tiled_swiglu_residual(const void* tiled, const float* gate, const float* up, float* resid,
                                          int64_t n, int64_t k, rt_hip_stream stream);
int rt_hip_gemv_bf16_swiglu_residual(const uint16_t* w, const float* gate, const float* up, float* resid, int64_t n,
                                     int64_t k, rt_hip_stream stream);

/* rt_hip_attention_decode: one query token's grouped-query attention over
 * positions [0, seq_len) of a layer's KV cache.
 * Replace: gqa_attention_cached's decode path (src/transformer4.cpp:379-432),
 * as LlamaAttention::forward_cached calls it (src/transformer5.cpp:152-172):
 * per query head h (KV head h / (n_q / n_kv)), s_c = (q_h . k_c) * scale,
 * p = softmax(s), out_h = sum_c p_c v_c.  q [n_q * 128], k_cache / v_cache
 * row-major [>= seq_len, n_kv * 128] f32 (LlamaLayerKvCache), out
 * [n_q * 128]; head_dim 128, n_q / n_kv in {1, 2, 3, 4}, seq_len >= 1.
 * Results match to f32 rounding (online softmax over position splits,
 * merged in a fixed order: deterministic).  Uses the per-device workspace,
 * as the GEMM and batched GEMV do. */
int rt_hip_attention_decode(const float* q, const float* k_cache, const float* v_cache, float* out,
                            int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int64_t seq_len, float scale,
                            rt_hip_stream stream);

/* rt_hip_attention_decode_noalloc: rt_hip_attention_decode, same arguments
 * and the same results bit for bit, for callers that cannot allocate: code
 * under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  No counterpart in the reference.  It allocates nothing: the
 * split partials live in a library-owned device array of 1 MiB per device
 * (held until the process ends), whose address rt_hip_init looks up.  A
 * shape whose partials exceed 1 MiB (n_q_heads * splits * 528 bytes; about
 * one split per CU over the KV heads) fails with RT_HIP_E_SHAPE.  Every call
 * on a device shares that array, so calls that overlap on one device race:
 * issue them on one stream, or order the streams. */
int rt_hip_attention_decode_noalloc(const float* q, const float* k_cache, const float* v_cache, float* out,
                                    int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int64_t seq_len,
                                    float scale, rt_hip_stream stream);

/* rt_hip_flux_attention: FLUX's multi-head attention with no mask (every
 * token attends to every token).
 * Replace: the Metal flux_attention kernel (src/shaders/flux.msl:145-331) as
 * MetalFluxContext::run_attention dispatches it (src/metal_flux.mm:254-272),
 * and the CPU attention it stands in for (src/flux.cpp:282-323), called by
 * the double and single blocks (src/flux.cpp:688, 743).
 * q, k, v, out: [t][n_heads * head_dim] f32 rows; per head h and query i,
 * s_j = (q_i . k_j) * scale with scale = 1 / sqrt(head_dim) in f32,
 * out_i = sum_j softmax(s)_j v_j.  head_dim must be a multiple of 8 in
 * [8, 128] (the Metal path's limits, metal_flux.mm:443-452; else
 * RT_HIP_E_SHAPE); t = 0 is a no-op.  Buffers 16-byte aligned; out must not
 * overlap q, k or v.  Products and sums in f32 (matrix cores, online softmax
 * over tiles of 32 keys): results match the reference to f32 rounding and
 * are deterministic.  With more 128-query blocks (n_heads * ceil(t / 128))
 * than two per CU, the work is divided evenly over two workgroups per CU and
 * the blocks cut between two of them keep their partial states in the
 * library workspace (see above): rt_hip_flux_attention_workspace_bytes gives
 * the need for a shape (0 when none, -1 for invalid sizes), to reserve before
 * a graph capture. */
int rt_hip_flux_attention(const float* q, const float* k, const float* v, float* out, int64_t t, int32_t n_heads,
                          int32_t head_dim, rt_hip_stream stream);
int64_t rt_hip_flux_attention_workspace_bytes(int64_t t, int32_t n_heads, int32_t head_dim);

/* The same two operations for the BF16-widened projections of a Q4_K_M
 * model (src/transformer4_load.cpp:141-143): q/k (tiled Q4_K) and a BF16 v
 * on RMSNorm(x) in one launch, as rt_hip_gemv_q4k_tiled_bf16; and a BF16
 * down on silu(gate) * up, as rt_hip_gemv_bf16 at m = 1. */
int rt_hip_gemv_q4k_tiled_bf16_rmsnorm(int32_t count, const void* const* tiled, float* const* y,
                                       const int64_t* n, const uint16_t* w_bf16, float* y_bf16, int64_t n_bf16,
                                       const float* x, const float* gamma, float eps, int32_t gemma3, int64_t k,
                                       rt_hip_stream stream);
int rt_hip_gemv_bf16_swiglu(const uint16_t* w, const float* gate, const float* up, float* y, int64_t n, int64_t k,
                            rt_hip_stream stream);
/* rt_hip_gemv_q4k_tiled_bf16_rmsnorm_rope: rt_hip_gemv_q4k_tiled_bf16_rmsnorm
 * plus RoPE on the Q4_K jobs in rope_jobs, as rt_hip_gemv_q4k_tiled_rmsnorm_rope
 * (llama_rope, src/transformer5.cpp:95-125; RT_HIP_ROPE_HALF for the
 * half-split pairing), and the KV-cache append through the y pointers
 * (LlamaLayerKvCache::append, :59-68): the q/k/v launch of a Q4_K_M layer
 * whose v is BF16 (src/transformer4_load.cpp:141-143). */
int rt_hip_gemv_q4k_tiled_bf16_rmsnorm_rope(int32_t count, const void* const* tiled, float* const* y,
                                            const int64_t* n, const uint16_t* w_bf16, float* y_bf16,
                                            int64_t n_bf16, const float* x, const float* gamma, float eps,
                                            int32_t gemma3, const float* inv_freq, int32_t pos, int32_t head_dim,
                                            int32_t rope_jobs, int64_t k, rt_hip_stream stream);

/* Replace: MatBf16::matmul_by_t for M <= 8 (src/mat.cpp:318-414); Metal
 * metal_gemv_bf16_t (metal_ops.hpp:64-65) and gemv_bf16_t / _batch
 * (decode_gemma3.msl:390-518).  Requires K % 8 == 0. */
int rt_hip_gemv_bf16(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                     int32_t m, rt_hip_stream stream);

/* Q4Mat weights (RT_HIP_Q4MAT layout above), M <= 8: each byte read once for
 * all M rows.  Replace: Q4Mat::matmul_q4_t / matmul_q4_t_blas for small M
 * (src/quant_q4.cpp:92-156) and metal_matmul_q4_t (metal_ops.hpp:54-55,
 * src/metal_ops.mm:117-161, 578-619).  w = s(nibble) * scale, summed in f32
 * (factorized: agreement to f32 rounding, normwise 1e-5).  K % 32 == 0 and
 * K up to what one workgroup's LDS holds for one row of x and its group
 * sums (4.125 bytes per value: K up to about 39 700 in gfx950's 160 KB);
 * larger M is split into launches that fit.
 * rt_hip_q4mat_bytes / _scales_offset: the buffer size and where the
 * scales start (-1 for invalid n, k). */
int64_t rt_hip_q4mat_bytes(int64_t n, int64_t k);
int64_t rt_hip_q4mat_scales_offset(int64_t n, int64_t k);
int rt_hip_gemv_q4mat(const void* w, const float* x, float* y, int64_t n, int64_t k, int32_t m,
                      rt_hip_stream stream);

/* GGUF Q4_0 weights streamed as 18-byte blocks.
 * Replace: Q4Mat::matmul_q4_t on GgufFile::decode_q4_0_to_q4mat output
 * (src/quant_q4.cpp:92-114, src/gguf.cpp:392-450) and metal_matmul_q4_t
 * (metal_ops.hpp:54-55).  Requires K % 256 == 0. */
int rt_hip_gemv_q4_0(const void* blocks, const float* x, float* y, int64_t n, int64_t k,
                     int32_t m, rt_hip_stream stream);

/* ---- GGUF Q6_K -------------------------------------------------------------
 * 210-byte blocks, K/256 per row: ql[128] | qh[64] | sc[16] (int8) | d (f16)
 * (GgufFile::decode_q6k_to_f32, src/gguf.cpp:531-580).  The reference widens
 * a Q6_K projection to bf16 when it loads it (f32s_to_bf16_and_drop of the
 * decoded values, src/transformer4_load.cpp:33-41, 141-143) and then runs the
 * BF16 GEMV.  K % 256 == 0.
 * rt_hip_dequant_q6k_bf16: that widening on the device, bit-identical:
 *   out[n][k] = bf16_rne(decode(blocks)[n][k]).
 * rt_hip_q6k_tiled_bytes / rt_hip_q6k_tile: a size-preserving tiled copy
 *   (16-row tiles in the GEMV's lane order; no counterpart in the reference,
 *   made once at load like rt_hip_q4k_tile); -1 for invalid n, k.
 * rt_hip_gemv_q6k_tiled: y = x * W^T (M == 1, K <= 8192) reading the Q6_K
 *   bytes (0.82 byte per weight instead of 2) and widening each weight to the
 *   same bf16 value in registers; equals rt_hip_gemv_bf16 on the widened
 *   weights to f32 rounding.  Replace: the BF16 GEMV of a Q6_K-widened v or
 *   down (MatBf16::matmul_by_t, src/mat.cpp:318-414).
 * rt_hip_gemv_q6k_tiled_swiglu_residual: resid += W . (silu(gate) * up),
 *   the same product on the Q6_K bytes with the MLP's gating applied while x
 *   is staged and the rows added to resid in the store: the Q6_K counterpart
 *   of rt_hip_gemv_bf16_swiglu_residual.  Replace: LlamaMlp::forward's down
 *   projection of silu(gate) * up (src/transformer5.cpp:186-190) and the
 *   residual add after it (:205-212), for a Q6_K down widened at load.
 *   resid [n] is read and written; it must not overlap gate or up. */
int rt_hip_dequant_q6k_bf16(const void* blocks, uint16_t* out, int64_t n, int64_t k, rt_hip_stream stream);
int64_t rt_hip_q6k_tiled_bytes(int64_t n, int64_t k);
int rt_hip_q6k_tile(const void* blocks, void* tiled, int64_t n, int64_t k, rt_hip_stream stream);
int rt_hip_gemv_q6k_tiled(const void* tiled, const float* x, float* y, int64_t n, int64_t k,
                          rt_hip_stream stream);
int rt_hip_gemv_q6k_tiled_swiglu_residual(const void* tiled, const float* gate, const float* up, float* resid,
                                          int64_t n, int64_t k, rt_hip_stream stream);

/* ---- GGUF files: reading and uploading weights ------------------------------
 * Replace: GgufFile::open, find_tensor, read_tensor_bytes and the metadata
 * accessors (include/rt/gguf.hpp:130-200, src/gguf.cpp:100-368), and the
 * engine's verbatim upload (upload_linear_detect_type,
 * src/metal_decode.mm:157-176).  GGUF v2/v3: header, typed metadata (nested
 * arrays), tensor infos, data at an aligned offset (metadata
 * "general.alignment", default 32).  The file is mapped read-only; a file
 * that is not GGUF ("not a GGUF file: <path>"), an unsupported version, or a
 * header or tensor running past the end of the file fails with
 * RT_HIP_E_FORMAT.  Tensor types are the ggml ids (gguf.hpp:46-77); bytes
 * are sized for F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q5_K and Q6_K
 * (gguf_block_info, gguf.cpp:81-93) and -1 otherwise.
 * The layer formats: a Q4_K tensor's bytes are rt_hip_gemv_q4k's blocks; a
 * Q4_0 tensor's, rt_hip_gemv_q4_0's; BF16, rt_hip_gemv_bf16's; a Q6_K
 * tensor is widened by rt_hip_dequant_q6k_bf16 (or tiled for
 * rt_hip_gemv_q6k_tiled).  A 2-D tensor [in, out] is the [out, in] weight
 * of y = x W^T (rt_hip_gguf_linear_shape, as the reference's
 * transposed_shape, gguf.cpp:371-381). */
enum {
    RT_HIP_GGUF_F32 = 0, RT_HIP_GGUF_F16 = 1, RT_HIP_GGUF_Q4_0 = 2, RT_HIP_GGUF_Q8_0 = 8,
    RT_HIP_GGUF_Q4_K = 12, RT_HIP_GGUF_Q5_K = 13, RT_HIP_GGUF_Q6_K = 14, RT_HIP_GGUF_BF16 = 30
};
#define RT_HIP_GGUF_MAX_DIMS 4

typedef struct rt_hip_gguf rt_hip_gguf;

typedef struct rt_hip_gguf_tensor {
    const char* name;     /* valid until rt_hip_gguf_close */
    int32_t type;         /* ggml type id */
    int32_t n_dims;
    int64_t dims[RT_HIP_GGUF_MAX_DIMS];  /* GGUF order: dims[0] is the fastest */
    int64_t n_elements;
    int64_t bytes;        /* -1 for a type this reader does not size */
    int64_t file_offset;  /* of the data in the file, -1 if not sized */
} rt_hip_gguf_tensor;

int64_t rt_hip_gguf_type_bytes(int32_t type, int64_t n_elements);
int rt_hip_gguf_open(const char* path, rt_hip_gguf** out);
void rt_hip_gguf_close(rt_hip_gguf* file);
int64_t rt_hip_gguf_tensor_count(const rt_hip_gguf* file);
int64_t rt_hip_gguf_find_tensor(const rt_hip_gguf* file, const char* name); /* -1 if absent */
int rt_hip_gguf_tensor_info(const rt_hip_gguf* file, int64_t index, rt_hip_gguf_tensor* out);
int rt_hip_gguf_linear_shape(const rt_hip_gguf* file, int64_t index, int64_t* rows, int64_t* cols);
/* bytes must equal the tensor's size.  read: into host memory; upload: to
 * device memory (returns once the copy is complete). */
int rt_hip_gguf_read_tensor(const rt_hip_gguf* file, int64_t index, void* host_dst, int64_t bytes);
int rt_hip_gguf_upload(const rt_hip_gguf* file, int64_t index, void* device_dst, int64_t bytes,
                       rt_hip_stream stream);
/* Metadata by key; index >= 0 selects an element of an array value.  Strings
 * stay valid until rt_hip_gguf_close.  As the reference's accessors
 * (GgufMetaValue::as_u64 / as_f32 / as_str, gguf.cpp:104-128): u64 reads
 * u8, u16, u32, u64, i32 and i64 (signed ones sign-extended), f32 reads
 * f32 and f64; other types are RT_HIP_E_UNSUPPORTED. */
int rt_hip_gguf_meta_u64(const rt_hip_gguf* file, const char* key, int64_t index, uint64_t* out);
int rt_hip_gguf_meta_f32(const rt_hip_gguf* file, const char* key, int64_t index, float* out);
int rt_hip_gguf_meta_str(const rt_hip_gguf* file, const char* key, int64_t index, const char** out);
int64_t rt_hip_gguf_meta_array_len(const rt_hip_gguf* file, const char* key); /* -1 if not an array */

/* ---- argmax ---------------------------------------------------------------
 * Replace: greedy sampling, src/transformer5.cpp:382-391 -- the first index
 * of the strict maximum of each row; NaN never wins; a row with no value
 * above -inf gives 0.  idx[rows] (int64) and val[rows] (f32, may be NULL) are
 * device pointers.  Uses a library-owned device workspace. */
int rt_hip_argmax(const float* logits, int64_t rows, int64_t cols, int64_t* idx, float* val,
                  rt_hip_stream stream);

/* BF16 GEMV (M == 1) with the argmax of y fused into the same pass: y as
 * rt_hip_gemv_bf16, plus idx[0]/val[0] as rt_hip_argmax over y.  The
 * lm_head + greedy step of transformer5.cpp:262-266 and :382-391. */
int rt_hip_gemv_bf16_argmax(const uint16_t* w, const float* x, float* y, int64_t n,
                            int64_t k, int64_t* idx, float* val, rt_hip_stream stream);

/* ---- dequantization and quantization ---------------------------------- */

/* Q4_K -> f32, [N, K]: Q4KMat::dequantize_row_into for every row
 * (src/quant_q4k.cpp:280-317).  Bit-exact. */
int rt_hip_dequant_q4k_f32(const void* blocks, float* out, int64_t n, int64_t k,
                           rt_hip_stream stream);
/* Q4_K -> bf16 (RNE), [N, K]: flux_dequant_q4k (src/shaders/flux.msl:51-82). */
int rt_hip_dequant_q4k_bf16(const void* blocks, uint16_t* out, int64_t n, int64_t k,
                            rt_hip_stream stream);
/* f32 [N, K] -> Q4_K blocks, byte-identical to Q4KMat::quantize
 * (src/quant_q4k.cpp:71-205).  Requires K % 256 == 0. */
int rt_hip_quantize_q4k(const float* w, void* blocks, int64_t n, int64_t k,
                        rt_hip_stream stream);

/* ---- GEMM: any M ----------------------------------------------------------
 * C[M,N] = A[M,K] * W^T (+ bias[N]).  A is f32 (a_dtype RT_HIP_F32) or bf16
 * bits (RT_HIP_BF16).  Operands are rounded to bf16 (RNE) and contracted on
 * bf16 MFMA with f32 accumulation.
 * Replace: Q4KMat::matmul_q4k_t_exact (src/quant_q4k.cpp:636-710) and
 * QLinear::forward (src/qlinear.cpp:55-80); the FLUX gemm_into sequence
 * flux_dequant_q4k + flux_gemm_bt + flux_add_bias (src/metal_flux.mm:155-185,
 * src/shaders/flux.msl:51-143).  When M fits one 128-row tile the Q4_K
 * weight is dequantized into LDS tile by tile; for larger M it is dequantized
 * once into the library workspace as bf16 (the same bits), as
 * flux_dequant_q4k does, and shared by every M tile.  K % 256 == 0. */
int rt_hip_gemm_q4k(const void* a, int32_t a_dtype, const void* blocks, const float* bias,
                    float* c, int64_t m, int64_t n, int64_t k, rt_hip_stream stream);
/* rt_hip_gemm: the GEMM for any weight format -- RT_HIP_Q4K and RT_HIP_BF16
 * as rt_hip_gemm_q4k / rt_hip_gemm_bf16; RT_HIP_Q4_0 (GGUF blocks) and
 * RT_HIP_Q4MAT are dequantized once per call into the workspace as bf16 (the
 * f32 values rounded to nearest-even) and run on the bf16 GEMM.
 * Replace: Q4Mat::matmul_q4_t / _blas for M > 4 (src/quant_q4.cpp:92-151:
 * dequantize, then one sgemm) and metal_matmul_q4_t at any M
 * (src/metal_ops.mm:578-619).  K % 64 == 0.
 * rt_hip_dequant: weight bytes -> f32 or bf16 [N, K] (out_dtype RT_HIP_F32
 * or RT_HIP_BF16) for RT_HIP_Q4K (bit-exact dequantize_row_into),
 * RT_HIP_Q4_0 (decode_q4_0_to_f32, gguf.cpp:495-529) and RT_HIP_Q4MAT
 * (Q4Mat::dequantize, quant_q4.cpp:67-74). */
int rt_hip_gemm(int32_t format, const void* a, int32_t a_dtype, const void* w, const float* bias, float* c,
                int64_t m, int64_t n, int64_t k, rt_hip_stream stream);
int rt_hip_dequant(int32_t format, const void* w, void* out, int32_t out_dtype, int64_t n, int64_t k,
                   rt_hip_stream stream);
/* Replace: MatBf16::matmul_by_t for M > 1 (src/mat.cpp:351-414).  K % 64 == 0. */
int rt_hip_gemm_bf16(const void* a, int32_t a_dtype, const uint16_t* w, const float* bias,
                     float* c, int64_t m, int64_t n, int64_t k, rt_hip_stream stream);

/* ---- weight handles ---------------------------------------------------------
 * A weight uploaded once to the current device: the verbatim bytes of any
 * format (the engines' upload_linear_detect_type, src/metal_decode.mm:
 * 157-176), and with flags & RT_HIP_WEIGHT_TILED a Q4_K weight's tiled copy
 * too, which the M == 1 GEMV then reads.  bytes must equal the format's size
 * for (n, k).  rt_hip_weight_linear runs y[m, n] = x[m, k] W^T (+ bias) on
 * device activations at any m, as rt_hip_linear_forward.
 * rt_hip_weight_data: the device copy of the verbatim bytes. */
#define RT_HIP_WEIGHT_TILED 1
typedef struct rt_hip_weight rt_hip_weight;
int rt_hip_weight_upload(int32_t format, const void* host, int64_t bytes, int64_t n, int64_t k, int32_t flags,
                         rt_hip_weight** out);
int rt_hip_weight_free(rt_hip_weight* w);
const void* rt_hip_weight_data(const rt_hip_weight* w);
int rt_hip_weight_linear(const rt_hip_weight* w, const float* x, const float* bias, float* y, int64_t m,
                         rt_hip_stream stream);

/* ---- host drop-ins ------------------------------------------------------------
 * rt_hip_host_matmul: y[m, n] = x[m, k] W^T with host x and y, synchronous.
 * The weight is uploaded on first use and found again by (host pointer, byte
 * length) on the current device, exactly the reference's cached_weights
 * (src/metal_ops.mm:425-434), so the caller keeps the host bytes unchanged
 * at that address while it uses the cache.  w_host / w_bytes are the
 * weight's bytes in `format`; for RT_HIP_Q4MAT they are Q4Mat's `packed`
 * array and w2_host its `scales` (else w2_host is NULL).
 * Replace: metal_gemv_q4k_t, metal_gemv_bf16_t and metal_matmul_q4_t
 * (include/rt/metal_ops.hpp:47-68, src/metal_ops.mm:578-675), at any m.
 * rt_hip_host_cache_clear frees the current device's cached weights;
 * rt_hip_host_cache_bytes is their total size.  Calls on one device are
 * serialized by the library. */
int rt_hip_host_matmul(int32_t format, const void* w_host, int64_t w_bytes, const void* w2_host, int64_t n,
                       int64_t k, const float* x_host, float* y_host, int64_t m);
int rt_hip_host_cache_clear(void);
int64_t rt_hip_host_cache_bytes(void);

/* ---- graphs -------------------------------------------------------------------
 * Capture a sequence of library calls on `stream` into a hipGraph and replay
 * it with one launch: the analogue of the decode engine encoding a whole
 * step into one command buffer (src/metal_decode.mm:436-482).  Pointers and
 * scalar arguments are fixed at capture.  Reserve the workspace first (see
 * above); calls that would grow it fail inside a capture. */
typedef struct rt_hip_graph rt_hip_graph;
int rt_hip_graph_begin(rt_hip_stream stream);
int rt_hip_graph_end(rt_hip_stream stream, rt_hip_graph** out);
int rt_hip_graph_launch(const rt_hip_graph* graph, rt_hip_stream stream);
int rt_hip_graph_destroy(rt_hip_graph* graph);

/* ---- decode engine -------------------------------------------------------------
 * A model's decode step on the device: weights uploaded once, a KV cache of
 * max_seq positions, and the whole step -- embedding, every layer, the final
 * norm and the lm_head -- replayed as one captured hipGraph per token.  The
 * token and its position are written to device memory before each replay,
 * so the graph is captured once (per batch size) and never again.
 * Replace: MetalDecodeContext::create / decode_step / decode_step_batch /
 * sync_kv_from_cpu (include/rt/metal_decode.hpp:41-69, src/metal_decode.mm:
 * 436-938) for Gemma 3, and the Llama 3.2 decode loop
 * (src/transformer5.cpp:152-266) for Llama.
 *
 * RT_HIP_ARCH_GEMMA3 is the Metal engine's layer (metal_decode.mm:436-482):
 * RMSNorm x (1 + gamma); q/k/v; per-head RMSNorm of q and k (1 + gamma);
 * NeoX RoPE with angle (pos * scale) / theta^(2i/d); the KV append; attention
 * scaled by attn_scale over the window [pos + 1 - sliding_window, pos] on
 * local layers and every position on global ones (layer % global_every ==
 * global_every - 1: theta rope_theta, scale rope_freq_scale; local layers
 * rope_theta_local, rope_freq_scale_local); o; the post-attention norm then
 * the residual add; the pre-FFN norm; gate/up; gelu_tanh(gate) * up; down;
 * the post-FFN norm then the residual add.  The embedding is scaled by
 * embed_scale (sqrt(hidden) for Gemma 3).
 * RT_HIP_ARCH_LLAMA is LlamaBlock::forward_cached (transformer5.cpp:198-212):
 * RMSNorm x gamma, q/k/v, RoPE (interleaved pairing, or half-split with
 * rope_half; angle pos * inv_freq[i], inv_freq from llama_inv_freq or
 * 1 / theta^(2i/d)), attention (1/sqrt(head_dim) unless attn_scale is set),
 * o + residual, RMSNorm, gate/up, silu(gate) * up, down + residual.
 * kv_f16 keeps the cache in f16 (RNE), as the Metal engine does.
 * Projections are Q4_K or BF16 (metal_decode.mm:157-176), the embedding BF16
 * or F32, norms F32.  head_dim 64, 128 or 256; n_heads = 1..4 x n_kv_heads;
 * hidden, ffn and n_heads x head_dim multiples of 256.
 * step returns when the logits are on the host (as decode_step does);
 * argmax_host receives the first-max index (transformer5.cpp:382-391).
 * step_batch runs count <= max_batch tokens at positions start_pos.. in one
 * graph, each weight byte read once for all of them (decode_step_batch,
 * metal_decode.mm:887-938); logits are [count][vocab].
 * set_kv loads prefilled cache rows (f32, converted to f16 when kv_f16).
 * Calls on one decoder must not overlap. */
enum { RT_HIP_ARCH_LLAMA = 0, RT_HIP_ARCH_GEMMA3 = 1 };
enum {
    RT_HIP_T_EMBED = 0, RT_HIP_T_OUTPUT_NORM = 1, RT_HIP_T_LM_HEAD = 2,
    RT_HIP_T_ATTN_NORM = 3, RT_HIP_T_Q = 4, RT_HIP_T_K = 5, RT_HIP_T_V = 6, RT_HIP_T_O = 7,
    RT_HIP_T_Q_NORM = 8, RT_HIP_T_K_NORM = 9, RT_HIP_T_POST_ATTN_NORM = 10, RT_HIP_T_FFN_NORM = 11,
    RT_HIP_T_GATE = 12, RT_HIP_T_UP = 13, RT_HIP_T_DOWN = 14, RT_HIP_T_POST_FFN_NORM = 15
};
typedef struct rt_hip_decoder_config {
    int32_t arch;
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq;
    float norm_eps;
    float rope_theta, rope_theta_local;
    float rope_freq_scale, rope_freq_scale_local;
    int32_t rope_half;
    int32_t sliding_window;   /* 0: none */
    int32_t global_every;     /* Gemma 3: 6 */
    float attn_scale;         /* 0: 1/sqrt(head_dim) */
    float embed_scale;        /* 0: 1 */
    int32_t kv_f16;
    int32_t max_batch;        /* 0..8 */
    const float* llama_inv_freq;  /* [head_dim / 2] or NULL (copied at create) */
} rt_hip_decoder_config;
typedef struct rt_hip_decoder rt_hip_decoder;
int rt_hip_decoder_create(const rt_hip_decoder_config* cfg, rt_hip_decoder** out);
int rt_hip_decoder_set_tensor(rt_hip_decoder* dec, int32_t layer, int32_t tensor, int32_t format, const void* host,
                              int64_t bytes);
int rt_hip_decoder_set_kv(rt_hip_decoder* dec, int32_t layer, const float* k_host, const float* v_host, int64_t rows);
int rt_hip_decoder_step(rt_hip_decoder* dec, int32_t token, int32_t pos, float* logits_host, int64_t* argmax_host,
                        rt_hip_stream stream);
int rt_hip_decoder_step_batch(rt_hip_decoder* dec, const int32_t* tokens, int32_t count, int32_t start_pos,
                              float* logits_host, rt_hip_stream stream);
int64_t rt_hip_decoder_vocab(const rt_hip_decoder* dec);
const float* rt_hip_decoder_logits(const rt_hip_decoder* dec);
int rt_hip_decoder_destroy(rt_hip_decoder* dec);

/* ---- linear dispatch ------------------------------------------------------
 * The QLinear / Linear2::fused_linear dispatch over whichever weight format
 * is loaded (src/qlinear.cpp:55-80, src/nn2.cpp:143-203: Q4Mat, Q4_K, BF16;
 * GGUF Q4_0 as decoded into Q4Mat by gguf.cpp:495-529): M <= 8 takes the GEMV
 * kernels, larger M the MFMA GEMM (rt_hip_gemm); the bias (may be NULL) is
 * added to every row (qlinear.cpp:42-53).  x is f32.  Every format at any M. */
int rt_hip_linear_forward(int32_t format, const void* w, const float* bias, const float* x,
                          float* y, int64_t m, int64_t n, int64_t k, rt_hip_stream stream);

/* ---- launch-ceiling calibration --------------------------------------------
 * No counterpart in the reference: two kernels that do none of the path's
 * arithmetic, so that a graph of the decode step's launch sequence built
 * from them measures what the launch structure itself allows on the device.
 * rt_hip_probe_read streams `bytes` (a multiple of 16) of `buf` with 16-byte
 * loads over about `workgroups` workgroups of 256 threads, then writes
 * `out_bytes` (a multiple of 4) of `out` from what it read, as a GEMV stores
 * its rows; with out_bytes 0 it writes nothing (out then needs one u32 per
 * workgroup, named only so the loads stay live).
 * rt_hip_probe_empty launches an empty kernel of the given shape. */
int rt_hip_probe_read(const void* buf, int64_t bytes, int32_t workgroups, uint32_t* out, int64_t out_bytes,
                      rt_hip_stream stream);
int rt_hip_probe_empty(int32_t workgroups, int32_t threads, rt_hip_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* RT_HIP_H */
