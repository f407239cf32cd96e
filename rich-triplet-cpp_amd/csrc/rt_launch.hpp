// rt_launch.hpp -- internal launcher declarations (host side of each .hip
// file); the C ABI in api.cpp validates arguments and calls these.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "rt_hip.h"

namespace rt_hip {

// Device facts used for launch sizing (filled once per device by api.cpp).
struct DeviceInfo {
    int ordinal = -1;
    int cus = 256;
    size_t lds_per_block = 65536;  // the device's, read at first use
};
const DeviceInfo& device_info();
// LDS one workgroup may allocate on the current device (160 KB on gfx950):
// the bound of every kernel that stages its activation in LDS.
size_t lds_cap();

// Records `msg` as the calling thread's last error (rt_hip_last_error) and
// returns `code` (host code outside api.cpp).
int set_error(int code, const std::string& msg);

// Launch-shape knob: `fallback` (the measured best) in the shipped library;
// in a sweep build (-DRT_HIP_TUNING) the environment's RT_HIP_<name>.
int tune_param(const char* name, int fallback);

// Library-owned device workspace, one per device.  It grows on demand
// unless `s` is being captured into a hipGraph (then the call fails with
// hipErrorStreamCaptureUnsupported); a replaced buffer is kept until the
// process ends, since a captured graph may still write it.
void* workspace(size_t bytes, hipStream_t s, hipError_t* err);
// kArrivalCounters zeroed u32 counters per device (made by rt_hip_init).
// A kernel that counts arrivals in them returns each to zero before it ends.
constexpr size_t kArrivalCounters = 16384;
uint32_t* arrival_counters(hipStream_t s, hipError_t* err);

// Largest M*K the GEMV kernels stage in LDS (f32 activations + 16-value sums).
size_t gemv_lds_bytes(int fmt, int m, int64_t k);

hipError_t launch_gemv_q4k(const void* w, const float* x, float* y, int64_t n, int64_t k,
                           int m, hipStream_t s);
hipError_t launch_gemv_q4k_mfma(const void* w, const float* x, float* y, int64_t n, int64_t k,
                                hipStream_t s);
// Up to four M = 1 Q4_K GEMVs sharing x, K; `tiled`: the weights are in the
// tiled layout (q4k_mfma.hpp) rather than reference row-major blocks.
// FLUX attention (flux_attention.hip): q, k, v, out [t][n_heads * head_dim]
// f32, head_dim a multiple of 8 in [8, 128], no mask, 16-byte aligned.
// With more query blocks than workgroup slots the work is split evenly over
// the slots: part (flux_attention_workspace bytes) holds the states of the
// blocks cut in two, and counters (kArrivalCounters) their arrivals; both
// null otherwise.
size_t flux_attention_workspace(int64_t t, int n_heads, int head_dim);
hipError_t launch_flux_attention(const float* q, const float* k, const float* v, float* out, int64_t t, int n_heads,
                                 int head_dim, float scale, float* part, uint32_t* counters, hipStream_t s);

// Decode attention (attention.hip): head_dim 128, n_q / n_kv in {1, 2, 3, 4};
// `part` holds attention_decode_workspace(...) bytes.
void attention_decode_shape(int64_t n_kv, int64_t seq_len, int* splits, int* chunk);
size_t attention_decode_workspace(int64_t n_q, int64_t n_kv, int64_t seq_len);
// The allocation-free variant's per-device scratch (a file-scope device
// array of attention_scratch_bytes()): setup looks up its device address for
// device `dev`, which must be current, once, and returns it in *out.
size_t attention_scratch_bytes();
hipError_t attention_scratch_setup(int dev, void** out);
hipError_t launch_attention_decode(const float* q, const float* kc, const float* vc, float* out, float* part,
                                   int64_t n_q, int64_t n_kv, int64_t seq_len, float scale, hipStream_t s);
// M = 1 BF16 GEMV with a layer operation applied to x while it is staged
// (xop as below); LDS: bf16_m1_lds_bytes(k).
hipError_t launch_gemv_bf16_xop(int xop, const uint16_t* w, const float* x, const float* aux, float eps, float* y,
                                int64_t n, int64_t k, hipStream_t s, bool add = false);
// Tiled Q4_K GEMVs sharing x, with a layer operation applied to x while it
// is staged: xop 1 RMSNorm * gamma, 2 RMSNorm * (1 + gamma), 3 silu(x) * aux,
// 4 gelu_tanh(x) * aux (aux = gamma or up; eps for the norms).
// rope_jobs != 0: interleaved RoPE (position pos, inv_freq [head_dim / 2])
// on the outputs of the jobs in that bit mask; only with an RMSNorm xop.
// add: y += the product (the residual add); with xop 0 (none) or 3 (SwiGLU).
// cache.pos != null (RoPE launches only): the position is read from device
// memory at run time instead of pos, and the outputs of the jobs in
// cache.jobs (bit kRopeCacheBf16: the BF16 rows of the fused launch below)
// are stored at y + position * cache.row -- the KV-cache row of the token,
// so a captured graph serves every position.
struct RopeCache {
    const int32_t* pos = nullptr;
    int64_t row = 0;
    int jobs = 0;
};
constexpr int kRopeCacheBf16Bit = 4;
constexpr int kRopeCacheBf16 = 1 << kRopeCacheBf16Bit;
// argmax_keys (RMSNorm xops only, no RoPE or add, one job): every 16-row
// tile also stores its greedy-argmax key there (q4k_argmax_partials(n)
// slots); launch_argmax_reduce(keys, q4k_argmax_partials(n)) then gives the
// index.
hipError_t launch_gemv_q4k_xop(int xop, int count, const void* const* w, float* const* y, const int64_t* n,
                              const float* x, const float* aux, float eps, int64_t k, hipStream_t s,
                              const float* inv_freq = nullptr, int pos = 0, int head_dim = 0, int rope_jobs = 0,
                              bool add = false, const RopeCache& cache = {}, uint64_t* argmax_keys = nullptr);
// Argmax key slots of a one-job Q4_K GEMV of n rows: its tiles.
inline int64_t q4k_argmax_partials(int64_t n) { return (n + 15) / 16; }
// Up to four tiled-Q4_K GEMVs on RMSNorm(x) * (1 + gamma) where
// x = a + RMSNorm(b) * (1 + g2) (the Gemma 3 post-norm residual step of the
// previous sub-layer, folded into this launch's staging); x is also stored
// to x_out (k floats).  Runs only on the launch shapes with converter
// waves (q4k_postnorm_fits); hipErrorNotSupported otherwise, nothing
// launched.
bool q4k_postnorm_fits(int count, const int64_t* n, int64_t k);
hipError_t launch_gemv_q4k_postnorm(int count, const void* const* w, float* const* y, const int64_t* n,
                                    const float* a, const float* b, const float* g2, const float* gamma, float eps,
                                    int64_t k, float* x_out, hipStream_t s);
hipError_t launch_gemv_q4k_mfma_multi(int count, const void* const* w, float* const* y,
                                      const int64_t* n, const float* x, int64_t k, hipStream_t s,
                                      bool tiled);
// LDS of the M = 1 Q4_K GEMV for `waves` waves per workgroup, and its
// worst case over the splits it picks (the callers' K bound: <= lds_cap()).
size_t mfma_gemv_lds_bytes(int64_t k, int waves);
size_t q4k_m1_lds_bytes(int64_t k);
// head_dim > 0: interleave each head's rows (2j <- j, 2j + 1 <- j + head_dim / 2).
hipError_t launch_q4k_tile(const void* blocks, void* tiled, int64_t n, int64_t k, hipStream_t s, int head_dim = 0);
// Up to four tiled-Q4_K GEMVs and one BF16 GEMV sharing x (K <= 8192) in one
// launch; LDS: q4k_bf16_fused_lds_bytes(k).
size_t q4k_bf16_fused_lds_bytes(int64_t k);
// xop: kXNone, or an RMSNorm form (1, 2) with gamma in aux, applied on both
// sides of the launch.
hipError_t launch_gemv_q4k_bf16_fused(int count, const void* const* w, float* const* y, const int64_t* n,
                                      const uint16_t* wb, float* yb, int64_t nb_rows, const float* x,
                                      int64_t k, hipStream_t s, int xop = 0, const float* aux = nullptr,
                                      float eps = 0.0f, const float* inv_freq = nullptr, int pos = 0,
                                      int head_dim = 0, int rope_jobs = 0, const RopeCache& cache = {});

hipError_t launch_gemv_bf16(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                            int m, uint64_t* argmax_key, hipStream_t s);
// M = 1 BF16 GEMV (gemv_bf16.hip); `key` (may be null) receives the fused
// argmax.  LDS: bf16_m1_lds_bytes(k).
size_t bf16_m1_lds_bytes(int64_t k);
hipError_t launch_gemv_bf16_m1(const uint16_t* w, const float* x, float* y, int64_t n, int64_t k,
                               uint64_t* key, hipStream_t s);
hipError_t launch_gemv_q4_0(const void* w, const float* x, float* y, int64_t n, int64_t k,
                            int m, hipStream_t s);
// Batched GEMV, 2 <= m <= 8, Q4_K (K % 256 == 0) or BF16 (K % 8 == 0) on
// bf16 MFMA (gemv_batch.hip): every weight byte is read once for all m rows;
// K-slices beyond the LDS budget are summed through the library workspace.
hipError_t launch_gemv_batch(int fmt, const void* w, const float* x, float* y, int64_t n, int64_t k, int m,
                             hipStream_t s);
// Workspace bytes one launch_gemv_batch call needs (0 when K fits one slice).
size_t gemv_batch_workspace_bytes(int fmt, int64_t n, int64_t k, int m);
// M = 1 GGUF Q4_0 GEMV (gemv_q40.hip); LDS q40_m1_lds_bytes(k).
size_t q40_m1_lds_bytes(int64_t k);
hipError_t launch_gemv_q4_0_m1(const void* w, const float* x, float* y, int64_t n, int64_t k, hipStream_t s);

// GGUF Q6_K (gemv_q6k.hip): the widening to bf16 (the reference's load),
// the tiled copy and the M = 1 GEMV on it (K % 256 == 0, K <= 8192).
size_t q6k_gemv_lds_bytes(int64_t k);
int64_t q6k_tiled_bytes(int64_t n, int64_t k);
hipError_t launch_q6k_tile(const void* blocks, void* tiled, int64_t n, int64_t k, hipStream_t s);
hipError_t launch_q6k_to_bf16(const void* blocks, uint16_t* dst, int64_t n, int64_t k, hipStream_t s);
// With `up`: y += W . (silu(x) * up) (the MLP's down projection and its
// residual add).
hipError_t launch_gemv_q6k(const void* tiled, const float* x, float* y, int64_t n, int64_t k, hipStream_t s,
                           const float* up = nullptr);

// The fused BF16 GEMV + argmax writes one partial key per workgroup
// (bf16_argmax_partials(n, k) of them); launch_argmax_reduce folds them.
int64_t bf16_argmax_partials(int64_t n, int64_t k);
// The BF16 GEMV with an RMSNorm xop (1 or 2, gamma) and the argmax epilogue:
// each workgroup's best key (of the rows as stored) into keys
// (bf16_xop_argmax_partials(n, k) of them); launch_argmax_reduce folds them.
int64_t bf16_xop_argmax_partials(int64_t n, int64_t k);
hipError_t launch_gemv_bf16_xop_argmax(int xop, const uint16_t* w, const float* x, const float* gamma, float eps,
                                       float* y, int64_t n, int64_t k, uint64_t* keys, hipStream_t s);
hipError_t launch_argmax_reduce(const uint64_t* part, int64_t count, int64_t* idx, float* val, hipStream_t s);
hipError_t launch_argmax_init(uint64_t* keys, int64_t rows, hipStream_t s);
hipError_t launch_argmax_scan(const float* v, int64_t rows, int64_t cols, uint64_t* keys,
                              hipStream_t s);
hipError_t launch_argmax_finalize(uint64_t* keys, int64_t rows, int64_t* idx, float* val,
                                  hipStream_t s);

hipError_t launch_dequant_q4k(const void* w, void* out, bool bf16, int64_t n, int64_t k,
                              hipStream_t s);
// Dequantize w (n x k Q4_K) to bf16 and convert a_elems f32 activations to
// bf16 in one launch (a_elems % 8 == 0).
hipError_t launch_dequant_q4k_cvt(const void* w, uint16_t* wout, int64_t n, int64_t k, const float* a,
                                  uint16_t* aout, int64_t a_elems, hipStream_t s);
hipError_t launch_quantize_q4k(const float* w, void* blocks, int64_t n, int64_t k,
                               hipStream_t s);

// Q8 activations (gemv_q8.hip): quantize_activation_q8 for any k (q8 padded
// with zeros to whole 32-value blocks), and the M = 1 Q4_K x Q8 GEMV on
// row-major or tiled blocks (k % 256 == 0, k <= 16384).
hipError_t launch_quantize_q8(const float* a, int64_t k, int8_t* q8, float* scales, float* sums, hipStream_t s);
hipError_t launch_gemv_q4k_q8(const void* w, bool tiled, const float* x, float* y, int64_t n, int64_t k,
                              hipStream_t s);

// Q4Mat (q4mat.hip): one buffer of packed nibbles then f32 scales at
// q4mat_scales_offset; K % 32 == 0.  The M <= 8 GEMV stages x [M][K] in LDS
// (q4mat_gemv_lds_bytes).  launch_dequant_4bit: Q4Mat or GGUF Q4_0 -> bf16
// or f32 [N, K].
size_t q4mat_scales_offset(int64_t n, int64_t k);
size_t q4mat_bytes(int64_t n, int64_t k);
size_t q4mat_gemv_lds_bytes(int m, int64_t k);
hipError_t launch_gemv_q4mat(const void* w, const float* x, float* y, int64_t n, int64_t k, int m, hipStream_t s);
hipError_t launch_dequant_4bit(int fmt, const void* w, void* out, bool bf16, int64_t n, int64_t k, hipStream_t s);

// ---- decode-step operations (decoder_ops.hip) ----------------------------------
// Embedding rows: out[m][i] = table[tokens[m]][i] * scale (bf16 or f32 table).
hipError_t launch_embed(const void* table, bool bf16, const int32_t* tokens, float scale, float* out, int64_t h,
                        int m, hipStream_t s);
// RMSNorm of `rows` rows of d (gamma or 1 + gamma); with resid: out = resid + norm.
hipError_t launch_rmsnorm_rows(const float* x, const float* gamma, const float* resid, float* out, int64_t d,
                               int rows, float eps, bool gemma, hipStream_t s);
// q/k preparation for m rows at positions pos[0] + row: optional per-head
// RMSNorm (1 + gamma), RoPE, and the K/V append into the cache.
struct QkPrep {
    const float* q = nullptr;  // [m][n_q * d] raw projections
    const float* k = nullptr;  // [m][n_kv * d]
    const float* v = nullptr;  // [m][n_kv * d]
    float* q_out = nullptr;    // [m][n_q * d] rotated queries
    void* k_cache = nullptr;   // [cap][n_kv * d] f32 or f16
    void* v_cache = nullptr;
    const int32_t* pos = nullptr;   // device: position of row 0
    const float* q_gamma = nullptr; // [d] per-head norm (null: none)
    const float* k_gamma = nullptr;
    const float* rope_tab = nullptr;  // [d / 2]: inv_freq, or pow denominators (pow_angle)
    float freq_scale = 1.0f, eps = 0.0f;
    int n_q = 0, n_kv = 0, head_dim = 0, m = 1;
    bool half_split = false, pow_angle = false, f16 = false;
};
hipError_t launch_qk_prep(const QkPrep& p, hipStream_t s);
// Attention of m query rows over a KV cache (head_dim 64/128/256, f32 or
// f16, optional sliding window); row r ends at pos[0] + r + 1 (or
// k_end + r with pos null).  `part` holds attention2_workspace(...) bytes.
struct Attn2 {
    const float* q = nullptr;  // [m][n_q * d]
    const void* k_cache = nullptr;
    const void* v_cache = nullptr;
    float* out = nullptr;      // [m][n_q * d]
    const int32_t* pos = nullptr;
    int k_end = 0, window = 0;
    int n_q = 0, n_kv = 0, head_dim = 0, m = 1, splits = 1;
    // rows the caches hold (0: not stated); with no window and splits of one
    // round covering them, the first round's loads leave before the
    // position is read
    int cache_rows = 0;
    float scale = 1.0f;
    bool f16 = false;
    // m = 1 with pos: the q/k preparation of launch_qk_prep (same operands,
    // same caches) runs inside the attention launch; q is then its raw q,
    // and q_out is not written.
    const QkPrep* prep = nullptr;
};
int attention2_splits(int n_kv, int m, int64_t max_len, int head_dim);
size_t attention2_workspace(int n_q, int head_dim, int splits, int m);
// part: attention2_workspace bytes; counters: m * n_kv zeroed words (each
// launch leaves them zero).
hipError_t launch_attention2(const Attn2& p, float* part, uint32_t* counters, hipStream_t s);
// out = gelu_tanh(gate) * up (the Gemma 3 MLP activation); silu(gate) * up
// (the Llama one); a + b.
hipError_t launch_gelu_mul(const float* gate, const float* up, float* out, int64_t n, hipStream_t s);
hipError_t launch_swiglu(const float* gate, const float* up, float* out, int64_t n, hipStream_t s);
hipError_t launch_add(const float* a, const float* b, float* out, int64_t n, hipStream_t s);

hipError_t launch_gemm(int w_fmt, const void* a, bool a_bf16, const void* w, const float* bias,
                       float* c, int64_t m, int64_t n, int64_t k, hipStream_t s);
// Whether launch_gemm dequantizes this 4-bit weight inside the GEMM (small
// M, or wide N); otherwise a Q4Mat / Q4_0 caller dequantizes into the
// workspace first.
bool gemm_dequant_in_kernel(int w_fmt, bool a_bf16, int64_t m, int64_t n, int64_t k);
// Workspace bytes one launch_gemm call needs.
size_t gemm_workspace_bytes(int w_fmt, bool a_bf16, int64_t m, int64_t n, int64_t k);
hipError_t launch_add_bias(float* y, const float* bias, int64_t m, int64_t n, hipStream_t s);

}  // namespace rt_hip
