// decoder.cpp -- the decode engine behind the C ABI (rt_hip_decoder_*): a
// model's weights uploaded once, its KV cache, and one decode step (or a
// batch of up to 8 tokens) run as a captured hipGraph that is replayed for
// every token.  The MI355X counterpart of the reference's MetalDecodeContext
// (include/rt/metal_decode.hpp:41-69, src/metal_decode.mm:436-938), which
// encodes a whole step into one Metal command buffer; here the token and its
// position live in device memory, so the graph is captured once per batch
// size and never again.
//
// Architectures: the Gemma 3 layer of the Metal engine (metal_decode.mm:
// 436-482: RMSNorm (1 + gamma), q/k/v, per-head q/k RMSNorm, NeoX RoPE with
// per-layer theta and scale, f16 KV cache, sliding-window attention on local
// layers, o, post-attention norm and residual, pre-FFN norm, gate/up,
// GELU-tanh, down, post-FFN norm and residual), and the Llama layer of
// transformer5.cpp:152-212 (RMSNorm, q/k/v, RoPE, attention, o + residual,
// RMSNorm, gate/up, SwiGLU, down + residual).  Projection weights are Q4_K or
// BF16, as the Metal engine's upload_linear_detect_type (metal_decode.mm:
// 157-176) allows; a Llama down projection may also keep its GGUF Q6_K bytes
// (the reference widens them to BF16 at load).
//
// Single-token step: the library's fused launches where the formats allow
// (RMSNorm inside the q/k/v and gate/up GEMVs' activation staging; the Llama
// residual adds and SwiGLU inside the o and down GEMVs), the tiled Q4_K
// layout, and the decode-step operations of decoder_ops.hip.  Batch step:
// the batched GEMVs (each weight byte read once for all rows) on the
// row-major weights.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "rt_hip.h"
#include "rt_launch.hpp"

namespace rt_hip {
namespace {

int fail(int code, const std::string& msg) { return set_error(code, msg); }
int hip_fail(hipError_t e, const std::string& what) {
    return set_error(RT_HIP_E_HIP, what + ": " + hipGetErrorString(e));
}

struct Proj {
    int32_t format = -1;
    void* data = nullptr;   // verbatim bytes (row-major Q4_K blocks or bf16)
    void* tiled = nullptr;  // Q4_K: tiled copy for the M = 1 GEMV
    int64_t n = 0, k = 0;
    bool set() const { return data != nullptr; }
    bool q4k() const { return format == RT_HIP_Q4K; }
};

struct Layer {
    Proj q, k, v, o, gate, up, down;
    float* attn_norm = nullptr;
    float* q_norm = nullptr;
    float* k_norm = nullptr;
    float* post_attn_norm = nullptr;
    float* ffn_norm = nullptr;
    float* post_ffn_norm = nullptr;
    void* kc = nullptr;
    void* vc = nullptr;
    float* rope_tab = nullptr;  // [head_dim / 2] device
    float freq_scale = 1.0f;
    int window = 0;
};

}  // namespace
}  // namespace rt_hip

using namespace rt_hip;

struct rt_hip_decoder {
    rt_hip_decoder_config cfg;
    int device = -1;
    bool gemma = false;
    std::vector<Layer> layers;
    Proj lm_head;
    void* embed = nullptr;
    int32_t embed_format = -1;
    float* out_norm = nullptr;
    // activations, [max rows][...]
    int rows = 1;  // max(1, max_batch)
    float *hidden = nullptr, *hidden2 = nullptr, *normed = nullptr, *q = nullptr, *k = nullptr, *v = nullptr,
          *q_rot = nullptr, *attn = nullptr, *o = nullptr, *gate = nullptr, *up = nullptr, *act = nullptr,
          *down = nullptr, *logits = nullptr, *part = nullptr;
    size_t part_bytes = 0;
    uint32_t* attn_cnt = nullptr;  // attention arrival counters, [max rows][n_kv], zero between launches
    int32_t* dstate = nullptr;  // [0] position of row 0, [1..8] tokens
    int32_t* hstate = nullptr;  // pinned host mirror
    float* logits_stage = nullptr;  // pinned host staging for the logits readback, [max rows][vocab]
    uint64_t* argmax_part = nullptr;  // per-workgroup keys of the lm_head (zeroed at create)
    int64_t* argmax_idx = nullptr;
    hipStream_t stream = nullptr;  // used when the caller passes the legacy stream (not capturable)
    rt_hip_graph* graphs[RT_HIP_GEMV_MAX_M + 1] = {};
    std::vector<void*> allocations;
};

namespace {

int64_t format_bytes(int32_t f, int64_t n, int64_t k) {
    if (f == RT_HIP_Q4K) return k % 256 ? -1 : n * (k / 256) * 144;
    if (f == RT_HIP_BF16) return n * k * 2;
    if (f == RT_HIP_F32) return n * k * 4;
    if (f == RT_HIP_Q6K) return k % 256 ? -1 : n * (k / 256) * 210;
    return -1;
}

hipError_t dev_alloc(rt_hip_decoder* d, void** p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes < 16 ? 16 : bytes);
    if (e == hipSuccess) d->allocations.push_back(*p);
    return e;
}

// Frees one of the decoder's allocations (no captured graph may still use it).
void dev_free(rt_hip_decoder* d, void** p) {
    if (!*p) return;
    for (auto it = d->allocations.begin(); it != d->allocations.end(); ++it)
        if (*it == *p) {
            d->allocations.erase(it);
            break;
        }
    (void)hipFree(*p);
    *p = nullptr;
}

template <typename T>
hipError_t dev_alloc_t(rt_hip_decoder* d, T** p, size_t count) {
    void* v = nullptr;
    hipError_t e = dev_alloc(d, &v, count * sizeof(T));
    *p = static_cast<T*>(v);
    return e;
}

// A window of max_seq positions or more covers every position a step can
// reach (pos < max_seq), so it is no window: 0.  The attention's split count
// and its partials buffer then both follow max_seq.
int clamp_window(const rt_hip_decoder_config& c) {
    return c.sliding_window >= c.max_seq ? 0 : c.sliding_window;
}

bool is_global_layer(const rt_hip_decoder_config& c, int i) {
    return c.global_every <= 0 || i % c.global_every == c.global_every - 1;
}

// ---- launch helpers (each returns an rt_hip status) ---------------------------

int chk(hipError_t e, const char* what) { return e == hipSuccess ? RT_HIP_OK : hip_fail(e, what); }

// y = W x for one projection, M = 1 (tiled Q4_K or BF16).
int gemv1(const Proj& p, const float* x, float* y, hipStream_t s) {
    if (p.q4k()) return rt_hip_gemv_q4k_tiled(p.tiled, x, y, p.n, p.k, s);
    return rt_hip_gemv_bf16(static_cast<const uint16_t*>(p.data), x, y, p.n, p.k, 1, s);
}

// y[m] = W x[m], m rows (batched GEMV on row-major weights).
int gemvm(const Proj& p, const float* x, float* y, int m, hipStream_t s) {
    if (m == 1) return gemv1(p, x, y, s);
    if (p.q4k()) return rt_hip_gemv_q4k(p.data, x, y, p.n, p.k, m, s);
    return rt_hip_gemv_bf16(static_cast<const uint16_t*>(p.data), x, y, p.n, p.k, m, s);
}

// Split count of a layer's attention for m rows: the window bounds the
// positions a row reads, else the cache length.  The partials buffer was
// sized at create for the cache length, and create clamps every window to
// below max_seq, so the count never needs more; the check keeps a future
// change from writing past the buffer.
int attn_splits(const rt_hip_decoder* d, const Layer& L, int m, int* splits) {
    const auto& c = d->cfg;
    const int S = attention2_splits(c.n_kv_heads, m, L.window > 0 ? L.window : c.max_seq, c.head_dim);
    if (attention2_workspace(c.n_heads, c.head_dim, S, m) > d->part_bytes)
        return fail(RT_HIP_E_SHAPE, "decoder: attention partials exceed the buffer sized at create");
    *splits = S;
    return RT_HIP_OK;
}

// Gemma 3's post-attention and post-FFN norms with their residual adds
// (metal_decode.mm:467-480) run inside the next launch that reads their
// result: gate/up, and the next layer's q/k/v, stage
// x = a + RMSNorm(b) * (1 + g2) and normalize it in one pass, one workgroup
// storing x for the residual add after (launch_gemv_q4k_postnorm).  Only
// where that launch is all Q4_K on a shape with converter waves; otherwise
// the separate norm launch runs.
bool postnorm_into_qkv(const rt_hip_decoder* d, int li) {
    if (!d->gemma || li < 1 || li >= d->cfg.n_layers) return false;
    const Layer& L = d->layers[li];
    if (!(L.q.q4k() && L.k.q4k() && L.v.q4k())) return false;
    const int64_t n[3] = {L.q.n, L.k.n, L.v.n};
    return q4k_postnorm_fits(3, n, d->cfg.hidden);
}

bool postnorm_into_gate_up(const rt_hip_decoder* d, int li) {
    if (!d->gemma) return false;
    const Layer& L = d->layers[li];
    if (!(L.gate.q4k() && L.up.q4k())) return false;
    const int64_t n[2] = {L.gate.n, L.up.n};
    return q4k_postnorm_fits(2, n, d->cfg.hidden);
}

// ---- one layer, single token ------------------------------------------------
int layer_step1(rt_hip_decoder* d, int li, hipStream_t s) {
    const auto& c = d->cfg;
    Layer& L = d->layers[li];
    const int H = c.hidden, nq = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim, F = c.ffn;
    const int xop_gemma = d->gemma ? 1 : 0;
    int rc;
    // Llama with an f32 cache and the interleaved pairing: q/k/v, RoPE and
    // the KV append in one launch -- the epilogue rotates q and k at the
    // position it reads from device memory and stores k and v straight into
    // the cache row of that position (LlamaAttention::forward_cached,
    // transformer5.cpp:152-172), so no separate q/k pass runs.
    const bool fused_kv = !d->gemma && !c.kv_f16 && !c.rope_half && L.q.q4k() && L.k.q4k();
    constexpr int kXopRmsNorm = 1;  // launch_gemv_q4k_xop's xop 1: RMSNorm(x) * gamma
    if (fused_kv) {
        const int64_t kvd = static_cast<int64_t>(nkv) * hd;
        const int64_t n[3] = {L.q.n, L.k.n, L.v.n};
        if (L.v.q4k()) {
            const void* w[3] = {L.q.tiled, L.k.tiled, L.v.tiled};
            float* y[3] = {d->q_rot, static_cast<float*>(L.kc), static_cast<float*>(L.vc)};
            rc = chk(launch_gemv_q4k_xop(kXopRmsNorm, 3, w, y, n, d->hidden, L.attn_norm, c.norm_eps, H, s, L.rope_tab,
                                         0, hd, 0x3, false, RopeCache{d->dstate, kvd, 0x6}),
                     "decoder: q/k/v + RoPE + KV append");
        } else {
            const void* w[2] = {L.q.tiled, L.k.tiled};
            float* y[2] = {d->q_rot, static_cast<float*>(L.kc)};
            rc = chk(launch_gemv_q4k_bf16_fused(2, w, y, n, static_cast<const uint16_t*>(L.v.data),
                                                static_cast<float*>(L.vc), L.v.n, d->hidden, H, s, kXopRmsNorm,
                                                L.attn_norm, c.norm_eps, L.rope_tab, 0, hd, 0x3,
                                                RopeCache{d->dstate, kvd, 0x2 | kRopeCacheBf16}),
                     "decoder: q/k/v + RoPE + KV append");
        }
    } else if (postnorm_into_qkv(d, li)) {
        // the previous layer's post-FFN norm and residual add, then this
        // layer's attention norm
        const void* w[3] = {L.q.tiled, L.k.tiled, L.v.tiled};
        float* y[3] = {d->q, d->k, d->v};
        const int64_t n[3] = {L.q.n, L.k.n, L.v.n};
        rc = chk(launch_gemv_q4k_postnorm(3, w, y, n, d->hidden2, d->down, d->layers[li - 1].post_ffn_norm,
                                          L.attn_norm, c.norm_eps, H, d->hidden, s),
                 "decoder: post-FFN norm + q/k/v");
    } else if (L.q.q4k() && L.k.q4k() && L.v.q4k()) {
        const void* w[3] = {L.q.tiled, L.k.tiled, L.v.tiled};
        float* y[3] = {d->q, d->k, d->v};
        const int64_t n[3] = {L.q.n, L.k.n, L.v.n};
        rc = rt_hip_gemv_q4k_tiled_rmsnorm_multi(3, w, y, n, d->hidden, L.attn_norm, c.norm_eps, xop_gemma, H, s);
    } else if (L.q.q4k() && L.k.q4k() && !L.v.q4k()) {
        const void* w[2] = {L.q.tiled, L.k.tiled};
        float* y[2] = {d->q, d->k};
        const int64_t n[2] = {L.q.n, L.k.n};
        rc = rt_hip_gemv_q4k_tiled_bf16_rmsnorm(2, w, y, n, static_cast<const uint16_t*>(L.v.data), d->v, L.v.n,
                                                d->hidden, L.attn_norm, c.norm_eps, xop_gemma, H, s);
    } else {
        rc = chk(launch_rmsnorm_rows(d->hidden, L.attn_norm, nullptr, d->normed, H, 1, c.norm_eps, d->gemma, s),
                 "decoder: rmsnorm");
        if (!rc) rc = gemv1(L.q, d->normed, d->q, s);
        if (!rc) rc = gemv1(L.k, d->normed, d->k, s);
        if (!rc) rc = gemv1(L.v, d->normed, d->v, s);
    }
    if (rc) return rc;
    // per-head norms, RoPE, KV append: inside the attention launch
    QkPrep p;
    if (!fused_kv) {
        p.q = d->q;
        p.k = d->k;
        p.v = d->v;
        p.q_out = d->q_rot;
        p.k_cache = L.kc;
        p.v_cache = L.vc;
        p.pos = d->dstate;
        p.q_gamma = L.q_norm;
        p.k_gamma = L.k_norm;
        p.rope_tab = L.rope_tab;
        p.freq_scale = L.freq_scale;
        p.eps = c.norm_eps;
        p.n_q = nq;
        p.n_kv = nkv;
        p.head_dim = hd;
        p.m = 1;
        p.half_split = d->gemma || c.rope_half;
        p.pow_angle = d->gemma;
        p.f16 = c.kv_f16 != 0;
    }
    Attn2 a;
    a.q = fused_kv ? d->q_rot : d->q;
    a.prep = fused_kv ? nullptr : &p;
    a.k_cache = L.kc;
    a.v_cache = L.vc;
    a.out = d->attn;
    a.pos = d->dstate;
    a.window = L.window;
    a.n_q = nq;
    a.n_kv = nkv;
    a.head_dim = hd;
    a.m = 1;
    a.cache_rows = c.max_seq;
    rc = attn_splits(d, L, 1, &a.splits);
    if (rc) return rc;
    a.scale = c.attn_scale > 0.0f ? c.attn_scale : 1.0f / std::sqrt(static_cast<float>(hd));
    a.f16 = c.kv_f16 != 0;
    rc = chk(launch_attention2(a, d->part, d->attn_cnt, s), "decoder: attention");
    if (rc) return rc;
    // o
    if (!d->gemma) {
        if (L.o.q4k()) {
            rc = rt_hip_gemv_q4k_tiled_residual(L.o.tiled, d->attn, d->hidden, H, nq * hd, s);
        } else {
            rc = gemv1(L.o, d->attn, d->o, s);
            if (!rc) rc = chk(launch_add(d->hidden, d->o, d->hidden, H, s), "decoder: residual");
        }
    } else {
        rc = gemv1(L.o, d->attn, d->o, s);
        if (!rc && !postnorm_into_gate_up(d, li))
            rc = chk(launch_rmsnorm_rows(d->o, L.post_attn_norm, d->hidden, d->hidden2, H, 1, c.norm_eps, true, s),
                     "decoder: post-attention norm");
    }
    if (rc) return rc;
    // gate/up on RMSNorm of the residual stream
    float* h = d->gemma ? d->hidden2 : d->hidden;
    if (postnorm_into_gate_up(d, li)) {
        const void* w[2] = {L.gate.tiled, L.up.tiled};
        float* y[2] = {d->gate, d->up};
        const int64_t n[2] = {L.gate.n, L.up.n};
        rc = chk(launch_gemv_q4k_postnorm(2, w, y, n, d->hidden, d->o, L.post_attn_norm, L.ffn_norm, c.norm_eps, H,
                                          d->hidden2, s),
                 "decoder: post-attention norm + gate/up");
    } else if (L.gate.q4k() && L.up.q4k()) {
        const void* w[2] = {L.gate.tiled, L.up.tiled};
        float* y[2] = {d->gate, d->up};
        const int64_t n[2] = {L.gate.n, L.up.n};
        rc = rt_hip_gemv_q4k_tiled_rmsnorm_multi(2, w, y, n, h, L.ffn_norm, c.norm_eps, xop_gemma, H, s);
    } else {
        rc = chk(launch_rmsnorm_rows(h, L.ffn_norm, nullptr, d->normed, H, 1, c.norm_eps, d->gemma, s),
                 "decoder: rmsnorm");
        if (!rc) rc = gemv1(L.gate, d->normed, d->gate, s);
        if (!rc) rc = gemv1(L.up, d->normed, d->up, s);
    }
    if (rc) return rc;
    // down
    if (!d->gemma) {
        if (L.down.q4k())
            return rt_hip_gemv_q4k_tiled_swiglu_residual(L.down.tiled, d->gate, d->up, d->hidden, H, F, s);
        if (L.down.format == RT_HIP_Q6K)
            return rt_hip_gemv_q6k_tiled_swiglu_residual(L.down.tiled, d->gate, d->up, d->hidden, H, F, s);
        return rt_hip_gemv_bf16_swiglu_residual(static_cast<const uint16_t*>(L.down.data), d->gate, d->up, d->hidden,
                                                H, F, s);
    }
    // gelu_tanh(gate) * up applied while down stages its input (xop 4);
    // a BF16 down wider than the fused launch's 8192 takes the separate pass
    constexpr int kXopGelu = 4;
    if (L.down.q4k()) {
        const void* w[1] = {L.down.tiled};
        float* y[1] = {d->down};
        const int64_t n[1] = {L.down.n};
        rc = chk(launch_gemv_q4k_xop(kXopGelu, 1, w, y, n, d->gate, d->up, 0.0f, F, s), "decoder: gelu + down");
    } else if (F <= 8192) {
        rc = chk(launch_gemv_bf16_xop(kXopGelu, static_cast<const uint16_t*>(L.down.data), d->gate, d->up, 0.0f,
                                      d->down, L.down.n, F, s),
                 "decoder: gelu + down");
    } else {
        rc = chk(launch_gelu_mul(d->gate, d->up, d->act, F, s), "decoder: gelu");
        if (!rc) rc = gemv1(L.down, d->act, d->down, s);
    }
    if (!rc && !postnorm_into_qkv(d, li + 1))
        rc = chk(launch_rmsnorm_rows(d->down, L.post_ffn_norm, d->hidden2, d->hidden, H, 1, c.norm_eps, true, s),
                 "decoder: post-FFN norm");
    return rc;
}

// ---- one layer, m tokens -----------------------------------------------------
int layer_stepm(rt_hip_decoder* d, int li, int m, hipStream_t s) {
    const auto& c = d->cfg;
    Layer& L = d->layers[li];
    const int H = c.hidden, nq = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim, F = c.ffn;
    int rc = chk(launch_rmsnorm_rows(d->hidden, L.attn_norm, nullptr, d->normed, H, m, c.norm_eps, d->gemma, s),
                 "decoder: rmsnorm");
    if (!rc) rc = gemvm(L.q, d->normed, d->q, m, s);
    if (!rc) rc = gemvm(L.k, d->normed, d->k, m, s);
    if (!rc) rc = gemvm(L.v, d->normed, d->v, m, s);
    if (rc) return rc;
    QkPrep p;
    p.q = d->q;
    p.k = d->k;
    p.v = d->v;
    p.q_out = d->q_rot;
    p.k_cache = L.kc;
    p.v_cache = L.vc;
    p.pos = d->dstate;
    p.q_gamma = L.q_norm;
    p.k_gamma = L.k_norm;
    p.rope_tab = L.rope_tab;
    p.freq_scale = L.freq_scale;
    p.eps = c.norm_eps;
    p.n_q = nq;
    p.n_kv = nkv;
    p.head_dim = hd;
    p.m = m;
    p.half_split = d->gemma || c.rope_half;
    p.pow_angle = d->gemma;
    p.f16 = c.kv_f16 != 0;
    rc = chk(launch_qk_prep(p, s), "decoder: q/k prep");
    if (rc) return rc;
    Attn2 a;
    a.q = d->q_rot;
    a.k_cache = L.kc;
    a.v_cache = L.vc;
    a.out = d->attn;
    a.pos = d->dstate;
    a.window = L.window;
    a.n_q = nq;
    a.n_kv = nkv;
    a.head_dim = hd;
    a.m = m;
    a.cache_rows = c.max_seq;
    rc = attn_splits(d, L, m, &a.splits);
    if (rc) return rc;
    a.scale = c.attn_scale > 0.0f ? c.attn_scale : 1.0f / std::sqrt(static_cast<float>(hd));
    a.f16 = c.kv_f16 != 0;
    rc = chk(launch_attention2(a, d->part, d->attn_cnt, s), "decoder: attention");
    if (!rc) rc = gemvm(L.o, d->attn, d->o, m, s);
    if (rc) return rc;
    if (!d->gemma)
        rc = chk(launch_add(d->hidden, d->o, d->hidden, static_cast<int64_t>(m) * H, s), "decoder: residual");
    else
        rc = chk(launch_rmsnorm_rows(d->o, L.post_attn_norm, d->hidden, d->hidden2, H, m, c.norm_eps, true, s),
                 "decoder: post-attention norm");
    if (rc) return rc;
    float* h = d->gemma ? d->hidden2 : d->hidden;
    rc = chk(launch_rmsnorm_rows(h, L.ffn_norm, nullptr, d->normed, H, m, c.norm_eps, d->gemma, s), "decoder: rmsnorm");
    if (!rc) rc = gemvm(L.gate, d->normed, d->gate, m, s);
    if (!rc) rc = gemvm(L.up, d->normed, d->up, m, s);
    if (rc) return rc;
    const int64_t mf = static_cast<int64_t>(m) * F;
    rc = d->gemma ? chk(launch_gelu_mul(d->gate, d->up, d->act, mf, s), "decoder: gelu")
                  : chk(launch_swiglu(d->gate, d->up, d->act, mf, s), "decoder: swiglu");
    if (!rc) rc = gemvm(L.down, d->act, d->down, m, s);
    if (rc) return rc;
    if (!d->gemma) return chk(launch_add(d->hidden, d->down, d->hidden, static_cast<int64_t>(m) * H, s), "decoder: residual");
    return chk(launch_rmsnorm_rows(d->down, L.post_ffn_norm, d->hidden2, d->hidden, H, m, c.norm_eps, true, s),
               "decoder: post-FFN norm");
}

// The whole step for m rows (m = 1: the single-token path).
int record_step(rt_hip_decoder* d, int m, hipStream_t s) {
    const auto& c = d->cfg;
    const float escale = c.embed_scale > 0.0f ? c.embed_scale : 1.0f;
    int rc = chk(launch_embed(d->embed, d->embed_format == RT_HIP_BF16, d->dstate + 1, escale, d->hidden, c.hidden, m, s),
                 "decoder: embedding");
    for (int li = 0; li < c.n_layers && !rc; ++li) rc = m == 1 ? layer_step1(d, li, s) : layer_stepm(d, li, m, s);
    if (rc) return rc;
    const int64_t V = d->lm_head.n, H = c.hidden;
    if (m == 1) {
        // final norm inside the lm_head GEMV's staging
        if (d->lm_head.q4k()) {
            // the argmax of the logits (transformer5.cpp:382-391) rides in
            // the GEMV's epilogue, one key per workgroup, and one launch
            // folds them
            const void* w[1] = {d->lm_head.tiled};
            float* y[1] = {d->logits};
            const int64_t n[1] = {V};
            rc = chk(launch_gemv_q4k_xop(d->gemma ? 2 : 1, 1, w, y, n, d->hidden, d->out_norm, c.norm_eps, H, s,
                                         nullptr, 0, 0, 0, false, RopeCache{}, d->argmax_part),
                     "decoder: lm_head + argmax");
            if (!rc)
                rc = chk(launch_argmax_reduce(d->argmax_part, q4k_argmax_partials(V), d->argmax_idx, nullptr, s),
                         "decoder: argmax");
            return rc;
        }
        // BF16 (the tied embedding): the same, one key per workgroup
        rc = chk(launch_gemv_bf16_xop_argmax(d->gemma ? 2 : 1, static_cast<const uint16_t*>(d->lm_head.data),
                                             d->hidden, d->out_norm, c.norm_eps, d->logits, V, H, d->argmax_part, s),
                 "decoder: lm_head + argmax");
        if (!rc)
            rc = chk(launch_argmax_reduce(d->argmax_part, bf16_xop_argmax_partials(V, H), d->argmax_idx, nullptr, s),
                     "decoder: argmax");
        return rc;
    }
    rc = chk(launch_rmsnorm_rows(d->hidden, d->out_norm, nullptr, d->normed, H, m, c.norm_eps, d->gemma, s),
             "decoder: final norm");
    if (!rc) rc = gemvm(d->lm_head, d->normed, d->logits, m, s);
    return rc;
}

// Queues the copy of `elems` logits to the caller's host buffer.  A pinned
// (page-locked) destination takes the copy directly; pageable memory would
// make the runtime stage the copy itself at a fraction of the bandwidth, so
// it goes through the decoder's pinned staging buffer and *staged is set: the
// caller copies from there after the stream has synchronised.
hipError_t logits_readback(rt_hip_decoder* d, float* dst, int64_t elems, hipStream_t s, float** staged) {
    hipPointerAttribute_t attr{};
    const bool pinned = hipPointerGetAttributes(&attr, dst) == hipSuccess && attr.type == hipMemoryTypeHost;
    (void)hipGetLastError();  // an unregistered pointer may leave an error behind: clear it
    *staged = pinned ? nullptr : d->logits_stage;
    return hipMemcpyAsync(pinned ? dst : d->logits_stage, d->logits, static_cast<size_t>(elems) * 4,
                          hipMemcpyDeviceToHost, s);
}

bool complete(const rt_hip_decoder* d, std::string* what) {
    auto need = [&](bool ok, const char* name, int layer) {
        if (!ok && what->empty()) *what = std::string(name) + (layer >= 0 ? " of layer " + std::to_string(layer) : "");
        return ok;
    };
    bool ok = need(d->embed != nullptr, "embedding", -1) && need(d->out_norm != nullptr, "output norm", -1) &&
              need(d->lm_head.set(), "lm_head", -1);
    for (int i = 0; i < d->cfg.n_layers && ok; ++i) {
        const Layer& L = d->layers[i];
        ok = need(L.q.set() && L.k.set() && L.v.set() && L.o.set(), "attention projections", i) &&
             need(L.gate.set() && L.up.set() && L.down.set(), "MLP projections", i) &&
             need(L.attn_norm && L.ffn_norm, "norms", i);
        if (ok && d->gemma)
            ok = need(L.q_norm && L.k_norm && L.post_attn_norm && L.post_ffn_norm, "Gemma 3 norms", i);
    }
    return ok;
}

int run_step(rt_hip_decoder* d, const int32_t* tokens, int m, int32_t pos, hipStream_t s) {
    const char* fn = "rt_hip_decoder_step";
    std::string missing;
    if (!complete(d, &missing)) return fail(RT_HIP_E_ARG, std::string(fn) + ": weights not set: " + missing);
    if (pos < 0 || static_cast<int64_t>(pos) + m > d->cfg.max_seq)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": position beyond the KV cache (max_seq)");
    for (int i = 0; i < m; ++i)
        if (tokens[i] < 0 || tokens[i] >= d->cfg.vocab)
            return fail(RT_HIP_E_ARG, std::string(fn) + ": token id out of range");
    hipError_t e = hipSetDevice(d->device);
    if (e != hipSuccess) return hip_fail(e, fn);
    // The previous step finished (steps are synchronous), so the pinned
    // mirror can be rewritten.
    d->hstate[0] = pos;
    for (int i = 0; i < m; ++i) d->hstate[1 + i] = tokens[i];
    e = hipMemcpyAsync(d->dstate, d->hstate, sizeof(int32_t) * (1 + m), hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_fail(e, fn);
    if (!d->graphs[m]) {
        // Nothing inside the capture may allocate: size the library workspace
        // for the batched GEMVs' K-slice partials first.
        if (m > 1) {
            int64_t need = 0;
            auto take = [&](const Proj& p) {
                const int64_t b = rt_hip_gemv_workspace_bytes(p.format, p.n, p.k, m);
                need = b > need ? b : need;
            };
            take(d->lm_head);
            for (const Layer& L : d->layers)
                for (const Proj* p : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down}) take(*p);
            const int rc = rt_hip_reserve_workspace(need);
            if (rc) return rc;
        }
        int rc = rt_hip_graph_begin(s);
        if (rc) return rc;
        rc = record_step(d, m, s);
        rt_hip_graph* g = nullptr;
        const int rc_end = rt_hip_graph_end(s, &g);
        if (rc) {
            rt_hip_graph_destroy(g);
            return rc;
        }
        if (rc_end) return rc_end;
        d->graphs[m] = g;
    }
    return rt_hip_graph_launch(d->graphs[m], s);
}

}  // namespace

extern "C" {

int rt_hip_decoder_create(const rt_hip_decoder_config* cfg, rt_hip_decoder** out) {
    const char* fn = "rt_hip_decoder_create";
    if (!out || !cfg) return fail(RT_HIP_E_ARG, std::string(fn) + ": null argument");
    *out = nullptr;
    const auto& c = *cfg;
    if (c.arch != RT_HIP_ARCH_LLAMA && c.arch != RT_HIP_ARCH_GEMMA3)
        return fail(RT_HIP_E_ARG, std::string(fn) + ": unknown architecture");
    if (c.n_layers < 1 || c.hidden < 1 || c.n_heads < 1 || c.n_kv_heads < 1 || c.ffn < 1 || c.vocab < 1 ||
        c.max_seq < 1)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": sizes must be positive");
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": head_dim must be 64, 128 or 256");
    if (c.n_heads % c.n_kv_heads || c.n_heads / c.n_kv_heads > 4)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": n_heads must be 1..4 times n_kv_heads");
    if (c.hidden % 256 || c.ffn % 256 || (static_cast<int64_t>(c.n_heads) * c.head_dim) % 256)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": hidden, ffn and n_heads * head_dim must be multiples of 256");
    if (c.max_batch < 0 || c.max_batch > RT_HIP_GEMV_MAX_M)
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": max_batch must be in [0, 8]");
    if (!(c.norm_eps >= 0.0f)) return fail(RT_HIP_E_ARG, std::string(fn) + ": norm_eps must be >= 0");
    if (c.sliding_window < 0) return fail(RT_HIP_E_ARG, std::string(fn) + ": sliding_window must be >= 0");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, fn);

    auto* d = new rt_hip_decoder();
    d->cfg = c;
    d->cfg.llama_inv_freq = nullptr;  // copied below
    d->device = dev;
    d->gemma = c.arch == RT_HIP_ARCH_GEMMA3;
    d->rows = c.max_batch > 1 ? c.max_batch : 1;
    d->layers.resize(c.n_layers);
    const int R = d->rows, H = c.hidden, F = c.ffn, hd = c.head_dim;
    // per-workgroup argmax keys of the lm_head, Q4_K or BF16
    const size_t argmax_slots = static_cast<size_t>(
        std::max(q4k_argmax_partials(c.vocab), bf16_xop_argmax_partials(c.vocab, c.hidden)));
    const int64_t qd = static_cast<int64_t>(c.n_heads) * hd, kvd = static_cast<int64_t>(c.n_kv_heads) * hd;
    const size_t kv_elem = c.kv_f16 ? 2 : 4;
    auto cleanup = [&](hipError_t err) {
        rt_hip_decoder_destroy(d);
        return err == hipErrorOutOfMemory ? fail(RT_HIP_E_OOM, std::string(fn) + ": out of device memory")
                                          : hip_fail(err, fn);
    };
    float** bufs[] = {&d->hidden, &d->hidden2, &d->normed, &d->o, &d->down};
    for (float** b : bufs)
        if ((e = dev_alloc_t(d, b, static_cast<size_t>(R) * H)) != hipSuccess) return cleanup(e);
    if ((e = dev_alloc_t(d, &d->q, R * qd)) != hipSuccess || (e = dev_alloc_t(d, &d->q_rot, R * qd)) != hipSuccess ||
        (e = dev_alloc_t(d, &d->attn, R * qd)) != hipSuccess || (e = dev_alloc_t(d, &d->k, R * kvd)) != hipSuccess ||
        (e = dev_alloc_t(d, &d->v, R * kvd)) != hipSuccess ||
        (e = dev_alloc_t(d, &d->gate, static_cast<size_t>(R) * F)) != hipSuccess ||
        (e = dev_alloc_t(d, &d->up, static_cast<size_t>(R) * F)) != hipSuccess ||
        (e = dev_alloc_t(d, &d->act, static_cast<size_t>(R) * F)) != hipSuccess ||
        (e = dev_alloc_t(d, &d->logits, static_cast<size_t>(R) * c.vocab)) != hipSuccess ||
        (e = dev_alloc_t(d, &d->dstate, 16)) != hipSuccess ||
        (e = dev_alloc_t(d, &d->argmax_part, argmax_slots)) != hipSuccess ||
        (e = hipMemset(d->argmax_part, 0, argmax_slots * 8)) != hipSuccess ||
        (e = dev_alloc_t(d, &d->argmax_idx, 16)) != hipSuccess)
        return cleanup(e);
    if ((e = hipHostMalloc(reinterpret_cast<void**>(&d->hstate), 16 * sizeof(int32_t))) != hipSuccess)
        return cleanup(e);
    if ((e = hipHostMalloc(reinterpret_cast<void**>(&d->logits_stage), static_cast<size_t>(R) * c.vocab * 4)) !=
        hipSuccess)
        return cleanup(e);
    if ((e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking)) != hipSuccess) return cleanup(e);
    // attention partials for the largest split count of any batch size
    size_t pb = 0;
    for (int m = 1; m <= R; ++m) {
        const int S = attention2_splits(c.n_kv_heads, m, c.max_seq, hd);
        const size_t b = attention2_workspace(c.n_heads, hd, S, m);
        pb = b > pb ? b : pb;
    }
    d->part_bytes = pb;
    if ((e = dev_alloc(d, reinterpret_cast<void**>(&d->part), pb)) != hipSuccess) return cleanup(e);
    const size_t cb = static_cast<size_t>(R) * c.n_kv_heads * sizeof(uint32_t);
    if ((e = dev_alloc(d, reinterpret_cast<void**>(&d->attn_cnt), cb)) != hipSuccess ||
        (e = hipMemset(d->attn_cnt, 0, cb)) != hipSuccess)
        return cleanup(e);
    // KV caches (zeroed) and RoPE tables, per layer
    std::vector<float> tab(hd / 2);
    for (int i = 0; i < c.n_layers; ++i) {
        Layer& L = d->layers[i];
        const size_t kvb = static_cast<size_t>(c.max_seq) * kvd * kv_elem;
        if ((e = dev_alloc(d, &L.kc, kvb)) != hipSuccess || (e = dev_alloc(d, &L.vc, kvb)) != hipSuccess)
            return cleanup(e);
        if ((e = hipMemset(L.kc, 0, kvb)) != hipSuccess || (e = hipMemset(L.vc, 0, kvb)) != hipSuccess)
            return cleanup(e);
        if (d->gemma) {
            // rope_neox (decode_gemma3.msl:99-126): the pow(theta, 2i/d)
            // denominators, computed once here in f32; global layers
            // (layer % global_every == global_every - 1, Config4::
            // is_global_layer) use rope_theta and rope_freq_scale and no
            // window, local ones the _local values and sliding_window.
            const bool global = is_global_layer(c, i);
            const float theta = global ? c.rope_theta : c.rope_theta_local;
            L.freq_scale = global ? c.rope_freq_scale : c.rope_freq_scale_local;
            L.window = global ? 0 : clamp_window(c);
            for (int j = 0; j < hd / 2; ++j)
                tab[j] = std::pow(theta, 2.0f * static_cast<float>(j) / static_cast<float>(hd));
        } else {
            // Config5::inv_freq (transformer5.cpp:36-52), or the caller's table
            for (int j = 0; j < hd / 2; ++j)
                tab[j] = cfg->llama_inv_freq
                             ? cfg->llama_inv_freq[j]
                             : 1.0f / std::pow(c.rope_theta, 2.0f * static_cast<float>(j) / static_cast<float>(hd));
            L.window = clamp_window(c);
        }
        if ((e = dev_alloc_t(d, &L.rope_tab, hd / 2)) != hipSuccess) return cleanup(e);
        if ((e = hipMemcpy(L.rope_tab, tab.data(), tab.size() * 4, hipMemcpyHostToDevice)) != hipSuccess)
            return cleanup(e);
    }
    *out = d;
    return RT_HIP_OK;
}

int rt_hip_decoder_set_tensor(rt_hip_decoder* d, int32_t layer, int32_t tensor, int32_t format, const void* host,
                              int64_t bytes) {
    const char* fn = "rt_hip_decoder_set_tensor";
    if (!d || !host) return fail(RT_HIP_E_ARG, std::string(fn) + ": null argument");
    const auto& c = d->cfg;
    const int64_t H = c.hidden, F = c.ffn, qd = static_cast<int64_t>(c.n_heads) * c.head_dim,
                  kvd = static_cast<int64_t>(c.n_kv_heads) * c.head_dim;
    const bool global = tensor == RT_HIP_T_EMBED || tensor == RT_HIP_T_OUTPUT_NORM || tensor == RT_HIP_T_LM_HEAD;
    if (global != (layer < 0)) return fail(RT_HIP_E_ARG, std::string(fn) + ": layer must be -1 for model tensors");
    if (!global && layer >= c.n_layers) return fail(RT_HIP_E_ARG, std::string(fn) + ": layer out of range");
    hipError_t e = hipSetDevice(d->device);
    if (e != hipSuccess) return hip_fail(e, fn);
    for (auto& g : d->graphs) {  // new weights: record the step again
        rt_hip_graph_destroy(g);
        g = nullptr;
    }
    auto upload = [&](void** dst, int64_t need) -> int {
        if (bytes != need)
            return fail(RT_HIP_E_SHAPE, std::string(fn) + ": " + std::to_string(bytes) + " bytes given, " +
                                            std::to_string(need) + " expected");
        if (!*dst) {
            hipError_t er = dev_alloc(d, dst, static_cast<size_t>(need));
            if (er != hipSuccess) return hip_fail(er, fn);
        }
        hipError_t er = hipMemcpy(*dst, host, static_cast<size_t>(need), hipMemcpyHostToDevice);
        return er == hipSuccess ? RT_HIP_OK : hip_fail(er, fn);
    };
    auto norm = [&](float** dst, int64_t n) -> int {
        if (format != RT_HIP_F32) return fail(RT_HIP_E_UNSUPPORTED, std::string(fn) + ": norm weights are f32");
        return upload(reinterpret_cast<void**>(dst), n * 4);
    };
    auto proj = [&](Proj& p, int64_t n, int64_t k) -> int {
        // A Q6_K down projection stays in its GGUF bytes (tiled once here)
        // instead of the reference's load-time widening: Llama's SwiGLU down
        // + residual, single-token steps only (no batched Q6_K GEMV).
        const bool q6_ok = tensor == RT_HIP_T_DOWN && !d->gemma && c.max_batch <= 1;
        if (format != RT_HIP_Q4K && format != RT_HIP_BF16 && !(format == RT_HIP_Q6K && q6_ok))
            return fail(RT_HIP_E_UNSUPPORTED, std::string(fn) + ": projections are Q4_K or BF16 (Q6_K: a Llama "
                                                                "down projection with max_batch <= 1)");
        const int64_t need = format_bytes(format, n, k);
        if (need < 0) return fail(RT_HIP_E_ALIGN, std::string(fn) + ": Q4_K and Q6_K need k % 256 == 0");
        if (format == RT_HIP_Q6K && k > 8192) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": Q6_K k above 8192");
        // Every check comes before the tensor changes, so a rejected call
        // leaves the previous weight in place.
        if (bytes != need)
            return fail(RT_HIP_E_SHAPE, std::string(fn) + ": " + std::to_string(bytes) + " bytes given, " +
                                            std::to_string(need) + " expected");
        if (p.set() && p.format != format) {
            // Format change: the old buffers are freed (the graphs that read
            // them were destroyed above, and steps are synchronous).
            dev_free(d, &p.data);
            dev_free(d, &p.tiled);
        }
        p.format = format;
        p.n = n;
        p.k = k;
        int rc = upload(&p.data, need);
        if (rc || (format != RT_HIP_Q4K && format != RT_HIP_Q6K)) return rc;
        const bool q6 = format == RT_HIP_Q6K;
        if (!p.tiled) {
            const int64_t tb = q6 ? rt_hip_q6k_tiled_bytes(n, k) : rt_hip_q4k_tiled_bytes(n, k);
            hipError_t er = dev_alloc(d, &p.tiled, static_cast<size_t>(tb));
            if (er != hipSuccess) return hip_fail(er, fn);
        }
        rc = q6 ? rt_hip_q6k_tile(p.data, p.tiled, n, k, nullptr) : rt_hip_q4k_tile(p.data, p.tiled, n, k, nullptr);
        if (!rc) rc = chk(hipDeviceSynchronize(), fn);
        return rc;
    };
    if (tensor == RT_HIP_T_EMBED) {
        if (format != RT_HIP_BF16 && format != RT_HIP_F32)
            return fail(RT_HIP_E_UNSUPPORTED, std::string(fn) + ": the embedding is BF16 or F32");
        const int64_t need = format_bytes(format, c.vocab, H);
        if (bytes != need)
            return fail(RT_HIP_E_SHAPE, std::string(fn) + ": " + std::to_string(bytes) + " bytes given, " +
                                            std::to_string(need) + " expected");
        if (d->embed && d->embed_format != format) dev_free(d, &d->embed);
        d->embed_format = format;
        return upload(&d->embed, need);
    }
    if (tensor == RT_HIP_T_OUTPUT_NORM) return norm(&d->out_norm, H);
    if (tensor == RT_HIP_T_LM_HEAD) return proj(d->lm_head, c.vocab, H);
    Layer& L = d->layers[layer];
    switch (tensor) {
        case RT_HIP_T_ATTN_NORM: return norm(&L.attn_norm, H);
        case RT_HIP_T_Q: return proj(L.q, qd, H);
        case RT_HIP_T_K: return proj(L.k, kvd, H);
        case RT_HIP_T_V: return proj(L.v, kvd, H);
        case RT_HIP_T_O: return proj(L.o, H, qd);
        case RT_HIP_T_Q_NORM: return norm(&L.q_norm, c.head_dim);
        case RT_HIP_T_K_NORM: return norm(&L.k_norm, c.head_dim);
        case RT_HIP_T_POST_ATTN_NORM: return norm(&L.post_attn_norm, H);
        case RT_HIP_T_FFN_NORM: return norm(&L.ffn_norm, H);
        case RT_HIP_T_GATE: return proj(L.gate, F, H);
        case RT_HIP_T_UP: return proj(L.up, F, H);
        case RT_HIP_T_DOWN: return proj(L.down, H, F);
        case RT_HIP_T_POST_FFN_NORM: return norm(&L.post_ffn_norm, H);
        default: return fail(RT_HIP_E_ARG, std::string(fn) + ": unknown tensor");
    }
}

int rt_hip_decoder_set_kv(rt_hip_decoder* d, int32_t layer, const float* k_host, const float* v_host, int64_t rows) {
    const char* fn = "rt_hip_decoder_set_kv";
    if (!d || !k_host || !v_host) return fail(RT_HIP_E_ARG, std::string(fn) + ": null argument");
    if (layer < 0 || layer >= d->cfg.n_layers) return fail(RT_HIP_E_ARG, std::string(fn) + ": layer out of range");
    if (rows < 0 || rows > d->cfg.max_seq) return fail(RT_HIP_E_SHAPE, std::string(fn) + ": rows beyond max_seq");
    hipError_t e = hipSetDevice(d->device);
    if (e != hipSuccess) return hip_fail(e, fn);
    const int64_t n = rows * d->cfg.n_kv_heads * d->cfg.head_dim;
    Layer& L = d->layers[layer];
    if (!d->cfg.kv_f16) {
        e = hipMemcpy(L.kc, k_host, n * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(L.vc, v_host, n * 4, hipMemcpyHostToDevice);
        return e == hipSuccess ? RT_HIP_OK : hip_fail(e, fn);
    }
    // sync_kv_from_cpu (metal_decode.mm:840-861): f32 rows converted to the
    // f16 cache on the device (RNE, as half()).
    std::vector<uint16_t> h(static_cast<size_t>(n));
    for (const float* src : {k_host, v_host}) {
        for (int64_t i = 0; i < n; ++i) h[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(src[i]));
        e = hipMemcpy(src == k_host ? L.kc : L.vc, h.data(), n * 2, hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_fail(e, fn);
    }
    return RT_HIP_OK;
}

int rt_hip_decoder_step(rt_hip_decoder* d, int32_t token, int32_t pos, float* logits_host, int64_t* argmax_host,
                        rt_hip_stream stream) {
    if (!d) return fail(RT_HIP_E_ARG, "rt_hip_decoder_step: null decoder");
    const hipStream_t s = stream ? static_cast<hipStream_t>(stream) : d->stream;
    int rc = run_step(d, &token, 1, pos, s);
    if (rc) return rc;
    hipError_t e = hipSuccess;
    float* staged = nullptr;
    if (logits_host) e = logits_readback(d, logits_host, d->lm_head.n, s, &staged);
    if (e == hipSuccess && argmax_host) e = hipMemcpyAsync(argmax_host, d->argmax_idx, 8, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess && staged) std::memcpy(logits_host, staged, static_cast<size_t>(d->lm_head.n) * 4);
    return e == hipSuccess ? RT_HIP_OK : hip_fail(e, "rt_hip_decoder_step");
}

int rt_hip_decoder_step_batch(rt_hip_decoder* d, const int32_t* tokens, int32_t count, int32_t start_pos,
                              float* logits_host, rt_hip_stream stream) {
    const char* fn = "rt_hip_decoder_step_batch";
    if (!d || !tokens) return fail(RT_HIP_E_ARG, std::string(fn) + ": null argument");
    if (count < 1 || count > d->rows || (count > 1 && d->cfg.max_batch < count))
        return fail(RT_HIP_E_SHAPE, std::string(fn) + ": count must be in [1, max_batch]");
    const hipStream_t s = stream ? static_cast<hipStream_t>(stream) : d->stream;
    int rc = run_step(d, tokens, count, start_pos, s);
    if (rc) return rc;
    hipError_t e = hipSuccess;
    float* staged = nullptr;
    const int64_t elems = static_cast<int64_t>(count) * d->lm_head.n;
    if (logits_host) e = logits_readback(d, logits_host, elems, s, &staged);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess && staged) std::memcpy(logits_host, staged, static_cast<size_t>(elems) * 4);
    return e == hipSuccess ? RT_HIP_OK : hip_fail(e, fn);
}

int64_t rt_hip_decoder_vocab(const rt_hip_decoder* d) { return d ? d->lm_head.n : -1; }

const float* rt_hip_decoder_logits(const rt_hip_decoder* d) { return d ? d->logits : nullptr; }

int rt_hip_decoder_destroy(rt_hip_decoder* d) {
    if (!d) return RT_HIP_OK;
    if (d->device >= 0) (void)hipSetDevice(d->device);
    (void)hipDeviceSynchronize();
    for (auto& g : d->graphs) rt_hip_graph_destroy(g);
    for (void* p : d->allocations) (void)hipFree(p);
    if (d->hstate) (void)hipHostFree(d->hstate);
    if (d->logits_stage) (void)hipHostFree(d->logits_stage);
    if (d->stream) (void)hipStreamDestroy(d->stream);
    delete d;
    return RT_HIP_OK;
}

}  // extern "C"
