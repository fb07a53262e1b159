// kiln_gpu.hpp - C++ host mirror of the reference op layer for the attention path (engine/src/gpu.h:133-156),
// over the C ABI of libkiln_attn.so (include/kiln_attn.h). Same names, argument order and meaning as the
// reference's free functions; failures throw std::runtime_error like the reference's CK/CB macros
// (engine/src/gpu.h:15-16) and attention16's shape check (engine/src/kernels.cu:870).
//
// The reference keeps its stream in a global (G.stream, engine/src/gpu.h:51-89); here it is set once with
// kiln::set_stream() and defaults to the null stream.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <string>

#include "../../include/kiln_attn.h"

namespace kiln {

inline hipStream_t& stream_ref() {
    static thread_local hipStream_t s = nullptr;
    return s;
}
inline void set_stream(hipStream_t s) { stream_ref() = s; }

inline void check(int rc, const char* what) {
    if (rc != KILN_OK)
        throw std::runtime_error(std::string(what) + ": " + kiln_attn_status_string(rc) + " (" + kiln_attn_last_error() +
                                 ")");
}

// Multi-head attention, fp32 rows; npad extra all-zero keys accounted for analytically.
inline void attention(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v, int ldv,
                      int Tq, int Tk, int H, int Dh, bool causal, int npad = 0) {
    check(kiln_attn_fwd_f32out(out, ldo, q, ldq, k, ldk, v, ldv, Tq, Tk, H, Dh, causal ? 1 : 0, npad,
                               (kiln_stream_t)stream_ref()),
          "attention");
}

// The same with an fp16 output (Dh = 128, not causal); throws on an unsupported shape.
inline void attention16(uint16_t* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                        int ldv, int Tq, int Tk, int H, int Dh, int npad = 0) {
    check(kiln_attn_fwd_f16out(out, ldo, q, ldq, k, ldk, v, ldv, Tq, Tk, H, Dh, npad, (kiln_stream_t)stream_ref()),
          "attention16");
}

// Exact fp32 attention (the reference's --fp32 mode).
inline void attention_exact(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                            int ldv, int Tq, int Tk, int H, int Dh, bool causal, int npad = 0) {
    check(kiln_attn_fwd_exact(out, ldo, q, ldq, k, ldk, v, ldv, Tq, Tk, H, Dh, causal ? 1 : 0, npad,
                              (kiln_stream_t)stream_ref()),
          "attention_exact");
}

// Per-row RMSNorm with bf16 weights (w may be null); in place allowed.
inline void rmsnorm(float* y, const float* x, const uint16_t* w_bf16, int rows, int dim, float eps) {
    check(kiln_rmsnorm_rows(y, x, w_bf16, rows, dim, eps, (kiln_stream_t)stream_ref()), "rmsnorm");
}

// Rotate-half RoPE over pairs (i, i + Dh/2), tables [T, Dh/2].
inline void rope_half(float* x, int T, int H, int Dh, const float* cos_t, const float* sin_t) {
    check(kiln_rope_half(x, T, H, Dh, cos_t, sin_t, (kiln_stream_t)stream_ref()), "rope_half");
}

// Modulated LayerNorm of the DiT block, fp32 or fp16 output (scale/shift fp32 per column).
inline void layernorm_mod(float* y, const float* x, const float* scale, const float* shift, int rows, int dim,
                          float eps) {
    check(kiln_layernorm_mod(y, x, scale, shift, rows, dim, eps, (kiln_stream_t)stream_ref()), "layernorm_mod");
}
inline void layernorm_mod16(uint16_t* y, const float* x, const float* scale, const float* shift, int rows, int dim,
                            float eps) {
    check(kiln_layernorm_mod16(y, x, scale, shift, rows, dim, eps, (kiln_stream_t)stream_ref()), "layernorm_mod16");
}

// Gated residual x += gate * y (gate may be null).
inline void add_gated(float* x, const float* y, const float* gate, int rows, int dim) {
    check(kiln_add_gated(x, y, gate, rows, dim, (kiln_stream_t)stream_ref()), "add_gated");
}

// ---- linear16 (engine/src/gpu.h:125-127, kernels.cu:573-609): fp16 GEMM with fused epilogue ----

enum class Epi16 { F32 = KILN_EPI_F32, F16 = KILN_EPI_F16, Gelu16 = KILN_EPI_GELU16, Resid = KILN_EPI_RESID };

// A linear16 weight converted at load (the reference's weight_to_f16, kernels.cu:531-544) into the prepared
// layout; owns its device buffer. src: [rows, cols] fp16, or bf16 when src_bf16.
class Linear16Weight {
   public:
    Linear16Weight(const uint16_t* src, int rows, int cols, bool src_bf16) : rows_(rows), cols_(cols) {
        const size_t n = kiln_linear16_prepped_weight_bytes(rows, cols);
        if (!n || hipMalloc(&p_, n) != hipSuccess) throw std::runtime_error("kiln: linear16 weight allocation failed");
        check(kiln_linear16_prepare_weight(p_, src, rows, cols, src_bf16 ? 1 : 0, (kiln_stream_t)stream_ref()),
              "linear16_prepare_weight");
    }
    ~Linear16Weight() {
        if (p_) (void)hipFree(p_);
    }
    Linear16Weight(const Linear16Weight&) = delete;
    Linear16Weight& operator=(const Linear16Weight&) = delete;
    const uint16_t* data() const { return p_; }
    int rows() const { return rows_; }
    int cols() const { return cols_; }

   private:
    uint16_t* p_ = nullptr;
    int rows_, cols_;
};

// y [T, ldy] (fp32 for F32/Resid, fp16 for F16/Gelu16) from x16 [T, W.cols()] (dense fp16 rows). The folded
// LoRA product (kernels.cu:564-600) comes in as a2 [T, k2] and w2 [W.rows(), k2] (fp16, k2 % 32 == 0).
inline void linear16(void* y, int ldy, const uint16_t* x16, int T, const Linear16Weight& W, Epi16 epi,
                     const float* gate = nullptr, float beta = 0.f, const uint16_t* a2 = nullptr,
                     const uint16_t* w2 = nullptr, int k2 = 0) {
    check(kiln_linear16_prepped(y, ldy, x16, T, W.data(), W.rows(), W.cols(), (int)epi, gate, beta, a2, w2, k2,
                                (kiln_stream_t)stream_ref()),
          "linear16");
}
// The same on a plain fp16 weight [rows, cols].
inline void linear16(void* y, int ldy, const uint16_t* x16, int T, const uint16_t* w16, int rows, int cols, Epi16 epi,
                     const float* gate = nullptr, float beta = 0.f) {
    check(kiln_linear16(y, ldy, x16, T, w16, rows, cols, (int)epi, gate, beta, nullptr, nullptr, 0,
                        (kiln_stream_t)stream_ref()),
          "linear16");
}

// The DiT self-attention section from the block's fp16 LayerNorm output (engine/src/dit.cu:460-469): the
// stacked Q/K/V projection with QK-RMSNorm, RoPE and K/V preparation in its epilogue, then the attention.
inline void dit_self_attention_x16(uint16_t* out, int ldo, const uint16_t* x16, const Linear16Weight& wqkv,
                                   const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps, const float* rcos,
                                   const float* rsin, int B, int T, int H, void* workspace, size_t ws_bytes) {
    check(kiln_dit_self_attn_x16(out, KILN_F16, ldo, x16, wqkv.data(), q_norm_w, k_norm_w, eps, rcos, rsin, B, T, H,
                                 workspace, ws_bytes, (kiln_stream_t)stream_ref()),
          "dit_self_attn_x16");
}

// NAG combine of fp16 rows (the k_nag<__half> launch of the fp16-activation forward).
inline void nag16(uint16_t* a, const uint16_t* an, int T, int dim, float scale, float tau, float alpha) {
    check(kiln_nag_combine(a, dim, an, dim, KILN_F16, T, dim, scale, tau, alpha, (kiln_stream_t)stream_ref()),
          "nag");
}

// ---- the DiT block's attention section (engine/src/dit.cu:458-488) and its per-generation state ----

// Cross-attention context of one generation: the reference's Dit::Context (rows [real, len) are zero padding,
// engine/src/models.h:26) together with its Dit::KVCache (models.h:56-58): every block's K/V, prepared once by
// prepare() (Dit::cache_context, engine/src/dit.cu:217-234) in the attention kernel's tiled layout. The padding
// rows are never stored: they enter the softmax analytically as npad = len - real zero keys.
class ContextKV {
   public:
    ContextKV(int nblocks, int len, int real, int H) : nblocks_(nblocks), len_(len), real_(real), H_(H) {
        if (nblocks <= 0 || real <= 0 || len < real || H <= 0) throw std::runtime_error("ContextKV: bad sizes");
        per_ = kiln_kv_prepped_bytes(real, H);
        if (hipMalloc(&buf_, per_ * nblocks) != hipSuccess) throw std::runtime_error("ContextKV: hipMalloc failed");
    }
    ~ContextKV() {
        if (buf_) (void)hipFree(buf_);
    }
    ContextKV(const ContextKV&) = delete;
    ContextKV& operator=(const ContextKV&) = delete;

    // block i's raw context projections K, V [real, ld] (in_dtype KILN_F32 or KILN_F16, head h at column
    // h*128); K is RMS-normed per head with the bf16 weights k_norm_w (null: no norm).
    void prepare(int block, const void* k, const void* v, int ld, int in_dtype, const uint16_t* k_norm_w, float eps) {
        if (block < 0 || block >= nblocks_) throw std::runtime_error("ContextKV::prepare: block out of range");
        check(kiln_kv_prepare(kv_mut(block), k, ld, v, ld, in_dtype, real_, H_, k_norm_w, eps, nullptr, nullptr,
                              (kiln_stream_t)stream_ref()),
              "cache_context");
    }
    const uint16_t* kv(int block) const { return reinterpret_cast<const uint16_t*>((const char*)buf_ + per_ * block); }
    int len() const { return len_; }
    int real() const { return real_; }
    int npad() const { return len_ - real_; }
    int heads() const { return H_; }

   private:
    uint16_t* kv_mut(int block) { return reinterpret_cast<uint16_t*>((char*)buf_ + per_ * block); }
    int nblocks_, len_, real_, H_;
    size_t per_ = 0;
    void* buf_ = nullptr;
};

// Normalized Attention Guidance settings of the reference (Dit::Nag, engine/src/models.h:80): with `neg` set,
// batch item 0's cross-attention output becomes the NAG blend of its positive and negative attentions.
struct Nag {
    const ContextKV* neg = nullptr;
    float scale = 5.f, tau = 2.5f, alpha = 0.25f;
};

// Self-attention of a CFG batch (engine/src/dit.cu:458-470): raw projections q, k, v [B*T, ld] (item b at
// rows b*T), QK-RMSNorm with bf16 weights and RoPE tables [T, 64] applied inside, fp16 out [B*T, ldo].
// ws may be null (library-owned workspace) or kiln_dit_self_attn_workspace_bytes(B, T, H) bytes.
inline void dit_self_attention(uint16_t* out, int ldo, const void* q, const void* k, const void* v, int in_dtype,
                               int ld, const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps,
                               const float* rope_cos, const float* rope_sin, int B, int T, int H, void* ws = nullptr,
                               size_t ws_bytes = 0) {
    check(kiln_dit_self_attn_fused(out, KILN_F16, ldo, q, k, v, in_dtype, ld, q_norm_w, k_norm_w, eps, rope_cos,
                                   rope_sin, B, T, H, ws, ws_bytes, (kiln_stream_t)stream_ref()),
          "self-attention");
}

// Cross-attention of a CFG batch for block `block` (engine/src/dit.cu:473-487): item b's queries (rows b*T of
// q, RMS-normed inside with q_norm_w) attend to cs[b]; with nag.neg, item 0 also attends to the negative
// context into out_neg [T, ldo] (caller scratch) and its output becomes the NAG blend.
inline void dit_cross_attention(uint16_t* out, uint16_t* out_neg, int ldo, const void* q, int in_dtype, int ldq,
                                const uint16_t* q_norm_w, float eps, int B, int T, int H, int block,
                                const ContextKV* const* cs, const Nag& nag = Nag()) {
    if (B <= 0 || B > 3) throw std::runtime_error("dit_cross_attention: B outside 1..3");
    const uint16_t* kvp[3];
    int Lk[3], np[3];
    for (int b = 0; b < B; b++) {
        if (cs[b]->heads() != H) throw std::runtime_error("dit_cross_attention: context prepared for other heads");
        kvp[b] = cs[b]->kv(block);
        Lk[b] = cs[b]->real();
        np[b] = cs[b]->npad();
    }
    const ContextKV* n = nag.neg;
    check(kiln_cross_attn_nag(out, out_neg, KILN_F16, ldo, q, in_dtype, ldq, q_norm_w, eps, B, T, H, kvp, Lk, np,
                              n ? n->kv(block) : nullptr, n ? n->real() : 0, n ? n->npad() : 0, nag.scale, nag.tau,
                              nag.alpha, (kiln_stream_t)stream_ref()),
          "cross-attention");
}

}  // namespace kiln
