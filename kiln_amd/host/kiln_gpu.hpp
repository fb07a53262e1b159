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

// NAG combine of fp16 rows (the k_nag<__half> launch of the fp16-activation forward).
inline void nag16(uint16_t* a, const uint16_t* an, int T, int dim, float scale, float tau, float alpha) {
    check(kiln_nag_combine(a, dim, an, dim, KILN_F16, T, dim, scale, tau, alpha, (kiln_stream_t)stream_ref()),
          "nag");
}

}  // namespace kiln
