// C ABI of libkiln_attn.so: argument checks, workspace handling and kernel dispatch.
// Declarations and contracts: include/kiln_attn.h.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "../../include/kiln_attn.h"
#include "common.hpp"
#include "capi_util.hpp"
#include "internal.hpp"

using kiln::DT;

namespace kiln::capi {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return KILN_OK;
    return fail(KILN_EHIP, "%s: %s", what, hipGetErrorString(e));
}

// Per-device workspace of the entry points that take none (the drop-ins among them): the prepared K/V tiles
// and key-split partials. Three modes per device:
//   * bound: kiln_attn_set_workspace gave a caller-owned buffer (e.g. a slice of the engine's arena);
//   * reserved: kiln_attn_workspace_reserve allocated one at set-up;
//   * neither: the first call that needs more allocates (grow-only; the outgrown buffer is kept, not freed, so
//     nothing has to wait for earlier stream-ordered users of it; kiln_attn_workspace_release frees them).
// Once bound or reserved, no call allocates or synchronizes: one whose need exceeds the buffer fails with
// KILN_ENOMEM. Calls are stream-ordered on the caller's stream; concurrent calls on different streams of one
// device must pass their own workspaces.
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool fixed = false;      // bound or reserved: never grows
    bool owned = false;      // ptr was allocated by the library
    std::vector<void*> old;  // outgrown library buffers
};
std::mutex g_ws_mu;
std::vector<Workspace> g_ws;

int current_device(int* dev) {
    hipError_t e = hipGetDevice(dev);
    if (e != hipSuccess) return hip_check(e, "hipGetDevice");
    return KILN_OK;
}

Workspace& ws_of(int dev) {
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
    return g_ws[dev];
}

int get_workspace(size_t need, void** out) {
    int dev = 0;
    if (int r = current_device(&dev)) return r;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = ws_of(dev);
    if (w.bytes < need) {
        if (w.fixed)
            return fail(KILN_ENOMEM, "workspace of device %d holds %zu bytes, this call needs %zu (set up with "
                        "kiln_attn_workspace_reserve / kiln_attn_set_workspace)", dev, w.bytes, need);
        const size_t sz = need + need / 4;
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, sz);
        if (e != hipSuccess) return fail(KILN_ENOMEM, "workspace hipMalloc(%zu): %s", sz, hipGetErrorString(e));
        if (w.ptr) w.old.push_back(w.ptr);
        w.ptr = p;
        w.bytes = sz;
        w.owned = true;
    }
    *out = w.ptr;
    return KILN_OK;
}

// frees every library-owned buffer of device dev (the caller has synchronized)
void drop_owned(Workspace& w) {
    for (void* p : w.old) (void)hipFree(p);
    w.old.clear();
    if (w.owned && w.ptr) (void)hipFree(w.ptr);
    w = Workspace{};
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// row alignment for 16-byte vector loads of 8-element chunks
bool rows_ok(const void* p, int ld, DT dt) {
    if (!aligned16(p)) return false;
    return dt == DT::F16 ? (ld % 8) == 0 : (ld % 4) == 0;
}

// Keys per head of the flash path: the attention kernel addresses a head's prepared K/V block (32 KB per 64
// keys) with 32-bit buffer offsets.
constexpr int MAX_TK = 1 << 22;

int check_common(int Tq, int Tk, int H, int npad) {
    if (Tq < 0 || Tk < 0 || H <= 0 || npad < 0) return fail(KILN_EINVAL, "bad sizes Tq=%d Tk=%d H=%d npad=%d", Tq, Tk, H, npad);
    if (Tk > MAX_TK) return fail(KILN_EUNSUPPORTED, "Tk=%d above %d keys per head", Tk, MAX_TK);
    if (Tk == 0 && npad == 0 && Tq > 0) return fail(KILN_EINVAL, "no keys (Tk=0, npad=0): softmax undefined");
    return KILN_OK;
}

// output when there are no real keys but npad zero keys: softmax mass all on zero values -> 0
int zero_rows(void* out, int ldo, size_t esz, int Tq, int H, int Dh, hipStream_t s) {
    return hip_check(kiln::launch_zero_rows(out, (size_t)ldo * esz, (size_t)H * Dh * esz, Tq, s), "zero_rows launch");
}

int flash_self(void* out, DT od, int ldo, long long bso, const void* q, int ldq, long long bsq, const void* k, int ldk,
               long long bsk, const void* v, int ldv, long long bsv, DT in, int B, int Tq, int Tk, int H, int npad,
               const uint16_t* qw, const uint16_t* kw, float eps, const float* rc, const float* rs, void* ws,
               size_t ws_bytes, hipStream_t stream) {
    if (B <= 0 || B > kiln::MAX_JOBS) return fail(KILN_EUNSUPPORTED, "batch %d outside 1..%d", B, kiln::MAX_JOBS);
    const size_t per = kiln_kv_prepped_bytes(Tk, H);
    const size_t need = per * B;
    // small grids split every unit's keys (partials behind the prepared K/V); a caller's workspace takes the
    // split only if it is large enough for the partials too (the *_workspace_bytes functions that know Tq
    // include them)
    int ks = kiln::attn_key_split(B, Tq, Tk, H);
    size_t split = kiln::attn_split_bytes(ks, B, Tq, H);
    if (!ws) {
        int rc2 = get_workspace(need + split, &ws);
        if (rc2) return rc2;
    } else if (ws_bytes < need) {
        return fail(KILN_ENOMEM, "workspace %zu bytes < %zu needed", ws_bytes, need);
    } else if (ws_bytes < need + split) {
        ks = 1;
        split = 0;
    }
    const size_t isz = in == DT::F16 ? 2 : 4, osz = od == DT::F16 ? 2 : 4;
    kiln::AttnLaunch a{};
    kiln::KVPrepJob pj[kiln::MAX_JOBS];
    for (int b = 0; b < B; b++) {
        uint16_t* kvp = reinterpret_cast<uint16_t*>((char*)ws + per * b);
        pj[b] = {kvp, (const char*)k + bsk * b * isz, (const char*)v + bsv * b * isz, ldk, ldv};
        a.job[b] = {(const char*)q + bsq * b * isz, kvp, (char*)out + bso * b * osz, Tk, npad};
    }
    int r = hip_check(kiln::launch_kv_prep(pj, B, in, Tk, H, kw, eps, rc, rs, stream), "kv_prep launch");
    if (r) return r;
    a.njobs = B;
    a.Tq = Tq;
    a.H = H;
    a.ldq = ldq;
    a.ldo = ldo;
    a.in = in;
    a.out = od;
    a.qw = qw;
    a.eps = eps;
    a.rcos = rc;
    a.rsin = rs;
    a.ksplit = ks;
    a.part = ks > 1 ? reinterpret_cast<float*>((char*)ws + need) : nullptr;
    return hip_check(kiln::launch_attn_fwd(a, stream), "attn_fwd launch");
}

}  // namespace kiln::capi

using namespace kiln::capi;

extern "C" {

const char* kiln_attn_status_string(int status) {
    switch (status) {
        case KILN_OK: return "ok";
        case KILN_EINVAL: return "invalid argument";
        case KILN_EUNSUPPORTED: return "unsupported shape, stride or alignment";
        case KILN_EHIP: return "HIP runtime error";
        case KILN_ENOMEM: return "out of device memory / workspace too small";
        default: return "unknown status";
    }
}

const char* kiln_attn_last_error(void) { return g_err; }

size_t kiln_attn_dropin_workspace_bytes(int Tq, int Tk, int H) {
    if (Tq <= 0 || Tk <= 0 || H <= 0) return 0;
    const int ks = kiln::attn_key_split(1, Tq, Tk, H);
    return kiln_kv_prepped_bytes(Tk, H) + kiln::attn_split_bytes(ks, 1, Tq, H);
}

int kiln_attn_workspace_reserve(size_t bytes) {
    int dev = 0;
    if (int r = current_device(&dev)) return r;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = ws_of(dev);
    if (w.fixed && !w.owned) return fail(KILN_EINVAL, "device %d has a caller-bound workspace", dev);
    if (w.bytes < bytes) {
        // set-up time: earlier users of the library's buffers finish before they are released
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_check(e, "hipDeviceSynchronize");
        drop_owned(w);
        void* p = nullptr;
        e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return fail(KILN_ENOMEM, "workspace hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        w.ptr = p;
        w.bytes = bytes;
        w.owned = true;
    }
    w.fixed = true;
    return KILN_OK;
}

int kiln_attn_set_workspace(void* ptr, size_t bytes) {
    int dev = 0;
    if (int r = current_device(&dev)) return r;
    if (ptr && ((uintptr_t)ptr & 255)) return fail(KILN_EUNSUPPORTED, "workspace must be 256-byte aligned");
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = ws_of(dev);
    if (w.owned) {
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_check(e, "hipDeviceSynchronize");
        drop_owned(w);
    }
    std::vector<void*> old;
    old.swap(w.old);
    w = Workspace{};
    w.old.swap(old);
    if (ptr) {
        w.ptr = ptr;
        w.bytes = bytes;
        w.fixed = true;
    }
    return KILN_OK;
}

int kiln_attn_workspace_release(void) {
    int dev = 0;
    if (int r = current_device(&dev)) return r;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = ws_of(dev);
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_check(e, "hipDeviceSynchronize");
    if (w.owned || !w.ptr) {
        drop_owned(w);
    } else {  // a caller-bound buffer stays bound; only outgrown library buffers go
        for (void* p : w.old) (void)hipFree(p);
        w.old.clear();
    }
    return KILN_OK;
}

int kiln_attn_device_arch(int dev, char* buf, int buflen) {
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_check(e, "hipGetDeviceProperties");
    snprintf(buf, buflen, "%s", prop.gcnArchName);
    return KILN_OK;
}

size_t kiln_kv_prepped_bytes(int Tk, int H) {
    if (Tk <= 0 || H <= 0) return 0;
    return (size_t)H * kiln::kv_head_stride(Tk) * 2;
}

int kiln_kv_prepare(uint16_t* kvp, const void* k, int ldk, const void* v, int ldv, int in_dtype, int Tk, int H,
                    const uint16_t* k_norm_w, float eps, const float* rope_cos, const float* rope_sin,
                    kiln_stream_t stream) {
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    if (in_dtype != KILN_F32 && in_dtype != KILN_F16) return fail(KILN_EINVAL, "in_dtype %d", in_dtype);
    DT in = (DT)in_dtype;
    if (Tk < 0 || H <= 0) return fail(KILN_EINVAL, "bad sizes Tk=%d H=%d", Tk, H);
    if (Tk > MAX_TK) return fail(KILN_EUNSUPPORTED, "Tk=%d above %d keys per head", Tk, MAX_TK);
    if (Tk == 0) return KILN_OK;
    if (!kvp || !k || !v) return fail(KILN_EINVAL, "null pointer");
    if (!aligned16(kvp)) return fail(KILN_EUNSUPPORTED, "kvp not 16-byte aligned");
    if (!rows_ok(k, ldk, in) || !rows_ok(v, ldv, in)) return fail(KILN_EUNSUPPORTED, "K/V rows not 16-byte aligned");
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) return fail(KILN_EINVAL, "rope tables: need both cos and sin");
    if (rope_cos && (!aligned16(rope_cos) || !aligned16(rope_sin))) return fail(KILN_EUNSUPPORTED, "rope tables not 16-byte aligned");
    const kiln::KVPrepJob pj{kvp, k, v, ldk, ldv};
    return hip_check(kiln::launch_kv_prep(&pj, 1, in, Tk, H, k_norm_w, eps, rope_cos, rope_sin, (hipStream_t)stream),
                     "kv_prep launch");
}

int kiln_attn_fwd_prepped(void* out, int out_dtype, int ldo, const void* q, int in_dtype, int ldq,
                          const uint16_t* q_norm_w, float eps, const float* rope_cos, const float* rope_sin,
                          const uint16_t* kvp, int Tq, int Tk, int H, int npad, kiln_stream_t stream) {
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    if ((in_dtype != KILN_F32 && in_dtype != KILN_F16) || (out_dtype != KILN_F32 && out_dtype != KILN_F16))
        return fail(KILN_EINVAL, "dtype");
    int r = check_common(Tq, Tk, H, npad);
    if (r) return r;
    if (Tq == 0) return KILN_OK;
    if (!out || !q || (Tk > 0 && !kvp)) return fail(KILN_EINVAL, "null pointer");
    const DT in = (DT)in_dtype, od = (DT)out_dtype;
    if (Tk == 0) return zero_rows(out, ldo, od == DT::F16 ? 2 : 4, Tq, H, 128, (hipStream_t)stream);
    if (!rows_ok(q, ldq, in) || !aligned16(kvp)) return fail(KILN_EUNSUPPORTED, "Q rows / kvp not 16-byte aligned");
    if (ldo % 2) return fail(KILN_EUNSUPPORTED, "ldo must be even");
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) return fail(KILN_EINVAL, "rope tables: need both cos and sin");
    kiln::AttnLaunch a{};
    a.job[0] = {q, kvp, out, Tk, npad};
    a.njobs = 1;
    a.Tq = Tq;
    a.H = H;
    a.ldq = ldq;
    a.ldo = ldo;
    a.in = in;
    a.out = od;
    a.qw = q_norm_w;
    a.eps = eps;
    a.rcos = rope_cos;
    a.rsin = rope_sin;
    return hip_check(kiln::launch_attn_fwd(a, (hipStream_t)stream), "attn_fwd launch");
}

int kiln_attn_fwd_prepped_batch(void* out, int out_dtype, int ldo, long long bso, const void* q, int in_dtype, int ldq,
                                long long bsq, const uint16_t* q_norm_w, float eps, const float* rope_cos,
                                const float* rope_sin, const uint16_t* const* kvp, int B, int Tq, int Tk, int H,
                                int npad, kiln_stream_t stream) {
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    if ((in_dtype != KILN_F32 && in_dtype != KILN_F16) || (out_dtype != KILN_F32 && out_dtype != KILN_F16))
        return fail(KILN_EINVAL, "dtype");
    int r = check_common(Tq, Tk, H, npad);
    if (r) return r;
    if (B <= 0 || B > kiln::MAX_JOBS) return fail(KILN_EUNSUPPORTED, "batch %d outside 1..%d", B, kiln::MAX_JOBS);
    if (Tq == 0) return KILN_OK;
    if (Tk == 0) return fail(KILN_EUNSUPPORTED, "batched prepped attention needs Tk > 0");
    if (!out || !q || !kvp) return fail(KILN_EINVAL, "null pointer");
    const DT in = (DT)in_dtype, od = (DT)out_dtype;
    const size_t isz = in == DT::F16 ? 2 : 4, osz = od == DT::F16 ? 2 : 4;
    if (!rows_ok(q, ldq, in) || ldo % 2 || (bsq * (long long)isz) % 16) return fail(KILN_EUNSUPPORTED, "Q rows not 16-byte aligned");
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) return fail(KILN_EINVAL, "rope tables: need both cos and sin");
    kiln::AttnLaunch a{};
    for (int b = 0; b < B; b++) {
        if (!kvp[b] || !aligned16(kvp[b])) return fail(KILN_EINVAL, "kvp[%d] null or misaligned", b);
        a.job[b] = {(const char*)q + bsq * b * isz, kvp[b], (char*)out + bso * b * osz, Tk, npad};
    }
    a.njobs = B;
    a.Tq = Tq;
    a.H = H;
    a.ldq = ldq;
    a.ldo = ldo;
    a.in = in;
    a.out = od;
    a.qw = q_norm_w;
    a.eps = eps;
    a.rcos = rope_cos;
    a.rsin = rope_sin;
    return hip_check(kiln::launch_attn_fwd(a, (hipStream_t)stream), "attn_fwd launch");
}

int kiln_attn_fwd_f32out(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                         int ldv, int Tq, int Tk, int H, int Dh, int causal, int npad, kiln_stream_t stream) {
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    int r = check_common(Tq, Tk, H, npad);
    if (r) return r;
    if (Tq == 0) return KILN_OK;
    if (!out || !q || (Tk > 0 && (!k || !v))) return fail(KILN_EINVAL, "null pointer");
    const bool flash = Dh == 128 && !causal && rows_ok(q, ldq, DT::F32) && rows_ok(k, ldk, DT::F32) &&
                       rows_ok(v, ldv, DT::F32) && ldo % 2 == 0;
    if (!flash) return kiln_attn_fwd_exact(out, ldo, q, ldq, k, ldk, v, ldv, Tq, Tk, H, Dh, causal, npad, stream);
    if (Tk == 0) return zero_rows(out, ldo, 4, Tq, H, Dh, (hipStream_t)stream);
    return flash_self(out, DT::F32, ldo, 0, q, ldq, 0, k, ldk, 0, v, ldv, 0, DT::F32, 1, Tq, Tk, H, npad, nullptr,
                      nullptr, 0.f, nullptr, nullptr, nullptr, 0, (hipStream_t)stream);
}

int kiln_attn_fwd_f16out(uint16_t* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                         int ldv, int Tq, int Tk, int H, int Dh, int npad, kiln_stream_t stream) {
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    int r = check_common(Tq, Tk, H, npad);
    if (r) return r;
    if (Dh != 128) return fail(KILN_EUNSUPPORTED, "attention16: unsupported head size %d (needs 128)", Dh);
    if (Tq == 0) return KILN_OK;
    if (!out || !q || (Tk > 0 && (!k || !v))) return fail(KILN_EINVAL, "null pointer");
    if (!rows_ok(q, ldq, DT::F32) || !rows_ok(k, ldk, DT::F32) || !rows_ok(v, ldv, DT::F32) || ldo % 2)
        return fail(KILN_EUNSUPPORTED, "attention16: unsupported row stride or alignment");
    if (Tk == 0) return zero_rows(out, ldo, 2, Tq, H, Dh, (hipStream_t)stream);
    return flash_self(out, DT::F16, ldo, 0, q, ldq, 0, k, ldk, 0, v, ldv, 0, DT::F32, 1, Tq, Tk, H, npad, nullptr,
                      nullptr, 0.f, nullptr, nullptr, nullptr, 0, (hipStream_t)stream);
}

int kiln_attn_fwd_exact(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                        int ldv, int Tq, int Tk, int H, int Dh, int causal, int npad, kiln_stream_t stream) {
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    int r = check_common(Tq, Tk, H, npad);
    if (r) return r;
    if (Dh <= 0 || Dh > 256) return fail(KILN_EUNSUPPORTED, "exact attention: head size %d outside 1..256", Dh);
    if (Tq == 0) return KILN_OK;
    if (!out || !q || (Tk > 0 && (!k || !v))) return fail(KILN_EINVAL, "null pointer");
    if (Tk == 0) return zero_rows(out, ldo, 4, Tq, H, Dh, (hipStream_t)stream);
    return hip_check(kiln::launch_exact_attn(out, ldo, q, ldq, k, ldk, v, ldv, Tq, Tk, H, Dh, causal != 0, npad,
                                             (hipStream_t)stream),
                     "exact_attn launch");
}

size_t kiln_attn_fwd_f16in_workspace_bytes(int B, int Tk, int H) {
    return B > 0 ? (size_t)B * kiln_kv_prepped_bytes(Tk, H) : 0;
}

int kiln_attn_fwd_f16in(void* out, int out_dtype, int ldo, long long bso, const uint16_t* q, int ldq, long long bsq,
                        const uint16_t* k, int ldk, long long bsk, const uint16_t* v, int ldv, long long bsv, int B,
                        int Tq, int Tk, int H, int npad, void* workspace, size_t ws_bytes, kiln_stream_t stream) {
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    if (out_dtype != KILN_F32 && out_dtype != KILN_F16) return fail(KILN_EINVAL, "out_dtype %d", out_dtype);
    int r = check_common(Tq, Tk, H, npad);
    if (r) return r;
    if (B <= 0) return fail(KILN_EINVAL, "B=%d", B);
    if (Tq == 0) return KILN_OK;
    if (!out || !q || (Tk > 0 && (!k || !v))) return fail(KILN_EINVAL, "null pointer");
    const DT od = (DT)out_dtype;
    if (Tk == 0) {
        for (int b = 0; b < B; b++) {
            r = zero_rows((char*)out + bso * b * (od == DT::F16 ? 2 : 4), ldo, od == DT::F16 ? 2 : 4, Tq, H, 128,
                          (hipStream_t)stream);
            if (r) return r;
        }
        return KILN_OK;
    }
    if (!rows_ok(q, ldq, DT::F16) || !rows_ok(k, ldk, DT::F16) || !rows_ok(v, ldv, DT::F16) || ldo % 2 ||
        bsq % 8 || bsk % 8 || bsv % 8 || bso % 2)
        return fail(KILN_EUNSUPPORTED, "rows / batch strides not 16-byte aligned");
    return flash_self(out, od, ldo, bso, q, ldq, bsq, k, ldk, bsk, v, ldv, bsv, DT::F16, B, Tq, Tk, H, npad, nullptr,
                      nullptr, 0.f, nullptr, nullptr, workspace, ws_bytes, (hipStream_t)stream);
}

size_t kiln_dit_self_attn_workspace_bytes(int B, int T, int H) {
    if (B <= 0 || T <= 0 || H <= 0) return 0;
    return (size_t)B * kiln_kv_prepped_bytes(T, H) +
           kiln::attn_split_bytes(kiln::attn_key_split(B, T, T, H), B, T, H);
}

int kiln_dit_self_attn_fused(void* out, int out_dtype, int ldo, const void* q, const void* k, const void* v,
                             int in_dtype, int ld, const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps,
                             const float* rope_cos, const float* rope_sin, int B, int T, int H, void* workspace,
                             size_t ws_bytes, kiln_stream_t stream) {
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    if ((in_dtype != KILN_F32 && in_dtype != KILN_F16) || (out_dtype != KILN_F32 && out_dtype != KILN_F16))
        return fail(KILN_EINVAL, "dtype");
    if (B <= 0 || T <= 0 || H <= 0) return fail(KILN_EINVAL, "bad sizes B=%d T=%d H=%d", B, T, H);
    if (!out || !q || !k || !v) return fail(KILN_EINVAL, "null pointer");
    const DT in = (DT)in_dtype, od = (DT)out_dtype;
    if (!rows_ok(q, ld, in) || !rows_ok(k, ld, in) || !rows_ok(v, ld, in) || ldo % 2)
        return fail(KILN_EUNSUPPORTED, "rows not 16-byte aligned");
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) return fail(KILN_EINVAL, "rope tables: need both cos and sin");
    if (rope_cos && (!aligned16(rope_cos) || !aligned16(rope_sin))) return fail(KILN_EUNSUPPORTED, "rope tables not 16-byte aligned");
    const long long bs = (long long)T * ld, bso = (long long)T * ldo;
    return flash_self(out, od, ldo, bso, q, ld, bs, k, ld, bs, v, ld, bs, in, B, T, T, H, 0, q_norm_w, k_norm_w, eps,
                      rope_cos, rope_sin, workspace, ws_bytes, (hipStream_t)stream);
}

static size_t align256(size_t n) { return (n + 255) / 256 * 256; }

size_t kiln_dit_self_attn_x16_workspace_bytes(int B, int T, int H) {
    if (B <= 0 || T <= 0 || H <= 0) return 0;
    const size_t q = align256((size_t)B * T * H * kiln::HD * 2), kv = align256(kiln_kv_prepped_bytes(T, H));
    const int ks = kiln::attn_key_split(B, T, T, H);
    return q + kv * B + kiln::attn_split_bytes(ks, B, T, H);
}

int kiln_dit_self_attn_x16(void* out, int out_dtype, int ldo, const uint16_t* x16, const uint16_t* wqkv_prepped,
                           const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps, const float* rope_cos,
                           const float* rope_sin, int B, int T, int H, void* workspace, size_t ws_bytes,
                           kiln_stream_t stream) {
    if (out_dtype != KILN_F32 && out_dtype != KILN_F16) return fail(KILN_EINVAL, "dtype");
    if (B <= 0 || T <= 0 || H <= 0) return fail(KILN_EINVAL, "bad sizes B=%d T=%d H=%d", B, T, H);
    if (B > kiln::MAX_JOBS || H % 2 || T > MAX_TK)
        return fail(KILN_EUNSUPPORTED, "dit_self_attn_x16: needs B <= %d, an even H and T <= %d (B=%d H=%d T=%d)",
                    kiln::MAX_JOBS, MAX_TK, B, H, T);
    if (!out || !x16 || !wqkv_prepped || !q_norm_w || !k_norm_w || !rope_cos || !rope_sin || !workspace)
        return fail(KILN_EINVAL, "null pointer");
    if (!aligned16(x16) || !aligned16(wqkv_prepped) || !aligned16(rope_cos) || !aligned16(rope_sin) ||
        !aligned16(workspace) || ldo % 2)
        return fail(KILN_EUNSUPPORTED, "operands not 16-byte aligned / ldo odd");
    if (ws_bytes < kiln_dit_self_attn_x16_workspace_bytes(B, T, H))
        return fail(KILN_ENOMEM, "workspace %zu bytes < %zu", ws_bytes, kiln_dit_self_attn_x16_workspace_bytes(B, T, H));
    const int D = H * kiln::HD;
    char* ws = static_cast<char*>(workspace);
    uint16_t* q16 = reinterpret_cast<uint16_t*>(ws);
    ws += align256((size_t)B * T * D * 2);
    const size_t kvb = align256(kiln_kv_prepped_bytes(T, H));
    uint16_t* kvp[kiln::MAX_JOBS] = {};
    for (int b = 0; b < B; b++) kvp[b] = reinterpret_cast<uint16_t*>(ws + kvb * b);
    float* part = reinterpret_cast<float*>(ws + kvb * B);
    hipStream_t s = (hipStream_t)stream;
    int rc = hip_check(kiln::launch_kv_zero_tail(kvp, B, T, H, s), "kv tail launch");
    if (rc) return rc;
    kiln::GemmLaunch g{};
    g.a = x16;
    g.w = wqkv_prepped;
    g.K = D;
    g.M = B * T;
    g.N = 3 * D;
    g.c = nullptr;
    g.ldc = 3 * D;
    g.epi = 4;
    g.wprep = true;
    g.q16 = q16;
    for (int b = 0; b < B; b++) g.kvp[b] = kvp[b];
    g.T = T;
    g.H = H;
    g.qw = q_norm_w;
    g.kw = k_norm_w;
    g.eps = eps;
    g.rcos = rope_cos;
    g.rsin = rope_sin;
    {
        kiln::prof::Scope prof_("gemm_tc16", s);
        rc = hip_check(kiln::launch_gemm16(g, s), "qkv projection launch");
    }
    if (rc) return rc;
    const DT od = (DT)out_dtype;
    const size_t osz = od == DT::F16 ? 2 : 4;
    kiln::AttnLaunch a{};
    for (int b = 0; b < B; b++) a.job[b] = {q16 + (size_t)b * T * D, kvp[b], (char*)out + (size_t)b * T * ldo * osz, T, 0};
    a.njobs = B;
    a.Tq = T;
    a.H = H;
    a.ldq = D;
    a.ldo = ldo;
    a.in = DT::F16;
    a.out = od;
    a.q_prescaled = true;
    a.ksplit = kiln::attn_key_split(B, T, T, H);
    a.part = a.ksplit > 1 ? part : nullptr;
    kiln::prof::Scope prof_("attention", s);
    return hip_check(kiln::launch_attn_fwd(a, s), "attn_fwd launch");
}

static int cross_attn_impl(void* out, void* out_neg, int out_dtype, int ldo, const void* q, int in_dtype, int ldq,
                           const uint16_t* q_norm_w, float eps, int B, int T, int H, const uint16_t* const* kvp,
                           const int* Lk, const int* npad, const uint16_t* kvp_neg, int Lk_neg, int npad_neg,
                           float nag_scale, float nag_tau, float nag_alpha, bool q_prescaled, kiln_stream_t stream) {
    if ((in_dtype != KILN_F32 && in_dtype != KILN_F16) || (out_dtype != KILN_F32 && out_dtype != KILN_F16))
        return fail(KILN_EINVAL, "dtype");
    const int nj = B + (kvp_neg ? 1 : 0);
    if (B <= 0 || nj > kiln::MAX_JOBS) return fail(KILN_EUNSUPPORTED, "B=%d (+NAG) outside 1..%d jobs", B, kiln::MAX_JOBS);
    if (T <= 0 || H <= 0 || !out || !q || !kvp || !Lk || !npad || (kvp_neg && !out_neg))
        return fail(KILN_EINVAL, "bad sizes or null pointer");
    const DT in = (DT)in_dtype, od = (DT)out_dtype;
    if (!rows_ok(q, ldq, in) || ldo % 2) return fail(KILN_EUNSUPPORTED, "Q rows not 16-byte aligned / ldo odd");
    const size_t isz = in == DT::F16 ? 2 : 4, osz = od == DT::F16 ? 2 : 4;
    kiln::AttnLaunch a{};
    // Context chains: one unit per query tile and head runs every context in turn (item 0's positive and
    // NAG-negative contexts, which share item 0's queries, back to back on the same Q registers), so a launch has a
    // third of the units, each three times longer: config 5's cross-attention + NAG 60.9 -> 58.1 us per block
    // (A/B on one box), bit-identical outputs. KILN_CHAIN=0 runs one unit per context (A/B measurements, tests).
    const char* ce = getenv("KILN_CHAIN");
    a.chain = !(ce && atoi(ce) == 0);
    int n = 0;
    for (int b = 0; b < B; b++) {
        if (Lk[b] <= 0 || Lk[b] > MAX_TK || npad[b] < 0 || !kvp[b] || !aligned16(kvp[b]))
            return fail(KILN_EINVAL, "context %d: Lk=%d npad=%d", b, Lk[b], npad[b]);
        a.job[n++] = {(const char*)q + (size_t)b * T * ldq * isz, kvp[b], (char*)out + (size_t)b * T * ldo * osz, Lk[b],
                      npad[b]};
        if (b == 0 && kvp_neg) {
            if (Lk_neg <= 0 || Lk_neg > MAX_TK || npad_neg < 0 || !aligned16(kvp_neg))
                return fail(KILN_EINVAL, "NAG context Lk=%d", Lk_neg);
            a.job[n++] = {q, kvp_neg, out_neg, Lk_neg, npad_neg};
        }
    }
    a.njobs = n;
    a.Tq = T;
    a.H = H;
    a.ldq = ldq;
    a.ldo = ldo;
    a.in = in;
    a.out = od;
    a.qw = q_norm_w;
    a.eps = eps;
    a.q_prescaled = q_prescaled;
    int r = hip_check(kiln::launch_attn_fwd(a, (hipStream_t)stream), "attn_fwd launch");
    if (r || !kvp_neg) return r;
    return hip_check(kiln::launch_nag(out, ldo, out_neg, ldo, od, T, H * 128, nag_scale, nag_tau, nag_alpha,
                                      (hipStream_t)stream),
                     "nag launch");
}

int kiln_cross_attn_nag(void* out, void* out_neg, int out_dtype, int ldo, const void* q, int in_dtype, int ldq,
                        const uint16_t* q_norm_w, float eps, int B, int T, int H, const uint16_t* const* kvp,
                        const int* Lk, const int* npad, const uint16_t* kvp_neg, int Lk_neg, int npad_neg,
                        float nag_scale, float nag_tau, float nag_alpha, kiln_stream_t stream) {
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    return cross_attn_impl(out, out_neg, out_dtype, ldo, q, in_dtype, ldq, q_norm_w, eps, B, T, H, kvp, Lk, npad,
                           kvp_neg, Lk_neg, npad_neg, nag_scale, nag_tau, nag_alpha, false, stream);
}

int kiln_dit_cross_attn_x16(void* out, void* out_neg, int out_dtype, int ldo, const uint16_t* x16,
                            const uint16_t* wq_prepped, const uint16_t* q_norm_w, float eps, int B, int T, int H,
                            const uint16_t* const* kvp, const int* Lk, const int* npad, const uint16_t* kvp_neg,
                            int Lk_neg, int npad_neg, float nag_scale, float nag_tau, float nag_alpha, void* workspace,
                            size_t ws_bytes, kiln_stream_t stream) {
    if (B <= 0 || T <= 0 || H <= 0 || H % 2) return fail(KILN_EINVAL, "bad sizes B=%d T=%d H=%d (H even)", B, T, H);
    if (!x16 || !wq_prepped || !q_norm_w || !workspace) return fail(KILN_EINVAL, "null pointer");
    if (!aligned16(x16) || !aligned16(wq_prepped) || !aligned16(workspace))
        return fail(KILN_EUNSUPPORTED, "operands not 16-byte aligned");
    const int D = H * kiln::HD;
    if (ws_bytes < (size_t)B * T * D * 2) return fail(KILN_ENOMEM, "workspace %zu < %zu bytes", ws_bytes, (size_t)B * T * D * 2);
    uint16_t* q16 = static_cast<uint16_t*>(workspace);
    kiln::GemmLaunch g{};
    g.a = x16;
    g.w = wq_prepped;
    g.K = D;
    g.M = B * T;
    g.N = D;
    g.ldc = D;
    g.epi = 4;
    g.wprep = true;
    g.q16 = q16;
    g.T = T;
    g.H = H;
    g.qw = q_norm_w;
    g.kw = q_norm_w;
    g.eps = eps;
    int rc;
    {
        kiln::prof::Scope prof_("gemm_tc16", (hipStream_t)stream);
        rc = hip_check(kiln::launch_gemm16(g, (hipStream_t)stream), "cross-Q projection launch");
    }
    if (rc) return rc;
    kiln::prof::Scope prof_("attention", (hipStream_t)stream);
    return cross_attn_impl(out, out_neg, out_dtype, ldo, q16, KILN_F16, D, nullptr, eps, B, T, H, kvp, Lk, npad, kvp_neg,
                           Lk_neg, npad_neg, nag_scale, nag_tau, nag_alpha, true, stream);
}

int kiln_rmsnorm_rows(float* y, const float* x, const uint16_t* w_bf16, int rows, int dim, float eps,
                      kiln_stream_t stream) {
    kiln::prof::Scope prof_("norm", (hipStream_t)stream);
    if (rows < 0 || dim <= 0) return fail(KILN_EINVAL, "bad sizes");
    if (rows && (!y || !x)) return fail(KILN_EINVAL, "null pointer");
    return hip_check(kiln::launch_rmsnorm_rows(y, x, w_bf16, rows, dim, eps, (hipStream_t)stream), "rmsnorm launch");
}

int kiln_layernorm_mod(float* y, const float* x, const float* scale, const float* shift, int rows, int dim, float eps,
                       kiln_stream_t stream) {
    kiln::prof::Scope prof_("layernorm", (hipStream_t)stream);
    if (rows < 0 || dim <= 0) return fail(KILN_EINVAL, "bad sizes rows=%d dim=%d", rows, dim);
    if (rows && (!y || !x || !scale || !shift)) return fail(KILN_EINVAL, "null pointer");
    return hip_check(kiln::launch_layernorm_mod(y, kiln::DT::F32, x, scale, shift, rows, dim, eps, (hipStream_t)stream),
                     "layernorm_mod launch");
}

int kiln_layernorm_mod16(uint16_t* y, const float* x, const float* scale, const float* shift, int rows, int dim,
                         float eps, kiln_stream_t stream) {
    kiln::prof::Scope prof_("layernorm", (hipStream_t)stream);
    if (rows < 0 || dim <= 0) return fail(KILN_EINVAL, "bad sizes rows=%d dim=%d", rows, dim);
    if (rows && (!y || !x || !scale || !shift)) return fail(KILN_EINVAL, "null pointer");
    return hip_check(kiln::launch_layernorm_mod(y, kiln::DT::F16, x, scale, shift, rows, dim, eps, (hipStream_t)stream),
                     "layernorm_mod16 launch");
}

int kiln_add_gated(float* x, const float* y, const float* gate, int rows, int dim, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (rows < 0 || dim <= 0) return fail(KILN_EINVAL, "bad sizes rows=%d dim=%d", rows, dim);
    if (rows && (!x || !y)) return fail(KILN_EINVAL, "null pointer");
    return hip_check(kiln::launch_add_gated(x, y, gate, rows, dim, (hipStream_t)stream), "add_gated launch");
}

static int linear16_impl(const char* fn, void* y, int ldy, const uint16_t* x16, int T, const uint16_t* w16, int rows,
                         int cols, int epi, const float* gate, float beta, const uint16_t* a2, const uint16_t* w2, int k2,
                         bool wprep, kiln_stream_t stream) {
    if (epi < KILN_EPI_F32 || epi > KILN_EPI_RESID) return fail(KILN_EINVAL, "%s: epilogue %d", fn, epi);
    if (T < 0 || rows <= 0 || cols <= 0 || k2 < 0)
        return fail(KILN_EINVAL, "%s: bad sizes T=%d rows=%d cols=%d k2=%d", fn, T, rows, cols, k2);
    if (rows % 128 || cols % 32 || k2 % 32)
        return fail(KILN_EUNSUPPORTED, "%s: needs rows %% 128 == 0, cols %% 32 == 0, k2 %% 32 == 0 (rows=%d cols=%d k2=%d)",
                    fn, rows, cols, k2);
    if (ldy < rows) return fail(KILN_EINVAL, "%s: ldy=%d < rows=%d", fn, ldy, rows);
    if (T == 0) return KILN_OK;
    if (!y || !x16 || !w16 || (k2 && (!a2 || !w2))) return fail(KILN_EINVAL, "%s: null pointer", fn);
    if (!aligned16(x16) || !aligned16(w16) || (k2 && (!aligned16(a2) || !aligned16(w2))))
        return fail(KILN_EUNSUPPORTED, "%s: operands must be 16-byte aligned", fn);
    const size_t esz = (epi == KILN_EPI_F32 || epi == KILN_EPI_RESID) ? 4 : 2;
    if (ldy % 2 || (size_t)y % (2 * esz)) return fail(KILN_EUNSUPPORTED, "%s: y rows must hold element pairs", fn);
    kiln::GemmLaunch g;
    g.a = x16;
    g.w = w16;
    g.K = cols;
    g.a2 = a2;
    g.w2 = w2;
    g.K2 = k2;
    g.c = y;
    g.ldc = ldy;
    g.gate = gate;
    g.beta = beta;
    g.M = T;
    g.N = rows;
    g.epi = epi;
    g.wprep = wprep;
    return hip_check(kiln::launch_gemm16(g, (hipStream_t)stream), "linear16 launch");
}

int kiln_linear16(void* y, int ldy, const uint16_t* x16, int T, const uint16_t* w16, int rows, int cols, int epi,
                  const float* gate, float beta, const uint16_t* a2, const uint16_t* w2, int k2, kiln_stream_t stream) {
    kiln::prof::Scope prof_("gemm_tc16", (hipStream_t)stream);
    return linear16_impl("linear16", y, ldy, x16, T, w16, rows, cols, epi, gate, beta, a2, w2, k2, false, stream);
}

int kiln_linear16_prepped(void* y, int ldy, const uint16_t* x16, int T, const uint16_t* wp, int rows, int cols,
                          int epi, const float* gate, float beta, const uint16_t* a2, const uint16_t* w2, int k2,
                          kiln_stream_t stream) {
    kiln::prof::Scope prof_("gemm_tc16", (hipStream_t)stream);
    return linear16_impl("linear16_prepped", y, ldy, x16, T, wp, rows, cols, epi, gate, beta, a2, w2, k2, true, stream);
}

size_t kiln_linear16_prepped_weight_bytes(int rows, int cols) {
    if (rows <= 0 || cols <= 0) return 0;
    return kiln::gemm16_prepped_bytes(rows, cols);
}

int kiln_linear16_prepare_weight(uint16_t* wp, const uint16_t* w, int rows, int cols, int src_bf16,
                                 kiln_stream_t stream) {
    kiln::prof::Scope prof_("w->f16", (hipStream_t)stream);
    if (rows <= 0 || cols <= 0) return fail(KILN_EINVAL, "linear16_prepare_weight: bad sizes rows=%d cols=%d", rows, cols);
    if (rows % 128 || cols % 32)
        return fail(KILN_EUNSUPPORTED, "linear16_prepare_weight: needs rows %% 128 == 0, cols %% 32 == 0 (rows=%d cols=%d)",
                    rows, cols);
    if (!wp || !w) return fail(KILN_EINVAL, "linear16_prepare_weight: null pointer");
    if (!aligned16(wp) || !aligned16(w)) return fail(KILN_EUNSUPPORTED, "linear16_prepare_weight: 16-byte alignment");
    const size_t nb = kiln::gemm16_prepped_bytes(rows, cols);
    if ((const char*)wp < (const char*)w + (size_t)rows * cols * 2 && (const char*)w < (const char*)wp + nb)
        return fail(KILN_EINVAL, "linear16_prepare_weight: wp overlaps w");
    return hip_check(kiln::launch_gemm_wprep(wp, w, rows, cols, src_bf16 != 0, (hipStream_t)stream),
                     "linear16_prepare_weight launch");
}

int kiln_matvec_bf16(float* y, const uint16_t* w_bf16, const float* x, const float* add, int rows, int cols,
                     kiln_stream_t stream) {
    kiln::prof::Scope prof_("matvec", (hipStream_t)stream);
    if (rows < 0 || cols <= 0) return fail(KILN_EINVAL, "matvec: bad sizes rows=%d cols=%d", rows, cols);
    if (rows && (!y || !w_bf16 || !x)) return fail(KILN_EINVAL, "matvec: null pointer");
    if (!rows) return KILN_OK;
    return hip_check(kiln::launch_matvec_bf16(y, w_bf16, x, add, rows, cols, 1, (hipStream_t)stream), "matvec launch");
}

int kiln_matvec_bf16_grouped(float* y, const uint16_t* w_bf16, const float* x, const float* add, int groups, int rows,
                             int cols, kiln_stream_t stream) {
    kiln::prof::Scope prof_("matvec", (hipStream_t)stream);
    if (groups < 0 || rows < 0 || cols <= 0 || (long)groups * rows > (1L << 30))
        return fail(KILN_EINVAL, "matvec_grouped: bad sizes groups=%d rows=%d cols=%d", groups, rows, cols);
    if (!groups || !rows) return KILN_OK;
    if (!y || !w_bf16 || !x) return fail(KILN_EINVAL, "matvec_grouped: null pointer");
    return hip_check(kiln::launch_matvec_bf16(y, w_bf16, x, add, rows, cols, groups, (hipStream_t)stream),
                     "matvec_grouped launch");
}

int kiln_silu(float* y, const float* x, size_t n, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && (!y || !x)) return fail(KILN_EINVAL, "silu: null pointer");
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_silu(y, x, n, (hipStream_t)stream), "silu launch");
}

int kiln_patchify(float* tok, const float* latent, int Hl, int Wl, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (Hl <= 0 || Wl <= 0 || Hl % 2 || Wl % 2) return fail(KILN_EINVAL, "patchify: Hl=%d Wl=%d (even, > 0)", Hl, Wl);
    if (!tok || !latent) return fail(KILN_EINVAL, "patchify: null pointer");
    return hip_check(kiln::launch_patchify(tok, latent, Hl, Wl, (hipStream_t)stream), "patchify launch");
}

int kiln_unpatchify(float* latent, const float* tok, int ldt, int Hl, int Wl, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (Hl <= 0 || Wl <= 0 || Hl % 2 || Wl % 2 || ldt < 64)
        return fail(KILN_EINVAL, "unpatchify: Hl=%d Wl=%d ldt=%d", Hl, Wl, ldt);
    if (!tok || !latent) return fail(KILN_EINVAL, "unpatchify: null pointer");
    return hip_check(kiln::launch_unpatchify(latent, tok, ldt, Hl, Wl, (hipStream_t)stream), "unpatchify launch");
}

int kiln_linear_f32(float* y, int ldy, const float* x, int ldx, const uint16_t* w_bf16, int T, int rows, int cols,
                    kiln_stream_t stream) {
    kiln::prof::Scope prof_("gemm_fp32", (hipStream_t)stream);
    if (T < 0 || rows <= 0 || cols <= 0 || ldy < rows || ldx < cols)
        return fail(KILN_EINVAL, "linear_f32: bad sizes T=%d rows=%d cols=%d ldy=%d ldx=%d", T, rows, cols, ldy, ldx);
    if (!T) return KILN_OK;
    if (!y || !x || !w_bf16) return fail(KILN_EINVAL, "linear_f32: null pointer");
    return hip_check(kiln::launch_linear_f32(y, ldy, x, ldx, w_bf16, T, rows, cols, (hipStream_t)stream),
                     "linear_f32 launch");
}

int kiln_cfg_combine(float* v, const float* vn, float cfg, size_t n, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && (!v || !vn)) return fail(KILN_EINVAL, "cfg_combine: null pointer");
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_cfg_combine(v, vn, cfg, n, (hipStream_t)stream), "cfg_combine launch");
}

int kiln_pad_circular(float* dst, const float* src, int Hs, int Ws, int Hd, int Wd, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (Hs <= 0 || Ws <= 0 || Hd <= 0 || Wd <= 0) return fail(KILN_EINVAL, "pad_circular: bad sizes");
    if (!dst || !src) return fail(KILN_EINVAL, "pad_circular: null pointer");
    return hip_check(kiln::launch_pad_circular(dst, src, Hs, Ws, Hd, Wd, (hipStream_t)stream), "pad_circular launch");
}

int kiln_crop(float* dst, const float* src, int Hs, int Ws, int Hd, int Wd, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (Hs <= 0 || Ws <= 0 || Hd <= 0 || Wd <= 0 || Hd > Hs || Wd > Ws) return fail(KILN_EINVAL, "crop: bad sizes");
    if (!dst || !src) return fail(KILN_EINVAL, "crop: null pointer");
    return hip_check(kiln::launch_crop(dst, src, Hs, Ws, Hd, Wd, (hipStream_t)stream), "crop launch");
}

int kiln_fill_uniform_bf16(uint16_t* p, size_t n, uint64_t seed, float lo, float hi, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && !p) return fail(KILN_EINVAL, "fill_uniform_bf16: null pointer");
    if (!(lo <= hi)) return fail(KILN_EINVAL, "fill_uniform_bf16: lo > hi");
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_fill_uniform_bf16(p, n, seed, lo, hi, (hipStream_t)stream), "fill_uniform launch");
}

int kiln_sub(float* y, const float* a, const float* b, size_t n, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && (!y || !a || !b)) return fail(KILN_EINVAL, "sub: null pointer");
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_sub(y, a, b, n, (hipStream_t)stream), "sub launch");
}

int kiln_rel_l1(const float* a, const float* b, size_t n, float* acc, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (!acc || (n && (!a || !b))) return fail(KILN_EINVAL, "rel_l1: null pointer");
    return hip_check(kiln::launch_rel_l1(a, b, n, acc, (hipStream_t)stream), "rel_l1 launch");
}

int kiln_torch_randn(float* host_out, uint64_t seed, size_t n) {
    if (!host_out) return fail(KILN_EINVAL, "torch_randn: null pointer");
    if (!kiln::host_torch_randn(host_out, seed, n)) return fail(KILN_EUNSUPPORTED, "torch_randn: n=%zu < 16", n);
    return KILN_OK;
}

int kiln_flow_start(float* x, const float* noise, const float* init, float sigma, size_t n, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && (!x || !noise)) return fail(KILN_EINVAL, "flow_start: null pointer");
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_flow_start(x, noise, init, sigma, n, (hipStream_t)stream), "flow_start launch");
}

int kiln_flow_ersde_step(float* x, const float* den, const float* old, float* oldd, const float* noise, float a,
                         float b, float c2, float inv2, float c3, float inv3, float cn, int stage, size_t n,
                         kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (stage < 1 || stage > 3) return fail(KILN_EINVAL, "flow_ersde_step: stage %d", stage);
    if (n && (!x || !den || (stage >= 2 && (!old || !oldd)))) return fail(KILN_EINVAL, "flow_ersde_step: null pointer");
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_flow_ersde(x, den, old, oldd, noise, a, b, c2, inv2, c3, inv3, cn, stage, n,
                                             (hipStream_t)stream),
                     "flow_ersde launch");
}

int kiln_gelu(float* x, size_t n, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && !x) return fail(KILN_EINVAL, "gelu: null pointer");
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_gelu(x, n, (hipStream_t)stream), "gelu launch");
}

int kiln_flow_inpaint_in(float* xin, const float* x, const float* noise, const float* init, const float* mask,
                         float sigma, int P, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (P < 0 || (P && (!xin || !x || !noise || !init || !mask))) return fail(KILN_EINVAL, "flow_inpaint_in: bad args");
    if (!P) return KILN_OK;
    return hip_check(kiln::launch_flow_inpaint_in(xin, x, noise, init, mask, sigma, P, (hipStream_t)stream),
                     "flow_inpaint_in launch");
}

int kiln_flow_denoised_masked(float* den, const float* xin, const float* v, const float* init, const float* mask,
                              float sigma, int P, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (P < 0 || (P && (!den || !xin || !v || !init || !mask))) return fail(KILN_EINVAL, "flow_denoised_masked: bad args");
    if (!P) return KILN_OK;
    return hip_check(kiln::launch_flow_denoised_masked(den, xin, v, init, mask, sigma, P, (hipStream_t)stream),
                     "flow_denoised_masked launch");
}

int kiln_flow_denoised(float* den, const float* x, const float* v, float sigma, size_t n, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && (!den || !x || !v)) return fail(KILN_EINVAL, "flow_denoised: null pointer");
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_flow_denoised(den, x, v, sigma, n, (hipStream_t)stream), "flow_denoised launch");
}

int kiln_flow_update(float* x, const float* den, const float* old, float a, float b, float c, size_t n,
                     kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && (!x || !den)) return fail(KILN_EINVAL, "flow_update: null pointer");
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_flow_update(x, den, old, a, b, c, n, (hipStream_t)stream), "flow_update launch");
}

int kiln_flow_euler_step(float* x, const float* v, float sigma, float sigma_next, size_t n, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && (!x || !v)) return fail(KILN_EINVAL, "flow_euler_step: null pointer");
    if (!(sigma > 0.f)) return fail(KILN_EINVAL, "flow_euler_step: sigma %g must be > 0", (double)sigma);
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_flow_euler(x, v, sigma, sigma_next, n, (hipStream_t)stream), "flow_euler launch");
}

int kiln_flow_euler_den(float* x, const float* den, float sigma, float sigma_next, size_t n, kiln_stream_t stream) {
    kiln::prof::Scope prof_("eltwise", (hipStream_t)stream);
    if (n && (!x || !den)) return fail(KILN_EINVAL, "flow_euler_den: null pointer");
    if (!(sigma > 0.f)) return fail(KILN_EINVAL, "flow_euler_den: sigma %g must be > 0", (double)sigma);
    if (!n) return KILN_OK;
    return hip_check(kiln::launch_flow_euler_den(x, den, sigma, sigma_next, n, (hipStream_t)stream),
                     "flow_euler_den launch");
}

int kiln_rope_half(float* x, int T, int H, int Dh, const float* cos_t, const float* sin_t, kiln_stream_t stream) {
    kiln::prof::Scope prof_("rope", (hipStream_t)stream);
    if (T < 0 || H <= 0 || Dh <= 0 || Dh % 2) return fail(KILN_EINVAL, "bad sizes");
    if (T && (!x || !cos_t || !sin_t)) return fail(KILN_EINVAL, "null pointer");
    return hip_check(kiln::launch_rope_half(x, T, H, Dh, cos_t, sin_t, (hipStream_t)stream), "rope launch");
}

int kiln_nag_combine(void* a, int lda, const void* an, int ldn, int dtype, int T, int dim, float s, float tau,
                     float alpha, kiln_stream_t stream) {
    kiln::prof::Scope prof_("nag", (hipStream_t)stream);
    if (dtype != KILN_F32 && dtype != KILN_F16) return fail(KILN_EINVAL, "dtype %d", dtype);
    if (T < 0 || dim <= 0) return fail(KILN_EINVAL, "bad sizes");
    if (T && (!a || !an)) return fail(KILN_EINVAL, "null pointer");
    return hip_check(kiln::launch_nag(a, lda, an, ldn, (DT)dtype, T, dim, s, tau, alpha, (hipStream_t)stream),
                     "nag launch");
}

// Cosmos 3D RoPE for one image (engine/src/dit.cu:196-215): 22 temporal (identity at T=1), 21 height and
// 21 width frequencies over the 64 rotated pairs of a 128-dim head; NTK-scaled theta for height/width.
int kiln_cosmos_rope_tables(float* cos_t, float* sin_t, int Hp, int Wp) {
    if (!cos_t || !sin_t || Hp <= 0 || Wp <= 0) return fail(KILN_EINVAL, "bad arguments");
    const int dh = 128 / 6 * 2, dt = 128 - 2 * dh, half = 64;
    const double ntk = pow(4.0, (double)dh / (dh - 2));
    const float theta = (float)(10000.0 * ntk);
    float freq[32];
    for (int j = 0; j < dh / 2; j++) freq[j] = 1.0f / powf(theta, (float)(2 * j) / (float)dh);
    for (int y = 0; y < Hp; y++)
        for (int x = 0; x < Wp; x++) {
            float* c = cos_t + ((size_t)y * Wp + x) * half;
            float* s = sin_t + ((size_t)y * Wp + x) * half;
            for (int i = 0; i < dt / 2; i++) { c[i] = 1.f; s[i] = 0.f; }
            for (int j = 0; j < dh / 2; j++) {
                const float ah = (float)y * freq[j], aw = (float)x * freq[j];
                c[dt / 2 + j] = cosf(ah);
                s[dt / 2 + j] = sinf(ah);
                c[dt / 2 + dh / 2 + j] = cosf(aw);
                s[dt / 2 + dh / 2 + j] = sinf(aw);
            }
        }
    return KILN_OK;
}

}  // extern "C"
