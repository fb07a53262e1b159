// kiln_attn_fwd_f16out_noalloc: attention16 (kiln_attn_fwd_f16out) for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Its scratch (the prepared
// K/V tiles and key-split partials) is a file-scope device array of a fixed size instead of a workspace.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/kiln_attn.h"
#include "capi_util.hpp"

using namespace kiln::capi;
using kiln::DT;

namespace {

// The scratch: each device holds its own copy at its own address. Host code uses only the per-device address
// that hipGetSymbolAddress returns; the array's name in host code is a host-side stand-in, not a device address.
constexpr size_t SCRATCH_BYTES = (size_t)64 << 20;
__device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* g_scratch[MAX_DEVICES] = {};

// the current device's scratch address, resolved on its first call on that device
int scratch_of_current_device(void** out) {
    int dev = 0;
    if (int r = current_device(&dev)) return r;
    if (dev < 0 || dev >= MAX_DEVICES) return fail(KILN_EUNSUPPORTED, "device %d beyond %d", dev, MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_check(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(KILN_EHIP, "hipGetSymbolAddress(scratch) returned null");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return KILN_OK;
}

}  // namespace

extern "C" {

size_t kiln_attn_noalloc_scratch_bytes(void) { return SCRATCH_BYTES; }

int kiln_attn_fwd_f16out_noalloc(uint16_t* out, int ldo, const float* q, int ldq, const float* k, int ldk,
                                 const float* v, int ldv, int Tq, int Tk, int H, int Dh, int npad,
                                 kiln_stream_t stream) {
    int r = check_common(Tq, Tk, H, npad);
    if (r) return r;
    if (Dh != 128) return fail(KILN_EUNSUPPORTED, "attention16: unsupported head size %d (needs 128)", Dh);
    if (Tq == 0) return KILN_OK;
    if (!out || !q || (Tk > 0 && (!k || !v))) return fail(KILN_EINVAL, "null pointer");
    if (!rows_ok(q, ldq, DT::F32) || !rows_ok(k, ldk, DT::F32) || !rows_ok(v, ldv, DT::F32) || ldo % 2)
        return fail(KILN_EUNSUPPORTED, "attention16: unsupported row stride or alignment");
    if (Tk == 0) return zero_rows(out, ldo, 2, Tq, H, Dh, (hipStream_t)stream);
    const size_t need = kiln_kv_prepped_bytes(Tk, H);
    if (need > SCRATCH_BYTES)
        return fail(KILN_ENOMEM, "attention16 (no-alloc): the prepared K/V of Tk=%d x H=%d take %zu bytes, above the "
                    "%zu-byte scratch", Tk, H, need, SCRATCH_BYTES);
    void* ws = nullptr;
    if ((r = scratch_of_current_device(&ws))) return r;
    // Every scratch byte the kernels read is written earlier in the same call (prepared K/V, then the partials
    // of a key split), so nothing is cleared. The key split is taken only when its partials fit behind the K/V.
    return flash_self(out, DT::F16, ldo, 0, q, ldq, 0, k, ldk, 0, v, ldv, 0, DT::F32, 1, Tq, Tk, H, npad, nullptr,
                      nullptr, 0.f, nullptr, nullptr, ws, SCRATCH_BYTES, (hipStream_t)stream);
}

}  // extern "C"
