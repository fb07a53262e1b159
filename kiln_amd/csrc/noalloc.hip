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
std::mutex g_mu;  // held for a whole call: calls from several host threads reach the device one after another

// Per device: the scratch address, and the stream and completion event of the last eager call. A call on another
// stream than the last one first makes its stream wait for that event, so two streams never use the scratch at
// once (calls on one stream are ordered by the stream itself and pay nothing).
struct DeviceState {
    void* scratch = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool pending = false;  // `done` was recorded after the last eager call
};
DeviceState g_dev[MAX_DEVICES];

// the current device's state, its scratch address and event set up on its first call on that device
int state_of_current_device(DeviceState** out) {
    int dev = 0;
    if (int r = current_device(&dev)) return r;
    if (dev < 0 || dev >= MAX_DEVICES) return fail(KILN_EUNSUPPORTED, "device %d beyond %d", dev, MAX_DEVICES);
    DeviceState& st = g_dev[dev];
    if (!st.scratch) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_check(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(KILN_EHIP, "hipGetSymbolAddress(scratch) returned null");
        e = hipEventCreateWithFlags(&st.done, hipEventDisableTiming);
        if (e != hipSuccess) return hip_check(e, "hipEventCreateWithFlags");
        st.scratch = p;
    }
    *out = &st;
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
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState* st = nullptr;
    if ((r = state_of_current_device(&st))) return r;
    const hipStream_t s = (hipStream_t)stream;
    // Under graph capture the ordering against other streams is the caller's (a captured wait on an event of an
    // eager call would tie the graph to that call): the guard covers eager calls only.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipError_t e = hipStreamIsCapturing(s, &cs); e != hipSuccess) return hip_check(e, "hipStreamIsCapturing");
    const bool eager = cs == hipStreamCaptureStatusNone;
    if (eager && st->pending && st->last != s) {
        if (hipError_t e = hipStreamWaitEvent(s, st->done, 0); e != hipSuccess) return hip_check(e, "hipStreamWaitEvent");
    }
    // Every scratch byte the kernels read is written earlier in the same call (prepared K/V, then the partials
    // of a key split), so nothing is cleared. The key split is taken only when its partials fit behind the K/V.
    r = flash_self(out, DT::F16, ldo, 0, q, ldq, 0, k, ldk, 0, v, ldv, 0, DT::F32, 1, Tq, Tk, H, npad, nullptr, nullptr,
                   0.f, nullptr, nullptr, st->scratch, SCRATCH_BYTES, s);
    if (r || !eager) return r;
    if (hipError_t e = hipEventRecord(st->done, s); e != hipSuccess) return hip_check(e, "hipEventRecord");
    st->last = s;
    st->pending = true;
    return KILN_OK;
}

}  // extern "C"
