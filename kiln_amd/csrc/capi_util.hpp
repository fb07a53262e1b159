// Helpers shared by the C-ABI source files of libkiln_attn.so (argument checks, the thread's error message,
// the fused self-attention launch). Not part of the public interface.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "internal.hpp"

namespace kiln::capi {

// sets the calling thread's kiln_attn_last_error() message and returns code
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// KILN_OK, or KILN_EHIP with the runtime's message
int hip_check(hipError_t e, const char* what);
int current_device(int* dev);
// 16-byte aligned rows of 8-element chunks
bool rows_ok(const void* p, int ld, DT dt);
// sizes of an attention call (Tq, Tk >= 0, H > 0, npad >= 0, some key)
int check_common(int Tq, int Tk, int H, int npad);
// zeros Tq rows of H * Dh elements of esz bytes (a call with only padding keys)
int zero_rows(void* out, int ldo, size_t esz, int Tq, int H, int Dh, hipStream_t s);
// K/V prepare pass + attention over B batch items; ws == nullptr takes the device's workspace
int flash_self(void* out, DT od, int ldo, long long bso, const void* q, int ldq, long long bsq, const void* k, int ldk,
               long long bsk, const void* v, int ldv, long long bsv, DT in, int B, int Tq, int Tk, int H, int npad,
               const uint16_t* qw, const uint16_t* kw, float eps, const float* rc, const float* rs, void* ws,
               size_t ws_bytes, hipStream_t stream);

}  // namespace kiln::capi

namespace kiln::prof {
// A timed scope of one category on a stream (kiln_prof_enable / kiln_prof_report).
class Scope {
   public:
    Scope(const char* name, hipStream_t s);
    ~Scope();
    Scope(const Scope&) = delete;
    Scope& operator=(const Scope&) = delete;

   private:
    int slot_ = -1;          // the event pair recording this scope, or -1
    unsigned gen_ = 0;       // the profile generation the slot belongs to (kiln_prof_enable starts a new one)
    bool counted_ = false;   // this scope raised the thread's nesting depth and lowers it again
    hipStream_t s_ = nullptr;
};
}  // namespace kiln::prof
