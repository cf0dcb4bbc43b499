// fa_scratch.hip -- the device-global scratch array behind the
// allocation-free entry point (fa_device_ex_noalloc in include/fa_hip.h).
//
// The split-KV decode and the prefill key split write per-split partials
// (O, m, l) that fa_merge combines.  The ordinary entry points keep those
// partials in a per-stream workspace they allocate with hipMalloc on first
// use; callers that cannot allocate (code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc) use this fixed array instead.
//
// `scratch` lives in the code object embedded in libfa_hip.so, so every GPU
// the library runs on holds its own copy, at its own address, until the
// process ends.  In host code the name `scratch` is only a host-side handle:
// its device address comes from hipGetSymbolAddress, taken once per device
// with that device current, and every kernel argument uses that address.
//
// Compiled by hipcc (-c, gfx950) and linked into libfa_hip.so with
// fa_host.cpp.

#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/fa_hip.h"
#include "fa_scratch.h"

static __device__ __align__(256) unsigned char scratch[FA_SCRATCH_BYTES];

namespace {

struct ScratchSlot {
    std::once_flag once;
    void* ptr = nullptr;   // device address of `scratch` on this device
    int status = FA_ERR_SCRATCH;
};

ScratchSlot g_slot[FA_SCRATCH_MAX_DEVICES];

}  // namespace

int fa_scratch_init(int dev) {
    if (dev < 0 || dev >= FA_SCRATCH_MAX_DEVICES) return FA_ERR_NO_DEVICE;
    ScratchSlot& s = g_slot[dev];
    std::call_once(s.once, [&] {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            s.status = FA_ERR_SCRATCH;
            return;
        }
        s.ptr = p;
        s.status = FA_OK;
    });
    return s.status;
}

void* fa_scratch_ptr(int dev) {
    if (dev < 0 || dev >= FA_SCRATCH_MAX_DEVICES) return nullptr;
    return g_slot[dev].ptr;
}
