// fa_scratch.h -- internal interface to the device-global scratch array
// defined in fa_scratch.hip (used by fa_device_ex_noalloc).
#ifndef FA_SCRATCH_H
#define FA_SCRATCH_H

#include <stddef.h>

// Bytes of the per-device scratch array: the largest split workspace
// (partials of the split-KV decode / prefill key split) an allocation-free
// call may use.  The largest benchmark shape that splits needs 48 MiB
// (16 heads of 1000 x 1000 at d_head 256, causal, prefill key split).
#define FA_SCRATCH_BYTES (size_t(64) << 20)
#define FA_SCRATCH_MAX_DEVICES 64

// With device `dev` current: look up the device address of the scratch
// array (once per device; later calls return the first result).  FA_OK or
// FA_ERR_SCRATCH.
__attribute__((visibility("hidden"))) int fa_scratch_init(int dev);
// The address fa_scratch_init found for `dev`, or nullptr.
__attribute__((visibility("hidden"))) void* fa_scratch_ptr(int dev);

#endif
