// qm_noalloc.h -- the fixed device scratch behind the allocation-free entry
// point (qm_gqa_decode_noalloc), shared between qm_noalloc.hip (which owns
// the device array) and qm_runtime.cpp (which launches into it).
#pragma once

#include <stddef.h>

// Bytes of the per-device scratch array: the split-K partials of one GQA
// decode launch, 4 query heads x 260 floats per (sequence, kv head, split),
// so at most 8065 such triples per call.
#define QM_NOALLOC_SCRATCH_BYTES (32u << 20)
#define QM_NOALLOC_MAX_DEVICES 64

#ifdef __cplusplus
extern "C" {
#endif
// The device address of `device`'s copy of the scratch array, resolved once
// per device with that device current and cached; returns a hipError_t.
__attribute__((visibility("hidden"))) int qm_noalloc_scratch(int device, void** ptr);
// Records `owner` (a context) as the one user of `device`'s scratch: 0 if it
// is free or already owned by `owner`, nonzero if another context holds it.
__attribute__((visibility("hidden"))) int qm_noalloc_claim(int device, const void* owner);
// Releases `device`'s scratch if `owner` holds it.
__attribute__((visibility("hidden"))) void qm_noalloc_release(int device, const void* owner);
#ifdef __cplusplus
}
#endif
