// qm_noalloc.hip -- the device scratch of qm_gqa_decode_noalloc.
//
// `scratch` is a file-scope device array of QM_NOALLOC_SCRATCH_BYTES: every
// GPU this library runs on holds its own copy, at its own address, until the
// process ends.  In host code the name `scratch` is only a host-side stand-in
// for the device symbol (a kernel given it would fault); qm_noalloc_scratch()
// resolves each device's address once, with that device current, and host
// code passes that address to the kernels.  This file is compiled with hipcc
// into libqora_mixer.so itself (not into a code object), so the runtime
// places the array on a device when the library's fat binary is first used
// there; nothing here allocates.
#include <hip/hip_runtime.h>

#include <mutex>

#include "qm_noalloc.h"

static __device__ __align__(256) unsigned char scratch[QM_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_mu;
void* g_ptr[QM_NOALLOC_MAX_DEVICES] = {};
const void* g_owner[QM_NOALLOC_MAX_DEVICES] = {};
}  // namespace

extern "C" int qm_noalloc_claim(int device, const void* owner) {
    if (device < 0 || device >= QM_NOALLOC_MAX_DEVICES || !owner) return 1;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_owner[device] && g_owner[device] != owner) return 1;
    g_owner[device] = owner;
    return 0;
}

extern "C" void qm_noalloc_release(int device, const void* owner) {
    if (device < 0 || device >= QM_NOALLOC_MAX_DEVICES) return;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_owner[device] == owner) g_owner[device] = nullptr;
}

extern "C" int qm_noalloc_scratch(int device, void** ptr) {
    if (!ptr || device < 0 || device >= QM_NOALLOC_MAX_DEVICES) return static_cast<int>(hipErrorInvalidValue);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[device]) {
        int cur = 0;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return static_cast<int>(e);
        if (cur != device && (e = hipSetDevice(device)) != hipSuccess) return static_cast<int>(e);
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != device) (void)hipSetDevice(cur);
        if (e != hipSuccess) return static_cast<int>(e);
        if (!p) return static_cast<int>(hipErrorInvalidSymbol);
        g_ptr[device] = p;
    }
    *ptr = g_ptr[device];
    return static_cast<int>(hipSuccess);
}
