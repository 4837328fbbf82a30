// Workspace of the entry points that allocate nothing (mvlm_gemm_packed_ex_noalloc).
//
// Callers under HIP graph capture, in tight serving loops or in harnesses that
// forbid device allocation cannot let a call grow the device workspace with
// hipMalloc.  For them the library reserves one fixed device array per GPU,
// `scratch` below, sized MVLM_NOALLOC_SCRATCH_BYTES, which lives until the
// process ends.  Host code never passes the array's name to a kernel (on the
// host it is only a stand-in symbol): its device address is looked up once per
// device handle at mvlm_device_create, with that device current, and kept in
// mvlm_device::noalloc_scratch; kernels receive that pointer.
//
// Every call on one GPU shares the array, and the array keeps whatever the
// last call left in it.  Calls through one device handle run in order on its
// stream; calls that overlap on one GPU (two handles, two streams) race.
#include "common.h"

namespace mvlm {

static __device__ __align__(256) unsigned char scratch[MVLM_NOALLOC_SCRATCH_BYTES];

int resolve_noalloc_scratch(mvlm_device* dev) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return set_error(MVLM_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev->ordinal,
                         hipGetErrorString(e));
    }
    dev->noalloc_scratch = p;
    return MVLM_OK;
}

}  // namespace mvlm
