// noalloc.hip - spinn_hip_conv_noalloc: the convolution entry point with its
// scratch (split-K partial sums, Winograd V and M) in one fixed device array
// instead of a caller-provided workspace, for callers that cannot allocate
// device memory: code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc.
//
// The array lives in this translation unit's code object, so a device holds it
// (SPINN_HIP_NOALLOC_SCRATCH_BYTES) from the first resolution of its address on
// that device until the process ends. Host code never passes the array's name
// to a kernel - on the host that is only a stand-in symbol - but the device
// address hipGetSymbolAddress returns, resolved once per device.
#include "spinn_hip_internal.h"
#include <mutex>

namespace spinn {

static __device__ __align__(256) unsigned char scratch[SPINN_HIP_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
struct ScratchSlot {
    std::once_flag once;
    void *ptr = nullptr;
    int rc = SPINN_HIP_OK;
};
ScratchSlot g_scratch[kMaxDevices];
} // namespace

// Device address of `scratch` on `device`, which must be the current device;
// resolved on the first call for that device, cached afterwards.
int noalloc_scratch(int device, void **ptr) {
    if (device < 0 || device >= kMaxDevices) return SPINN_HIP_EUNSUPPORTED;
    ScratchSlot &s = g_scratch[device];
    std::call_once(s.once, [&s]() {
        void *p = nullptr;
        s.rc = hip_code(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (s.rc == SPINN_HIP_OK) s.ptr = p;
    });
    *ptr = s.ptr;
    return s.rc;
}

} // namespace spinn

using namespace spinn;

extern "C" int spinn_hip_conv_noalloc(const SpinnHipConvDesc *d, const float *x, const float *w,
                                      const float *packed_w, const float *bias, const float *residual, float *y,
                                      void *stream) {
    // The descriptor is checked by spinn_hip_conv; an invalid one needs no scratch.
    const size_t need = spinn_hip_conv_workspace_size(d);
    if (need > SPINN_HIP_NOALLOC_SCRATCH_BYTES) return SPINN_HIP_EWORKSPACE;
    void *ws = nullptr;
    if (need > 0) {
        int dev = 0;
        int rc = hip_code(hipGetDevice(&dev));
        if (rc) return rc;
        rc = noalloc_scratch(dev, &ws);
        if (rc) return rc;
    }
    return spinn_hip_conv(d, x, w, packed_w, bias, residual, y, ws, need, stream);
}
