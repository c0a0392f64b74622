// kda_noalloc.hip -- kda_fwd_noalloc: kda_fwd's kernels on a file-scope device
// scratch array instead of a caller workspace.  It has no counterpart in the
// reference; it serves callers that cannot allocate device memory.
//
// The array lives in this translation unit only, so it belongs to this file's
// code object and nothing else in the library refers to it.  Host code never
// uses the name `scratch` as an address (on the host it is a stand-in, not
// device memory): the device address comes from hipGetSymbolAddress, once per
// device, with that device current.
#include <mutex>

#include "kda_hip.h"
#include "kda_internal.h"

namespace {

static __device__ __align__(256) unsigned char scratch[KDA_NOALLOC_MAX_WORKSPACE];

constexpr int kMaxDevices = 64;

// Device address of `scratch` on device `dev`, looked up once per device with
// `dev` current (the caller's current device is restored); nullptr with the
// HIP error in *err if the lookup failed.
void* scratch_ptr(int dev, hipError_t* err) {
    static std::once_flag once[kMaxDevices];
    static void* ptr[kMaxDevices];
    static hipError_t status[kMaxDevices];
    std::call_once(once[dev], [dev] {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        void* p = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur >= 0 && cur != dev) (void)hipSetDevice(cur);
        status[dev] = e;
        ptr[dev] = (e == hipSuccess) ? p : nullptr;
    });
    *err = status[dev];
    return ptr[dev];
}

// Whether p is device (or managed) memory that lives on device `dev`.  A
// pointer the runtime does not know (plain host memory) is "no"; the error
// such a query may record is cleared, so that the next launch check does not
// report it.
bool on_device(const void* p, int dev) {
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return (at.type == hipMemoryTypeDevice || at.type == hipMemoryTypeManaged) && at.device == dev;
}

}  // namespace

extern "C" int kda_fwd_noalloc(const void* q, const void* k, const void* v, const void* g, const void* beta,
                               const float* s0, void* o, float* s_final, int B, int T, int H, int D, int chunk,
                               int dtype, int g_dtype, void* stream) {
    int rc = KDA_OK;
    const size_t need = kda::api_fwd_workspace_bytes(B, T, H, D, chunk, dtype, g_dtype, &rc);
    if (rc != KDA_OK) return rc;
    if (need > KDA_NOALLOC_MAX_WORKSPACE)
        return kda::api_fail(KDA_E_WORKSPACE,
                             "kda_fwd_noalloc: B=%d T=%d H=%d D=%d needs %zu bytes of workspace, above the %zu bytes "
                             "of its static scratch; call kda_fwd with a caller workspace",
                             B, T, H, D, need, (size_t)KDA_NOALLOC_MAX_WORKSPACE);
    // the GPU whose scratch the kernels use is the stream's (the current
    // device for the NULL stream), and every buffer must live on it
    int dev = -1;
    hipError_t e = stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return kda::api_hip_fail(e, "kda_fwd_noalloc: device of the stream");
    if (dev < 0 || dev >= kMaxDevices)
        return kda::api_fail(KDA_E_UNSUPPORTED, "kda_fwd_noalloc: device %d >= %d", dev, kMaxDevices);
    if ((size_t)B * T * H > 0) {
        const void* bufs[] = {q, k, v, g, beta, o};
        const char* names[] = {"q", "k", "v", "g", "beta", "o"};
        for (int i = 0; i < 6; ++i)
            if (bufs[i] && !on_device(bufs[i], dev))
                return kda::api_fail(KDA_E_INVALID,
                                     "kda_fwd_noalloc: %s is not device memory of device %d, the stream's device",
                                     names[i], dev);
    }
    if (s0 && !on_device(s0, dev))
        return kda::api_fail(KDA_E_INVALID, "kda_fwd_noalloc: s0 is not device memory of device %d", dev);
    if (s_final && !on_device(s_final, dev))
        return kda::api_fail(KDA_E_INVALID, "kda_fwd_noalloc: s_final is not device memory of device %d", dev);
    void* ws = scratch_ptr(dev, &e);
    if (!ws) return kda::api_hip_fail(e, "kda_fwd_noalloc: hipGetSymbolAddress(scratch)");
    return kda::api_fwd_on_workspace(q, k, v, g, beta, s0, o, s_final, B, T, H, D, chunk, dtype, g_dtype, ws,
                                     KDA_NOALLOC_MAX_WORKSPACE, stream);
}
