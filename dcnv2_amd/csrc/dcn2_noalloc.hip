// dcn2_forward_noalloc: the forward of dcn2_forward with its workspace (the
// channels-last input copy, the packed weight and the chunk table) in a
// static device array instead of a caller-provided buffer, for callers that
// cannot allocate device memory.
//
// The array's name is only a host-side handle: its device address is looked
// up with hipGetSymbolAddress once per device (each GPU holds its own copy at
// its own address) and that address is what the kernels receive.  The pack
// kernel writes every byte of the workspace it uses (padding channels and
// rows included), so nothing needs clearing between calls.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/dcnv2_amd.h"
#include "dcn2_kernels.h"

namespace dcn2 {
namespace {

constexpr size_t kScratchBytes = DCN2_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device

// Device address of `scratch` on the current device (looked up on the first
// call there).
int scratch_on_current_device(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return fail(DCN2_ELAUNCH, "dcn2_forward_noalloc: hipGetDevice failed: %s",
                    hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(DCN2_ELAUNCH, "dcn2_forward_noalloc: device %d beyond the %d supported", dev,
                    kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
            return fail(DCN2_ELAUNCH, "dcn2_forward_noalloc: hipGetSymbolAddress failed: %s",
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return DCN2_OK;
}

}  // namespace
}  // namespace dcn2

extern "C" int dcn2_forward_noalloc(const dcn2_desc *d, const void *input, const void *weight,
                                    const void *mask, const void *offset, const void *bias,
                                    void *output, void *stream) {
    using namespace dcn2;
    Geo g;
    int rc = make_geo(d, g);
    if (rc) return rc;
    const size_t need = fwd_workspace(g).total;
    if (need > kScratchBytes)
        return fail(DCN2_EWORKSPACE,
                    "dcn2_forward_noalloc: this problem needs %zu bytes of workspace, more than "
                    "the %zu bytes of the static scratch array; use dcn2_forward with a workspace",
                    need, kScratchBytes);
    void *ws = nullptr;
    if ((rc = scratch_on_current_device(&ws))) return rc;
    return forward_impl(g, input, weight, mask, offset, bias, output, ws, kScratchBytes, stream);
}
