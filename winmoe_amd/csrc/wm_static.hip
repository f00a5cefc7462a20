// wm_static.hip -- the decode step for callers that cannot allocate device
// memory (code under HIP graph capture, serving loops that forbid hipMalloc):
// wm_moe_decode_noalloc runs wm_moe_decode with its workspace in a fixed,
// library-owned device array instead of a caller buffer.  Host code plus the
// array itself.
//
// The array is a file-scope __device__ object: every device the library runs
// on holds its own copy until the process ends.  Host code never uses the
// array's name as an address (on the host it names a stand-in, not device
// memory); the device address comes from hipGetSymbolAddress, once per
// device, with that device current, and is kept per device.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "../../include/winmoe_hip.h"
#include "wm_host.h"
#include "wm_launch.h"

using namespace wm;

// The workspace of every supported decode layer without WM_FLAG_TIMELINE fits:
// E <= 1024, K <= 16 and H, I, inter_shared <= 4096 need at most 2,685,440 B
// (about 2.6 MB, of the 3 MiB here).  A layer whose workspace is larger (a
// shared expert wider than 4096, or WM_FLAG_TIMELINE: 3,734,016 B at those
// sizes) is refused with WM_EINVAL.
static __device__ __align__(256) uint8_t scratch[WM_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};        // device address of `scratch` on each device (null: not set up)

// The current device's address of the array, looked up on its first use.
int scratch_on_current_device(void** out) {
    int dev = 0;
    WM_FAIL_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) {
        fprintf(stderr, "winmoe_hip: device %d is past the %d devices wm_moe_decode_noalloc serves\n", dev,
                kMaxDevices);
        return WM_EINVAL;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "winmoe_hip: hipGetSymbolAddress(scratch) failed on device %d: %s\n", dev,
                    hipGetErrorString(e));
            return WM_ERR;
        }
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return WM_OK;
}
}  // namespace

extern "C" int64_t wm_noalloc_scratch_bytes(void) { return WM_NOALLOC_SCRATCH_BYTES; }

extern "C" int wm_noalloc_init(void) {
    if (wm_init() != WM_OK) return WM_ERR;
    void* p = nullptr;
    if (int rc = scratch_on_current_device(&p)) return rc;
    return persist_order_prepare();
}

extern "C" int wm_moe_decode_noalloc(const wm_layer_desc* d, const float* x, float* out, int32_t* ids_out,
                                     float* w_out, void* stream) {
    WM_CHECK_ARG(d && x && out);
    const int64_t need = wm_workspace_size(d, 1);
    WM_CHECK_ARG(need > 0);
    if (need > WM_NOALLOC_SCRATCH_BYTES) {
        fprintf(stderr, "winmoe_hip: this layer's decode workspace is %lld bytes, more than the %d bytes of the "
                        "fixed scratch array (use wm_moe_decode with a caller workspace)\n",
                (long long)need, WM_NOALLOC_SCRATCH_BYTES);
        return WM_EINVAL;
    }
    if (int rc = wm_noalloc_init()) return rc;
    void* ws = nullptr;
    if (int rc = scratch_on_current_device(&ws)) return rc;
    hipStream_t s = (hipStream_t)stream;
    // the previous call may have left another layer's layout here: start from
    // zero (status, tags, epoch, counters), with a kernel rather than a memset
    WM_FAIL_HIP(launch_fill_i32((int32_t*)ws, 0, need / 4, s));
    if (int rc = wm_moe_decode(d, x, out, ws, need, 1, 0, stream)) return rc;
    if (ids_out || w_out) {
        int64_t ids_off = 0, w_off = 0;
        if (int rc = wm_workspace_trace(d, 1, &ids_off, &w_off, nullptr)) return rc;
        const size_t n = (size_t)d->top_k * 4;
        if (ids_out) WM_FAIL_HIP(hipMemcpyAsync(ids_out, (uint8_t*)ws + ids_off, n, hipMemcpyDeviceToDevice, s));
        if (w_out) WM_FAIL_HIP(hipMemcpyAsync(w_out, (uint8_t*)ws + w_off, n, hipMemcpyDeviceToDevice, s));
    }
    return WM_OK;
}

extern "C" int wm_noalloc_status(int32_t* status_out) {
    WM_CHECK_ARG(status_out);
    void* ws = nullptr;
    if (int rc = scratch_on_current_device(&ws)) return rc;
    return wm_workspace_status(ws, 4, status_out);
}
