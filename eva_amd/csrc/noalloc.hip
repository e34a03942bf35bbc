// evamx_moe_forward_static: the MoE forward of evamx_moe_forward on a fixed device scratch
// array instead of a caller's workspace, for callers that cannot allocate device memory (code
// under hipGraph capture, serving loops that forbid allocation). No counterpart in the
// reference, whose runners own their scratch tensors.
//
// The array is a file-scope __device__ object: every GPU the library runs on holds its own copy,
// at its own address, until the process ends. In host code its name stands for a host-side
// shadow, not for device memory, so the device address is looked up with hipGetSymbolAddress
// (with that device current) on the entry point's first call on each device, kept per device,
// and only that address is ever handed to kernels.
//
// Every call on one GPU uses that GPU's one array: calls that overlap on one GPU (two streams,
// two threads) race and corrupt each other's results. The array keeps the last call's contents;
// the forward writes every region it later reads (as with a fresh caller workspace), and only
// the sticky flag word must start at zero, which the first call on a device does.
#include <mutex>

#include "evamx_internal.hpp"

namespace evamx {

constexpr size_t STATIC_SCRATCH_BYTES = (size_t)64 << 20;   // DSv3 decode needs 44-53 MiB (1-32 rows)
constexpr int MAX_DEVICES = 64;

static __device__ __align__(256) unsigned char scratch[STATIC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES];

// The current device's scratch address; on the first call on a device also zeroes the flag
// word (offset 0 of every workspace layout) with a fill kernel on `stream`.
static int device_scratch(void** out, hipStream_t stream)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        set_error("evamx_moe_forward_static: no current device (or device index %d >= %d)", dev, MAX_DEVICES);
        return EVAMX_EINVAL;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_error("evamx_moe_forward_static: hipGetSymbolAddress of the scratch array failed on device %d: %s", dev,
                      hipGetErrorString(e));
            return EVAMX_ELAUNCH;
        }
        launch_fill_i32((int*)ptr, 64, 0, stream);
        const int rc = launched("evamx_moe_forward_static (scratch set-up)");
        if (rc != EVAMX_OK) return rc;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return EVAMX_OK;
}

}  // namespace evamx

using namespace evamx;

extern "C" int evamx_moe_forward_static(const evamx_moe_args* a, evamx_stream_t stream)
{
    set_error("%s", "");
    if (!a) {
        set_error("evamx_moe_forward_static: null args");
        return EVAMX_EINVAL;
    }
    if (a->workspace || a->workspace_bytes) {
        set_error("evamx_moe_forward_static: pass no workspace (this entry point uses the library's fixed scratch)");
        return EVAMX_EINVAL;
    }
    const size_t need = moe_workspace_bytes_of(&a->shape);
    if (need == 0) return EVAMX_EINVAL;           // message set by the shape check
    if (need > STATIC_SCRATCH_BYTES) {
        set_error("evamx_moe_forward_static: this shape needs %zu bytes of scratch, the fixed scratch holds %zu "
                  "(use evamx_moe_forward with a workspace)", need, STATIC_SCRATCH_BYTES);
        return EVAMX_ENOSPACE;
    }
    void* ws = nullptr;
    const int rc = device_scratch(&ws, (hipStream_t)stream);
    if (rc != EVAMX_OK) return rc;
    return moe_forward_ws(a, ws, STATIC_SCRATCH_BYTES, (hipStream_t)stream, "evamx_moe_forward_static", false);
}
