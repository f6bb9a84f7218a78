// qfm_noalloc.hip -- the fused forward for callers that cannot allocate.
//
// qfm_moe_forward_noalloc is qfm_moe_forward (same kernels, same arithmetic,
// same results) whose workspace is a file-scope device array instead of a
// caller buffer: for code under stream capture, tight serving loops and
// harnesses that forbid hipMalloc. The array holds the M <= 8 workspace
// (decode and fork rows) at either supported shape; prefill (M > 8) needs
// gigabytes and is rejected.
//
// Host code never passes the array's name to a kernel (in host code it is a
// stand-in, not a device address): qfm_init (for the device current then) and
// otherwise the first call on a device, with that device current, take the
// array's device address with hipGetSymbolAddress and keep it per device
// (each GPU holds its own copy). The array starts zeroed, as the workspace's
// tags require, and every call leaves them valid for the next.
// Every call on one GPU uses that GPU's array: calls that overlap on one GPU
// (two streams, two host threads) race and must be serialized by the caller.
#include <mutex>

#include "qfm_internal.h"

namespace qfm {

constexpr size_t kScratchBytes = size_t(3) << 20;   // the M <= 8 workspace at H = 2560, K = 10 is ~2.1 MiB
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

static void *g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// device address of this device's scratch array (nullptr and, when latch is
// set, an error latched on failure)
static void *scratch_for_current_device(bool latch = true) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        if (latch) set_error(-5, "qfm_moe_forward_noalloc: no current device (or device index >= %d)", kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            if (latch) set_error(-5, "qfm_moe_forward_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

// set-up from qfm_init: resolve the current device's array now (nothing
// latched when the host has no device)
void noalloc_prepare_current_device() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) return;
    (void)scratch_for_current_device(false);
}

}  // namespace qfm

using namespace qfm;

extern "C" int qfm_moe_forward_noalloc(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y, hipStream_t s) {
    if (M < 1 || M > 8) {
        set_error(-1, "qfm_moe_forward_noalloc: M = %d; the built-in workspace serves 1 <= M <= 8", M);
        return -1;
    }
    const size_t need = qfm_workspace_bytes(M);
    if (need > kScratchBytes) {
        set_error(-1, "qfm_moe_forward_noalloc: M = %d needs %zu workspace bytes, the built-in workspace has %zu", M,
                  need, kScratchBytes);
        return -1;
    }
    void *ws = scratch_for_current_device();
    if (!ws) return -5;
    return forward_on_workspace(L, x, M, y, ws, kScratchBytes, s);
}
