// noalloc.hip — split-KV decode for callers that cannot allocate device memory.
//
// int8k_decode_attention_forward takes a caller-owned workspace for its split
// partials (m, l, acc[D] per unit).  Code under HIP graph capture, tight
// serving loops and harnesses that forbid hipMalloc cannot provide one, so
// this entry point runs the same kernels with the partials in `scratch`, a
// file-scope device array the library reserves once per GPU for the life of
// the process.
//
// Host code never uses the array's name as an address: in host code `scratch`
// is the host-side stand-in that HIP registers for the symbol.  The device
// address of each GPU's copy comes from hipGetSymbolAddress, taken once per
// device with that device current, and only that address is passed on.
//
// Only plans of more than 16 chunks per (b,h) run the split kernel and write
// partials; the one-launch plans merge their chunks on chip, need no scratch
// and are never refused for size (the workspace query returns 0 for them).
// Every call on a GPU shares that GPU's array and leaves its partials there.
// Nothing in it has to start at zero: each unit of the split kernel writes its
// partial before the combine kernel reads it.  Two calls that overlap on one
// GPU (different streams, or different host threads) race on the array.
#include <atomic>

#include "int8k_common.h"

namespace int8k {
namespace {

constexpr size_t kScratchBytes = INT8K_DECODE_NOALLOC_SCRATCH_BYTES;

static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxTrackedDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxTrackedDevices];

// Device address of the current GPU's copy of `scratch`, looked up on the
// first call on that device (devices past kMaxTrackedDevices look it up on
// every call).
int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_last_error("hipGetDevice", e);
        return INT8K_ERR_HIP;
    }
    const bool tracked = dev >= 0 && dev < kMaxTrackedDevices;
    if (tracked) {
        void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
        if (p != nullptr) {
            *out = p;
            return INT8K_OK;
        }
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
        set_last_error("hipGetSymbolAddress(scratch)", e != hipSuccess ? e : hipErrorInvalidSymbol);
        return INT8K_ERR_HIP;
    }
    if (tracked) g_scratch_ptr[dev].store(p, std::memory_order_release);
    *out = p;
    return INT8K_OK;
}

}  // namespace
}  // namespace int8k

using namespace int8k;

extern "C" int int8k_decode_attention_forward_noalloc(
    const int8_t* Q, const int8_t* K, const int8_t* V, uint16_t* out,
    const float* scale_Q, const float* scale_K, const float* scale_V,
    int BH, int S, int head_dim, int nsplit, void* stream) {
    clear_last_error();
    if (!Q || !K || !V || !out || !scale_Q || !scale_K || !scale_V)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (BH <= 0 || S <= 0 || nsplit < 0) return INT8K_ERR_INVALID_ARGUMENT;
    if (head_dim != 64 && head_dim != 128) return INT8K_ERR_UNSUPPORTED;
    // the size check comes before any HIP call
    const size_t need = int8k_decode_attention_workspace_bytes(BH, S, head_dim, nsplit);
    if (need > kScratchBytes) {
        set_last_error_text(
            "int8k_decode_attention_forward_noalloc: the split partials of this call need more "
            "than the INT8K_DECODE_NOALLOC_SCRATCH_BYTES (8 MiB) of library scratch; use "
            "int8k_decode_attention_forward with a workspace, or a smaller nsplit");
        return INT8K_ERR_WORKSPACE;
    }
    void* ws = nullptr;
    const int st = scratch_address(&ws);
    if (st != INT8K_OK) return st;
    return int8k_decode_attention_forward(Q, K, V, out, scale_Q, scale_K, scale_V, BH, S,
                                          head_dim, nsplit, ws, kScratchBytes, stream);
}
