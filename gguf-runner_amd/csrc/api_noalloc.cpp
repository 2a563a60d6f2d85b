// gr_decode_attention_noalloc: split-K decode with the partials in a
// library-owned device array instead of a caller workspace, for callers that
// cannot allocate device memory (code under HIP graph capture, serving loops
// that forbid hipMalloc).  Same kernels and results as gr_decode_attention.
#include <hip/hip_runtime.h>

#include <mutex>

#include "gr_api_util.hpp"
#include "gr_attn.h"

// The partials (o, m, l) and the stream-schedule offsets of one decode call.
// Each GPU holds its own copy for the life of the process; every call on a GPU
// shares it, so calls that overlap on one GPU (two streams, two threads) race.
// The kernels write every word they later read within the call, so nothing
// needs clearing between calls.
static __device__ __align__(256) unsigned char scratch[GR_DECODE_NOALLOC_MAX_WORKSPACE];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, set once

// Device address of the current device's copy of `scratch`.  The array's name
// is a host-side stand-in; kernels get this address instead.
int scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return gr::hip_fail(e, "gr_decode_attention_noalloc: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return gr::fail(GR_ERR_ARG, "gr_decode_attention_noalloc: device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return gr::hip_fail(e, "gr_decode_attention_noalloc: hipGetSymbolAddress(scratch)");
        if (!p || (uintptr_t)p % 256 != 0)
            return gr::fail(GR_ERR_HIP, "gr_decode_attention_noalloc: scratch address %p not 256-byte aligned", p);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GR_OK;
}

}  // namespace

extern "C" int gr_decode_attention_noalloc(const gr_decode_args* a, void* stream) {
    gr::clear_error();
    if (!a) return gr::fail(GR_ERR_ARG, "gr_decode_attention_noalloc: null args");
    gr_decode_args b = *a;
    b.workspace = (void*)(uintptr_t)256;  // stand-in for the checks: the workspace argument is ignored
    int rc = gr::check_decode(&b);
    if (rc) return rc;
    const size_t need = gr::decode_ws_bytes(&b);
    if (need > (size_t)GR_DECODE_NOALLOC_MAX_WORKSPACE)
        return gr::fail(GR_ERR_ARG,
                        "gr_decode_attention_noalloc: this call needs %zu bytes of partials, more than the "
                        "%zu-byte built-in scratch; use gr_decode_attention with a caller workspace",
                        need, (size_t)GR_DECODE_NOALLOC_MAX_WORKSPACE);
    if ((rc = scratch_address(&b.workspace))) return rc;
    return gr::decode_enqueue(&b, (hipStream_t)stream);
}
