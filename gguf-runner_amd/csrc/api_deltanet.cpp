// C-ABI entry points of the gated DeltaNet path.
#include <hip/hip_runtime.h>

#include "gr_api_util.hpp"
#include "gr_attn.h"
#include "gr_internal.hpp"

namespace gr {

namespace {

// The chunked kernels are built for state size 128; other sizes run the token
// recurrence whatever the algorithm asked for (the same results to fp32 rounding).
bool use_chunked(const gr_deltanet_args* a) {
    return a->head_dim == 128 &&
           (a->algo == GR_DELTANET_CHUNKED || (a->algo == GR_DELTANET_AUTO && a->n_tokens >= 64));
}

int check_deltanet(const gr_deltanet_args* a) {
    if (!a) return fail(GR_ERR_ARG, "gr_deltanet_attention: null args");
    if (a->n_tokens < 0 || a->n_heads <= 0)
        return fail(GR_ERR_ARG, "gr_deltanet_attention: n_tokens >= 0 and n_heads > 0 required");
    if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
        return fail(GR_ERR_ARG, "gr_deltanet_attention: head_dim %d unsupported (64, 128, 256)", a->head_dim);
    if (a->in_dtype < GR_DTYPE_F32 || a->in_dtype > GR_DTYPE_BF16)
        return fail(GR_ERR_ARG, "gr_deltanet_attention: bad in_dtype %d", a->in_dtype);
    if (a->algo < GR_DELTANET_AUTO || a->algo > GR_DELTANET_CHUNKED)
        return fail(GR_ERR_ARG, "gr_deltanet_attention: bad algo %d", a->algo);
    if (a->n_tokens > 0 && (!a->q || !a->k || !a->v || !a->gate || !a->beta || !a->state || !a->out))
        return fail(GR_ERR_ARG, "gr_deltanet_attention: null buffer");
    if (a->n_tokens > 0 && use_chunked(a) && (!a->workspace || (uintptr_t)a->workspace % 256))
        return fail(GR_ERR_ARG, "gr_deltanet_attention: chunked algorithm needs a 256-byte aligned workspace");
    return GR_OK;
}

}  // namespace

size_t deltanet_ws(const gr_deltanet_args* a) {
    if (!a || a->n_tokens <= 0 || a->n_heads <= 0 || !use_chunked(a)) return 0;
    return deltanet_chunked_ws_bytes(a->n_tokens, a->n_heads, a->head_dim, 64);
}

int deltanet_enqueue(const gr_deltanet_args* a, hipStream_t st) {
    int rc = check_deltanet(a);
    if (rc) return rc;
    if (a->n_tokens == 0) return GR_OK;
    DeltaNetLaunch p{};
    p.n_tokens = a->n_tokens;
    p.n_heads = a->n_heads;
    p.head_dim = a->head_dim;
    p.in_dtype = a->in_dtype;
    p.l2norm = a->l2norm;
    p.eps = a->eps;
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.gate = a->gate;
    p.beta = a->beta;
    p.state = a->state;
    p.out = a->out;
    p.ws = (float*)a->workspace;
    p.chunk = 64;
    p.gate_is_log = 1;
    hipError_t e = use_chunked(a) ? launch_deltanet_chunked(p, st) : launch_deltanet_scan(p, st);
    if (e != hipSuccess) return hip_fail(e, "gr_deltanet_attention launch");
    return GR_OK;
}

}  // namespace gr

extern "C" {

size_t gr_deltanet_workspace_size(const gr_deltanet_args* a) { return gr::deltanet_ws(a); }

int gr_deltanet_attention(const gr_deltanet_args* a, void* stream) {
    gr::clear_error();
    return gr::deltanet_enqueue(a, (hipStream_t)stream);
}

}  // extern "C"
