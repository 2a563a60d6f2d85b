// C-ABI entry point of the encoder self-attention (encoder.hip).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gr_api_util.hpp"
#include "gr_attn.h"
#include "gr_internal.hpp"

namespace gr {

namespace {

// Shape checks of encoder_self_attention (multimodal/mod.rs:156-176), with the
// reference's messages; the buffers are device pointers without lengths, so
// the length check becomes "non-negative sizes and non-null buffers".
int check_encoder(float* out, const float* q, const float* k, const float* v, int32_t n_seq, int32_t tokens,
                  int32_t heads, int32_t head_dim) {
    if (n_seq < 0 || tokens < 0 || heads < 0 || head_dim < 0)
        return fail(GR_ERR_ARG, "encoder attention shape mismatch: sequences=%d tokens=%d heads=%d head_dim=%d",
                    n_seq, tokens, heads, head_dim);
    const int64_t dim = (int64_t)heads * head_dim;
    if (dim > INT32_MAX) return fail(GR_ERR_ARG, "encoder attention dimension overflow");
    const int64_t total = (int64_t)n_seq * tokens;
    if (total > INT32_MAX) return fail(GR_ERR_ARG, "encoder attention token count overflow");
    if (total * dim > ((int64_t)1 << 40)) return fail(GR_ERR_ARG, "encoder attention buffer size overflow");
    if (total * dim == 0) return GR_OK;
    if (head_dim > 256)
        return fail(GR_ERR_ARG, "gr_encoder_self_attention: head_dim %d unsupported (<= 256)", head_dim);
    if (!out || !q || !k || !v)
        return fail(GR_ERR_ARG, "encoder attention shape mismatch: sequences=%d tokens=%d heads=%d head_dim=%d",
                    n_seq, tokens, heads, head_dim);
    return GR_OK;
}

}  // namespace

}  // namespace gr

extern "C" int gr_encoder_self_attention(float* out, const float* q, const float* k, const float* v, int32_t n_seq,
                                         int32_t tokens, int32_t heads, int32_t head_dim, void* stream) {
    gr::clear_error();
    int rc = gr::check_encoder(out, q, k, v, n_seq, tokens, heads, head_dim);
    if (rc || (int64_t)n_seq * tokens * heads * head_dim == 0) return rc;
    gr::EncoderLaunch p{};
    p.n_seq = n_seq;
    p.tokens = tokens;
    p.heads = heads;
    p.head_dim = head_dim;
    p.q = q;
    p.k = k;
    p.v = v;
    p.out = out;
    hipError_t e = gr::launch_encoder_attention(p, (hipStream_t)stream);
    if (e != hipSuccess) return gr::hip_fail(e, "gr_encoder_self_attention launch");
    return GR_OK;
}
