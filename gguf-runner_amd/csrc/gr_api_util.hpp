// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "gr_attn.h"

namespace gr {

// Record `fmt` as this thread's last error and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);
void clear_error();
size_t align_up(size_t x, size_t a);

int check_decode_shape_only(const gr_decode_args* a);
// Full argument check of gr_decode_attention (no HIP calls); GR_OK or the error.
int check_decode(const gr_decode_args* a);
int decode_enqueue(const gr_decode_args* a, hipStream_t st);
int decode_enqueue_ex(const gr_decode_args* a, const int32_t* seq_slot, hipStream_t st);
// Turbo caches only: token-packed split kernel (DecodeLaunch::tok_pack).
int decode_enqueue_ex(const gr_decode_args* a, const int32_t* seq_slot, hipStream_t st, int tok_pack,
                      const int32_t* col_start, const int32_t* col_end);
size_t decode_ws_bytes(const gr_decode_args* a);
// turboquant_build_sign_table (inference.rs:370-395) into host memory.
void turbo_sign_table_host(int n_layers, int n_kv_heads, int head_size, uint8_t* table);

}  // namespace gr
