// src/engine/gpu/ffi.rs for gguf-runner: the declarations of include/gr_attn.h.
// Every struct is a #[repr(C)] copy of the header's struct, field for field and in
// order (tests/test_rust_ffi.py checks the field lists and the function list
// against the header on every test run); gr_abi_version() must return
// GR_ATTN_ABI_VERSION below.
#![allow(non_camel_case_types, dead_code)]
use std::ffi::{c_char, c_void};

pub const GR_ATTN_ABI_VERSION: i32 = 5;

pub const GR_OK: i32 = 0;
pub const GR_DTYPE_F32: i32 = 0;
pub const GR_DTYPE_F16: i32 = 1;
pub const GR_DTYPE_BF16: i32 = 2;
pub const GR_DTYPE_Q8: i32 = 3;
pub const GR_DTYPE_TURBO: i32 = 4;
pub const GR_DELTANET_AUTO: i32 = 0;
pub const GR_DELTANET_RECURRENT: i32 = 1;
pub const GR_DELTANET_CHUNKED: i32 = 2;

#[repr(C)]
pub struct GrRunState {
    _p: [u8; 0],
}

#[repr(C)]
pub struct GrDecodeArgs {
    pub n_seq: i32,
    pub n_heads: i32,
    pub n_kv_heads: i32,
    pub head_dim: i32,
    pub kv_dtype: i32,
    pub split_keys: i32,
    pub max_kv_len: i32,
    pub score_scale: f32,
    pub q: *const f32,
    pub k_cache: *const c_void,
    pub v_cache: *const c_void,
    pub seq_stride: i64,
    pub row_stride: i64,
    pub kv_start: *const i32,
    pub kv_end: *const i32,
    pub out: *mut f32,
    pub workspace: *mut c_void,
    pub k_scale: *const f32,
    pub v_scale: *const f32,
    pub scale_seq_stride: i64,
    pub scale_row_stride: i64,
    pub q8_block: i32,
    pub k_sign: *const c_void,
    pub v_sign: *const c_void,
    pub k_rnorm: *const f32,
    pub v_rnorm: *const f32,
    pub turbo_signs: *const u8,
    pub turbo_slot_stride: i64,
    pub out_gate: *const f32,
    pub out_gate_row_stride: i64,
    pub out_gate_head_stride: i32,
}

#[repr(C)]
pub struct GrPrefillArgs {
    pub n_tokens: i32,
    pub base_pos: i32,
    pub n_heads: i32,
    pub n_kv_heads: i32,
    pub head_dim: i32,
    pub dtype: i32,
    pub window: i32,
    pub rope_mode: i32,
    pub rope_dim: i32,
    pub rope_scale: f32,
    pub rope_freqs: *const f32,
    pub q_norm: *const f32,
    pub k_norm: *const f32,
    pub norm_eps: f32,
    pub is_gemma3: i32,
    pub q: *const c_void,
    pub k: *const c_void,
    pub v: *const c_void,
    pub k_cache: *mut c_void,
    pub v_cache: *mut c_void,
    pub cache_row_stride: i64,
    pub out: *mut f32,
    pub workspace: *mut c_void,
    pub bidirectional: i32,
    pub out_gate: *const f32,
    pub out_gate_row_stride: i64,
    pub out_gate_head_stride: i32,
    pub q_bias: *const f32,
    pub k_bias: *const f32,
    pub v_bias: *const f32,
}

#[repr(C)]
pub struct GrDeltaNetArgs {
    pub n_tokens: i32,
    pub n_heads: i32,
    pub head_dim: i32,
    pub in_dtype: i32,
    pub l2norm: i32,
    pub algo: i32,
    pub eps: f32,
    pub q: *const c_void,
    pub k: *const c_void,
    pub v: *const c_void,
    pub gate: *const f32,
    pub beta: *const f32,
    pub state: *mut f32,
    pub out: *mut f32,
    pub workspace: *mut c_void,
}

#[repr(C)]
pub struct GrAttnConfig {
    pub n_layers: i32,
    pub n_heads: i32,
    pub n_kv_heads: i32,
    pub head_dim: i32,
    pub seq_len: i32,
    pub n_seq: i32,
    pub kv_dtype: i32,
    pub rope_mode: i32,
    pub rope_dim: i32,
    pub rope_theta: f32,
    pub rope_theta_swa: f32,
    pub rope_scale_global: f32,
    pub rope_scale_local: f32,
    pub layer_windows: *const i32,
    pub swa_pattern: i32,
    pub is_gemma3: i32,
    pub online_attn_fusion: i32,
    pub rms_norm_eps: f32,
    pub q_norm: *const f32,
    pub k_norm: *const f32,
    pub qk_norm_present: *const u8,
    pub ssm_n_heads: i32,
    pub ssm_head_dim: i32,
    pub q8_block_scales: i32,
    pub ssm_n_k_heads: i32,
    pub ssm_conv_kernel: i32,
    pub ssm_conv1d: *const f32,
    pub ssm_a: *const f32,
    pub ssm_dt_bias: *const f32,
    pub ssm_norm: *const f32,
}

unsafe extern "C" {
    pub fn gr_last_error() -> *const c_char;
    pub fn gr_abi_version() -> i32;
    pub fn gr_decode_workspace_size(a: *const GrDecodeArgs) -> usize;
    pub fn gr_decode_attention(a: *const GrDecodeArgs, stream: *mut c_void) -> i32;
    pub fn gr_decode_attention_noalloc(a: *const GrDecodeArgs, stream: *mut c_void) -> i32;
    pub fn gr_prefill_workspace_size(a: *const GrPrefillArgs) -> usize;
    pub fn gr_prefill_attention(a: *const GrPrefillArgs, stream: *mut c_void) -> i32;
    pub fn gr_turbo_sign_table(n_layers: i32, n_kv_heads: i32, head_size: i32, out: *mut u8) -> i32;
    pub fn gr_rope_freqs(theta: f32, rope_dim: i32, freqs_out: *mut f32) -> i32;
    pub fn gr_encoder_self_attention(out: *mut f32, q: *const f32, k: *const f32, v: *const f32,
                                     n_seq: i32, tokens: i32, heads: i32, head_dim: i32,
                                     stream: *mut c_void) -> i32;
    pub fn gr_deltanet_workspace_size(a: *const GrDeltaNetArgs) -> usize;
    pub fn gr_deltanet_attention(a: *const GrDeltaNetArgs, stream: *mut c_void) -> i32;
    pub fn gr_malloc_run_state(cfg: *const GrAttnConfig, out: *mut *mut GrRunState) -> i32;
    pub fn gr_free_run_state(s: *mut GrRunState);
    pub fn gr_qkv_norm(s: *mut GrRunState, layer: i32, q: *mut f32, k: *mut f32) -> i32;
    pub fn gr_apply_rope_qk(s: *mut GrRunState, layer: i32, pos: i64, q: *mut f32, k: *mut f32) -> i32;
    pub fn gr_kv_write_token(s: *mut GrRunState, seq: i32, layer: i32, pos: i64, k: *const f32,
                             v: *const f32) -> i32;
    pub fn gr_attention_token(s: *mut GrRunState, seq: i32, layer: i32, pos: i64, q: *const f32,
                              xb: *mut f32) -> i32;
    pub fn gr_attention_layer_token(s: *mut GrRunState, seq: i32, layer: i32, pos: i64,
                                    q: *const f32, k: *const f32, v: *const f32, xb: *mut f32) -> i32;
    pub fn gr_prefill_attention_chunk(s: *mut GrRunState, seq: i32, layer: i32, base_pos: i64,
                                      m: i32, q: *const f32, k: *const f32, v: *const f32,
                                      xb: *mut f32) -> i32;
    pub fn gr_prefill_image_block(s: *mut GrRunState, seq: i32, layer: i32, base_pos: i64, m: i32,
                                  q: *const f32, k: *const f32, v: *const f32, xb: *mut f32) -> i32;
    pub fn gr_decode_layer_batch(s: *mut GrRunState, layer: i32, n: i32, seqs: *const i32,
                                 pos: *const i64, q: *const f32, k: *const f32, v: *const f32,
                                 xb: *mut f32) -> i32;
    pub fn gr_qwen3next_state_step(s: *mut GrRunState, layer: i32, q: *const f32, k: *const f32,
                                   v: *const f32, g: *const f32, beta: *const f32, out: *mut f32) -> i32;
    pub fn gr_qwen3next_prefill(s: *mut GrRunState, layer: i32, t: i32, q: *const f32, k: *const f32,
                                v: *const f32, gate: *const f32, beta: *const f32, out: *mut f32) -> i32;
    pub fn gr_qwen3next_ssm_layer(s: *mut GrRunState, layer: i32, t: i32, qkv: *const f32,
                                  z: *const f32, gate_a: *const f32, gate_b: *const f32,
                                  out: *mut f32) -> i32;
    pub fn gr_read_ssm_conv_state(s: *mut GrRunState, layer: i32, out: *mut f32) -> i32;
    pub fn gr_write_ssm_conv_state(s: *mut GrRunState, layer: i32, input: *const f32) -> i32;
    pub fn gr_read_kv_rows(s: *mut GrRunState, layer: i32, seq: i32, row0: i64, n_rows: i64,
                           k_out: *mut c_void, v_out: *mut c_void) -> i32;
    pub fn gr_read_kv_scales(s: *mut GrRunState, layer: i32, seq: i32, row0: i64, n_rows: i64,
                             k_scale_out: *mut f32, v_scale_out: *mut f32) -> i32;
    pub fn gr_read_turbo_rows(s: *mut GrRunState, layer: i32, seq: i32, row0: i64, n_rows: i64,
                              k_base: *mut u8, k_sign: *mut u8, k_rnorm: *mut f32, v_base: *mut u8,
                              v_sign: *mut u8, v_rnorm: *mut f32) -> i32;
    pub fn gr_read_ssm_state(s: *mut GrRunState, layer: i32, out: *mut f32) -> i32;
    pub fn gr_write_ssm_state(s: *mut GrRunState, layer: i32, input: *const f32) -> i32;
    pub fn gr_prefill_cache_snapshot(s: *mut GrRunState, seq: i32, tokens: *const i32, k: i32,
                                     model_len: u64, model_head_fnv: u64, out: *mut u8, cap: u64,
                                     size_out: *mut u64) -> i32;
    pub fn gr_prefill_cache_inject(s: *mut GrRunState, seq: i32, blob: *const u8, len: u64,
                                   k_out: *mut i32) -> i32;
}

/// Turns a status into a Result with gr_last_error()'s message.
pub fn check(rc: i32) -> Result<(), String> {
    if rc == GR_OK {
        return Ok(());
    }
    let msg = unsafe { std::ffi::CStr::from_ptr(gr_last_error()) };
    Err(msg.to_string_lossy().into_owned())
}
