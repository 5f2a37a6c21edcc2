//! Raw declarations of libqora_hip.so, one for each function of
//! include/qora_hip.h, in the header's order, with the header's argument
//! meanings (each header entry cites the reference function it replaces).
//! Every function returns a status (QORA_HIP_OK or a negative QORA_HIP_E_*)
//! unless noted; qora_hip_last_error(ctx) holds the message of the last
//! failure. No call panics or unwinds across the boundary.
//!
//! Safety: the usual FFI contract. Pointers must be valid for the lengths
//! the header states, `ctx` must come from qora_hip_create and be used from
//! one thread at a time, device pointers (`*mut c_void` from qora_hip_malloc,
//! qora_hip_weight_ptrs) must belong to that context's device, and `stream`
//! arguments are HIP streams of that device or null for the context's own.
#![allow(non_camel_case_types, non_snake_case)]

use std::ffi::{c_char, c_int, c_void};

pub const QORA_HIP_OK: c_int = 0;
pub const QORA_HIP_E_INVALID: c_int = -1;
pub const QORA_HIP_E_DEVICE: c_int = -2;
pub const QORA_HIP_E_NOMEM: c_int = -3;
pub const QORA_HIP_E_STATE: c_int = -4;
pub const QORA_HIP_E_IO: c_int = -5;
pub const QORA_HIP_E_RANGE: c_int = -6;

/// Opaque context: one device, its stream, uploaded weights, one model.
#[repr(C)]
pub struct qora_hip_ctx {
    _private: [u8; 0],
}

/// Model description for qora_hip_model_init (DecodeWeights::from_parts, gemv.rs:195-337).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct qora_model_desc {
    pub num_layers: u32,
    pub vocab: u32,
    pub hidden: u32,
    pub intermediate: u32,
    pub num_heads: u32,
    pub num_kv_heads: u32,
    pub head_dim: u32,
    pub num_kv_groups: u32,
    pub rope_half_dim: u32,
    /// 0 = F16, 1 = Q4 (save.rs:198-202)
    pub format: u32,
    /// [num_layers * 7] weight ids: q k v o gate up down
    pub layer_wids: *const u32,
    /// [num_layers] -> f16[hidden]
    pub input_norm: *const *const u16,
    pub post_attn_norm: *const *const u16,
    /// k = vocab, n = hidden
    pub embed_wid: u32,
    pub final_norm: *const u16,
    /// [rope_positions][rope_half_dim]
    pub rope_cos: *const f32,
    pub rope_sin: *const f32,
    pub rope_positions: u64,
    /// [num_layers]: the file's no_rope_layers (1 = rotate)
    pub use_rope: *const u8,
    /// positions held on the device; 0 = the RoPE table length
    pub kv_capacity: u32,
    /// 0 = f32 (the reference RawKvCache), 1 = f16
    pub kv_dtype: u32,
}

/// Sampling fields of GenerateParams (generate.rs:15-35, 345-395).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct qora_sample_params {
    /// <= 0: greedy, the first-max rule
    pub temperature: f32,
    pub top_p: f32,
    /// 0 = the whole vocabulary
    pub top_k: u32,
    /// <= 1: off
    pub repetition_penalty: f32,
    /// <= 0: off
    pub presence_penalty: f32,
}

/// Host-side model for qora_file_write (the .qora v1 writer, save.rs:119-152).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct qora_host_model {
    pub num_layers: u32,
    pub vocab: u32,
    pub hidden: u32,
    pub intermediate: u32,
    pub num_heads: u32,
    pub num_kv_heads: u32,
    pub head_dim: u32,
    pub num_kv_groups: u32,
    pub rope_half_dim: u32,
    pub format: u32,
    pub w_data: *const *const c_void,
    pub w_scales: *const *const u16,
    pub input_norm: *const *const u16,
    pub post_attn_norm: *const *const u16,
    pub embed_data: *const c_void,
    pub embed_scales: *const u16,
    pub final_norm: *const u16,
    pub rope_cos: *const f32,
    pub rope_sin: *const f32,
    pub rope_positions: u64,
    pub use_rope: *const u8,
}

extern "C" {
    // ---- context ----
    pub fn qora_hip_create(device: c_int, out: *mut *mut qora_hip_ctx) -> c_int;
    pub fn qora_hip_destroy(ctx: *mut qora_hip_ctx) -> c_int;
    /// The message of the context's last failure (never null).
    pub fn qora_hip_last_error(ctx: *const qora_hip_ctx) -> *const c_char;
    /// Compute units of the context's device (not a status).
    pub fn qora_hip_device_cus(ctx: *const qora_hip_ctx) -> c_int;

    // ---- weights ----
    pub fn qora_hip_upload_q4(ctx: *mut qora_hip_ctx, packed: *const u8, packed_len: usize, scales_f16: *const u16,
                              n_scales: usize, k: u64, n: u64, wid: *mut u32) -> c_int;
    pub fn qora_hip_upload_f16(ctx: *mut qora_hip_ctx, w: *const u16, len: usize, k: u64, n: u64, wid: *mut u32)
                               -> c_int;
    pub fn qora_hip_weight_ptrs(ctx: *mut qora_hip_ctx, wid: u32, packed_or_data: *mut *mut c_void,
                                scales: *mut *mut c_void) -> c_int;
    pub fn qora_hip_release_weight(ctx: *mut qora_hip_ctx, wid: u32) -> c_int;

    // ---- model: DecodeWeights, raw_prefill, forward_decode_raw, generation ----
    pub fn qora_hip_model_init(ctx: *mut qora_hip_ctx, desc: *const qora_model_desc) -> c_int;
    pub fn qora_hip_load_model(ctx: *mut qora_hip_ctx, path: *const c_char, kv_capacity: u32, kv_dtype: u32) -> c_int;
    pub fn qora_hip_prefill(ctx: *mut qora_hip_ctx, ids: *const u32, n: usize, logits_or_null: *mut f32,
                            argmax_or_null: *mut u32) -> c_int;
    pub fn qora_hip_decode(ctx: *mut qora_hip_ctx, token: u32, logits_or_null: *mut f32, argmax_or_null: *mut u32)
                           -> c_int;
    pub fn qora_hip_generate_greedy(ctx: *mut qora_hip_ctx, token: u32, steps: u32, tokens_out: *mut u32) -> c_int;
    pub fn qora_hip_sample(ctx: *mut qora_hip_ctx, logits: *const f32, vocab: u64, history: *const u32,
                           n_history: u64, params: *const qora_sample_params, rng_state: *mut u64, token: *mut u32,
                           stream: *mut c_void) -> c_int;
    pub fn qora_hip_decode_sample(ctx: *mut qora_hip_ctx, token: u32, history: *const u32, n_history: u64,
                                  params: *const qora_sample_params, rng_state: *mut u64, logits_or_null: *mut f32,
                                  token_out: *mut u32) -> c_int;
    /// Context bound of the fused short-context step (not a status; 0 = never).
    pub fn qora_hip_attn_o_limit(ctx: *const qora_hip_ctx) -> u32;
    /// Context bound of the chunked step (not a status; 0 = never).
    pub fn qora_hip_attn_chunk_limit(ctx: *const qora_hip_ctx) -> u32;

    // ---- KV cache (RawKvCache, gemv.rs:154-166) ----
    pub fn qora_hip_kv_len(ctx: *mut qora_hip_ctx, len: *mut u64) -> c_int;
    pub fn qora_hip_kv_reset(ctx: *mut qora_hip_ctx) -> c_int;
    pub fn qora_hip_kv_download(ctx: *mut qora_hip_ctx, layer: u32, k: *mut f32, v: *mut f32) -> c_int;
    pub fn qora_hip_kv_upload(ctx: *mut qora_hip_ctx, layer: u32, k: *const f32, v: *const f32, len: u64) -> c_int;

    // ---- device memory, stream and graphs ----
    pub fn qora_hip_malloc(ctx: *mut qora_hip_ctx, bytes: usize, dptr: *mut *mut c_void) -> c_int;
    pub fn qora_hip_free(ctx: *mut qora_hip_ctx, dptr: *mut c_void) -> c_int;
    pub fn qora_hip_memcpy_h2d(ctx: *mut qora_hip_ctx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn qora_hip_memcpy_d2h(ctx: *mut qora_hip_ctx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn qora_hip_synchronize(ctx: *mut qora_hip_ctx) -> c_int;
    /// The context's HIP stream (not a status).
    pub fn qora_hip_stream(ctx: *mut qora_hip_ctx) -> *mut c_void;
    pub fn qora_hip_capture_begin(ctx: *mut qora_hip_ctx) -> c_int;
    pub fn qora_hip_capture_end(ctx: *mut qora_hip_ctx, graph_exec: *mut *mut c_void) -> c_int;
    pub fn qora_hip_graph_launch(ctx: *mut qora_hip_ctx, graph_exec: *mut c_void, count: u32) -> c_int;
    pub fn qora_hip_graph_destroy(ctx: *mut qora_hip_ctx, graph_exec: *mut c_void) -> c_int;

    // ---- kernels of gemv.rs / simd.rs on device pointers ----
    pub fn qora_hip_gemv_q4(ctx: *mut qora_hip_ctx, packed: *const c_void, scales: *const c_void, x: *const f32,
                            y: *mut f32, k: u64, n: u64, stream: *mut c_void) -> c_int;
    /// qora_hip_gemv_q4 without allocating (no counterpart in the reference):
    /// for callers that cannot allocate; n <= 65536, calls on one device race.
    pub fn qora_hip_gemv_q4_noalloc(ctx: *mut qora_hip_ctx, packed: *const c_void, scales: *const c_void,
                                    x: *const f32, y: *mut f32, k: u64, n: u64, stream: *mut c_void) -> c_int;
    pub fn qora_hip_gemv_f16(ctx: *mut qora_hip_ctx, w: *const c_void, x: *const f32, y: *mut f32, k: u64, n: u64,
                             stream: *mut c_void) -> c_int;
    pub fn qora_hip_gemv_q4_accumulate(ctx: *mut qora_hip_ctx, packed: *const c_void, scales: *const c_void,
                                       x: *const f32, acc: *mut i64, k: u64, n: u64, stream: *mut c_void) -> c_int;
    pub fn qora_hip_gate_up_q4_accumulate(ctx: *mut qora_hip_ctx, gate_packed: *const c_void,
                                          gate_scales: *const c_void, up_packed: *const c_void,
                                          up_scales: *const c_void, x: *const f32, acc: *mut i64, k: u64, n: u64,
                                          stream: *mut c_void) -> c_int;
    pub fn qora_hip_acc_to_f32(ctx: *mut qora_hip_ctx, acc: *const i64, n: u64, paired: c_int, y: *mut f32,
                               stream: *mut c_void) -> c_int;
    pub fn qora_hip_gemv_prepare(ctx: *mut qora_hip_ctx, wid: u32, wid_up: u32, paired: c_int, gemv_id: *mut u32)
                                 -> c_int;
    pub fn qora_hip_gemv_run(ctx: *mut qora_hip_ctx, gemv_id: u32, x: *const f32, acc: *mut i64,
                             stream: *mut c_void) -> c_int;
    pub fn qora_hip_gemv_release(ctx: *mut qora_hip_ctx, gemv_id: u32) -> c_int;
    pub fn qora_hip_lm_head_prepare(ctx: *mut qora_hip_ctx, wid: u32, lm_id: *mut u32) -> c_int;
    pub fn qora_hip_lm_head_run(ctx: *mut qora_hip_ctx, lm_id: u32, x: *const f32, logits: *mut f32,
                                argmax_device: *mut i32, stream: *mut c_void) -> c_int;
    pub fn qora_hip_gemv_q4_rowdot(ctx: *mut qora_hip_ctx, packed: *const c_void, scales: *const c_void,
                                   x: *const f32, y: *mut f32, rows: u64, cols: u64, stream: *mut c_void) -> c_int;
    pub fn qora_hip_gemv_f16_rowdot(ctx: *mut qora_hip_ctx, w: *const c_void, x: *const f32, y: *mut f32, rows: u64,
                                    cols: u64, stream: *mut c_void) -> c_int;
    pub fn qora_hip_gate_up_q4(ctx: *mut qora_hip_ctx, gate_packed: *const c_void, gate_scales: *const c_void,
                               up_packed: *const c_void, up_scales: *const c_void, x: *const f32, out: *mut f32,
                               k: u64, n: u64, stream: *mut c_void) -> c_int;
    pub fn qora_hip_gate_up_f16(ctx: *mut qora_hip_ctx, gate_w: *const c_void, up_w: *const c_void, x: *const f32,
                                out: *mut f32, k: u64, n: u64, stream: *mut c_void) -> c_int;
    pub fn qora_hip_dequant_q4(ctx: *mut qora_hip_ctx, packed: *const c_void, scales: *const c_void, k: u64, n: u64,
                               out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn qora_hip_rmsnorm(ctx: *mut qora_hip_ctx, x: *const f32, gamma: *const c_void, n: u64, out: *mut f32,
                            stream: *mut c_void) -> c_int;
    pub fn qora_hip_rope(ctx: *mut qora_hip_ctx, data: *mut f32, num_heads: u32, head_dim: u32, cos_t: *const f32,
                         sin_t: *const f32, half_dim: u32, position: u32, stream: *mut c_void) -> c_int;
    pub fn qora_hip_attn_decode(ctx: *mut qora_hip_ctx, q: *const f32, kc: *const c_void, vc: *const c_void,
                                kv_f16: c_int, L: u32, num_heads: u32, num_kv_heads: u32, head_dim: u32,
                                out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn qora_hip_gemm(ctx: *mut qora_hip_ctx, wid: u32, x: *const f32, y: *mut f32, T: u64, stream: *mut c_void)
                         -> c_int;
    pub fn qora_hip_attn_prefill(ctx: *mut qora_hip_ctx, q: *const f32, kc: *const c_void, vc: *const c_void,
                                 kv_f16: c_int, pos0: u32, T: u32, num_heads: u32, num_kv_heads: u32, head_dim: u32,
                                 out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn qora_hip_argmax(ctx: *mut qora_hip_ctx, logits: *const f32, n: u64, out_device: *mut i32,
                           stream: *mut c_void) -> c_int;

    // ---- host utilities (no device; no status) ----
    pub fn qora_synth_q4(seed: u64, tensor_id: u64, k: u64, n: u64, packed: *mut u8, scales: *mut u16);
    pub fn qora_synth_f16(seed: u64, tensor_id: u64, count: u64, stddev: f32, out: *mut u16);
    pub fn qora_synth_f32(seed: u64, tensor_id: u64, count: u64, out: *mut f32);
    pub fn qora_synth_tokens(seed: u64, tensor_id: u64, count: u64, vocab: u32, out: *mut u32);
    pub fn qora_rope_tables(positions: u64, half_dim: u32, theta: f64, cos_out: *mut f32, sin_out: *mut f32);
    pub fn qora_file_write(path: *const c_char, m: *const qora_host_model) -> c_int;
}
