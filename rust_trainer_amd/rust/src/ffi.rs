//! Raw declarations of `include/rtq.h` (every function of the C ABI, in header order).  Pointers
//! are plain; `*mut c_void` streams are `hipStream_t` (null: the HIP null stream).

#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub type rtq_status = c_int;
pub const RTQ_OK: rtq_status = 0;
pub const RTQ_ERR_INVALID: rtq_status = 1;
pub const RTQ_ERR_UNSUPPORTED: rtq_status = 2;
pub const RTQ_ERR_HIP: rtq_status = 3;
pub const RTQ_ERR_NO_DEVICE: rtq_status = 4;

pub const RTQ_TYPE_F32: c_int = 0;
pub const RTQ_TYPE_Q4_0: c_int = 2;
pub const RTQ_TYPE_Q8_0: c_int = 8;
pub const RTQ_TYPE_Q4_K: c_int = 12;
pub const RTQ_TYPE_Q6_K: c_int = 14;
pub const RTQ_TYPE_TQ8_0: c_int = 264;

#[repr(C)]
pub struct rtq_ctx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct rtq_weight {
    _p: [u8; 0],
}
#[repr(C)]
pub struct rtq_gguf {
    _p: [u8; 0],
}
#[repr(C)]
pub struct rtq_gguf_writer {
    _p: [u8; 0],
}
#[repr(C)]
pub struct rtq_model {
    _p: [u8; 0],
}

/// `Lora` as the library reads it (src/linear.rs:8-16): a is [rank x in], b is [out x rank].
#[repr(C)]
#[derive(Clone, Copy)]
pub struct rtq_lora {
    pub rank: i64,
    pub alpha: f32,
    pub a: *const f32,
    pub b: *const f32,
    pub enabled: c_int,
}

#[repr(C)]
#[derive(Clone, Copy, Default, Debug)]
pub struct rtq_model_config {
    pub n_layer: i64,
    pub n_embd: i64,
    pub n_head: i64,
    pub n_head_kv: i64,
    pub head_dim: i64,
    pub rope_dim: i64,
    pub n_ff: i64,
    pub n_vocab: i64,
    pub rms_eps: f32,
    pub norm_offset: f32,
    pub rope_base: f32,
    pub rope_freq_scale: f32,
    pub rope_neox: c_int,
    pub qk_norm: c_int,
    pub kv_f16: c_int,
    pub tied: c_int,
    pub n_rope_factors: i64,
}

extern "C" {
    // library / context
    pub fn rtq_version() -> *const c_char;
    pub fn rtq_last_error() -> *const c_char;
    pub fn rtq_ctx_create(device: c_int, out: *mut *mut rtq_ctx) -> rtq_status;
    pub fn rtq_ctx_destroy(ctx: *mut rtq_ctx);
    pub fn rtq_ctx_stream(ctx: *mut rtq_ctx) -> *mut c_void;
    pub fn rtq_ctx_reserve(ctx: *mut rtq_ctx, max_t: i64, max_rows: i64, max_cols: i64, max_rank: i64) -> rtq_status;
    pub fn rtq_ctx_set_timing(ctx: *mut rtq_ctx, enable: c_int, only_kernel: *const c_char) -> rtq_status;
    pub fn rtq_ctx_timing_count(ctx: *mut rtq_ctx) -> c_int;
    pub fn rtq_ctx_timing_get(ctx: *mut rtq_ctx, i: c_int, name: *mut *const c_char, launches: *mut i64,
                              total_ms: *mut f64) -> rtq_status;
    pub fn rtq_ctx_timing_work(ctx: *mut rtq_ctx, i: c_int, flops: *mut f64, bytes: *mut f64) -> rtq_status;
    pub fn rtq_ctx_timing_reset(ctx: *mut rtq_ctx);

    // weights (FrozenMatmul)
    pub fn rtq_weight_create(ctx: *mut rtq_ctx, ggml_type: c_int, blocks: *const c_void, nbytes: usize, rows: i64,
                             cols: i64, out: *mut *mut rtq_weight) -> rtq_status;
    pub fn rtq_weight_destroy(w: *mut rtq_weight);
    pub fn rtq_weight_out_dim(w: *const rtq_weight) -> i64;
    pub fn rtq_weight_in_dim(w: *const rtq_weight) -> i64;
    pub fn rtq_weight_nbytes(w: *const rtq_weight) -> usize;
    pub fn rtq_weight_type(w: *const rtq_weight) -> c_int;
    pub fn rtq_frozen_forward(ctx: *mut rtq_ctx, w: *const rtq_weight, x: *const f32, t: i64, y: *mut f32) -> rtq_status;
    pub fn rtq_frozen_backward_input(ctx: *mut rtq_ctx, w: *const rtq_weight, dy: *const f32, t: i64,
                                     dx: *mut f32) -> rtq_status;
    pub fn rtq_frozen_row(ctx: *mut rtq_ctx, w: *const rtq_weight, r: i64, out: *mut f32) -> rtq_status;

    // Linear (LoRA)
    pub fn rtq_linear_forward(ctx: *mut rtq_ctx, w: *const rtq_weight, bias: *const f32, lora: *const rtq_lora,
                              x: *const f32, t: i64, y: *mut f32) -> rtq_status;
    pub fn rtq_linear_backward(ctx: *mut rtq_ctx, w: *const rtq_weight, lora: *const rtq_lora, x: *const f32,
                               dy: *const f32, t: i64, dx: *mut f32, ga: *mut f32, gb: *mut f32) -> rtq_status;

    // device pointers + stream
    pub fn rtq_frozen_forward_d(ctx: *mut rtq_ctx, w: *const rtq_weight, x: *const f32, t: i64, y: *mut f32,
                                stream: *mut c_void) -> rtq_status;
    pub fn rtq_frozen_backward_input_d(ctx: *mut rtq_ctx, w: *const rtq_weight, dy: *const f32, t: i64, dx: *mut f32,
                                       stream: *mut c_void) -> rtq_status;
    pub fn rtq_frozen_rows_d(ctx: *mut rtq_ctx, w: *const rtq_weight, r0: i64, count: i64, out: *mut f32,
                             stream: *mut c_void) -> rtq_status;
    pub fn rtq_linear_forward_d(ctx: *mut rtq_ctx, w: *const rtq_weight, bias: *const f32, lora: *const rtq_lora,
                                x: *const f32, t: i64, y: *mut f32, stream: *mut c_void) -> rtq_status;
    pub fn rtq_linear_backward_d(ctx: *mut rtq_ctx, w: *const rtq_weight, lora: *const rtq_lora, x: *const f32,
                                 dy: *const f32, t: i64, dx: *mut f32, ga: *mut f32, gb: *mut f32,
                                 stream: *mut c_void) -> rtq_status;
    pub fn rtq_linear_forward_noalloc_d(ctx: *mut rtq_ctx, w: *const rtq_weight, bias: *const f32,
                                        lora: *const rtq_lora, x: *const f32, t: i64, y: *mut f32,
                                        stream: *mut c_void) -> rtq_status;

    // embedding gather, LM head + cross-entropy (Model::embed_tokens, Model::head)
    pub fn rtq_frozen_gather(ctx: *mut rtq_ctx, w: *const rtq_weight, ids: *const i32, count: i64,
                             out: *mut f32) -> rtq_status;
    pub fn rtq_frozen_gather_d(ctx: *mut rtq_ctx, w: *const rtq_weight, ids: *const i32, count: i64, out: *mut f32,
                               stream: *mut c_void) -> rtq_status;
    pub fn rtq_lm_head(ctx: *mut rtq_ctx, lm_head: *const rtq_weight, norm_w: *const f32, eps: f32, offset: f32,
                       x: *const f32, t: i64, pos: *const i32, tok: *const i32, weights: *const f32, n: i64,
                       logp: *mut f32, hits: *mut i64, dx: *mut f32) -> rtq_status;
    pub fn rtq_lm_head_d(ctx: *mut rtq_ctx, lm_head: *const rtq_weight, norm_w: *const f32, eps: f32, offset: f32,
                         x: *const f32, t: i64, pos: *const i32, tok: *const i32, weights: *const f32, n: i64,
                         logp: *mut f32, hit: *mut i32, dx: *mut f32, stream: *mut c_void) -> rtq_status;

    // the device-resident training step (Model::forward_backward)
    pub fn rtq_model_from_gguf(ctx: *mut rtq_ctx, g: *const rtq_gguf, out: *mut *mut rtq_model) -> rtq_status;
    pub fn rtq_model_config_from_gguf(g: *const rtq_gguf, out: *mut rtq_model_config) -> rtq_status;
    pub fn rtq_model_destroy(m: *mut rtq_model);
    pub fn rtq_model_get_config(m: *const rtq_model, out: *mut rtq_model_config) -> rtq_status;
    pub fn rtq_model_attach_lora(m: *mut rtq_model, rank: i64, alpha: f32, target_mask: u32, seed: u64,
                                 n_params: *mut i64) -> rtq_status;
    pub fn rtq_model_lora_count(m: *const rtq_model) -> i64;
    pub fn rtq_model_lora_info(m: *const rtq_model, i: i64, layer: *mut c_int, which: *mut c_int, rank: *mut i64,
                               in_: *mut i64, out: *mut i64, alpha: *mut f32) -> rtq_status;
    pub fn rtq_model_lora_get(m: *mut rtq_model, i: i64, a: *mut f32, b: *mut f32, ga: *mut f32,
                              gb: *mut f32) -> rtq_status;
    pub fn rtq_model_lora_set(m: *mut rtq_model, i: i64, a: *const f32, b: *const f32) -> rtq_status;
    pub fn rtq_model_lora_device(m: *mut rtq_model, i: i64, a: *mut *mut f32, b: *mut *mut f32, ga: *mut *mut f32,
                                 gb: *mut *mut f32, ldb: *mut i64) -> rtq_status;
    pub fn rtq_model_zero_grad(m: *mut rtq_model) -> rtq_status;
    pub fn rtq_model_forward_backward(m: *mut rtq_model, tokens: *const i32, t: i64, pos: *const i32,
                                      tok: *const i32, weights: *const f32, n: i64, logp: *mut f32,
                                      hits: *mut i64) -> rtq_status;
    pub fn rtq_model_forward_backward_packed(m: *mut rtq_model, tokens: *const i32, t: i64, positions: *const i32,
                                             segments: *const i32, pos: *const i32, tok: *const i32,
                                             weights: *const f32, n: i64, logp: *mut f32,
                                             hits: *mut i64) -> rtq_status;
    pub fn rtq_model_set_checkpointing(m: *mut rtq_model, mode: c_int) -> rtq_status;
    pub fn rtq_model_checkpointing(m: *const rtq_model) -> c_int;
    pub fn rtq_model_set_attention(m: *mut rtq_model, mode: c_int) -> rtq_status;
    pub fn rtq_model_attention_fused(m: *const rtq_model) -> c_int;
    pub fn rtq_model_graph_replays(m: *const rtq_model) -> i64;
    pub fn rtq_model_debug_capture(m: *mut rtq_model, layer: i64) -> rtq_status;
    pub fn rtq_model_debug_tensor(m: *mut rtq_model, name: *const c_char, out: *mut f32, nfloats: i64) -> rtq_status;

    // parity / debug
    pub fn rtq_debug_quantize_acts(ctx: *mut rtq_ctx, w: *const rtq_weight, x: *const f32, t: i64,
                                   out: *mut c_void) -> rtq_status;
    pub fn rtq_debug_isums_per_row(w: *const rtq_weight) -> i64;
    pub fn rtq_debug_block_isums(ctx: *mut rtq_ctx, w: *const rtq_weight, x: *const f32, t: i64,
                                 out: *mut i32) -> rtq_status;

    // GGUF v3 container (rie_core::gguf::{GgufFile, GgufWriter})
    pub fn rtq_gguf_open(path: *const c_char, out: *mut *mut rtq_gguf) -> rtq_status;
    pub fn rtq_gguf_from_bytes(data: *const c_void, nbytes: usize, out: *mut *mut rtq_gguf) -> rtq_status;
    pub fn rtq_gguf_close(g: *mut rtq_gguf);
    pub fn rtq_gguf_version(g: *const rtq_gguf) -> u32;
    pub fn rtq_gguf_kv_count(g: *const rtq_gguf) -> i64;
    pub fn rtq_gguf_find_kv(g: *const rtq_gguf, key: *const c_char) -> i64;
    pub fn rtq_gguf_kv(g: *const rtq_gguf, i: i64, key: *mut *const c_char, type_: *mut c_int, elem_type: *mut c_int,
                       count: *mut u64, data: *mut *const c_void) -> rtq_status;
    pub fn rtq_gguf_get_str(g: *const rtq_gguf, key: *const c_char, s: *mut *const c_char, len: *mut u64) -> rtq_status;
    pub fn rtq_gguf_get_f64(g: *const rtq_gguf, key: *const c_char, v: *mut f64) -> rtq_status;
    pub fn rtq_gguf_tensor_count(g: *const rtq_gguf) -> i64;
    pub fn rtq_gguf_find_tensor(g: *const rtq_gguf, name: *const c_char) -> i64;
    pub fn rtq_gguf_tensor(g: *const rtq_gguf, i: i64, name: *mut *const c_char, type_: *mut c_int,
                           n_dims: *mut c_int, ne: *mut i64, data: *mut *const c_void, nbytes: *mut usize) -> rtq_status;
    pub fn rtq_weight_from_gguf(ctx: *mut rtq_ctx, g: *const rtq_gguf, name: *const c_char,
                                out: *mut *mut rtq_weight) -> rtq_status;
    pub fn rtq_gguf_writer_create(out: *mut *mut rtq_gguf_writer) -> rtq_status;
    pub fn rtq_gguf_writer_destroy(w: *mut rtq_gguf_writer);
    pub fn rtq_gguf_writer_kv(w: *mut rtq_gguf_writer, key: *const c_char, type_: c_int, elem_type: c_int, count: u64,
                              data: *const c_void) -> rtq_status;
    pub fn rtq_gguf_writer_tensor(w: *mut rtq_gguf_writer, name: *const c_char, type_: c_int, n_dims: c_int,
                                  ne: *const i64, data: *const c_void, nbytes: usize) -> rtq_status;
    pub fn rtq_gguf_writer_bytes(w: *mut rtq_gguf_writer, data: *mut *const c_void, nbytes: *mut usize) -> rtq_status;
    pub fn rtq_gguf_writer_write(w: *mut rtq_gguf_writer, path: *const c_char) -> rtq_status;
}
