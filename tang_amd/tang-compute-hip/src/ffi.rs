//! Raw bindings of the gfx950 backend's C ABI (`include/tang_hip.h`, built
//! as `libtang_hip.so`): one `extern "C"` declaration per entry point, with
//! the header's types.  Every function returns a status (`TH_OK` = 0) except
//! `th_last_error` and `th_synth_seed`; the message of the last failure on
//! the calling thread is `th_last_error()`.  `tests/test_rust_ffi.py` checks
//! this block against the header: same names, same argument counts and
//! kinds.
#![allow(non_camel_case_types, non_snake_case, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

pub const TH_OK: c_int = 0;
pub const TH_ERR_INVALID: c_int = 1;
pub const TH_ERR_HIP: c_int = 2;
pub const TH_ERR_OOM: c_int = 3;
pub const TH_ERR_UNSUPPORTED: c_int = 4;

// th_dtype
pub const TH_F32: c_int = 0;
pub const TH_BF16: c_int = 1;
pub const TH_F16: c_int = 2;
pub const TH_U8: c_int = 3;
pub const TH_I8: c_int = 4;
pub const TH_U32: c_int = 5;
pub const TH_I32: c_int = 6;

/// Size of the per-GPU workspace of `th_gemm_q4_noalloc`.
pub const TH_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

// safetensors dtypes (th_st_info)
pub const TH_ST_F64: c_int = 0;
pub const TH_ST_F32: c_int = 1;
pub const TH_ST_F16: c_int = 2;
pub const TH_ST_BF16: c_int = 3;

/// Opaque handles owned by the library.
#[repr(C)]
pub struct th_device {
    _private: [u8; 0],
}
#[repr(C)]
pub struct th_buffer {
    _private: [u8; 0],
}
#[repr(C)]
pub struct th_qweight {
    _private: [u8; 0],
}
#[repr(C)]
pub struct th_kernel {
    _private: [u8; 0],
}
#[repr(C)]
pub struct th_st_file {
    _private: [u8; 0],
}
#[repr(C)]
pub struct th_llama {
    _private: [u8; 0],
}
#[repr(C)]
pub struct th_sampler {
    _private: [u8; 0],
}
#[repr(C)]
pub struct th_moe {
    _private: [u8; 0],
}
#[repr(C)]
pub struct th_graph {
    _private: [u8; 0],
}

/// `Q8Block` (crates/tang-infer/src/quantize.rs:15-19) as a C struct.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct th_q8_block {
    pub scale: f32,
    pub values: [i8; 32],
}

/// `Q4Block` (quantize.rs:25-29): values[i] = (q[2i]+8) | (q[2i+1]+8) << 4.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct th_q4_block {
    pub scale: f32,
    pub values: [u8; 16],
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct th_llama_config {
    pub n_layers: c_int,
    pub d_model: c_int,
    pub n_heads: c_int,
    pub n_kv_heads: c_int,
    pub head_dim: c_int,
    pub d_ff: c_int,
    pub vocab: c_int,
    pub max_seq: c_int,
    pub eps: f32,
    pub rope_theta: f64,
}

/// `SamplingConfig` (crates/tang-infer/src/sampling.rs:6-20).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct th_sampling_config {
    pub temperature: f64,
    pub top_k: usize,
    pub top_p: f64,
    pub repetition_penalty: f64,
    pub stop_token: i64,
    pub max_tokens: usize,
}

// th_expr_node.op: the tang-expr node kinds (crates/tang-expr/src/node.rs:58-90)
pub const TH_EXPR_VAR: u32 = 0;
pub const TH_EXPR_LIT: u32 = 1;
pub const TH_EXPR_ADD: u32 = 2;
pub const TH_EXPR_MUL: u32 = 3;
pub const TH_EXPR_NEG: u32 = 4;
pub const TH_EXPR_RECIP: u32 = 5;
pub const TH_EXPR_SQRT: u32 = 6;
pub const TH_EXPR_SIN: u32 = 7;
pub const TH_EXPR_ATAN2: u32 = 8;
pub const TH_EXPR_EXP2: u32 = 9;
pub const TH_EXPR_LOG2: u32 = 10;
pub const TH_EXPR_SELECT: u32 = 11;

/// One node of an expression graph: operands are indices of earlier nodes
/// (`Var`: `a` is the input index; `Lit`: the value is `lit`).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct th_expr_node {
    pub op: u32,
    pub a: u32,
    pub b: u32,
    pub c: u32,
    pub lit: f64,
}

#[link(name = "tang_hip")]
extern "C" {
    pub fn th_last_error() -> *const c_char;
    pub fn th_device_count(n: *mut c_int) -> c_int;
    pub fn th_device_create(ordinal: c_int, out: *mut *mut th_device) -> c_int;
    pub fn th_device_destroy(dev: *mut th_device) -> c_int;
    pub fn th_sync(dev: *mut th_device) -> c_int;
    pub fn th_memory_info(dev: *mut th_device, free_bytes: *mut usize, total_bytes: *mut usize) -> c_int;
    pub fn th_timer_start(dev: *mut th_device) -> c_int;
    pub fn th_timer_stop(dev: *mut th_device, ms: *mut f32) -> c_int;
    pub fn th_capture_begin(dev: *mut th_device) -> c_int;
    pub fn th_capture_end(dev: *mut th_device, out: *mut *mut th_graph) -> c_int;
    pub fn th_graph_launch(g: *mut th_graph) -> c_int;
    pub fn th_graph_destroy(g: *mut th_graph) -> c_int;
    pub fn th_buffer_alloc(dev: *mut th_device, dtype: c_int, n: usize, out: *mut *mut th_buffer) -> c_int;
    pub fn th_buffer_free(buf: *mut th_buffer) -> c_int;
    pub fn th_buffer_upload(buf: *mut th_buffer, host: *const c_void, n: usize) -> c_int;
    pub fn th_buffer_download(buf: *mut th_buffer, host: *mut c_void, n: usize) -> c_int;
    pub fn th_buffer_info(buf: *const th_buffer, dtype: *mut c_int, n: *mut usize) -> c_int;
    pub fn th_buffer_zero(buf: *mut th_buffer) -> c_int;
    pub fn th_buffer_copy(dst: *mut th_buffer, src: *const th_buffer) -> c_int;
    pub fn th_buffer_copy_region(dst: *mut th_buffer, dst_offset: usize, src: *const th_buffer, src_offset: usize, n: usize) -> c_int;
    pub fn th_convert(dev: *mut th_device, src: *const th_buffer, dst: *mut th_buffer) -> c_int;
    pub fn th_q4_upload_blocks(dev: *mut th_device, blocks: *const th_q4_block, rows: usize, cols: usize, scale_dtype: c_int, out: *mut *mut th_qweight) -> c_int;
    pub fn th_q4_upload_packed(dev: *mut th_device, nib: *const u8, scales: *const c_void, scale_dtype: c_int, rows: usize, cols: usize, out: *mut *mut th_qweight) -> c_int;
    pub fn th_q8_upload_blocks(dev: *mut th_device, blocks: *const th_q8_block, rows: usize, cols: usize, out: *mut *mut th_qweight) -> c_int;
    pub fn th_q8_upload_rowwise(dev: *mut th_device, q: *const i8, row_scale: *const f32, rows: usize, cols: usize, out: *mut *mut th_qweight) -> c_int;
    pub fn th_q4_download_blocks(w: *const th_qweight, blocks: *mut th_q4_block) -> c_int;
    pub fn th_qweight_info(w: *const th_qweight, rows: *mut usize, cols: *mut usize, bits: *mut c_int) -> c_int;
    pub fn th_qweight_free(w: *mut th_qweight) -> c_int;
    pub fn th_quantize_q4(data: *const f32, rows: usize, cols: usize, out: *mut th_q4_block) -> c_int;
    pub fn th_quantize_q8(data: *const f32, rows: usize, cols: usize, out: *mut th_q8_block) -> c_int;
    pub fn th_st_open(path: *const c_char, out: *mut *mut th_st_file) -> c_int;
    pub fn th_st_close(f: *mut th_st_file) -> c_int;
    pub fn th_st_count(f: *const th_st_file, n: *mut usize) -> c_int;
    pub fn th_st_info(f: *const th_st_file, index: usize, name: *mut *const c_char, dtype: *mut c_int, ndim: *mut usize, shape: *mut usize, max_dims: usize) -> c_int;
    pub fn th_st_read_f32(f: *const th_st_file, name: *const c_char, out: *mut f32, n: usize) -> c_int;
    pub fn th_st_upload(dev: *mut th_device, f: *const th_st_file, name: *const c_char, dtype: c_int, out: *mut *mut th_buffer) -> c_int;
    pub fn th_st_upload_q4(dev: *mut th_device, f: *const th_st_file, name: *const c_char, out: *mut *mut th_qweight) -> c_int;
    pub fn th_st_upload_q8(dev: *mut th_device, f: *const th_st_file, name: *const c_char, out: *mut *mut th_qweight) -> c_int;
    pub fn th_gemm_q4(dev: *mut th_device, x: *const th_buffer, m: usize, w: *const th_qweight, y: *mut th_buffer) -> c_int;
    pub fn th_gemv_q8(dev: *mut th_device, x: *const th_buffer, m: usize, w: *const th_qweight, y: *mut th_buffer) -> c_int;
    pub fn th_gemm_q4_noalloc(dev: *mut th_device, x: *const th_buffer, m: usize, w: *const th_qweight, y: *mut th_buffer) -> c_int;
    pub fn th_bench_linear(dev: *mut th_device, x: *const th_buffer, m: usize, ws: *const *mut th_qweight, n_w: usize, y: *mut th_buffer, iters: usize, use_graph: c_int, ms: *mut f32) -> c_int;
    pub fn th_matmul_ex(dev: *mut th_device, a: *const th_buffer, b: *const th_buffer, m: usize, k: usize, n: usize, trans_a: c_int, trans_b: c_int, accumulate: c_int, c: *mut th_buffer) -> c_int;
    pub fn th_matmul(dev: *mut th_device, a: *const th_buffer, b: *const th_buffer, m: usize, k: usize, n: usize, c: *mut th_buffer) -> c_int;
    pub fn th_matmul_b_transposed(dev: *mut th_device, a: *const th_buffer, b: *const th_buffer, m: usize, k: usize, n: usize, c: *mut th_buffer) -> c_int;
    pub fn th_transpose_2d(dev: *mut th_device, in_: *const th_buffer, rows: usize, cols: usize, out: *mut th_buffer) -> c_int;
    pub fn th_reduce_sum(dev: *mut th_device, in_: *const th_buffer, shape: *const usize, ndim: usize, axis: usize, accumulate: c_int, out: *mut th_buffer) -> c_int;
    pub fn th_bias_add(dev: *mut th_device, matrix: *const th_buffer, bias: *const th_buffer, numel: usize, dim: usize, out: *mut th_buffer) -> c_int;
    pub fn th_add_assign(dev: *mut th_device, dst: *mut th_buffer, src: *const th_buffer) -> c_int;
    pub fn th_expr_source(nodes: *const th_expr_node, n_nodes: usize, output: u32, n_inputs: usize, buf: *mut c_char, cap: usize, len: *mut usize) -> c_int;
    pub fn th_elementwise_expr(dev: *mut th_device, nodes: *const th_expr_node, n_nodes: usize, output: u32, inputs: *const *const th_buffer, n_inputs: usize, numel: usize, out: *mut th_buffer) -> c_int;
    pub fn th_kernel_compile(dev: *mut th_device, source: *const c_char, entry: *const c_char, out: *mut *mut th_kernel) -> c_int;
    pub fn th_kernel_free(k: *mut th_kernel) -> c_int;
    pub fn th_elementwise(k: *mut th_kernel, inputs: *const *const th_buffer, n_inputs: usize, numel: usize, out: *mut th_buffer) -> c_int;
    pub fn th_rms_norm(dev: *mut th_device, x: *const th_buffer, weight: *const th_buffer, n_groups: usize, dim: usize, eps: f32, out: *mut th_buffer) -> c_int;
    pub fn th_rms_norm_residual(dev: *mut th_device, in_: *const th_buffer, residual: *const th_buffer, weight: *const th_buffer, n_groups: usize, dim: usize, eps: f32, out: *mut th_buffer, sum_out: *mut th_buffer) -> c_int;
    pub fn th_rope_tables(head_dim: usize, max_seq: usize, base: f64, cos_table: *mut f32, sin_table: *mut f32) -> c_int;
    pub fn th_rope_forward(dev: *mut th_device, in_: *const th_buffer, cos_buf: *const th_buffer, sin_buf: *const th_buffer, seq_len: usize, n_heads: usize, head_dim: usize, start_pos: usize, out: *mut th_buffer) -> c_int;
    pub fn th_kv_attention(dev: *mut th_device, q: *const th_buffer, k_cache: *const th_buffer, v_cache: *const th_buffer, cache_start: usize, q_len: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize, out: *mut th_buffer) -> c_int;
    pub fn th_swiglu(dev: *mut th_device, gate: *const th_buffer, up: *const th_buffer, n: usize, out: *mut th_buffer) -> c_int;
    pub fn th_swiglu_bf16(dev: *mut th_device, gate: *const th_buffer, up: *const th_buffer, n: usize, out: *mut th_buffer) -> c_int;
    pub fn th_add(dev: *mut th_device, a: *const th_buffer, b: *const th_buffer, n: usize, out: *mut th_buffer) -> c_int;
    pub fn th_embedding(dev: *mut th_device, weight: *const th_buffer, ids: *const th_buffer, seq_len: usize, dim: usize, out: *mut th_buffer) -> c_int;
    pub fn th_softmax(dev: *mut th_device, x: *const th_buffer, n_rows: usize, row_len: usize, out: *mut th_buffer) -> c_int;
    pub fn th_argmax(dev: *mut th_device, x: *const th_buffer, n_rows: usize, n: usize, out: *mut th_buffer) -> c_int;
    pub fn th_llama_create(dev: *mut th_device, cfg: *const th_llama_config, out: *mut *mut th_llama) -> c_int;
    pub fn th_llama_destroy(m: *mut th_llama) -> c_int;
    pub fn th_llama_init_synthetic(m: *mut th_llama, seed: u64) -> c_int;
    pub fn th_llama_load_safetensors(m: *mut th_llama, f: *const th_st_file) -> c_int;
    pub fn th_llama_fill_kv_synthetic(m: *mut th_llama, len: usize, seed: u64) -> c_int;
    pub fn th_llama_generate(m: *mut th_llama, token: i32, pos: usize, n_steps: usize, tokens_out: *mut i32, last_logits: *mut f32) -> c_int;
    pub fn th_llama_step_device(m: *mut th_llama, pos: usize) -> c_int;
    pub fn th_llama_set_token(m: *mut th_llama, token: i32) -> c_int;
    pub fn th_llama_time_steps(m: *mut th_llama, token: i32, pos: usize, n_steps: usize, ms: *mut f32) -> c_int;
    pub fn th_llama_prefill(m: *mut th_llama, tokens: *const i32, n: usize, pos: usize, next_token: *mut i32, last_logits: *mut f32) -> c_int;
    pub fn th_llama_time_prefill(m: *mut th_llama, tokens: *const i32, n: usize, pos: usize, ms: *mut f32) -> c_int;
    pub fn th_sampler_create(cfg: *const th_sampling_config, seed: u64, out: *mut *mut th_sampler) -> c_int;
    pub fn th_sampler_destroy(s: *mut th_sampler) -> c_int;
    pub fn th_sampler_sample(s: *mut th_sampler, logits: *const f32, vocab: usize, past: *const i32, n_past: usize, token: *mut i32) -> c_int;
    pub fn th_llama_generate_sampled(m: *mut th_llama, s: *mut th_sampler, prompt: *const i32, n_prompt: usize, pos: usize, tokens_out: *mut i32, n_out: *mut usize) -> c_int;
    pub fn th_moe_create(dev: *mut th_device, d_model: usize, d_ff: usize, n_experts: usize, n_shared: usize, top_k: usize, out: *mut *mut th_moe) -> c_int;
    pub fn th_moe_destroy(moe: *mut th_moe) -> c_int;
    pub fn th_moe_init_synthetic(moe: *mut th_moe, seed: u64) -> c_int;
    pub fn th_moe_forward(moe: *mut th_moe, h: *const th_buffer, T: usize, out: *mut th_buffer, topk_idx: *mut th_buffer, topk_w: *mut th_buffer) -> c_int;
    pub fn th_mla_decode(dev: *mut th_device, q_nope: *const th_buffer, q_rope: *const th_buffer, cache: *const th_buffer, B: usize, H: usize, L: usize, dn: usize, dr: usize, r: usize, dv: usize, w_uk: *const th_qweight, w_uv: *const th_qweight, sm_scale: f32, out: *mut th_buffer) -> c_int;
    pub fn th_synth_seed(base: u64, layer: u64, tensor: u64) -> u64;
    pub fn th_synth_q4(seed: u64, rows: usize, cols: usize, smin: f32, smax: f32, nib: *mut u8, scales_f16: *mut u16) -> c_int;
    pub fn th_synth_q8_rowwise(seed: u64, rows: usize, cols: usize, smin: f32, smax: f32, q: *mut i8, row_scale: *mut f32) -> c_int;
    pub fn th_synth_normal(seed: u64, n: usize, std: f32, dtype: c_int, out: *mut c_void) -> c_int;
}
