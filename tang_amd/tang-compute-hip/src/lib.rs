//! tang-compute-hip: a `tang_compute::ComputeDevice` backend for AMD MI355X
//! (gfx950), forwarding every operator to the C ABI of `libtang_hip.so`
//! (`include/tang_hip.h`, raw declarations in `ffi`).
//!
//! Model code written against `ComputeDevice` (crates/tang-compute/src/device.rs)
//! runs on this device unchanged: buffers are device allocations, operators
//! are HIP kernels on the device's one stream, `download` and `sync` are the
//! synchronisation points (device.rs:75, :367).  The quantized decode path the
//! reference runs on the CPU (`q4_matvec` / `q8_matvec`,
//! crates/tang-infer/src/quantize.rs:227-289) is the `QuantizedCompute`
//! extension trait below; `LatentAttention` adds MLA decode, `HipMoe` a MoE
//! layer, and `HipLlama` the device-resident decode engine whose `generate`
//! replaces `tang_infer::generate` (crates/tang-infer/src/sampling.rs:229-256)
//! for a Llama-shaped model.
//!
//! Errors panic with the library's message, as the reference backends do
//! (e.g. crates/tang-compute/src/cuda.rs:385).  Like `CudaComputeDevice`, the
//! device is `Send` but not `Sync` (one device per thread).  The engines
//! borrow the device they run on, so it outlives them.
//!
//! Training-only operators (the backward passes, cross-entropy, AdamW) are
//! outside this backend, which serves the inference path: they panic with
//! that reason rather than fall back to the host.
#![allow(clippy::too_many_arguments)]

pub mod ffi;

use std::ffi::{CStr, CString};
use std::marker::PhantomData;
use std::path::Path;
use std::os::raw::{c_int, c_void};
use std::ptr;

use tang_compute::{ComputeBuffer, ComputeDevice};
use tang_expr::codegen::Dialect;
use tang_expr::node::{ExprId, Node};
use tang_expr::trace;
use tang_infer::quantize::{QuantizedQ4, QuantizedQ8};
use tang_infer::SamplingConfig;

fn last_error() -> String {
    unsafe { CStr::from_ptr(ffi::th_last_error()).to_string_lossy().into_owned() }
}

/// Panic with the library's message unless `rc` is `TH_OK`.
#[track_caller]
fn check(rc: c_int) {
    if rc != ffi::TH_OK {
        panic!("tang-hip error {}: {}", rc, last_error());
    }
}

// ---------------------------------------------------------------------------
// Buffers
// ---------------------------------------------------------------------------

/// A device allocation.  `ComputeDevice` buffers hold f32 values; token ids
/// from `upload_u32` are u32 on the device and read back as their f32 bit
/// patterns, as the reference stores them (crates/tang-compute/src/cpu.rs:51-56).
pub struct HipBuffer {
    raw: *mut ffi::th_buffer,
    len: usize,
    dtype: c_int,
}

unsafe impl Send for HipBuffer {}

impl HipBuffer {
    pub fn raw(&self) -> *mut ffi::th_buffer {
        self.raw
    }
    pub fn dtype(&self) -> c_int {
        self.dtype
    }
}

impl Drop for HipBuffer {
    fn drop(&mut self) {
        // drains the stream before the memory returns to HIP
        unsafe {
            ffi::th_buffer_free(self.raw);
        }
    }
}

impl ComputeBuffer for HipBuffer {
    fn len(&self) -> usize {
        self.len
    }

    fn to_vec(&self) -> Vec<f32> {
        match self.dtype {
            ffi::TH_U32 | ffi::TH_I32 | ffi::TH_F32 => {
                let mut out = vec![0.0f32; self.len];
                check(unsafe { ffi::th_buffer_download(self.raw, out.as_mut_ptr() as *mut c_void, self.len) });
                out
            }
            ffi::TH_BF16 => {
                let mut h = vec![0u16; self.len];
                check(unsafe { ffi::th_buffer_download(self.raw, h.as_mut_ptr() as *mut c_void, self.len) });
                h.iter().map(|&b| f32::from_bits((b as u32) << 16)).collect()
            }
            other => panic!("tang-hip: to_vec on a buffer of dtype {}", other),
        }
    }
}

// ---------------------------------------------------------------------------
// Device
// ---------------------------------------------------------------------------

/// One MI355X (HIP device ordinal) with one stream.
pub struct HipComputeDevice {
    dev: *mut ffi::th_device,
}

unsafe impl Send for HipComputeDevice {}

impl HipComputeDevice {
    /// `CudaComputeDevice::new` (cuda.rs:151) for a HIP device ordinal.
    pub fn new(ordinal: usize) -> Self {
        let mut dev = ptr::null_mut();
        check(unsafe { ffi::th_device_create(ordinal as c_int, &mut dev) });
        HipComputeDevice { dev }
    }

    pub fn raw(&self) -> *mut ffi::th_device {
        self.dev
    }

    fn buffer(&self, dtype: c_int, len: usize) -> HipBuffer {
        let mut raw = ptr::null_mut();
        check(unsafe { ffi::th_buffer_alloc(self.dev, dtype, len, &mut raw) });
        HipBuffer { raw, len, dtype }
    }

    fn zeros(&self, len: usize) -> HipBuffer {
        let b = self.buffer(ffi::TH_F32, len);
        check(unsafe { ffi::th_buffer_zero(b.raw) });
        b
    }

    fn matmul_ex(&self, a: &HipBuffer, b: &HipBuffer, c: &mut HipBuffer, m: usize, k: usize, n: usize, ta: bool,
                 tb: bool, accumulate: bool) {
        check(unsafe {
            ffi::th_matmul_ex(self.dev, a.raw, b.raw, m, k, n, ta as c_int, tb as c_int, accumulate as c_int, c.raw)
        });
    }
}

impl Drop for HipComputeDevice {
    fn drop(&mut self) {
        // buffers still alive keep the library's device state until they drop
        unsafe {
            ffi::th_device_destroy(self.dev);
        }
    }
}

/// A tang-expr node (node.rs:58-90) as the C ABI's `th_expr_node`.
fn expr_node(n: &Node) -> ffi::th_expr_node {
    let mk = |op: u32, a: ExprId, b: ExprId, c: ExprId| ffi::th_expr_node { op, a: a.index(), b: b.index(),
                                                                            c: c.index(), lit: 0.0 };
    let z = ExprId::ZERO;
    match *n {
        Node::Var(i) => ffi::th_expr_node { op: ffi::TH_EXPR_VAR, a: i as u32, b: 0, c: 0, lit: 0.0 },
        Node::Lit(bits) => ffi::th_expr_node { op: ffi::TH_EXPR_LIT, a: 0, b: 0, c: 0, lit: f64::from_bits(bits) },
        Node::Add(a, b) => mk(ffi::TH_EXPR_ADD, a, b, z),
        Node::Mul(a, b) => mk(ffi::TH_EXPR_MUL, a, b, z),
        Node::Neg(a) => mk(ffi::TH_EXPR_NEG, a, z, z),
        Node::Recip(a) => mk(ffi::TH_EXPR_RECIP, a, z, z),
        Node::Sqrt(a) => mk(ffi::TH_EXPR_SQRT, a, z, z),
        Node::Sin(a) => mk(ffi::TH_EXPR_SIN, a, z, z),
        Node::Atan2(y, x) => mk(ffi::TH_EXPR_ATAN2, y, x, z),
        Node::Exp2(a) => mk(ffi::TH_EXPR_EXP2, a, z, z),
        Node::Log2(a) => mk(ffi::TH_EXPR_LOG2, a, z, z),
        Node::Select(c, a, b) => mk(ffi::TH_EXPR_SELECT, c, a, b),
    }
}

fn training_only(op: &str) -> ! {
    panic!(
        "tang-hip: {} is a training operator; this backend implements the inference path \
         (run training on CpuDevice or CudaComputeDevice)",
        op
    )
}

impl ComputeDevice for HipComputeDevice {
    type Buffer = HipBuffer;

    /// No `Dialect` variant names HIP, and this device consumes no shader
    /// text: `elementwise` hands the traced `ExprGraph` itself to the library,
    /// which generates gfx950 code for it.  `C` is reported because the
    /// device evaluates a graph as the C / CPU path does (f64 per node, one
    /// rounding to f32 at the end).
    fn dialect(&self) -> Dialect {
        Dialect::C
    }

    fn total_memory_bytes(&self) -> usize {
        let (mut free, mut total) = (0usize, 0usize);
        check(unsafe { ffi::th_memory_info(self.dev, &mut free, &mut total) });
        total
    }

    fn free_memory_bytes(&self) -> usize {
        let (mut free, mut total) = (0usize, 0usize);
        check(unsafe { ffi::th_memory_info(self.dev, &mut free, &mut total) });
        free
    }

    /// Dense FP32 matrix peak of MI355X (MFMA), for MFU figures.
    fn peak_flops_f32(&self) -> Option<f64> {
        Some(157.3e12)
    }

    // -- buffer lifecycle (device.rs:44-80) --

    fn upload(&self, data: &[f32]) -> HipBuffer {
        let b = self.buffer(ffi::TH_F32, data.len());
        check(unsafe { ffi::th_buffer_upload(b.raw, data.as_ptr() as *const c_void, data.len()) });
        b
    }

    fn upload_u32(&self, data: &[u32]) -> HipBuffer {
        let b = self.buffer(ffi::TH_U32, data.len());
        check(unsafe { ffi::th_buffer_upload(b.raw, data.as_ptr() as *const c_void, data.len()) });
        b
    }

    fn alloc(&self, len: usize) -> HipBuffer {
        self.zeros(len)
    }

    fn alloc_uninit(&self, len: usize) -> HipBuffer {
        self.buffer(ffi::TH_F32, len)
    }

    fn download(&self, buf: &HipBuffer) -> Vec<f32> {
        buf.to_vec()
    }

    fn upload_into_f32(&self, buf: &mut HipBuffer, data: &[f32]) {
        if buf.len == data.len() && buf.dtype == ffi::TH_F32 {
            check(unsafe { ffi::th_buffer_upload(buf.raw, data.as_ptr() as *const c_void, data.len()) });
        } else {
            *buf = self.upload(data);
        }
    }

    fn upload_into_u32(&self, buf: &mut HipBuffer, data: &[u32]) {
        if buf.len == data.len() && buf.dtype == ffi::TH_U32 {
            check(unsafe { ffi::th_buffer_upload(buf.raw, data.as_ptr() as *const c_void, data.len()) });
        } else {
            *buf = self.upload_u32(data);
        }
    }

    // -- element-wise via tang-expr (device.rs:93; the CPU semantics cpu.rs:68-97) --

    /// Traces the closure as every backend does (`trace`, tang-expr/src/lib.rs:61)
    /// and passes the graph's nodes, in graph order, to `th_elementwise_expr`:
    /// the library generates the HIP kernel from them, compiles it once per
    /// distinct graph and runs it.
    fn elementwise(&self, inputs: &[&HipBuffer], numel: usize, f: &dyn Fn(&[ExprId]) -> ExprId) -> HipBuffer {
        let n_inputs = inputs.len();
        let (graph, output) = trace(|| {
            let vars: Vec<ExprId> = (0..n_inputs as u16).map(ExprId::var).collect();
            f(&vars)
        });
        let nodes: Vec<ffi::th_expr_node> = graph.nodes_slice().iter().map(expr_node).collect();
        let raw: Vec<*const ffi::th_buffer> = inputs.iter().map(|b| b.raw as *const ffi::th_buffer).collect();
        let out = self.buffer(ffi::TH_F32, numel);
        check(unsafe {
            ffi::th_elementwise_expr(self.dev, nodes.as_ptr(), nodes.len(), output.index(), raw.as_ptr(), n_inputs,
                                     numel, out.raw)
        });
        out
    }

    // -- dense operators --

    fn matmul(&self, a: &HipBuffer, b: &HipBuffer, m: usize, k: usize, n: usize) -> HipBuffer {
        let mut c = self.buffer(ffi::TH_F32, m * n);
        self.matmul_ex(a, b, &mut c, m, k, n, false, false, false);
        c
    }

    fn matmul_accumulate(&self, a: &HipBuffer, b: &HipBuffer, c: &mut HipBuffer, m: usize, k: usize, n: usize) {
        self.matmul_ex(a, b, c, m, k, n, false, false, true);
    }

    fn matmul_b_transposed(&self, a: &HipBuffer, b: &HipBuffer, m: usize, k: usize, n: usize) -> HipBuffer {
        let mut c = self.buffer(ffi::TH_F32, m * n);
        self.matmul_ex(a, b, &mut c, m, k, n, false, true, false);
        c
    }

    fn matmul_a_transposed(&self, a: &HipBuffer, b: &HipBuffer, m: usize, k: usize, n: usize) -> HipBuffer {
        let mut c = self.buffer(ffi::TH_F32, m * n);
        self.matmul_ex(a, b, &mut c, m, k, n, true, false, false);
        c
    }

    fn matmul_accumulate_a_transposed(&self, a: &HipBuffer, b: &HipBuffer, c: &mut HipBuffer, m: usize, k: usize,
                                      n: usize) {
        self.matmul_ex(a, b, c, m, k, n, true, false, true);
    }

    fn transpose_2d(&self, buf: &HipBuffer, rows: usize, cols: usize) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, rows * cols);
        check(unsafe { ffi::th_transpose_2d(self.dev, buf.raw, rows, cols, out.raw) });
        out
    }

    fn reduce_sum(&self, data: &HipBuffer, shape: &[usize], axis: usize) -> HipBuffer {
        assert!(axis < shape.len());
        let n_out: usize = shape.iter().enumerate().filter(|&(i, _)| i != axis).map(|(_, &d)| d).product();
        let out = self.buffer(ffi::TH_F32, n_out);
        check(unsafe { ffi::th_reduce_sum(self.dev, data.raw, shape.as_ptr(), shape.len(), axis, 0, out.raw) });
        out
    }

    fn reduce_sum_accumulate(&self, data: &HipBuffer, shape: &[usize], axis: usize, dst: &mut HipBuffer) {
        check(unsafe { ffi::th_reduce_sum(self.dev, data.raw, shape.as_ptr(), shape.len(), axis, 1, dst.raw) });
    }

    fn bias_add(&self, matrix: &HipBuffer, bias: &HipBuffer, numel: usize, dim: usize) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, numel);
        check(unsafe { ffi::th_bias_add(self.dev, matrix.raw, bias.raw, numel, dim, out.raw) });
        out
    }

    fn add_assign(&self, dst: &mut HipBuffer, src: &HipBuffer) {
        check(unsafe { ffi::th_add_assign(self.dev, dst.raw, src.raw) });
    }

    fn zero_buffer(&self, buf: &mut HipBuffer) {
        check(unsafe { ffi::th_buffer_zero(buf.raw) });
    }

    fn copy_buffer(&self, src: &HipBuffer) -> HipBuffer {
        let out = self.buffer(src.dtype, src.len);
        check(unsafe { ffi::th_buffer_copy(out.raw, src.raw) });
        out
    }

    fn slice_buffer(&self, buf: &HipBuffer, offset: usize, len: usize) -> HipBuffer {
        let out = self.buffer(buf.dtype, len);
        check(unsafe { ffi::th_buffer_copy_region(out.raw, 0, buf.raw, offset, len) });
        out
    }

    fn write_into(&self, dst: &mut HipBuffer, offset: usize, src: &HipBuffer) {
        check(unsafe { ffi::th_buffer_copy_region(dst.raw, offset, src.raw, 0, src.len) });
    }

    fn extract_columns(&self, buf: &HipBuffer, batch: usize, total_cols: usize, col_start: usize,
                       col_count: usize) -> HipBuffer {
        let out = self.buffer(buf.dtype, batch * col_count);
        for row in 0..batch {
            check(unsafe {
                ffi::th_buffer_copy_region(out.raw, row * col_count, buf.raw, row * total_cols + col_start, col_count)
            });
        }
        out
    }

    fn concat_columns(&self, dst: &mut HipBuffer, src: &HipBuffer, batch: usize, total_cols: usize,
                      col_start: usize, col_count: usize) {
        for row in 0..batch {
            check(unsafe {
                ffi::th_buffer_copy_region(dst.raw, row * total_cols + col_start, src.raw, row * col_count, col_count)
            });
        }
    }

    // -- decode operators --

    fn softmax(&self, data: &HipBuffer, n_rows: usize, row_len: usize) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, n_rows * row_len);
        check(unsafe { ffi::th_softmax(self.dev, data.raw, n_rows, row_len, out.raw) });
        out
    }

    fn rms_norm(&self, data: &HipBuffer, weight: &HipBuffer, n_groups: usize, dim: usize, eps: f32) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, n_groups * dim);
        check(unsafe { ffi::th_rms_norm(self.dev, data.raw, weight.raw, n_groups, dim, eps, out.raw) });
        out
    }

    fn rms_norm_residual(&self, input: &HipBuffer, residual: &HipBuffer, weight: &HipBuffer, n_groups: usize,
                         dim: usize, eps: f32) -> (HipBuffer, HipBuffer) {
        let out = self.buffer(ffi::TH_F32, n_groups * dim);
        let sum = self.buffer(ffi::TH_F32, n_groups * dim);
        check(unsafe {
            ffi::th_rms_norm_residual(self.dev, input.raw, residual.raw, weight.raw, n_groups, dim, eps, out.raw,
                                      sum.raw)
        });
        (out, sum)
    }

    fn embedding(&self, weight: &HipBuffer, ids: &HipBuffer, seq_len: usize, dim: usize) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, seq_len * dim);
        check(unsafe { ffi::th_embedding(self.dev, weight.raw, ids.raw, seq_len, dim, out.raw) });
        out
    }

    fn rope_forward(&self, input: &HipBuffer, cos_table: &[f32], sin_table: &[f32], seq_len: usize,
                    n_heads: usize, head_dim: usize, start_pos: usize) -> HipBuffer {
        let cos_buf = self.upload(cos_table);
        let sin_buf = self.upload(sin_table);
        self.rope_forward_cached(input, &cos_buf, &sin_buf, seq_len, n_heads, head_dim, start_pos)
    }

    fn rope_forward_cached(&self, input: &HipBuffer, cos_buf: &HipBuffer, sin_buf: &HipBuffer, seq_len: usize,
                           n_heads: usize, head_dim: usize, start_pos: usize) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, seq_len * n_heads * head_dim);
        check(unsafe {
            ffi::th_rope_forward(self.dev, input.raw, cos_buf.raw, sin_buf.raw, seq_len, n_heads, head_dim,
                                 start_pos, out.raw)
        });
        out
    }

    /// Causal self-attention = kv_attention with an empty cache prefix:
    /// query i attends keys 0..=i in both (device.rs:147-158, :163-180).
    fn causal_attention(&self, q: &HipBuffer, k: &HipBuffer, v: &HipBuffer, seq_len: usize, n_heads: usize,
                        n_kv_heads: usize, head_dim: usize) -> HipBuffer {
        self.kv_attention(q, k, v, 0, seq_len, n_heads, n_kv_heads, head_dim)
    }

    fn kv_attention(&self, q: &HipBuffer, k_cache: &HipBuffer, v_cache: &HipBuffer, cache_start: usize,
                    q_len: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, q_len * n_heads * head_dim);
        check(unsafe {
            ffi::th_kv_attention(self.dev, q.raw, k_cache.raw, v_cache.raw, cache_start, q_len, n_heads,
                                 n_kv_heads, head_dim, out.raw)
        });
        out
    }

    fn add_tensors_buf(&self, a: &HipBuffer, b: &HipBuffer, numel: usize) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, numel);
        check(unsafe { ffi::th_add(self.dev, a.raw, b.raw, numel, out.raw) });
        out
    }

    fn swiglu_fused_buf(&self, gate: &HipBuffer, up: &HipBuffer, numel: usize) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, numel);
        check(unsafe { ffi::th_swiglu(self.dev, gate.raw, up.raw, numel, out.raw) });
        out
    }

    fn sync(&self) {
        check(unsafe { ffi::th_sync(self.dev) });
    }

    // -- training operators (required by the trait; not served here) --

    fn softmax_backward(&self, _softmax_out: &HipBuffer, _grad_output: &HipBuffer, _n_rows: usize,
                        _row_len: usize) -> HipBuffer {
        training_only("softmax_backward")
    }

    fn rms_norm_backward(&self, _input: &HipBuffer, _weight: &HipBuffer, _grad_output: &HipBuffer, _n_groups: usize,
                         _dim: usize, _eps: f32) -> (HipBuffer, HipBuffer) {
        training_only("rms_norm_backward")
    }

    fn embedding_backward(&self, _grad_output: &HipBuffer, _ids: &HipBuffer, _vocab_size: usize, _seq_len: usize,
                          _dim: usize) -> HipBuffer {
        training_only("embedding_backward")
    }

    fn causal_attention_backward(&self, _grad_output: &HipBuffer, _q: &HipBuffer, _k: &HipBuffer, _v: &HipBuffer,
                                 _seq_len: usize, _n_heads: usize, _n_kv_heads: usize,
                                 _head_dim: usize) -> (HipBuffer, HipBuffer, HipBuffer) {
        training_only("causal_attention_backward")
    }

    fn cross_entropy_forward_backward(&self, _logits: &HipBuffer, _targets: &HipBuffer, _n_positions: usize,
                                      _vocab_size: usize, _pad_id: u32) -> (f32, HipBuffer) {
        training_only("cross_entropy_forward_backward")
    }

    fn adamw_step(&self, _param: &mut HipBuffer, _grad: &HipBuffer, _m: &mut HipBuffer, _v: &mut HipBuffer,
                  _lr: f32, _beta1: f32, _beta2: f32, _eps: f32, _weight_decay: f32, _step_t: usize) {
        training_only("adamw_step")
    }
}

// ---------------------------------------------------------------------------
// Quantized extension (no counterpart in the reference trait)
// ---------------------------------------------------------------------------

/// A quantized weight matrix in the device layout.
pub struct HipQWeight {
    raw: *mut ffi::th_qweight,
    pub rows: usize,
    pub cols: usize,
    pub bits: u32,
}

unsafe impl Send for HipQWeight {}

impl Drop for HipQWeight {
    fn drop(&mut self) {
        unsafe {
            ffi::th_qweight_free(self.raw);
        }
    }
}

/// The quantized linear of tang-infer's decode (`q4_matvec` / `q8_matvec`,
/// crates/tang-infer/src/quantize.rs:227-289) as device operators:
/// y[m][n] = sum_k x[m][k] * dequant(W)[n][k], i.e. `matmul_b_transposed`
/// with a quantized B, f32 accumulation.
pub trait QuantizedCompute: ComputeDevice {
    type QWeight;
    /// A `[rows, cols]` `QuantizedQ4` (quantize_matrix_q4 layout); f32 block scales kept.
    fn upload_q4(&self, w: &QuantizedQ4) -> Self::QWeight;
    /// A `[rows, cols]` `QuantizedQ8`.
    fn upload_q8(&self, w: &QuantizedQ8) -> Self::QWeight;
    /// y = x . W^T for m activation rows (f32 or bf16 buffers of [m][cols]).
    fn quantized_matmul(&self, x: &Self::Buffer, m: usize, w: &Self::QWeight) -> Self::Buffer;
}

fn matrix_shape(shape: &[usize]) -> (usize, usize) {
    match shape {
        [rows, cols] => (*rows, *cols),
        [cols] => (1, *cols),
        _ => panic!("tang-hip: quantized weights must be 1-D or 2-D, got {:?}", shape),
    }
}

impl QuantizedCompute for HipComputeDevice {
    type QWeight = HipQWeight;

    fn upload_q4(&self, w: &QuantizedQ4) -> HipQWeight {
        let (rows, cols) = matrix_shape(&w.shape);
        assert_eq!(w.blocks.len(), rows * ((cols + 31) / 32), "block count does not match the shape");
        let blocks: Vec<ffi::th_q4_block> =
            w.blocks.iter().map(|b| ffi::th_q4_block { scale: b.scale, values: b.values }).collect();
        let mut raw = ptr::null_mut();
        check(unsafe { ffi::th_q4_upload_blocks(self.dev, blocks.as_ptr(), rows, cols, ffi::TH_F32, &mut raw) });
        HipQWeight { raw, rows, cols, bits: 4 }
    }

    fn upload_q8(&self, w: &QuantizedQ8) -> HipQWeight {
        let (rows, cols) = matrix_shape(&w.shape);
        assert_eq!(w.blocks.len(), rows * ((cols + 31) / 32), "block count does not match the shape");
        let blocks: Vec<ffi::th_q8_block> =
            w.blocks.iter().map(|b| ffi::th_q8_block { scale: b.scale, values: b.values }).collect();
        let mut raw = ptr::null_mut();
        check(unsafe { ffi::th_q8_upload_blocks(self.dev, blocks.as_ptr(), rows, cols, &mut raw) });
        HipQWeight { raw, rows, cols, bits: 8 }
    }

    fn quantized_matmul(&self, x: &HipBuffer, m: usize, w: &HipQWeight) -> HipBuffer {
        let y = self.buffer(ffi::TH_F32, m * w.rows);
        if w.bits == 4 {
            check(unsafe { ffi::th_gemm_q4(self.dev, x.raw, m, w.raw, y.raw) });
        } else {
            check(unsafe { ffi::th_gemv_q8(self.dev, x.raw, m, w.raw, y.raw) });
        }
        y
    }
}

impl HipComputeDevice {
    /// A copy of `src` in another element type (`ffi::TH_F32`, `TH_BF16`,
    /// `TH_F16`): f32 -> bf16 rounds as crates/tang-compute/src/cuda.rs:22-27.
    pub fn convert(&self, src: &HipBuffer, dtype: c_int) -> HipBuffer {
        let out = self.buffer(dtype, src.len);
        check(unsafe { ffi::th_convert(self.dev, src.raw, out.raw) });
        out
    }

    /// An int8 matrix with one f32 scale per row (the MLA projections of
    /// BASELINE config 5): `q` is `[rows][cols]` row-major.
    pub fn upload_q8_rowwise(&self, q: &[i8], row_scale: &[f32], rows: usize, cols: usize) -> HipQWeight {
        assert_eq!(q.len(), rows * cols, "q must be [rows][cols]");
        assert_eq!(row_scale.len(), rows, "one scale per row");
        let mut raw = ptr::null_mut();
        check(unsafe { ffi::th_q8_upload_rowwise(self.dev, q.as_ptr(), row_scale.as_ptr(), rows, cols, &mut raw) });
        HipQWeight { raw, rows, cols, bits: 8 }
    }
}

// ---------------------------------------------------------------------------
// MLA decode (no counterpart in the reference)
// ---------------------------------------------------------------------------

/// Absorbed multi-head latent attention for one decode position per
/// sequence (DeepSeek-V2 shape): for each sequence b and head h,
/// scores_j = (W_UK^T q_nope . c_j + q_rope . k_rope_j) * sm_scale over the
/// cache rows j = [c_j ; k_rope_j], softmax, o = W_UV (sum_j p_j c_j).
pub trait LatentAttention: QuantizedCompute {
    /// q_nope f32 `[B][H][dn]`, q_rope f32 `[B][H][dr]`, cache bf16
    /// `[B][L][r + dr]`, w_uk rowwise int8 `[H*r][dn]`, w_uv rowwise int8
    /// `[H*dv][r]`; returns f32 `[B][H][dv]`.
    fn mla_decode(&self, q_nope: &Self::Buffer, q_rope: &Self::Buffer, cache: &Self::Buffer, b: usize, h: usize,
                  l: usize, dn: usize, dr: usize, r: usize, dv: usize, w_uk: &Self::QWeight, w_uv: &Self::QWeight,
                  sm_scale: f32) -> Self::Buffer;
}

impl LatentAttention for HipComputeDevice {
    fn mla_decode(&self, q_nope: &HipBuffer, q_rope: &HipBuffer, cache: &HipBuffer, b: usize, h: usize, l: usize,
                  dn: usize, dr: usize, r: usize, dv: usize, w_uk: &HipQWeight, w_uv: &HipQWeight,
                  sm_scale: f32) -> HipBuffer {
        let out = self.buffer(ffi::TH_F32, b * h * dv);
        check(unsafe {
            ffi::th_mla_decode(self.dev, q_nope.raw, q_rope.raw, cache.raw, b, h, l, dn, dr, r, dv, w_uk.raw, w_uv.raw,
                               sm_scale, out.raw)
        });
        out
    }
}

// ---------------------------------------------------------------------------
// MoE layer (no counterpart in the reference)
// ---------------------------------------------------------------------------

/// The outputs of one MoE forward.
pub struct MoeOutput {
    /// f32 `[T][d_model]`.
    pub out: HipBuffer,
    /// i32 `[T][top_k]`: routed experts, probability descending (ties: lower index).
    pub topk_idx: HipBuffer,
    /// f32 `[T][top_k]`: their softmax probabilities (not renormalised).
    pub topk_w: HipBuffer,
}

/// A DeepSeek-style MoE layer: f32 router `[E][d]`, softmax over the router
/// logits, top-k routed SwiGLU experts weighted by their probabilities, plus
/// `n_shared` always-on experts; expert linears int4 group-32.
pub struct HipMoe<'d> {
    raw: *mut ffi::th_moe,
    pub d_model: usize,
    pub top_k: usize,
    dev: &'d HipComputeDevice,
}

impl<'d> HipMoe<'d> {
    pub fn new(dev: &'d HipComputeDevice, d_model: usize, d_ff: usize, n_experts: usize, n_shared: usize,
               top_k: usize) -> Self {
        let mut raw = ptr::null_mut();
        check(unsafe { ffi::th_moe_create(dev.dev, d_model, d_ff, n_experts, n_shared, top_k, &mut raw) });
        HipMoe { raw, d_model, top_k, dev }
    }

    /// Seeded synthetic weights (router N(0, 0.02), experts as th_synth_q4).
    pub fn init_synthetic(&mut self, seed: u64) {
        check(unsafe { ffi::th_moe_init_synthetic(self.raw, seed) });
    }

    /// `h`: `[t][d_model]` activations, f32 (rounded to bf16 here) or bf16.
    pub fn forward(&self, h: &HipBuffer, t: usize) -> MoeOutput {
        let hb;
        let h = if h.dtype == ffi::TH_BF16 {
            h
        } else {
            hb = self.dev.convert(h, ffi::TH_BF16);
            &hb
        };
        let out = self.dev.buffer(ffi::TH_F32, t * self.d_model);
        let topk_idx = self.dev.buffer(ffi::TH_I32, t * self.top_k);
        let topk_w = self.dev.buffer(ffi::TH_F32, t * self.top_k);
        check(unsafe { ffi::th_moe_forward(self.raw, h.raw, t, out.raw, topk_idx.raw, topk_w.raw) });
        MoeOutput { out, topk_idx, topk_w }
    }
}

impl Drop for HipMoe<'_> {
    fn drop(&mut self) {
        unsafe {
            ffi::th_moe_destroy(self.raw);
        }
    }
}

// ---------------------------------------------------------------------------
// Decode engine
// ---------------------------------------------------------------------------

/// The shape of a Llama-style decoder (crates/tang-train/examples/smollm.rs).
#[derive(Clone, Copy, Debug)]
pub struct LlamaConfig {
    pub n_layers: usize,
    pub d_model: usize,
    pub n_heads: usize,
    pub n_kv_heads: usize,
    pub head_dim: usize,
    pub d_ff: usize,
    pub vocab: usize,
    /// KV cache length: positions 0..max_seq.
    pub max_seq: usize,
    pub eps: f32,
    pub rope_theta: f64,
}

/// A whole Llama-shaped model resident on the device: int4 group-32 linears,
/// bf16 embeddings and norms, f16 KV cache; each decode step is one recorded
/// kernel sequence replayed on the device (the step of smollm.rs:215-300).
pub struct HipLlama<'d> {
    raw: *mut ffi::th_llama,
    cfg: LlamaConfig,
    _dev: PhantomData<&'d HipComputeDevice>,
}

fn token_i32(t: usize, vocab: usize) -> i32 {
    assert!(t < vocab, "token {} out of the vocabulary ({})", t, vocab);
    t as i32
}

impl<'d> HipLlama<'d> {
    pub fn new(dev: &'d HipComputeDevice, cfg: LlamaConfig) -> Self {
        let c = ffi::th_llama_config {
            n_layers: cfg.n_layers as c_int,
            d_model: cfg.d_model as c_int,
            n_heads: cfg.n_heads as c_int,
            n_kv_heads: cfg.n_kv_heads as c_int,
            head_dim: cfg.head_dim as c_int,
            d_ff: cfg.d_ff as c_int,
            vocab: cfg.vocab as c_int,
            max_seq: cfg.max_seq as c_int,
            eps: cfg.eps,
            rope_theta: cfg.rope_theta,
        };
        let mut raw = ptr::null_mut();
        check(unsafe { ffi::th_llama_create(dev.dev, &c, &mut raw) });
        HipLlama { raw, cfg, _dev: PhantomData }
    }

    pub fn config(&self) -> &LlamaConfig {
        &self.cfg
    }

    /// Seeded synthetic weights (the benchmark model of BASELINE config 3).
    pub fn init_synthetic(&mut self, seed: u64) {
        check(unsafe { ffi::th_llama_init_synthetic(self.raw, seed) });
    }

    /// Weights from a safetensors file with the Llama tensor names that
    /// `load_model` reads (smollm.rs:364-420), quantized to int4 on upload.
    pub fn load_safetensors(&mut self, path: &Path) {
        let p = CString::new(path.to_str().expect("path is not UTF-8")).expect("path holds a NUL byte");
        let mut f = ptr::null_mut();
        check(unsafe { ffi::th_st_open(p.as_ptr(), &mut f) });
        let rc = unsafe { ffi::th_llama_load_safetensors(self.raw, f) };
        unsafe {
            ffi::th_st_close(f);
        }
        check(rc);
    }

    /// The prompt through every layer at positions pos..pos+n (K/V appended);
    /// returns the greedy next token and its logits.
    pub fn prefill(&mut self, tokens: &[usize], pos: usize) -> (usize, Vec<f32>) {
        let t: Vec<i32> = tokens.iter().map(|&x| token_i32(x, self.cfg.vocab)).collect();
        let mut next = 0i32;
        let mut logits = vec![0.0f32; self.cfg.vocab];
        check(unsafe { ffi::th_llama_prefill(self.raw, t.as_ptr(), t.len(), pos, &mut next, logits.as_mut_ptr()) });
        (next as usize, logits)
    }

    /// n_steps greedy decode steps from `token` at `pos`; returns the tokens
    /// chosen after each step and the last step's logits.
    pub fn generate_greedy(&mut self, token: usize, pos: usize, n_steps: usize) -> (Vec<usize>, Vec<f32>) {
        let mut toks = vec![0i32; n_steps];
        let mut logits = vec![0.0f32; self.cfg.vocab];
        check(unsafe {
            ffi::th_llama_generate(self.raw, token_i32(token, self.cfg.vocab), pos, n_steps, toks.as_mut_ptr(),
                                   logits.as_mut_ptr())
        });
        (toks.into_iter().map(|t| t as usize).collect(), logits)
    }

    /// `tang_infer::generate` (sampling.rs:229-256) on this model from
    /// position 0: the prompt is prefilled, then each step samples with
    /// `Sampler::with_seed(config, seed)` (the reference's sampler, restated
    /// on the host) and decodes on the device, until `max_tokens` tokens or
    /// the stop token.  Returns prompt + generated tokens, as the reference.
    pub fn generate(&mut self, prompt: &[usize], config: &SamplingConfig, seed: u64) -> Vec<usize> {
        assert!(!prompt.is_empty(), "empty prompt");
        let cfg = ffi::th_sampling_config {
            temperature: config.temperature,
            top_k: config.top_k,
            top_p: config.top_p,
            repetition_penalty: config.repetition_penalty,
            stop_token: config.stop_token.map(|t| t as i64).unwrap_or(-1),
            max_tokens: config.max_tokens,
        };
        let p: Vec<i32> = prompt.iter().map(|&x| token_i32(x, self.cfg.vocab)).collect();
        // all but the last prompt token go through the prefill; the sampled
        // loop feeds the last one at its position
        if p.len() > 1 {
            check(unsafe {
                ffi::th_llama_prefill(self.raw, p.as_ptr(), p.len() - 1, 0, ptr::null_mut(), ptr::null_mut())
            });
        }
        let mut sampler = ptr::null_mut();
        check(unsafe { ffi::th_sampler_create(&cfg, seed, &mut sampler) });
        let mut out = vec![0i32; config.max_tokens];
        let mut n_out = 0usize;
        let rc = unsafe {
            ffi::th_llama_generate_sampled(self.raw, sampler, p.as_ptr(), p.len(), p.len() - 1, out.as_mut_ptr(),
                                           &mut n_out)
        };
        unsafe {
            ffi::th_sampler_destroy(sampler);
        }
        check(rc);
        let mut tokens = prompt.to_vec();
        tokens.extend(out[..n_out].iter().map(|&t| t as usize));
        tokens
    }
}

impl Drop for HipLlama<'_> {
    fn drop(&mut self) {
        unsafe {
            ffi::th_llama_destroy(self.raw);
        }
    }
}
