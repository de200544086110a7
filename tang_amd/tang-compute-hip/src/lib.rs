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
//! extension trait below, plus MoE, MLA and a whole-model decode engine.
//!
//! Errors panic with the library's message, as the reference backends do
//! (e.g. crates/tang-compute/src/cuda.rs:385).  Like `CudaComputeDevice`, the
//! device is `Send` but not `Sync` (one device per thread; the element-wise
//! kernel cache is a `RefCell`).
//!
//! Training-only operators (the backward passes, cross-entropy, AdamW) are
//! outside this backend, which serves the inference path: they panic with
//! that reason rather than fall back to the host.
#![allow(clippy::too_many_arguments)]

pub mod ffi;

use std::cell::RefCell;
use std::collections::HashMap;
use std::ffi::{CStr, CString};
use std::os::raw::{c_int, c_void};
use std::ptr;

use tang_compute::{ComputeBuffer, ComputeDevice};
use tang_expr::codegen::Dialect;
use tang_expr::node::ExprId;
use tang_expr::trace;
use tang_infer::quantize::{QuantizedQ4, QuantizedQ8};

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

struct Kernel(*mut ffi::th_kernel);

impl Drop for Kernel {
    fn drop(&mut self) {
        unsafe {
            ffi::th_kernel_free(self.0);
        }
    }
}

/// One MI355X (HIP device ordinal) with one stream.
pub struct HipComputeDevice {
    dev: *mut ffi::th_device,
    /// Element-wise kernels compiled by hiprtc, keyed by their source.
    kernels: RefCell<HashMap<String, Kernel>>,
}

unsafe impl Send for HipComputeDevice {}

impl HipComputeDevice {
    /// `CudaComputeDevice::new` (cuda.rs:151) for a HIP device ordinal.
    pub fn new(ordinal: usize) -> Self {
        let mut dev = ptr::null_mut();
        check(unsafe { ffi::th_device_create(ordinal as c_int, &mut dev) });
        HipComputeDevice { dev, kernels: RefCell::new(HashMap::new()) }
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

    fn compiled(&self, source: &str, entry: &str) -> *mut ffi::th_kernel {
        if let Some(k) = self.kernels.borrow().get(source) {
            return k.0;
        }
        let src = CString::new(source).expect("kernel source holds a NUL byte");
        let name = CString::new(entry).expect("entry name holds a NUL byte");
        let mut k = ptr::null_mut();
        check(unsafe { ffi::th_kernel_compile(self.dev, src.as_ptr(), name.as_ptr(), &mut k) });
        self.kernels.borrow_mut().insert(source.to_string(), Kernel(k));
        k
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
        self.kernels.borrow_mut().clear();
        // buffers still alive keep the library's device state until they drop
        unsafe {
            ffi::th_device_destroy(self.dev);
        }
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

    /// Element-wise kernels are generated as tang-expr's CUDA-dialect C
    /// (`extern "C" __global__`, blockIdx/threadIdx, libm names), which hiprtc
    /// compiles for gfx950 as it stands.
    fn dialect(&self) -> Dialect {
        Dialect::Cuda
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

    // -- element-wise via tang-expr (device.rs:93; the CUDA path is cuda.rs:1135-1190) --

    fn elementwise(&self, inputs: &[&HipBuffer], numel: usize, f: &dyn Fn(&[ExprId]) -> ExprId) -> HipBuffer {
        let n_inputs = inputs.len();
        let (graph, output) = trace(|| {
            let vars: Vec<ExprId> = (0..n_inputs as u16).map(ExprId::var).collect();
            f(&vars)
        });
        let kernel = graph.to_kernel(&[output], n_inputs, Dialect::Cuda);
        let k = self.compiled(&kernel.source, kernel.entry_point);
        let raw: Vec<*const ffi::th_buffer> = inputs.iter().map(|b| b.raw as *const ffi::th_buffer).collect();
        let out = self.buffer(ffi::TH_F32, numel);
        check(unsafe { ffi::th_elementwise(k, raw.as_ptr(), n_inputs, numel, out.raw) });
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
