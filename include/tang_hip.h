/*
 * tang_hip.h -- C ABI of the MI355X (gfx950) backend for tang-compute's
 * quantized-inference decode path.
 *
 * The entry points mirror `tang_compute::ComputeDevice`
 * (crates/tang-compute/src/device.rs:19-869) for the ops a decode step uses,
 * plus quantized-linear, MoE and MLA extensions the reference trait lacks.
 * A Rust `HipComputeDevice: ComputeDevice` forwards to these functions.
 *
 * Conventions
 *  - Every function returns an int status: TH_OK (0) or a TH_ERR_* code; the
 *    message of the last failure on the calling thread is th_last_error().
 *    Nothing unwinds across the ABI (the reference panics instead).
 *  - One device handle per host thread; each device owns one HIP stream.
 *    Calls enqueue work and return; th_sync / th_buffer_download synchronise
 *    (device.rs:367 sync, device.rs:75 download).
 *  - Outputs are caller-allocated buffers (the reference returns owned
 *    buffers; the shim allocates them with th_buffer_alloc first).
 *  - Sizes are element counts (usize in the reference).
 */
#ifndef TANG_HIP_H
#define TANG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TH_OK 0
#define TH_ERR_INVALID 1     /* bad argument, shape or dtype */
#define TH_ERR_HIP 2         /* HIP runtime error */
#define TH_ERR_OOM 3         /* device allocation failed */
#define TH_ERR_UNSUPPORTED 4 /* valid request this backend does not implement */

typedef enum {
    TH_F32 = 0,
    TH_BF16 = 1,
    TH_F16 = 2,
    TH_U8 = 3,
    TH_I8 = 4,
    TH_U32 = 5,
    TH_I32 = 6
} th_dtype;

typedef struct th_device th_device;
typedef struct th_buffer th_buffer;
typedef struct th_qweight th_qweight;
typedef struct th_graph th_graph;

/* Reference block layouts (crates/tang-infer/src/quantize.rs:15-29), as plain
 * C structs: Q8Block {scale; values[32]} and Q4Block {scale; values[16]} with
 * values[i] = (q[2i]+8) | (q[2i+1]+8) << 4. */
typedef struct { float scale; int8_t values[32]; } th_q8_block;
typedef struct { float scale; uint8_t values[16]; } th_q4_block;

/* ---- errors, devices, streams ------------------------------------------ */

/* Message of the last failed call on this thread ("" if none). */
const char* th_last_error(void);
/* Number of visible HIP devices. */
int th_device_count(int* n);
/* CudaComputeDevice::new (crates/tang-compute/src/cuda.rs:151). */
int th_device_create(int ordinal, th_device** out);
int th_device_destroy(th_device* dev);
/* ComputeDevice::sync (device.rs:367): wait for all work on the device stream. */
int th_sync(th_device* dev);
/* ComputeDevice::total_memory_bytes / free_memory_bytes (device.rs:27-30). */
int th_memory_info(th_device* dev, size_t* free_bytes, size_t* total_bytes);
/* Time the work enqueued between start and stop on the device stream with HIP
 * events; stop synchronises and returns elapsed milliseconds. */
int th_timer_start(th_device* dev);
int th_timer_stop(th_device* dev, float* ms);
/* Record the library calls made on the device stream between begin and end
 * into one HIP graph, replayed by th_graph_launch on the same stream.  No
 * counterpart in the reference (its backends launch every call): this is
 * for callers that repeat a fixed sequence of calls, as a decode loop does.
 * The recorded calls must not allocate: make each one once before capture
 * (workspaces grow on first use).  Replays read and write the same buffers
 * the recorded calls named. */
int th_capture_begin(th_device* dev);
int th_capture_end(th_device* dev, th_graph** out);
int th_graph_launch(th_graph* g);
int th_graph_destroy(th_graph* g);

/* ---- buffers (device.rs:44-80 upload/upload_u32/alloc/download) -------- */

int th_buffer_alloc(th_device* dev, th_dtype dtype, size_t n, th_buffer** out);
int th_buffer_free(th_buffer* buf);
/* Copy n elements of the buffer's dtype from host memory (synchronous). */
int th_buffer_upload(th_buffer* buf, const void* host, size_t n);
/* Copy n elements to host memory; synchronises the device stream first. */
int th_buffer_download(th_buffer* buf, void* host, size_t n);
int th_buffer_info(const th_buffer* buf, th_dtype* dtype, size_t* n);
/* ComputeDevice::zero_buffer. */
int th_buffer_zero(th_buffer* buf);
/* Device-to-device copy of min(src, dst) bytes on the device stream
 * (ComputeDevice::copy_buffer-style helper; also the known-size copy the
 * HBM-traffic counters are calibrated against). */
int th_buffer_copy(th_buffer* dst, const th_buffer* src);
/* Copy n elements src[src_offset..] -> dst[dst_offset..] (same dtype) on the
 * device stream: slice_buffer / write_into (device.rs:839-850) and the column
 * moves of extract_columns / concat_columns without a host round trip. */
int th_buffer_copy_region(th_buffer* dst, size_t dst_offset, const th_buffer* src, size_t src_offset, size_t n);
/* Element-wise dtype conversion between f32, bf16 and f16 buffers of equal
 * length; f32->bf16 rounds as crates/tang-compute/src/cuda.rs:22-27,
 * f32->f16 is IEEE round-to-nearest-even (kernels BF16_TO_F32_CUDA /
 * F32_TO_BF16_CUDA, util_cuda.rs:85,99). */
int th_convert(th_device* dev, const th_buffer* src, th_buffer* dst);

/* ---- quantized weights ------------------------------------------------- */

/* Upload a row-by-row quantized Q4 matrix in the reference block layout
 * (quantize_matrix_q4, quantize.rs:208): rows*ceil(cols/32) blocks.
 * scale_dtype TH_F32 keeps the f32 scales; TH_F16 stores them as f16 and
 * fails unless every scale is exactly representable. */
int th_q4_upload_blocks(th_device* dev, const th_q4_block* blocks, size_t rows, size_t cols,
                        th_dtype scale_dtype, th_qweight** out);
/* Same matrix as arrays: nib[rows][ceil(cols/32)*16] packed exactly like
 * Q4Block.values, scales[rows][ceil(cols/32)] of scale_dtype (f32 or f16). */
int th_q4_upload_packed(th_device* dev, const uint8_t* nib, const void* scales, th_dtype scale_dtype,
                        size_t rows, size_t cols, th_qweight** out);
/* Q8 (quantize_matrix_q8, quantize.rs:193), rows*ceil(cols/32) blocks. */
int th_q8_upload_blocks(th_device* dev, const th_q8_block* blocks, size_t rows, size_t cols,
                        th_qweight** out);
/* Q8 with one f32 scale per row: q[rows][cols], row_scale[rows].  Equivalent
 * to Q8 blocks whose scales within a row are all equal. */
int th_q8_upload_rowwise(th_device* dev, const int8_t* q, const float* row_scale, size_t rows,
                         size_t cols, th_qweight** out);
/* Read a Q4 weight back in the reference block layout (bit-exact round trip). */
int th_q4_download_blocks(const th_qweight* w, th_q4_block* blocks);
int th_qweight_info(const th_qweight* w, size_t* rows, size_t* cols, int* bits);
int th_qweight_free(th_qweight* w);

/* quantize_matrix_q4 / quantize_matrix_q8 (quantize.rs:193-220) on the host:
 * row-major f32 [rows][cols] -> rows*ceil(cols/32) reference blocks. */
int th_quantize_q4(const float* data, size_t rows, size_t cols, th_q4_block* out);
int th_quantize_q8(const float* data, size_t rows, size_t cols, th_q8_block* out);

/* ---- safetensors weights ---------------------------------------------------
 * The files tang-safetensors reads (crates/tang-safetensors/src/lib.rs:11-70):
 * F64, F32, F16 and BF16 tensors; other dtypes are rejected, as there. */
#define TH_ST_F64 0
#define TH_ST_F32 1
#define TH_ST_F16 2
#define TH_ST_BF16 3
typedef struct th_st_file th_st_file;
int th_st_open(const char* path, th_st_file** out);
int th_st_close(th_st_file* f);
int th_st_count(const th_st_file* f, size_t* n);
/* name stays valid until th_st_close; shape receives ndim values (max_dims room). */
int th_st_info(const th_st_file* f, size_t index, const char** name, int* dtype, size_t* ndim, size_t* shape,
               size_t max_dims);
/* The tensor's values as f32 (exact from F16/BF16/F32; F64 rounded). */
int th_st_read_f32(const th_st_file* f, const char* name, float* out, size_t n);
/* Into a device buffer of dtype TH_F32, TH_BF16 or TH_F16 (RNE). */
int th_st_upload(th_device* dev, const th_st_file* f, const char* name, th_dtype dtype, th_buffer** out);
/* A 2-D tensor quantized with quantize_matrix_q4 / _q8 and uploaded in the
 * device layout (f32 group scales). */
int th_st_upload_q4(th_device* dev, const th_st_file* f, const char* name, th_qweight** out);
int th_st_upload_q8(th_device* dev, const th_st_file* f, const char* name, th_qweight** out);

/* ---- quantized linear ---------------------------------------------------
 * y[m][n] = sum_k x[m][k] * dequant(W)[n][k]: the quantized form of
 * ComputeDevice::matmul_b_transposed (device.rs:407) with B = W [n,k]
 * row-major, i.e. Linear::forward_2d (modules.rs:56) without bias, and
 * m independent q4_matvec / q8_matvec calls (quantize.rs:227-289).
 * x: f32 or bf16 [m][k]; y: f32 [m][n].  Accumulation is f32. */
int th_gemm_q4(th_device* dev, const th_buffer* x, size_t m, const th_qweight* w, th_buffer* y);
int th_gemv_q8(th_device* dev, const th_buffer* x, size_t m, const th_qweight* w, th_buffer* y);

/* Allocation-free form of th_gemm_q4 (no counterpart in the reference): for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * kernels and results as th_gemm_q4, but the MFMA path's workspace (the
 * prepared activations, then the split-K partials) is a fixed per-GPU device
 * array of TH_NOALLOC_SCRATCH_BYTES, not an allocation: the call makes no
 * hipMalloc / hipFree.  Fails with TH_ERR_INVALID when the prepared
 * activations, about 2*m*K bytes, do not fit (split-K is narrowed to what
 * fits).  Every call on one GPU shares the array: calls that overlap on one
 * GPU (two streams, two threads) race. */
#define TH_NOALLOC_SCRATCH_BYTES (64u << 20)
int th_gemm_q4_noalloc(th_device* dev, const th_buffer* x, size_t m, const th_qweight* w, th_buffer* y);

/* Benchmark helper (no reference counterpart): enqueue `iters` calls of
 * th_gemm_q4 / th_gemv_q8 (by the weights' bit width) on x -> y, cycling
 * through the n_w weights (all of one shape) so the streamed bytes exceed the
 * last-level cache, and return the elapsed milliseconds between HIP events
 * recorded on the device stream around them.  use_graph == 1 captures the
 * calls into one HIP graph first and times its replay; use_graph == 2 records
 * them as one sequence on the library's own AQL queue (GEMV launches, q8 or
 * q4 at m <= 16, store their outputs write-through and read nothing another
 * launch writes, so the packets carry no fences between them) and
 * times its replay between device clock stamps.  Launch i reads weight
 * ws[i % n_w], and the untimed warm-up ends with one pass over ws[0..n_w) in
 * that order, so every timed launch's weights were last read n_w launches
 * earlier, for any iters. */
int th_bench_linear(th_device* dev, const th_buffer* x, size_t m, th_qweight* const* ws, size_t n_w,
                    th_buffer* y, size_t iters, int use_graph, float* ms);

/* ---- dense operators (ComputeDevice methods for unquantized weights) ------
 * f32 buffers unless stated; all calls enqueue on the device stream. */

/* C[m][n] (+)= op(A) . op(B): ComputeDevice::matmul (device.rs:103),
 * matmul_accumulate (:391), matmul_b_transposed (:407), matmul_a_transposed
 * (:422) and matmul_accumulate_a_transposed (:437) in one call.  A is [m][k]
 * (trans_a: stored [k][m]), B is [k][n] (trans_b: stored [n][k], the
 * Linear::forward_2d weight layout, modules.rs:56); A and B f32 or bf16, C
 * f32; accumulate != 0 adds to C.  f32 products, f32 accumulation on MFMA. */
int th_matmul_ex(th_device* dev, const th_buffer* a, const th_buffer* b, size_t m, size_t k, size_t n, int trans_a,
                 int trans_b, int accumulate, th_buffer* c);
/* ComputeDevice::matmul (device.rs:103; CpuDevice cpu.rs:99,760). */
int th_matmul(th_device* dev, const th_buffer* a, const th_buffer* b, size_t m, size_t k, size_t n, th_buffer* c);
/* ComputeDevice::matmul_b_transposed (device.rs:407). */
int th_matmul_b_transposed(th_device* dev, const th_buffer* a, const th_buffer* b, size_t m, size_t k, size_t n,
                           th_buffer* c);
/* ComputeDevice::transpose_2d (device.rs:183; cpu.rs:317). */
int th_transpose_2d(th_device* dev, const th_buffer* in, size_t rows, size_t cols, th_buffer* out);
/* ComputeDevice::reduce_sum (device.rs:140; cpu.rs:169) over axis of a
 * row-major tensor of ndim dims; accumulate != 0 is reduce_sum_accumulate
 * (device.rs:451).  Sums in the reference's order: bit-identical. */
int th_reduce_sum(th_device* dev, const th_buffer* in, const size_t* shape, size_t ndim, size_t axis, int accumulate,
                  th_buffer* out);
/* ComputeDevice::bias_add (device.rs:378): out[i] = matrix[i] + bias[i % dim]. */
int th_bias_add(th_device* dev, const th_buffer* matrix, const th_buffer* bias, size_t numel, size_t dim,
                th_buffer* out);
/* ComputeDevice::add_assign (device.rs:767; cpu.rs:650): dst += src, equal lengths. */
int th_add_assign(th_device* dev, th_buffer* dst, const th_buffer* src);

/* ComputeDevice::elementwise (device.rs:93; the CPU backend's semantics,
 * cpu.rs:68-97): the closure's tang-expr graph (trace(), tang-expr/src/lib.rs:61)
 * is handed over as its nodes in graph order (node.rs:58-90), operands
 * indexing earlier nodes.  The library generates the HIP kernel, compiles it
 * for gfx950 once per distinct graph (hiprtc, cached per device) and runs it
 * over numel elements: out[i] = f(in0[i], ..., in{n-1}[i]), each input widened
 * to f64, every node evaluated in f64, the result rounded to f32 once.
 * th_expr_source returns the generated source (len = its length; up to cap-1
 * bytes and a NUL are written to buf when buf is not NULL). */
enum {
    TH_EXPR_VAR = 0,  /* input a */
    TH_EXPR_LIT = 1,  /* the value lit */
    TH_EXPR_ADD = 2,  /* a + b */
    TH_EXPR_MUL = 3,  /* a * b */
    TH_EXPR_NEG = 4,  /* -a */
    TH_EXPR_RECIP = 5, /* 1 / a */
    TH_EXPR_SQRT = 6,
    TH_EXPR_SIN = 7,
    TH_EXPR_ATAN2 = 8, /* atan2(a = y, b = x) */
    TH_EXPR_EXP2 = 9,
    TH_EXPR_LOG2 = 10,
    TH_EXPR_SELECT = 11 /* a > 0 ? b : c */
};
typedef struct th_expr_node {
    uint32_t op;      /* TH_EXPR_* */
    uint32_t a, b, c; /* operand node indices; TH_EXPR_VAR: a = input index */
    double lit;       /* TH_EXPR_LIT */
} th_expr_node;
int th_expr_source(const th_expr_node* nodes, size_t n_nodes, uint32_t output, size_t n_inputs, char* buf,
                   size_t cap, size_t* len);
int th_elementwise_expr(th_device* dev, const th_expr_node* nodes, size_t n_nodes, uint32_t output,
                        const th_buffer* const* inputs, size_t n_inputs, size_t numel, th_buffer* out);

/* Run-time compiled kernels from HIP source: a kernel
 *   extern "C" __global__ void <entry>(const float* in0, ..., float* outputs,
 *                                      const unsigned int count)
 * with one thread per element, compiled for gfx950 with hiprtc and loaded as a
 * hipModule.  th_elementwise launches it over numel elements (256-thread
 * workgroups) with the n_inputs f32 input buffers and the f32 output. */
typedef struct th_kernel th_kernel;
int th_kernel_compile(th_device* dev, const char* source, const char* entry, th_kernel** out);
int th_kernel_free(th_kernel* k);
int th_elementwise(th_kernel* k, const th_buffer* const* inputs, size_t n_inputs, size_t numel, th_buffer* out);

/* ---- decode ops (f32 buffers unless stated) ---------------------------- */

/* CpuDevice::rms_norm (crates/tang-compute/src/cpu.rs:126); weight f32 or bf16. */
int th_rms_norm(th_device* dev, const th_buffer* x, const th_buffer* weight, size_t n_groups,
                size_t dim, float eps, th_buffer* out);
/* ComputeDevice::rms_norm_residual (device.rs:546): out = norm(in+res),
 * sum_out = in+res. */
int th_rms_norm_residual(th_device* dev, const th_buffer* in, const th_buffer* residual,
                         const th_buffer* weight, size_t n_groups, size_t dim, float eps,
                         th_buffer* out, th_buffer* sum_out);
/* InterleavedRoPE::new tables (modules.rs:495-511), host-side:
 * cos/sin [max_seq][head_dim/2]. */
int th_rope_tables(size_t head_dim, size_t max_seq, double base, float* cos_table, float* sin_table);
/* ComputeDevice::rope_forward_cached (device.rs:678 -> :582). */
int th_rope_forward(th_device* dev, const th_buffer* in, const th_buffer* cos_buf,
                    const th_buffer* sin_buf, size_t seq_len, size_t n_heads, size_t head_dim,
                    size_t start_pos, th_buffer* out);
/* ComputeDevice::kv_attention (cpu.rs:257): q [q_len][n_heads*head_dim] f32,
 * caches [>= cache_start+q_len][n_kv_heads*head_dim] of f32 or f16; query i
 * attends to positions 0..cache_start+i.  No length limit. */
int th_kv_attention(th_device* dev, const th_buffer* q, const th_buffer* k_cache,
                    const th_buffer* v_cache, size_t cache_start, size_t q_len, size_t n_heads,
                    size_t n_kv_heads, size_t head_dim, th_buffer* out);
/* swiglu_fused_buf (device.rs:727): out = g*sigmoid(g)*u. */
int th_swiglu(th_device* dev, const th_buffer* gate, const th_buffer* up, size_t n, th_buffer* out);
/* swiglu_fused_buf (device.rs:727) as a linear's input: out (bf16) =
 * bf16(f32(g*sigmoid(g)*u)) with the cuda.rs:22 rounding -- the SwiGLU the
 * decode, prefill and MoE epilogues apply; the same bits as th_swiglu's f32
 * output rounded to bf16. */
int th_swiglu_bf16(th_device* dev, const th_buffer* gate, const th_buffer* up, size_t n, th_buffer* out);
/* add_tensors_buf (device.rs:721). */
int th_add(th_device* dev, const th_buffer* a, const th_buffer* b, size_t n, th_buffer* out);
/* CpuDevice::embedding (cpu.rs:151): weight f32 or bf16 [vocab][dim], ids u32. */
int th_embedding(th_device* dev, const th_buffer* weight, const th_buffer* ids, size_t seq_len,
                 size_t dim, th_buffer* out);
/* CpuDevice::softmax (cpu.rs:105). */
int th_softmax(th_device* dev, const th_buffer* x, size_t n_rows, size_t row_len, th_buffer* out);
/* Greedy Sampler argmax (crates/tang-infer/src/sampling.rs:184): first
 * maximum wins.  x f32 [n_rows][n]; out u32 [n_rows]. */
int th_argmax(th_device* dev, const th_buffer* x, size_t n_rows, size_t n, th_buffer* out);

/* ---- device-resident Llama-style decode engine --------------------------
 * The decode step of crates/tang-train/examples/smollm.rs:215-300 with every
 * linear int4 group-32, bf16 embeddings and norm weights, and an f16 KV cache
 * kept on the device.  Greedy loop as crates/tang-infer/src/sampling.rs:229. */
typedef struct {
    int n_layers, d_model, n_heads, n_kv_heads, head_dim, d_ff, vocab, max_seq;
    float eps;
    double rope_theta;
} th_llama_config;
typedef struct th_llama th_llama;

int th_llama_create(th_device* dev, const th_llama_config* cfg, th_llama** out);
int th_llama_destroy(th_llama* m);
/* Fill all weights with the seeded synthetic generator (th_synth_*): linear
 * tensor t of layer l uses seed th_synth_seed(seed, l, t). */
int th_llama_init_synthetic(th_llama* m, uint64_t seed);
/* Replaces load_model (crates/tang-train/examples/smollm.rs:364-420): the
 * weights of a safetensors file with Llama tensor names
 * (model.embed_tokens.weight, model.layers.{i}.self_attn.{q,k,v,o}_proj.weight,
 * model.layers.{i}.mlp.{gate,up,down}_proj.weight,
 * model.layers.{i}.{input,post_attention}_layernorm.weight, model.norm.weight
 * and, unless tied to the embedding, lm_head.weight; F64/F32/F16/BF16).
 * Linears go through quantize_matrix_q4 with f16 block scales, embeddings and
 * norm weights are stored as bf16.  Every tensor but lm_head is required and
 * shape-checked (the reference keeps its initial values for a missing one). */
int th_llama_load_safetensors(th_llama* m, const th_st_file* f);
/* Fill KV positions [0, len) of every layer with N(0,1) f16 values. */
int th_llama_fill_kv_synthetic(th_llama* m, size_t len, uint64_t seed);
/* Greedy decode: feed `token` at position `pos`, then n_steps-1 more steps on
 * the argmax; tokens_out[i] is the argmax after step i.  last_logits (may be
 * NULL) receives the final step's f32 logits [vocab]. */
int th_llama_generate(th_llama* m, int32_t token, size_t pos, size_t n_steps, int32_t* tokens_out,
                      float* last_logits);
/* One decode step without host round-trips, for timing: token is read from
 * and argmax written to the model's device-side token slot. */
int th_llama_step_device(th_llama* m, size_t pos);
int th_llama_set_token(th_llama* m, int32_t token);
/* Benchmark helper: run n_steps greedy steps from (token, pos) as in
 * th_llama_generate and return the milliseconds between device clock stamps
 * around the step replays on the library's AQL queue (between HIP events
 * around the graph launches when TANG_HIP_DISPATCH=graph). */
int th_llama_time_steps(th_llama* m, int32_t token, size_t pos, size_t n_steps, float* ms);

/* Prefill: the prompt tokens[0..n) at positions pos..pos+n-1 run through
 * every layer as M=n GEMMs (prompt chunks of up to 512 rows) with causal
 * split attention, appending their K/V rows; then the last row's final norm,
 * LM head and greedy argmax, as the decode step of smollm.rs:215-300 would
 * give for tokens[n-1].  next_token / last_logits (vocab f32) are optional.
 * The device state is left at position pos+n with next_token, so
 * th_llama_generate(next_token, pos+n, ...) continues the sequence. */
int th_llama_prefill(th_llama* m, const int32_t* tokens, size_t n, size_t pos, int32_t* next_token,
                     float* last_logits);
/* HIP-event time of one th_llama_prefill (after a warm-up call). */
int th_llama_time_prefill(th_llama* m, const int32_t* tokens, size_t n, size_t pos, float* ms);

/* ---- sampling (host, crates/tang-infer/src/sampling.rs) ------------------ */
/* SamplingConfig (sampling.rs:6-20); stop_token < 0 means None. */
typedef struct {
    double temperature;        /* 0 = greedy */
    size_t top_k;              /* 0 = off */
    double top_p;              /* 1 = off */
    double repetition_penalty; /* 1 = off */
    int64_t stop_token;        /* < 0: none */
    size_t max_tokens;
} th_sampling_config;
typedef struct th_sampler th_sampler;
/* Sampler::with_seed (sampling.rs:67-72). */
int th_sampler_create(const th_sampling_config* cfg, uint64_t seed, th_sampler** out);
int th_sampler_destroy(th_sampler* s);
/* Sampler::sample (sampling.rs:86-160) on host f32 logits [vocab]; past =
 * tokens seen so far (for the repetition penalty). */
int th_sampler_sample(th_sampler* s, const float* logits, size_t vocab, const int32_t* past, size_t n_past,
                      int32_t* token);
/* generate() (sampling.rs:229-256) on the decode engine: prompt_last is fed
 * at position pos (positions < pos already in the KV cache); each step runs on
 * the device, the logits come to the host and the sampler picks the next
 * token (past = prompt tokens, then the generated ones).  Stops after
 * cfg.max_tokens or before appending stop_token.  tokens_out receives the
 * generated tokens (up to max_tokens), *n_out their count. */
int th_llama_generate_sampled(th_llama* m, th_sampler* s, const int32_t* prompt, size_t n_prompt, size_t pos,
                              int32_t* tokens_out, size_t* n_out);

/* ---- MoE (DeepSeek-style; no reference implementation) ------------------ */
typedef struct th_moe th_moe;
int th_moe_create(th_device* dev, size_t d_model, size_t d_ff, size_t n_experts, size_t n_shared,
                  size_t top_k, th_moe** out);
int th_moe_destroy(th_moe* moe);
/* Router W ~ N(0,0.02) f32 [E][d]; expert linears int4 g32 from th_synth_q4. */
int th_moe_init_synthetic(th_moe* moe, uint64_t seed);
/* h bf16 [T][d] -> out f32 [T][d]; topk_idx i32 [T][k], topk_w f32 [T][k]. */
int th_moe_forward(th_moe* moe, const th_buffer* h, size_t T, th_buffer* out, th_buffer* topk_idx,
                   th_buffer* topk_w);

/* ---- MLA decode attention (absorbed; no reference implementation) ------ */
/* q_nope f32 [B][H][dn], q_rope f32 [B][H][dr], cache bf16 [B][L][r+dr];
 * w_uk Q8 rowwise [H*r][dn]; w_uv Q8 rowwise [H*dv][r]; out f32 [B][H][dv]. */
int th_mla_decode(th_device* dev, const th_buffer* q_nope, const th_buffer* q_rope,
                  const th_buffer* cache, size_t B, size_t H, size_t L, size_t dn, size_t dr,
                  size_t r, size_t dv, const th_qweight* w_uk, const th_qweight* w_uv,
                  float sm_scale, th_buffer* out);

/* ---- seeded synthetic data (host) ---------------------------------------
 * xoshiro256** seeded through SplitMix64, as crates/tang-bench/src/lib.rs:7-46.
 * uniform(a,b) = a + (b-a)*(f64()+1)/2 with f64() the reference's [-1,1] map;
 * normal = Box-Muller on two 53-bit uniforms. */
uint64_t th_synth_seed(uint64_t base, uint64_t layer, uint64_t tensor);
/* Packed int4: every byte is one draw-byte (two nibbles ~U[0,15], value-8 in
 * [-8,7]); scales f16 ~U[smin,smax] rounded to nearest. */
int th_synth_q4(uint64_t seed, size_t rows, size_t cols, float smin, float smax, uint8_t* nib,
                uint16_t* scales_f16);
/* int8 ~U[-127,127] and per-row f32 scales ~U[smin,smax]. */
int th_synth_q8_rowwise(uint64_t seed, size_t rows, size_t cols, float smin, float smax, int8_t* q,
                        float* row_scale);
/* N(0,std) values rounded to bf16 / f16 / f32 (dtype TH_BF16/TH_F16/TH_F32). */
int th_synth_normal(uint64_t seed, size_t n, float std, th_dtype dtype, void* out);

#ifdef __cplusplus
}
#endif

#endif /* TANG_HIP_H */
