// Element-wise and row-wise decode ops: rms_norm, rms_norm_residual, RoPE,
// SwiGLU, add, embedding, softmax, argmax, dtype conversion.
// Each kernel restates the CpuDevice / ComputeDevice default of the reference
// (file:line at each kernel); row reductions run as 256-thread trees in f32.
#include <cmath>

#include "capi_util.hpp"
#include "ops.hpp"

namespace th {

__global__ void rms_norm_kernel(const float* __restrict__ x, const void* __restrict__ w, int w_bf16, int dim,
                                float eps, float* __restrict__ out) {
    __shared__ float red[256];
    const float* xr = x + (size_t)blockIdx.x * dim;
    float s = 0.0f;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) s += xr[i] * xr[i];
    s = block_sum_256(s, red);
    // cpu.rs:134-136: rms = sqrt(sum/dim + eps); inv = 1/rms
    const float inv = 1.0f / sqrtf(s / (float)dim + eps);
    for (int i = threadIdx.x; i < dim; i += blockDim.x) out[(size_t)blockIdx.x * dim + i] = xr[i] * inv * load_w(w, w_bf16, i);
}

__global__ void rms_norm_residual_kernel(const float* __restrict__ in, const float* __restrict__ res,
                                         const void* __restrict__ w, int w_bf16, int dim, float eps,
                                         float* __restrict__ out, float* __restrict__ sum_out) {
    __shared__ float red[256];
    const size_t base = (size_t)blockIdx.x * dim;
    float s = 0.0f;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        float v = in[base + i] + res[base + i];
        sum_out[base + i] = v;
        s += v * v;
    }
    s = block_sum_256(s, red);
    const float inv = 1.0f / sqrtf(s / (float)dim + eps);
    for (int i = threadIdx.x; i < dim; i += blockDim.x) out[base + i] = sum_out[base + i] * inv * load_w(w, w_bf16, i);
}

// device.rs:582-610: rotate interleaved pairs (2i, 2i+1) with cos/sin[pos*half+i].
__global__ void rope_kernel(const float* __restrict__ in, const float* __restrict__ cs, const float* __restrict__ sn,
                            int seq_len, int n_heads, int head_dim, int start_pos, float* __restrict__ out) {
    const int half = head_dim / 2;
    const size_t total = (size_t)seq_len * n_heads * half;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
        const int i = (int)(idx % half);
        const size_t sh = idx / half;
        const int s = (int)(sh / n_heads);
        const size_t base = sh * head_dim;
        const int pos = start_pos + s;
        const float c = cs[(size_t)pos * half + i], sv = sn[(size_t)pos * half + i];
        const float x0 = in[base + 2 * i], x1 = in[base + 2 * i + 1];
        out[base + 2 * i] = x0 * c - x1 * sv;
        out[base + 2 * i + 1] = x0 * sv + x1 * c;
    }
}

__global__ void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, size_t n, float* __restrict__ out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = swiglu_f64(g[i], u[i]);
}

__global__ void swiglu_bf16_kernel(const float* __restrict__ g, const float* __restrict__ u, size_t n,
                                   uint16_t* __restrict__ out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = swiglu_bf16(g[i], u[i]);
}

__global__ void add_kernel(const float* __restrict__ a, const float* __restrict__ b, size_t n, float* __restrict__ out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = a[i] + b[i];
}

// cpu.rs:151-168: row copy by id.
__global__ void embedding_kernel(const void* __restrict__ w, int w_bf16, const uint32_t* __restrict__ ids, int seq_len,
                                 int dim, float* __restrict__ out) {
    const size_t total = (size_t)seq_len * dim;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
        const size_t s = idx / dim, d = idx - s * dim;
        out[idx] = load_w(w, w_bf16, (size_t)ids[s] * dim + d);
    }
}

// cpu.rs:105-124: max-subtracted softmax per row.
__global__ void softmax_kernel(const float* __restrict__ x, int len, float* __restrict__ out) {
    __shared__ float red[256];
    const float* xr = x + (size_t)blockIdx.x * len;
    float* o = out + (size_t)blockIdx.x * len;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < len; i += blockDim.x) mx = fmaxf(mx, xr[i]);
    mx = block_max_256(mx, red);
    float s = 0.0f;
    for (int i = threadIdx.x; i < len; i += blockDim.x) {
        float e = expf(xr[i] - mx);
        o[i] = e;
        s += e;
    }
    s = block_sum_256(s, red);
    const float inv = 1.0f / s;
    for (int i = threadIdx.x; i < len; i += blockDim.x) o[i] *= inv;
}

__global__ void argmax_kernel(const float* __restrict__ x, int n, uint32_t* __restrict__ out) {
    __shared__ float rv[256];
    __shared__ int ri[256];
    const float* xr = x + (size_t)blockIdx.x * n;
    float bv; int bi;
    argmax_block_256(xr, n, rv, ri, bv, bi);
    if (threadIdx.x == 0) out[blockIdx.x] = (uint32_t)bi;
}

__global__ void convert_kernel(const void* __restrict__ src, th_dtype sdt, void* __restrict__ dst, th_dtype ddt, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float v;
        if (sdt == TH_F32) v = ((const float*)src)[i];
        else if (sdt == TH_BF16) v = __uint_as_float((uint32_t)((const uint16_t*)src)[i] << 16);
        else v = (float)((const _Float16*)src)[i];
        if (ddt == TH_F32) ((float*)dst)[i] = v;
        else if (ddt == TH_BF16) ((uint16_t*)dst)[i] = f32_to_bf16_rne(v);
        else ((_Float16*)dst)[i] = (_Float16)v;
    }
}

__global__ void fill_zero_kernel(uint32_t* __restrict__ p, size_t n_words) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n_words; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

static unsigned grid_for(size_t n) { return (unsigned)std::max<size_t>(1, std::min<size_t>(ceil_div(n, 256), 8192)); }

static int weight_flag(const th_buffer* w) {
    if (w->dtype == TH_F32) return 0;
    if (w->dtype == TH_BF16) return 1;
    throw Error(TH_ERR_INVALID, "weight buffer must be f32 or bf16");
}

}  // namespace th

using namespace th;

extern "C" {

int th_buffer_zero(th_buffer* b) {
    TH_API_BEGIN
    TH_REQUIRE(b, "null buffer");
    const size_t bytes = b->n * dtype_size(b->dtype);
    if (bytes == 0) return TH_OK;
    // A fill kernel, not hipMemsetAsync, so the call is safe inside graph capture.
    if (bytes % 4 == 0) {
        TH_LAUNCH(fill_zero_kernel, dim3(grid_for(bytes / 4)), dim3(256), 0, b->dev->stream,
                           (uint32_t*)b->ptr, bytes / 4);
        TH_LAUNCH_CHECK();
    } else {
        TH_HIP(hipMemsetAsync(b->ptr, 0, bytes, b->dev->stream));
    }
    TH_API_END
}

int th_convert(th_device* dev, const th_buffer* src, th_buffer* dst) {
    TH_API_BEGIN
    TH_REQUIRE(dev && src && dst, "null argument");
    auto ok = [](th_dtype t) { return t == TH_F32 || t == TH_BF16 || t == TH_F16; };
    TH_REQUIRE(ok(src->dtype) && ok(dst->dtype), "convert supports f32, bf16 and f16");
    TH_REQUIRE(dst->n >= src->n, "destination too small");
    if (src->n == 0) return TH_OK;
    TH_LAUNCH(convert_kernel, dim3(grid_for(src->n)), dim3(256), 0, dev->stream, src->ptr, src->dtype,
                       dst->ptr, dst->dtype, src->n);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_rms_norm(th_device* dev, const th_buffer* x, const th_buffer* w, size_t groups, size_t dim, float eps,
                th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && x && w && out, "null argument");
    require_len(x, TH_F32, groups * dim, "x");
    require_len_any(w, dim, "weight");
    require_len(out, TH_F32, groups * dim, "out");
    if (groups * dim == 0) return TH_OK;
    TH_LAUNCH(rms_norm_kernel, dim3((unsigned)groups), dim3(256), 0, dev->stream, (const float*)x->ptr,
                       w->ptr, weight_flag(w), (int)dim, eps, (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_rms_norm_residual(th_device* dev, const th_buffer* in, const th_buffer* res, const th_buffer* w, size_t groups,
                         size_t dim, float eps, th_buffer* out, th_buffer* sum_out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && in && res && w && out && sum_out, "null argument");
    require_len(in, TH_F32, groups * dim, "input");
    require_len(res, TH_F32, groups * dim, "residual");
    require_len_any(w, dim, "weight");
    require_len(out, TH_F32, groups * dim, "out");
    require_len(sum_out, TH_F32, groups * dim, "sum_out");
    if (groups * dim == 0) return TH_OK;
    TH_LAUNCH(rms_norm_residual_kernel, dim3((unsigned)groups), dim3(256), 0, dev->stream,
                       (const float*)in->ptr, (const float*)res->ptr, w->ptr, weight_flag(w), (int)dim, eps,
                       (float*)out->ptr, (float*)sum_out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_rope_tables(size_t head_dim, size_t max_seq, double base, float* cos_t, float* sin_t) {
    TH_API_BEGIN
    TH_REQUIRE(cos_t && sin_t, "null table");
    TH_REQUIRE(head_dim % 2 == 0, "head_dim must be even");
    rope_tables_host(head_dim, max_seq, base, cos_t, sin_t);
    TH_API_END
}

int th_rope_forward(th_device* dev, const th_buffer* in, const th_buffer* cs, const th_buffer* sn, size_t seq_len,
                    size_t n_heads, size_t head_dim, size_t start_pos, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && in && cs && sn && out, "null argument");
    TH_REQUIRE(head_dim % 2 == 0, "head_dim must be even");
    const size_t n = seq_len * n_heads * head_dim;
    require_len(in, TH_F32, n, "input");
    require_len(out, TH_F32, n, "out");
    require_len(cs, TH_F32, (start_pos + seq_len) * (head_dim / 2), "cos table");
    require_len(sn, TH_F32, (start_pos + seq_len) * (head_dim / 2), "sin table");
    if (n == 0) return TH_OK;
    TH_LAUNCH(rope_kernel, dim3(grid_for(n / 2)), dim3(256), 0, dev->stream, (const float*)in->ptr,
                       (const float*)cs->ptr, (const float*)sn->ptr, (int)seq_len, (int)n_heads, (int)head_dim,
                       (int)start_pos, (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_swiglu(th_device* dev, const th_buffer* g, const th_buffer* u, size_t n, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && g && u && out, "null argument");
    require_len(g, TH_F32, n, "gate");
    require_len(u, TH_F32, n, "up");
    require_len(out, TH_F32, n, "out");
    if (n == 0) return TH_OK;
    TH_LAUNCH(swiglu_kernel, dim3(grid_for(n)), dim3(256), 0, dev->stream, (const float*)g->ptr,
                       (const float*)u->ptr, n, (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_swiglu_bf16(th_device* dev, const th_buffer* g, const th_buffer* u, size_t n, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && g && u && out, "null argument");
    require_len(g, TH_F32, n, "gate");
    require_len(u, TH_F32, n, "up");
    require_len(out, TH_BF16, n, "out");
    if (n == 0) return TH_OK;
    TH_LAUNCH(swiglu_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, dev->stream, (const float*)g->ptr,
              (const float*)u->ptr, n, (uint16_t*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_add(th_device* dev, const th_buffer* a, const th_buffer* b, size_t n, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && a && b && out, "null argument");
    require_len(a, TH_F32, n, "a");
    require_len(b, TH_F32, n, "b");
    require_len(out, TH_F32, n, "out");
    if (n == 0) return TH_OK;
    TH_LAUNCH(add_kernel, dim3(grid_for(n)), dim3(256), 0, dev->stream, (const float*)a->ptr,
                       (const float*)b->ptr, n, (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_embedding(th_device* dev, const th_buffer* w, const th_buffer* ids, size_t seq_len, size_t dim, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && w && ids && out, "null argument");
    // u32 ids, or an f32 buffer holding their bit patterns (cpu.rs:160, to_bits)
    TH_REQUIRE(ids->dtype == TH_U32 || ids->dtype == TH_I32 || ids->dtype == TH_F32, "ids must be u32");
    require_len_any(ids, seq_len, "ids");
    require_len(out, TH_F32, seq_len * dim, "out");
    TH_REQUIRE(dim > 0 && w->n % dim == 0, "weight length must be a multiple of dim");
    // Validate ids on the host before any gather (an out-of-range id must not
    // reach the kernel).
    std::vector<uint32_t> h(seq_len);
    if (seq_len) {
        TH_HIP(hipStreamSynchronize(dev->stream));
        TH_HIP(hipMemcpy(h.data(), ids->ptr, seq_len * 4, hipMemcpyDeviceToHost));
    }
    const size_t vocab = w->n / dim;
    for (size_t i = 0; i < seq_len; i++) TH_REQUIRE(h[i] < vocab, "token id out of range");
    if (seq_len * dim == 0) return TH_OK;
    TH_LAUNCH(embedding_kernel, dim3(grid_for(seq_len * dim)), dim3(256), 0, dev->stream, w->ptr,
                       weight_flag(w), (const uint32_t*)ids->ptr, (int)seq_len, (int)dim, (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_softmax(th_device* dev, const th_buffer* x, size_t rows, size_t len, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && x && out, "null argument");
    require_len(x, TH_F32, rows * len, "x");
    require_len(out, TH_F32, rows * len, "out");
    if (rows * len == 0) return TH_OK;
    TH_LAUNCH(softmax_kernel, dim3((unsigned)rows), dim3(256), 0, dev->stream, (const float*)x->ptr, (int)len,
                       (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_argmax(th_device* dev, const th_buffer* x, size_t rows, size_t n, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && x && out, "null argument");
    TH_REQUIRE(n > 0, "empty row");
    require_len(x, TH_F32, rows * n, "x");
    TH_REQUIRE(out->dtype == TH_U32 || out->dtype == TH_I32, "out must be u32");
    require_len_any(out, rows, "out");
    if (rows == 0) return TH_OK;
    TH_LAUNCH(argmax_kernel, dim3((unsigned)rows), dim3(256), 0, dev->stream, (const float*)x->ptr, (int)n,
                       (uint32_t*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

}  // extern "C"
