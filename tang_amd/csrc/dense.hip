// Dense (unquantized) ComputeDevice operators, so that model code written
// against tang_compute::ComputeDevice (crates/tang-compute/src/device.rs)
// runs on this backend without a CPU round trip: matmul and its transposed /
// accumulating forms, transpose_2d, reduce_sum, bias_add, add_assign, and the
// tang-expr element-wise kernels (compiled at run time with hiprtc).
#include <hip/hiprtc.h>

#include <cmath>
#include <string>
#include <vector>

#include "capi_util.hpp"
#include "ops.hpp"

struct th_kernel {
    th_device* dev = nullptr;
    hipModule_t module = nullptr;
    hipFunction_t fn = nullptr;
};

namespace th {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// matmul: C[m][n] (+)= op(A)[m][k] . op(B)[k][n] on v_mfma_f32_16x16x4_f32
// (f32 products exact, f32 accumulation).  A is [m][k] row-major, or [k][m]
// with TA; B is [k][n], or [n][k] with TB (device.rs:103,407,425).  A and B
// are f32 or bf16 (converted exactly on load).
// Workgroup: 256 threads = 4 waves in a 2x2 grid, 64x64 output tile, each
// wave 32x32 = 2x2 MFMA tiles; K in steps of 16 staged through LDS with
// padded rows (stride 68 floats: the MFMA operand reads hit distinct banks).
// ---------------------------------------------------------------------------

template <bool BF16>
__device__ __forceinline__ float ld_el(const void* p, size_t i) {
    if constexpr (BF16) return __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16);
    else return ((const float*)p)[i];
}

constexpr int MM_T = 64, MM_K = 16, MM_LD = MM_T + 4;

template <bool TA, bool TB, bool ABF, bool BBF>
__global__ __launch_bounds__(256) void matmul_kernel(const void* __restrict__ a, const void* __restrict__ b,
                                                     float* __restrict__ c, int M, int N, int K, int accumulate) {
    __shared__ float As[MM_K][MM_LD];  // As[kk][row]
    __shared__ float Bs[MM_K][MM_LD];  // Bs[kk][col]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * MM_T, n0 = blockIdx.x * MM_T;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    f32x4_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // staging: each thread moves 4 elements of each 64x16 tile; the fast
    // index follows the contiguous dimension of the source
    auto stage = [&](int k0, float ra[4], float rb[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = tid + 256 * u;
            int row, kk;
            if (TA) { row = e & 63; kk = e >> 6; }   // A[k][m]: m contiguous
            else { kk = e & 15; row = e >> 4; }      // A[m][k]: k contiguous
            const int gm = m0 + row, gk = k0 + kk;
            ra[u] = (gm < M && gk < K) ? ld_el<ABF>(a, TA ? (size_t)gk * M + gm : (size_t)gm * K + gk) : 0.0f;
            int col, kb;
            if (TB) { kb = e & 15; col = e >> 4; }   // B[n][k]: k contiguous
            else { col = e & 63; kb = e >> 6; }      // B[k][n]: n contiguous
            const int gn = n0 + col, gkb = k0 + kb;
            rb[u] = (gn < N && gkb < K) ? ld_el<BBF>(b, TB ? (size_t)gn * K + gkb : (size_t)gkb * N + gn) : 0.0f;
        }
    };
    auto store = [&](const float ra[4], const float rb[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = tid + 256 * u;
            if (TA) As[e >> 6][e & 63] = ra[u];
            else As[e & 15][e >> 4] = ra[u];
            if (TB) Bs[e & 15][e >> 4] = rb[u];
            else Bs[e >> 6][e & 63] = rb[u];
        }
    };
    float ra[4], rb[4];
    stage(0, ra, rb);
    for (int k0 = 0; k0 < K; k0 += MM_K) {
        store(ra, rb);
        __syncthreads();
        if (k0 + MM_K < K) stage(k0 + MM_K, ra, rb);  // next tile's loads in flight during the MFMAs
#pragma unroll
        for (int ks = 0; ks < MM_K; ks += 4) {
            // 16x16x4: lane (g, r) supplies A[row r][k g] and B[k g][col r]
            const int g = lane >> 4, r = lane & 15;
            float av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; i++) av[i] = As[ks + g][wm + 16 * i + r];
#pragma unroll
            for (int j = 0; j < 2; j++) bv[j] = Bs[ks + g][wn + 16 * j + r];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // D: lane (g, r) holds rows 4g..4g+3 of column r
    const int g = lane >> 4, r = lane & 15;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + wn + 16 * j + r;
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int row = m0 + wm + 16 * i + 4 * g + e;
                if (row < M) {
                    float* p = c + (size_t)row * N + col;
                    *p = accumulate ? *p + acc[i][j][e] : acc[i][j][e];
                }
            }
        }
}

template <bool TA, bool TB>
static void matmul_launch2(const th_buffer* a, const th_buffer* b, th_buffer* c, size_t m, size_t k, size_t n,
                           int acc, hipStream_t s) {
    const dim3 grid((unsigned)ceil_div(n, MM_T), (unsigned)ceil_div(m, MM_T));
    const bool abf = a->dtype == TH_BF16, bbf = b->dtype == TH_BF16;
#define TH_MM(AB, BB)                                                                                          \
    TH_LAUNCH((matmul_kernel<TA, TB, AB, BB>), grid, dim3(256), 0, s, a->ptr, b->ptr, (float*)c->ptr, \
                       (int)m, (int)n, (int)k, acc)
    if (abf && bbf) TH_MM(true, true);
    else if (abf) TH_MM(true, false);
    else if (bbf) TH_MM(false, true);
    else TH_MM(false, false);
#undef TH_MM
    TH_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// transpose_2d (cpu.rs:317-326): out[c][r] = in[r][c], 32x32 LDS tiles.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ in, float* __restrict__ out, int rows,
                                                        int cols) {
    __shared__ float t[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int y = ty; y < 32; y += 8)
        if (r0 + y < rows && c0 + tx < cols) t[y][tx] = in[(size_t)(r0 + y) * cols + c0 + tx];
    __syncthreads();
    for (int y = ty; y < 32; y += 8)
        if (c0 + y < cols && r0 + tx < rows) out[(size_t)(c0 + y) * rows + r0 + tx] = t[tx][y];
}

// ---------------------------------------------------------------------------
// reduce_sum (cpu.rs:169-199): out[o][i] = sum over a of in[o][a][i], added
// in order a = 0, 1, ... in f32 from 0 (bit-identical to the reference).
// One thread per output; neighbouring threads read neighbouring i.
// ---------------------------------------------------------------------------
__global__ void reduce_sum_kernel(const float* __restrict__ in, float* __restrict__ out, size_t outer, size_t len,
                                  size_t inner, int accumulate) {
    const size_t total = outer * inner;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
        const size_t o = idx / inner, i = idx - o * inner;
        const float* p = in + o * len * inner + i;
        float s = 0.0f;
        for (size_t a = 0; a < len; a++) s += p[a * inner];
        out[idx] = accumulate ? out[idx] + s : s;
    }
}

// bias_add (device.rs:378-386): out[i] = matrix[i] + bias[i % dim].
__global__ void bias_add_kernel(const float* __restrict__ m, const float* __restrict__ bias, float* __restrict__ out,
                                size_t numel, size_t dim) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < numel; i += (size_t)gridDim.x * blockDim.x)
        out[i] = m[i] + bias[i % dim];
}

// add_assign (cpu.rs:650-655): dst[i] += src[i].
__global__ void add_assign_kernel(float* __restrict__ dst, const float* __restrict__ src, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = dst[i] + src[i];
}

static unsigned grid_of(size_t n) { return (unsigned)std::max<size_t>(1, std::min<size_t>(ceil_div(n, 256), 8192)); }

}  // namespace th

using namespace th;

extern "C" {

int th_matmul_ex(th_device* dev, const th_buffer* a, const th_buffer* b, size_t m, size_t k, size_t n, int trans_a,
                 int trans_b, int accumulate, th_buffer* c) {
    TH_API_BEGIN
    TH_REQUIRE(dev && a && b && c, "null argument");
    TH_REQUIRE(a->dtype == TH_F32 || a->dtype == TH_BF16, "a must be f32 or bf16");
    TH_REQUIRE(b->dtype == TH_F32 || b->dtype == TH_BF16, "b must be f32 or bf16");
    require_len_any(a, m * k, "a");
    require_len_any(b, k * n, "b");
    require_len(c, TH_F32, m * n, "c");
    TH_REQUIRE(m < (1u << 31) / MM_T && n < (1u << 31) / MM_T && k < (1u << 31), "matmul: dimension too large");
    if (m == 0 || n == 0) return TH_OK;
    hipStream_t s = dev->stream;
    if (k == 0) {  // an empty sum: C = 0 (or C unchanged when accumulating)
        if (!accumulate) check_status(th_buffer_zero(c));
        return TH_OK;
    }
    if (trans_a && trans_b) matmul_launch2<true, true>(a, b, c, m, k, n, accumulate, s);
    else if (trans_a) matmul_launch2<true, false>(a, b, c, m, k, n, accumulate, s);
    else if (trans_b) matmul_launch2<false, true>(a, b, c, m, k, n, accumulate, s);
    else matmul_launch2<false, false>(a, b, c, m, k, n, accumulate, s);
    TH_API_END
}

int th_matmul(th_device* dev, const th_buffer* a, const th_buffer* b, size_t m, size_t k, size_t n, th_buffer* c) {
    return th_matmul_ex(dev, a, b, m, k, n, 0, 0, 0, c);
}

int th_matmul_b_transposed(th_device* dev, const th_buffer* a, const th_buffer* b, size_t m, size_t k, size_t n,
                           th_buffer* c) {
    return th_matmul_ex(dev, a, b, m, k, n, 0, 1, 0, c);
}

int th_transpose_2d(th_device* dev, const th_buffer* in, size_t rows, size_t cols, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && in && out, "null argument");
    require_len(in, TH_F32, rows * cols, "in");
    require_len(out, TH_F32, rows * cols, "out");
    TH_REQUIRE(rows < (1u << 31) && cols < (1u << 31), "transpose: dimension too large");
    if (rows == 0 || cols == 0) return TH_OK;
    TH_REQUIRE(ceil_div(rows, 32) < 65536, "transpose: more than 2^21 rows");
    TH_LAUNCH(transpose_kernel, dim3((unsigned)ceil_div(cols, 32), (unsigned)ceil_div(rows, 32)), dim3(256), 0,
                       dev->stream, (const float*)in->ptr, (float*)out->ptr, (int)rows, (int)cols);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_reduce_sum(th_device* dev, const th_buffer* in, const size_t* shape, size_t ndim, size_t axis, int accumulate,
                  th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && in && out && (shape || ndim == 0), "null argument");
    TH_REQUIRE(axis < ndim, "reduce_sum: axis out of range");
    size_t outer = 1, inner = 1;
    for (size_t i = 0; i < axis; i++) outer *= shape[i];
    for (size_t i = axis + 1; i < ndim; i++) inner *= shape[i];
    const size_t len = shape[axis];
    require_len(in, TH_F32, outer * len * inner, "in");
    require_len(out, TH_F32, outer * inner, "out");
    if (outer * inner == 0) return TH_OK;
    TH_LAUNCH(reduce_sum_kernel, dim3(grid_of(outer * inner)), dim3(256), 0, dev->stream,
                       (const float*)in->ptr, (float*)out->ptr, outer, len, inner, accumulate);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_bias_add(th_device* dev, const th_buffer* matrix, const th_buffer* bias, size_t numel, size_t dim,
                th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && matrix && bias && out, "null argument");
    TH_REQUIRE(dim > 0 || numel == 0, "bias_add: dim is 0");
    require_len(matrix, TH_F32, numel, "matrix");
    require_len(bias, TH_F32, dim, "bias");
    require_len(out, TH_F32, numel, "out");
    if (numel == 0) return TH_OK;
    TH_LAUNCH(bias_add_kernel, dim3(grid_of(numel)), dim3(256), 0, dev->stream, (const float*)matrix->ptr,
                       (const float*)bias->ptr, (float*)out->ptr, numel, dim);
    TH_LAUNCH_CHECK();
    TH_API_END
}

int th_add_assign(th_device* dev, th_buffer* dst, const th_buffer* src) {
    TH_API_BEGIN
    TH_REQUIRE(dev && dst && src, "null argument");
    TH_REQUIRE(dst->dtype == TH_F32 && src->dtype == TH_F32, "add_assign: f32 buffers");
    TH_REQUIRE(dst->n == src->n, "add_assign: lengths differ");  // cpu.rs:651 asserts equal lengths
    if (dst->n == 0) return TH_OK;
    TH_LAUNCH(add_assign_kernel, dim3(grid_of(dst->n)), dim3(256), 0, dev->stream, (float*)dst->ptr,
                       (const float*)src->ptr, dst->n);
    TH_LAUNCH_CHECK();
    TH_API_END
}

// ---- run-time compiled element-wise kernels --------------------------------

int th_kernel_compile(th_device* dev, const char* source, const char* entry, th_kernel** out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && source && entry && out, "null argument");
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, source, "elementwise.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
        throw Error(TH_ERR_HIP, "hiprtcCreateProgram failed");
    // gfx950 only; no packed-FP32 instructions and no FMA contraction, as
    // the library's own kernels
    const char* opts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-Xclang", "-target-feature",
                          "-Xclang", "-packed-fp32-ops"};
    const hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof(opts) / sizeof(opts[0])), opts);
    if (rc != HIPRTC_SUCCESS) {
        size_t n = 0;
        std::string log;
        if (hiprtcGetProgramLogSize(prog, &n) == HIPRTC_SUCCESS && n > 1) {
            log.resize(n);
            hiprtcGetProgramLog(prog, &log[0]);
        }
        hiprtcDestroyProgram(&prog);
        throw Error(TH_ERR_INVALID, std::string("kernel compile failed: ") + hiprtcGetErrorString(rc) + "\n" + log);
    }
    size_t code_size = 0;
    hiprtcGetCodeSize(prog, &code_size);
    std::vector<char> code(code_size);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    th_kernel* k = new th_kernel();
    k->dev = dev;
    hipError_t e = hipModuleLoadData(&k->module, code.data());
    if (e == hipSuccess) e = hipModuleGetFunction(&k->fn, k->module, entry);
    if (e != hipSuccess) {
        if (k->module) (void)hipModuleUnload(k->module);
        delete k;
        throw Error(TH_ERR_HIP, std::string("module load: ") + hipGetErrorString(e));
    }
    device_retain(dev);
    *out = k;
    TH_API_END
}

int th_kernel_free(th_kernel* k) {
    TH_API_BEGIN
    if (!k) return TH_OK;
    th_device* d = k->dev;
    device_drain(d);
    (void)hipModuleUnload(k->module);
    delete k;
    device_release(d);
    TH_API_END
}

int th_elementwise(th_kernel* k, const th_buffer* const* inputs, size_t n_inputs, size_t numel, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(k && out && (inputs || n_inputs == 0), "null argument");
    TH_REQUIRE(n_inputs <= 64, "elementwise: at most 64 inputs");
    TH_REQUIRE(numel <= 0xFFFFFFFFu, "elementwise: count is a 32-bit kernel argument");
    for (size_t i = 0; i < n_inputs; i++) require_len(inputs[i], TH_F32, numel, "input");
    require_len(out, TH_F32, numel, "out");
    if (numel == 0) return TH_OK;
    // argument block of the generated signature: in0..in{n-1}, outputs, count
    std::vector<char> args;
    auto put = [&](const void* p, size_t sz, size_t align) {
        args.resize(round_up(args.size(), align));
        const size_t o = args.size();
        args.resize(o + sz);
        std::memcpy(&args[o], p, sz);
    };
    for (size_t i = 0; i < n_inputs; i++) put(&inputs[i]->ptr, sizeof(void*), sizeof(void*));
    put(&out->ptr, sizeof(void*), sizeof(void*));
    const unsigned count = (unsigned)numel;
    put(&count, sizeof(count), sizeof(count));
    size_t bytes = args.size();
    void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args.data(), HIP_LAUNCH_PARAM_BUFFER_SIZE, &bytes,
                   HIP_LAUNCH_PARAM_END};
    TH_HIP(hipModuleLaunchKernel(k->fn, (unsigned)ceil_div(numel, 256), 1, 1, 256, 1, 1, 0, k->dev->stream, nullptr,
                                 cfg));
    TH_API_END
}

}  // extern "C"
