// Device, buffer and quantized-weight management behind the C ABI.
//
// Mirrors the buffer lifecycle of tang_compute::ComputeDevice
// (crates/tang-compute/src/device.rs:44-80): upload / alloc / download, with
// one HIP stream per device (the reference CUDA backend also uses a single
// stream, crates/tang-compute/src/cuda.rs:155-158).
#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "capi_util.hpp"
#include "aql.hpp"
#include "qlinear.hpp"

namespace th {

// Workspace of th_gemm_q4_noalloc (the allocation-free GEMM): a file-scope
// device array, TH_NOALLOC_SCRATCH_BYTES per GPU, held by every GPU the
// library runs on until the process ends.  Host code never uses its name as
// an address: th_device_create looks up the array's address on its device
// (th_device::noalloc_scratch) and kernels receive that.  Every call on one
// GPU shares it.
static __device__ __align__(256) unsigned char scratch[TH_NOALLOC_SCRATCH_BYTES];

static thread_local std::string g_last_error;
void set_last_error(const std::string& msg) { g_last_error = msg; }

void* device_scratch(th_device* dev, size_t bytes) {
    if (bytes <= dev->scratch_bytes) return dev->scratch;
    if (dev->scratch) {
        TH_HIP(hipStreamSynchronize(dev->stream));
        TH_HIP(hipFree(dev->scratch));
        dev->scratch = nullptr;
        dev->scratch_bytes = 0;
    }
    size_t want = std::max(bytes, (size_t)1 << 20);
    TH_HIP(hipMalloc(&dev->scratch, want));
    dev->scratch_bytes = want;
    return dev->scratch;
}

void* device_scratch_x(th_device* dev, size_t bytes) {
    if (bytes <= dev->scratch_x_bytes) return dev->scratch_x;
    if (dev->scratch_x) {
        TH_HIP(hipStreamSynchronize(dev->stream));
        TH_HIP(hipFree(dev->scratch_x));
        dev->scratch_x = nullptr;
        dev->scratch_x_bytes = 0;
    }
    size_t want = std::max(bytes, (size_t)1 << 20);
    TH_HIP(hipMalloc(&dev->scratch_x, want));
    dev->scratch_x_bytes = want;
    return dev->scratch_x;
}

int* device_counters(th_device* dev, size_t n) {
    if (n <= dev->n_counters) return dev->counters;
    if (dev->counters) {
        TH_HIP(hipStreamSynchronize(dev->stream));
        TH_HIP(hipFree(dev->counters));
        dev->counters = nullptr;
        dev->n_counters = 0;
    }
    const size_t want = std::max(n, (size_t)4096);
    TH_HIP(hipMalloc(&dev->counters, want * sizeof(int)));
    TH_HIP(hipMemset(dev->counters, 0, want * sizeof(int)));
    dev->n_counters = want;
    return dev->counters;
}

static void check_buf(const th_buffer* b, const char* what) {
    if (!b || !b->ptr && b->n) throw Error(TH_ERR_INVALID, std::string("null buffer: ") + what);
}

void require_len(const th_buffer* b, th_dtype dt, size_t n, const char* what) {
    if (!b) throw Error(TH_ERR_INVALID, std::string("null buffer: ") + what);
    if (b->dtype != dt)
        throw Error(TH_ERR_INVALID, std::string("buffer ") + what + " has the wrong dtype");
    if (b->n < n)
        throw Error(TH_ERR_INVALID, std::string("buffer ") + what + " too small: " + std::to_string(b->n) +
                                        " < " + std::to_string(n));
}

void require_len_any(const th_buffer* b, size_t n, const char* what) {
    check_buf(b, what);
    if (b->n < n)
        throw Error(TH_ERR_INVALID, std::string("buffer ") + what + " too small: " + std::to_string(b->n) +
                                        " < " + std::to_string(n));
}

// ---------------------------------------------------------------------------
// Quantized weight packing (host side), see the th_qweight comment.
// ---------------------------------------------------------------------------

th_qweight* q4_pack(th_device* dev, const uint8_t* nib, const void* scales, th_dtype sdt, size_t rows,
                    size_t cols) {
    TH_REQUIRE(rows > 0 && cols > 0, "empty matrix");
    TH_REQUIRE(sdt == TH_F16 || sdt == TH_F32, "scale dtype must be f16 or f32");
    const size_t bpr = ceil_div(cols, 32);
    const size_t Np = round_up(rows, 16), Kp = round_up(cols, 128);
    const size_t GQ = Kp / 128, NT = Np / 16;
    std::vector<uint8_t> tiles(NT * GQ * 1024, 0x88);
    const size_t ssz = dtype_size(sdt);
    const bool f16 = sdt == TH_F16;
    std::vector<uint8_t> stile(q4_scale_count(f16, NT, GQ) * ssz, 0);
#pragma omp parallel for schedule(static)
    for (long rowl = 0; rowl < (long)rows; rowl++) {
        const size_t row = (size_t)rowl;
        const size_t t = row / 16, rr = row % 16;
        for (size_t g = 0; g < bpr; g++) {
            const size_t gq = g / 4, j = g % 4;
            const uint8_t* src = nib + (row * bpr + g) * 16;
            uint8_t tail[16];
            if (g == bpr - 1 && cols % 32) {
                // Elements past `cols` are ignored by q4_matvec (quantize.rs:277-282):
                // store them as the zero code so the kernels may read any finite x there.
                std::memcpy(tail, src, 16);
                for (size_t e = cols % 32; e < 32; e++)
                    tail[e / 2] = (e & 1) ? (uint8_t)((tail[e / 2] & 0x0F) | 0x80) : (uint8_t)((tail[e / 2] & 0xF0) | 0x08);
                src = tail;
            }
            uint8_t* tb = tiles.data() + (t * GQ + gq) * 1024;
            for (size_t q = 0; q < 4; q++) std::memcpy(tb + (q * 16 + rr) * 16 + j * 4, src + q * 4, 4);
            const uint8_t* s = (const uint8_t*)scales + (row * bpr + g) * ssz;
            std::memcpy(stile.data() + q4_scale_index(f16, t, gq, rr, j, GQ) * ssz, s, ssz);
        }
    }
    // per-row scale exponents for the MFMA GEMM's f16 operands (row maximum
    // scale brought to [2^8, 2^9); padding rows 0)
    std::vector<int> rexp(Np, 0);
    for (size_t row = 0; row < rows; row++) {
        float mx = 0.0f;
        for (size_t g = 0; g < bpr; g++) {
            const uint8_t* sp = (const uint8_t*)scales + (row * bpr + g) * ssz;
            float v;
            if (f16) { uint16_t h; std::memcpy(&h, sp, 2); v = f16_to_f32_host(h); }
            else std::memcpy(&v, sp, 4);
            mx = std::max(mx, std::fabs(v));
        }
        rexp[row] = range_exp(mx, WSCALE_TOP);
    }
    th_qweight* w = new th_qweight();
    w->dev = dev; w->bits = 4; w->rows = rows; w->cols = cols; w->Np = Np; w->Kp = Kp;
    w->scale_dtype = sdt;
    w->data_bytes = tiles.size(); w->scale_bytes = stile.size();
    try {
        TH_HIP(hipMalloc(&w->data, w->data_bytes));
        TH_HIP(hipMalloc(&w->scales, w->scale_bytes));
        TH_HIP(hipMalloc(&w->row_exp, Np * sizeof(int)));
        TH_HIP(hipMemcpy(w->data, tiles.data(), w->data_bytes, hipMemcpyHostToDevice));
        TH_HIP(hipMemcpy(w->scales, stile.data(), w->scale_bytes, hipMemcpyHostToDevice));
        TH_HIP(hipMemcpy(w->row_exp, rexp.data(), Np * sizeof(int), hipMemcpyHostToDevice));
    } catch (...) {
        if (w->data) (void)hipFree(w->data);
        if (w->scales) (void)hipFree(w->scales);
        if (w->row_exp) (void)hipFree(w->row_exp);
        delete w;
        throw;
    }
    device_retain(dev);
    return w;
}

void q4_unpack(const th_qweight* w, th_q4_block* out) {
    TH_REQUIRE(w && w->bits == 4, "not a q4 weight");
    const size_t bpr = ceil_div(w->cols, 32), GQ = w->Kp / 128, NT = w->Np / 16;
    const size_t ssz = dtype_size(w->scale_dtype);
    std::vector<uint8_t> tiles(w->data_bytes), stile(w->scale_bytes);
    TH_HIP(hipMemcpy(tiles.data(), w->data, w->data_bytes, hipMemcpyDeviceToHost));
    TH_HIP(hipMemcpy(stile.data(), w->scales, w->scale_bytes, hipMemcpyDeviceToHost));
    (void)NT;
    for (size_t row = 0; row < w->rows; row++) {
        const size_t t = row / 16, rr = row % 16;
        for (size_t g = 0; g < bpr; g++) {
            const size_t gq = g / 4, j = g % 4;
            th_q4_block& b = out[row * bpr + g];
            const uint8_t* tb = tiles.data() + (t * GQ + gq) * 1024;
            for (size_t q = 0; q < 4; q++) std::memcpy(b.values + q * 4, tb + (q * 16 + rr) * 16 + j * 4, 4);
            const uint8_t* s = stile.data() + q4_scale_index(w->scale_dtype == TH_F16, t, gq, rr, j, GQ) * ssz;
            if (w->scale_dtype == TH_F32) std::memcpy(&b.scale, s, 4);
            else { uint16_t h; std::memcpy(&h, s, 2); b.scale = f16_to_f32_host(h); }
        }
    }
}

th_qweight* q8_pack(th_device* dev, const int8_t* q, size_t ldq, const float* scales, bool per_row,
                    size_t rows, size_t cols) {
    TH_REQUIRE(rows > 0 && cols > 0, "empty matrix");
    const size_t Np = round_up(rows, 16), Kp = round_up(cols, 64);
    const size_t NCH = Kp / 64, NT = Np / 16, GPR = Kp / 32, bpr = ceil_div(cols, 32);
    std::vector<uint8_t> tiles(NT * NCH * 1024, 0);
    for (size_t row = 0; row < rows; row++) {
        const size_t t = row / 16, rr = row % 16;
        for (size_t k = 0; k < cols; k++) {
            const size_t c = k / 64, q4 = (k % 64) / 16, e = k % 16;
            tiles[(t * NCH + c) * 1024 + (q4 * 16 + rr) * 16 + e] = (uint8_t)q[row * ldq + k];
        }
    }
    std::vector<float> st(per_row ? Np : Np * GPR, 0.0f);
    for (size_t row = 0; row < rows; row++) {
        if (per_row) st[row] = scales[row];
        else for (size_t g = 0; g < bpr; g++) st[row * GPR + g] = scales[row * bpr + g];
    }
    th_qweight* w = new th_qweight();
    w->dev = dev; w->bits = 8; w->rows = rows; w->cols = cols; w->Np = Np; w->Kp = Kp;
    w->scale_dtype = TH_F32; w->per_row = per_row;
    w->data_bytes = tiles.size(); w->scale_bytes = st.size() * 4;
    try {
        TH_HIP(hipMalloc(&w->data, w->data_bytes));
        TH_HIP(hipMalloc(&w->scales, w->scale_bytes));
        TH_HIP(hipMemcpy(w->data, tiles.data(), w->data_bytes, hipMemcpyHostToDevice));
        TH_HIP(hipMemcpy(w->scales, st.data(), w->scale_bytes, hipMemcpyHostToDevice));
    } catch (...) {
        if (w->data) (void)hipFree(w->data);
        if (w->scales) (void)hipFree(w->scales);
        delete w;
        throw;
    }
    device_retain(dev);
    return w;
}

}  // namespace th

using namespace th;

extern "C" {

const char* th_last_error(void) { return g_last_error.c_str(); }

int th_device_count(int* n) {
    TH_API_BEGIN
    TH_REQUIRE(n, "null out");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) c = 0;
    *n = c;
    TH_API_END
}

int th_device_create(int ordinal, th_device** out) {
    TH_API_BEGIN
    TH_REQUIRE(out, "null out");
    int c = 0;
    TH_HIP(hipGetDeviceCount(&c));
    TH_REQUIRE(ordinal >= 0 && ordinal < c, "device ordinal out of range");
    TH_HIP(hipSetDevice(ordinal));
    // this GPU's copy of the allocation-free GEMM's workspace (device current)
    void* noalloc = nullptr;
    TH_HIP(hipGetSymbolAddress(&noalloc, HIP_SYMBOL(scratch)));
    th_device* d = new th_device();
    d->ordinal = ordinal;
    d->noalloc_scratch = noalloc;
    TH_HIP(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking));
    TH_HIP(hipEventCreate(&d->ev_start));
    TH_HIP(hipEventCreate(&d->ev_stop));
    hipDeviceProp_t prop;
    TH_HIP(hipGetDeviceProperties(&prop, ordinal));
    d->num_cus = prop.multiProcessorCount;
    *out = d;
    TH_API_END
}

int th_device_destroy(th_device* d) {
    TH_API_BEGIN
    if (!d) return TH_OK;
    (void)hipSetDevice(d->ordinal);
    TH_REQUIRE(!d->closed, "device already destroyed");
    th::aql_release(d);
    (void)hipStreamSynchronize(d->stream);
    th::expr_release(d);
    if (d->scratch) (void)hipFree(d->scratch);
    if (d->scratch_x) (void)hipFree(d->scratch_x);
    if (d->counters) (void)hipFree(d->counters);
    (void)hipEventDestroy(d->ev_start);
    (void)hipEventDestroy(d->ev_stop);
    (void)hipStreamDestroy(d->stream);
    d->stream = nullptr;
    d->scratch = d->scratch_x = nullptr;
    d->counters = nullptr;
    d->closed = true;
    if (d->live == 0) delete d;
    TH_API_END
}

int th_sync(th_device* d) {
    TH_API_BEGIN
    TH_REQUIRE(d, "null device");
    th::device_sync(d);
    TH_API_END
}

int th_memory_info(th_device* d, size_t* free_b, size_t* total_b) {
    TH_API_BEGIN
    TH_REQUIRE(d, "null device");
    TH_HIP(hipSetDevice(d->ordinal));
    size_t f = 0, t = 0;
    TH_HIP(hipMemGetInfo(&f, &t));
    if (free_b) *free_b = f;
    if (total_b) *total_b = t;
    TH_API_END
}

int th_timer_start(th_device* d) {
    TH_API_BEGIN
    TH_REQUIRE(d, "null device");
    TH_HIP(hipEventRecord(d->ev_start, d->stream));
    TH_API_END
}

int th_timer_stop(th_device* d, float* ms) {
    TH_API_BEGIN
    TH_REQUIRE(d && ms, "null argument");
    TH_HIP(hipEventRecord(d->ev_stop, d->stream));
    TH_HIP(hipEventSynchronize(d->ev_stop));
    TH_HIP(hipEventElapsedTime(ms, d->ev_start, d->ev_stop));
    TH_API_END
}

int th_capture_begin(th_device* d) {
    TH_API_BEGIN
    TH_REQUIRE(d, "null device");
    TH_HIP(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
    TH_API_END
}

int th_capture_end(th_device* d, th_graph** out) {
    TH_API_BEGIN
    TH_REQUIRE(d && out, "null argument");
    hipGraph_t g = nullptr;
    TH_HIP(hipStreamEndCapture(d->stream, &g));
    hipGraphExec_t ge = nullptr;
    const hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    TH_HIP(e);
    th_graph* r = new th_graph();
    r->dev = d;
    r->exec = ge;
    device_retain(d);
    *out = r;
    TH_API_END
}

int th_graph_launch(th_graph* g) {
    TH_API_BEGIN
    TH_REQUIRE(g && !g->dev->closed, "null graph or closed device");
    TH_HIP(hipGraphLaunch(g->exec, g->dev->stream));
    TH_API_END
}

int th_graph_destroy(th_graph* g) {
    TH_API_BEGIN
    if (!g) return TH_OK;
    device_drain(g->dev);
    (void)hipGraphExecDestroy(g->exec);
    th_device* d = g->dev;
    delete g;
    device_release(d);
    TH_API_END
}

int th_buffer_alloc(th_device* d, th_dtype dt, size_t n, th_buffer** out) {
    TH_API_BEGIN
    TH_REQUIRE(d && out, "null argument");
    TH_REQUIRE(dtype_size(dt) > 0, "bad dtype");
    th_buffer* b = new th_buffer();
    b->dev = d; b->dtype = dt; b->n = n;
    if (n) {
        hipError_t e = hipMalloc(&b->ptr, n * dtype_size(dt));
        if (e != hipSuccess) {
            delete b;
            throw Error(e == hipErrorOutOfMemory ? TH_ERR_OOM : TH_ERR_HIP,
                        std::string("hipMalloc: ") + hipGetErrorString(e));
        }
    }
    device_retain(d);
    *out = b;
    TH_API_END
}

int th_buffer_free(th_buffer* b) {
    TH_API_BEGIN
    if (!b) return TH_OK;
    th_device* d = b->dev;
    if (b->ptr) {
        device_drain(d);
        (void)hipFree(b->ptr);
    }
    delete b;
    device_release(d);
    TH_API_END
}

int th_buffer_upload(th_buffer* b, const void* host, size_t n) {
    TH_API_BEGIN
    TH_REQUIRE(b && (host || n == 0), "null argument");
    TH_REQUIRE(n <= b->n, "upload larger than buffer");
    if (n) {
        TH_HIP(hipMemcpyAsync(b->ptr, host, n * dtype_size(b->dtype), hipMemcpyHostToDevice, b->dev->stream));
        TH_HIP(hipStreamSynchronize(b->dev->stream));
    }
    TH_API_END
}

int th_buffer_download(th_buffer* b, void* host, size_t n) {
    TH_API_BEGIN
    TH_REQUIRE(b && (host || n == 0), "null argument");
    TH_REQUIRE(n <= b->n, "download larger than buffer");
    TH_HIP(hipStreamSynchronize(b->dev->stream));
    if (n) {
        TH_HIP(hipMemcpyAsync(host, b->ptr, n * dtype_size(b->dtype), hipMemcpyDeviceToHost, b->dev->stream));
        TH_HIP(hipStreamSynchronize(b->dev->stream));
    }
    TH_API_END
}

int th_buffer_copy(th_buffer* dst, const th_buffer* src) {
    TH_API_BEGIN
    TH_REQUIRE(dst && src && dst->dev == src->dev, "buffers must share a device");
    const size_t bytes = std::min(dst->n * dtype_size(dst->dtype), src->n * dtype_size(src->dtype));
    if (bytes) TH_HIP(hipMemcpyAsync(dst->ptr, src->ptr, bytes, hipMemcpyDeviceToDevice, dst->dev->stream));
    TH_API_END
}

int th_buffer_copy_region(th_buffer* dst, size_t dst_offset, const th_buffer* src, size_t src_offset, size_t n) {
    TH_API_BEGIN
    TH_REQUIRE(dst && src && dst->dev == src->dev, "buffers must share a device");
    TH_REQUIRE(dst->dtype == src->dtype, "buffers must share a dtype");
    TH_REQUIRE(src_offset <= src->n && n <= src->n - src_offset, "source range out of bounds");
    TH_REQUIRE(dst_offset <= dst->n && n <= dst->n - dst_offset, "destination range out of bounds");
    const size_t es = dtype_size(dst->dtype);
    if (n)
        TH_HIP(hipMemcpyAsync((char*)dst->ptr + dst_offset * es, (const char*)src->ptr + src_offset * es, n * es,
                              hipMemcpyDeviceToDevice, dst->dev->stream));
    TH_API_END
}

int th_buffer_info(const th_buffer* b, th_dtype* dt, size_t* n) {
    TH_API_BEGIN
    TH_REQUIRE(b, "null buffer");
    if (dt) *dt = b->dtype;
    if (n) *n = b->n;
    TH_API_END
}

int th_q4_upload_blocks(th_device* d, const th_q4_block* blocks, size_t rows, size_t cols,
                        th_dtype sdt, th_qweight** out) {
    TH_API_BEGIN
    TH_REQUIRE(d && blocks && out, "null argument");
    const size_t bpr = ceil_div(cols, 32), nb = rows * bpr;
    std::vector<uint8_t> nib(nb * 16);
    std::vector<uint8_t> sc(nb * dtype_size(sdt));
    for (size_t i = 0; i < nb; i++) {
        std::memcpy(nib.data() + i * 16, blocks[i].values, 16);
        if (sdt == TH_F32) {
            std::memcpy(sc.data() + i * 4, &blocks[i].scale, 4);
        } else if (sdt == TH_F16) {
            uint16_t h = f32_to_f16_host(blocks[i].scale);
            if (f16_to_f32_host(h) != blocks[i].scale)
                throw Error(TH_ERR_INVALID, "th_q4_upload_blocks: scale not exactly representable in f16");
            std::memcpy(sc.data() + i * 2, &h, 2);
        } else {
            throw Error(TH_ERR_INVALID, "th_q4_upload_blocks: scale dtype must be f16 or f32");
        }
    }
    *out = q4_pack(d, nib.data(), sc.data(), sdt, rows, cols);
    TH_API_END
}

int th_q4_upload_packed(th_device* d, const uint8_t* nib, const void* scales, th_dtype sdt, size_t rows,
                        size_t cols, th_qweight** out) {
    TH_API_BEGIN
    TH_REQUIRE(d && nib && scales && out, "null argument");
    *out = q4_pack(d, nib, scales, sdt, rows, cols);
    TH_API_END
}

int th_q8_upload_blocks(th_device* d, const th_q8_block* blocks, size_t rows, size_t cols,
                        th_qweight** out) {
    TH_API_BEGIN
    TH_REQUIRE(d && blocks && out, "null argument");
    TH_REQUIRE(rows > 0 && cols > 0, "empty matrix");
    const size_t bpr = ceil_div(cols, 32);
    std::vector<int8_t> q(rows * bpr * 32);
    std::vector<float> sc(rows * bpr);
    bool per_row = true;
    for (size_t r = 0; r < rows; r++) {
        for (size_t b = 0; b < bpr; b++) {
            const th_q8_block& blk = blocks[r * bpr + b];
            std::memcpy(q.data() + (r * bpr + b) * 32, blk.values, 32);
            sc[r * bpr + b] = blk.scale;
            if (blk.scale != blocks[r * bpr].scale) per_row = false;
        }
    }
    std::vector<float> rs;
    if (per_row) {
        rs.resize(rows);
        for (size_t r = 0; r < rows; r++) rs[r] = sc[r * bpr];
    }
    *out = q8_pack(d, q.data(), bpr * 32, per_row ? rs.data() : sc.data(), per_row, rows, cols);
    TH_API_END
}

int th_q8_upload_rowwise(th_device* d, const int8_t* q, const float* row_scale, size_t rows, size_t cols,
                         th_qweight** out) {
    TH_API_BEGIN
    TH_REQUIRE(d && q && row_scale && out, "null argument");
    *out = q8_pack(d, q, cols, row_scale, true, rows, cols);
    TH_API_END
}

int th_q4_download_blocks(const th_qweight* w, th_q4_block* blocks) {
    TH_API_BEGIN
    TH_REQUIRE(w && blocks, "null argument");
    q4_unpack(w, blocks);
    TH_API_END
}

int th_qweight_info(const th_qweight* w, size_t* rows, size_t* cols, int* bits) {
    TH_API_BEGIN
    TH_REQUIRE(w, "null weight");
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (bits) *bits = w->bits;
    TH_API_END
}

int th_qweight_free(th_qweight* w) {
    TH_API_BEGIN
    if (!w) return TH_OK;
    th_device* d = w->dev;
    device_drain(d);
    if (w->data) (void)hipFree(w->data);
    if (w->scales) (void)hipFree(w->scales);
    if (w->row_exp) (void)hipFree(w->row_exp);
    delete w;
    device_release(d);
    TH_API_END
}

}  // extern "C"
