// Weights from files into the device layout:
//  * the reference quantizers quantize_matrix_q4 / quantize_matrix_q8
//    (crates/tang-infer/src/quantize.rs:47-118,193-220), restated on the host;
//  * a safetensors reader (the format tang-safetensors loads through the
//    `safetensors` crate, crates/tang-safetensors/src/lib.rs:11-70): an
//    8-byte little-endian header length, a JSON header mapping each tensor
//    name to {dtype, shape, data_offsets}, then the data.  F64, F32, F16 and
//    BF16 are read, as the reference does; other dtypes are rejected.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <memory>
#include <string>
#include <vector>

#include "capi_util.hpp"

namespace th {

// One quantized block of at most 32 values (quantize.rs:84-118 / :47-70).
static void quant_q4_block(const float* x, size_t n, th_q4_block& b) {
    float amax = 0.0f;
    for (size_t i = 0; i < n; i++) amax = std::fmax(amax, std::fabs(x[i]));
    const float scale = amax == 0.0f ? 1.0f : amax / 7.0f;
    const float inv = 1.0f / scale;
    auto q = [&](size_t i) -> int {
        if (i >= n) return 0;
        const float r = std::round(x[i] * inv);  // f32::round: half away from zero
        if (std::isnan(r)) return 0;            // Rust's saturating cast maps NaN to 0
        return (int)std::fmin(std::fmax(r, -8.0f), 7.0f);
    };
    b.scale = scale;
    for (size_t i = 0; i < 16; i++) b.values[i] = (uint8_t)((q(2 * i) + 8) | ((q(2 * i + 1) + 8) << 4));
}

static void quant_q8_block(const float* x, size_t n, th_q8_block& b) {
    float amax = 0.0f;
    for (size_t i = 0; i < n; i++) amax = std::fmax(amax, std::fabs(x[i]));
    const float scale = amax == 0.0f ? 1.0f : amax / 127.0f;
    const float inv = 1.0f / scale;
    b.scale = scale;
    for (size_t i = 0; i < 32; i++) {
        int v = 0;
        if (i < n) {
            const float r = std::round(x[i] * inv);
            v = std::isnan(r) ? 0 : (int)std::fmin(std::fmax(r, -128.0f), 127.0f);
        }
        b.values[i] = (int8_t)v;
    }
}

// ---- safetensors ------------------------------------------------------------

struct StTensor {
    std::string name;
    int dtype = 0;  // TH_ST_*
    std::vector<size_t> shape;
    size_t begin = 0, end = 0;
};

// Minimal JSON reader for the safetensors header: objects, arrays, strings
// (with escapes), integers; anything else is skipped as a bare token.
struct Json {
    const std::string& s;
    size_t i = 0;
    explicit Json(const std::string& str) : s(str) {}
    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) i++;
    }
    void expect(char c) {
        ws();
        TH_REQUIRE(i < s.size() && s[i] == c, "safetensors header: malformed JSON");
        i++;
    }
    bool peek(char c) {
        ws();
        return i < s.size() && s[i] == c;
    }
    std::string str() {
        expect('"');
        std::string out;
        while (i < s.size() && s[i] != '"') {
            if (s[i] == '\\') {
                TH_REQUIRE(i + 1 < s.size(), "safetensors header: bad escape");
                const char e = s[i + 1];
                if (e == 'u') {  // keep \uXXXX verbatim: names are compared as written
                    out += s.substr(i, 6);
                    i += 6;
                    continue;
                }
                out += e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e == 'b' ? '\b' : e == 'f' ? '\f' : e;
                i += 2;
            } else {
                out += s[i++];
            }
        }
        expect('"');
        return out;
    }
    size_t uint() {
        ws();
        TH_REQUIRE(i < s.size() && s[i] >= '0' && s[i] <= '9', "safetensors header: expected an integer");
        size_t v = 0;
        while (i < s.size() && s[i] >= '0' && s[i] <= '9') v = v * 10 + (size_t)(s[i++] - '0');
        return v;
    }
    void skip() {  // any value
        ws();
        TH_REQUIRE(i < s.size(), "safetensors header: truncated");
        if (s[i] == '"') {
            str();
        } else if (s[i] == '{' || s[i] == '[') {
            const char close = s[i] == '{' ? '}' : ']';
            i++;
            if (peek(close)) { i++; return; }
            for (;;) {
                if (close == '}') { str(); expect(':'); }
                skip();
                if (peek(',')) { i++; continue; }
                expect(close);
                return;
            }
        } else {
            while (i < s.size() && s[i] != ',' && s[i] != '}' && s[i] != ']') i++;
        }
    }
};

static int st_dtype(const std::string& d) {
    if (d == "F64") return TH_ST_F64;
    if (d == "F32") return TH_ST_F32;
    if (d == "F16") return TH_ST_F16;
    if (d == "BF16") return TH_ST_BF16;
    return -1;
}

static size_t st_dtype_bytes(int d) { return d == TH_ST_F64 ? 8 : d == TH_ST_F32 ? 4 : 2; }

static float st_elem_f32(int dtype, const uint8_t* p) {
    switch (dtype) {
        case TH_ST_F64: { double v; std::memcpy(&v, p, 8); return (float)v; }
        case TH_ST_F32: { float v; std::memcpy(&v, p, 4); return v; }
        case TH_ST_F16: { uint16_t h; std::memcpy(&h, p, 2); return (float)__builtin_bit_cast(_Float16, h); }
        default: { uint16_t h; std::memcpy(&h, p, 2); uint32_t u = (uint32_t)h << 16; float v; std::memcpy(&v, &u, 4); return v; }
    }
}

}  // namespace th

using namespace th;

struct th_st_file {
    std::vector<uint8_t> data;  // bytes after the header
    std::vector<StTensor> tensors;
};

static const StTensor& st_find(const th_st_file* f, const char* name) {
    for (const StTensor& t : f->tensors)
        if (t.name == name) return t;
    throw Error(TH_ERR_INVALID, std::string("safetensors: no tensor named ") + name);
}

static std::vector<float> st_read(const th_st_file* f, const StTensor& t) {
    const size_t n = (t.end - t.begin) / st_dtype_bytes(t.dtype);
    std::vector<float> out(n);
    const uint8_t* p = f->data.data() + t.begin;
    for (size_t i = 0; i < n; i++) out[i] = st_elem_f32(t.dtype, p + i * st_dtype_bytes(t.dtype));
    return out;
}

namespace th {

bool st_has(const th_st_file* f, const std::string& name) {
    for (const StTensor& t : f->tensors)
        if (t.name == name) return true;
    return false;
}

std::vector<float> st_read_shaped(const th_st_file* f, const std::string& name, std::initializer_list<size_t> shape) {
    const StTensor& t = st_find(f, name.c_str());
    TH_REQUIRE(t.shape == std::vector<size_t>(shape), "safetensors: " + name + " has an unexpected shape");
    return st_read(f, t);
}

}  // namespace th

extern "C" {

int th_quantize_q4(const float* data, size_t rows, size_t cols, th_q4_block* out) {
    TH_API_BEGIN
    TH_REQUIRE(data && out && rows > 0 && cols > 0, "null argument");
    const size_t bpr = ceil_div(cols, (size_t)32);
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < bpr; b++)
            quant_q4_block(data + r * cols + b * 32, std::min<size_t>(32, cols - b * 32), out[r * bpr + b]);
    TH_API_END
}

int th_quantize_q8(const float* data, size_t rows, size_t cols, th_q8_block* out) {
    TH_API_BEGIN
    TH_REQUIRE(data && out && rows > 0 && cols > 0, "null argument");
    const size_t bpr = ceil_div(cols, (size_t)32);
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < bpr; b++)
            quant_q8_block(data + r * cols + b * 32, std::min<size_t>(32, cols - b * 32), out[r * bpr + b]);
    TH_API_END
}

int th_st_open(const char* path, th_st_file** out) {
    TH_API_BEGIN
    TH_REQUIRE(path && out, "null argument");
    std::ifstream in(path, std::ios::binary);
    TH_REQUIRE(in.good(), std::string("safetensors: cannot open ") + path);
    uint8_t lenb[8];
    in.read((char*)lenb, 8);
    TH_REQUIRE(in.gcount() == 8, "safetensors: file shorter than its header length");
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | lenb[i];
    TH_REQUIRE(hlen > 0 && hlen < (1ull << 30), "safetensors: implausible header length");
    std::string header(hlen, '\0');
    in.read(&header[0], (std::streamsize)hlen);
    TH_REQUIRE((uint64_t)in.gcount() == hlen, "safetensors: truncated header");
    std::unique_ptr<th_st_file> f(new th_st_file());
    f->data.assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
    Json j(header);
    j.expect('{');
    if (!j.peek('}')) {
        for (;;) {
            StTensor t;
            t.name = j.str();
            j.expect(':');
            if (t.name == "__metadata__") {
                j.skip();
            } else {
                bool have_dtype = false, have_shape = false, have_off = false;
                j.expect('{');
                for (;;) {
                    const std::string key = j.str();
                    j.expect(':');
                    if (key == "dtype") {
                        const std::string d = j.str();
                        t.dtype = st_dtype(d);
                        TH_REQUIRE(t.dtype >= 0, "safetensors: unsupported dtype " + d + " for " + t.name);
                        have_dtype = true;
                    } else if (key == "shape") {
                        j.expect('[');
                        if (!j.peek(']'))
                            for (;;) {
                                t.shape.push_back(j.uint());
                                if (j.peek(',')) { j.i++; continue; }
                                break;
                            }
                        j.expect(']');
                        have_shape = true;
                    } else if (key == "data_offsets") {
                        j.expect('[');
                        t.begin = j.uint();
                        j.expect(',');
                        t.end = j.uint();
                        j.expect(']');
                        have_off = true;
                    } else {
                        j.skip();
                    }
                    if (j.peek(',')) { j.i++; continue; }
                    j.expect('}');
                    break;
                }
                TH_REQUIRE(have_dtype && have_shape && have_off, "safetensors: incomplete entry " + t.name);
                size_t n = 1;
                for (size_t d : t.shape) n *= d;
                TH_REQUIRE(t.begin <= t.end && t.end <= f->data.size() && t.end - t.begin == n * st_dtype_bytes(t.dtype),
                           "safetensors: data_offsets do not match the shape of " + t.name);
                f->tensors.push_back(t);
            }
            if (j.peek(',')) { j.i++; continue; }
            j.expect('}');
            break;
        }
    }
    *out = f.release();
    TH_API_END
}

int th_st_close(th_st_file* f) {
    TH_API_BEGIN
    delete f;
    TH_API_END
}

int th_st_count(const th_st_file* f, size_t* n) {
    TH_API_BEGIN
    TH_REQUIRE(f && n, "null argument");
    *n = f->tensors.size();
    TH_API_END
}

int th_st_info(const th_st_file* f, size_t index, const char** name, int* dtype, size_t* ndim, size_t* shape,
               size_t max_dims) {
    TH_API_BEGIN
    TH_REQUIRE(f && name && dtype && ndim, "null argument");
    TH_REQUIRE(index < f->tensors.size(), "tensor index out of range");
    const StTensor& t = f->tensors[index];
    *name = t.name.c_str();
    *dtype = t.dtype;
    *ndim = t.shape.size();
    TH_REQUIRE(!shape || t.shape.size() <= max_dims, "shape buffer too small");
    if (shape)
        for (size_t i = 0; i < t.shape.size(); i++) shape[i] = t.shape[i];
    TH_API_END
}

int th_st_read_f32(const th_st_file* f, const char* name, float* out, size_t n) {
    TH_API_BEGIN
    TH_REQUIRE(f && name && out, "null argument");
    const StTensor& t = st_find(f, name);
    const std::vector<float> v = st_read(f, t);
    TH_REQUIRE(v.size() == n, "element count mismatch");
    std::memcpy(out, v.data(), n * sizeof(float));
    TH_API_END
}

int th_st_upload(th_device* dev, const th_st_file* f, const char* name, th_dtype dtype, th_buffer** out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && f && name && out, "null argument");
    TH_REQUIRE(dtype == TH_F32 || dtype == TH_BF16 || dtype == TH_F16, "device dtype must be f32, bf16 or f16");
    const std::vector<float> v = st_read(f, st_find(f, name));
    th_buffer* b = nullptr;
    check_status(th_buffer_alloc(dev, dtype, v.size(), &b));
    try {
        if (dtype == TH_F32) {
            check_status(th_buffer_upload(b, v.data(), v.size()));
        } else {
            std::vector<uint16_t> h(v.size());
            for (size_t i = 0; i < v.size(); i++)
                h[i] = dtype == TH_BF16 ? f32_to_bf16_host(v[i]) : __builtin_bit_cast(uint16_t, (_Float16)v[i]);
            check_status(th_buffer_upload(b, h.data(), h.size()));
        }
    } catch (...) {
        th_buffer_free(b);
        throw;
    }
    *out = b;
    TH_API_END
}

int th_st_upload_q4(th_device* dev, const th_st_file* f, const char* name, th_qweight** out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && f && name && out, "null argument");
    const StTensor& t = st_find(f, name);
    TH_REQUIRE(t.shape.size() == 2, "q4 upload needs a 2-D tensor");
    const std::vector<float> v = st_read(f, t);
    const size_t rows = t.shape[0], cols = t.shape[1];
    std::vector<th_q4_block> blocks(rows * ceil_div(cols, (size_t)32));
    check_status(th_quantize_q4(v.data(), rows, cols, blocks.data()));
    check_status(th_q4_upload_blocks(dev, blocks.data(), rows, cols, TH_F32, out));
    TH_API_END
}

int th_st_upload_q8(th_device* dev, const th_st_file* f, const char* name, th_qweight** out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && f && name && out, "null argument");
    const StTensor& t = st_find(f, name);
    TH_REQUIRE(t.shape.size() == 2, "q8 upload needs a 2-D tensor");
    const std::vector<float> v = st_read(f, t);
    const size_t rows = t.shape[0], cols = t.shape[1];
    std::vector<th_q8_block> blocks(rows * ceil_div(cols, (size_t)32));
    check_status(th_quantize_q8(v.data(), rows, cols, blocks.data()));
    check_status(th_q8_upload_blocks(dev, blocks.data(), rows, cols, out));
    TH_API_END
}

}  // extern "C"
