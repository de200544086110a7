// Helpers shared by the translation units that implement the C ABI.
#pragma once

#include "common.hpp"

#include <initializer_list>
#include <string>
#include <vector>

// Wrap a C entry point body: exceptions become status codes + last error.
#define TH_API_BEGIN try {
#define TH_API_END                                              \
    }                                                           \
    catch (const ::th::Error& e) {                              \
        ::th::set_last_error(e.what());                         \
        return e.code;                                          \
    }                                                           \
    catch (const std::exception& e) {                           \
        ::th::set_last_error(e.what());                         \
        return TH_ERR_INVALID;                                  \
    }                                                           \
    catch (...) {                                               \
        ::th::set_last_error("unknown error");                  \
        return TH_ERR_INVALID;                                  \
    }                                                           \
    ::th::set_last_error("");                                   \
    return TH_OK;

namespace th {

// Rethrow the failure of a nested C entry point.
inline void check_status(int rc) {
    if (rc != TH_OK) throw Error(rc, std::string("nested call failed: ") + th_last_error());
}

// Grow-only stream-ordered workspace owned by the device.
void* device_scratch(th_device* dev, size_t bytes);
// The configuration a sampler was created with (sampling.cpp).
const th_sampling_config& sampler_config(const th_sampler* s);
// Zero-initialised ints that kernels leave zero again on exit (arrival
// counters of the last-workgroup merges); grow-only.
int* device_counters(th_device* dev, size_t n);
// Second stream-ordered workspace, used for activations converted once per
// GEMM call (may be held at the same time as device_scratch).
void* device_scratch_x(th_device* dev, size_t bytes);
void require_len(const th_buffer* b, th_dtype dt, size_t n, const char* what);
// Unloads the device's compiled element-wise graphs (expr.cpp).
void expr_release(th_device* d);
void require_len_any(const th_buffer* b, size_t n, const char* what);

th_qweight* q4_pack(th_device* dev, const uint8_t* nib, const void* scales, th_dtype sdt, size_t rows,
                    size_t cols);

// safetensors helpers (loader.cpp): whether a tensor exists, and a tensor's
// values as f32 after checking that its shape is exactly `shape`.
bool st_has(const th_st_file* f, const std::string& name);
std::vector<float> st_read_shaped(const th_st_file* f, const std::string& name, std::initializer_list<size_t> shape);
th_qweight* q8_pack(th_device* dev, const int8_t* q, size_t ldq, const float* scales, bool per_row,
                    size_t rows, size_t cols);

// Quantized linear launchers (qlinear.hip).  x: [m][ldx] f32 or bf16,
// y: [m][ldy] f32.
// Activations in the MFMA GEMM's prepared layout: row r holds the f16 values
// x[r][k] * 2^-xexp[r] in rows of the weight's Kp (zero past K), each 8-value
// chunk ordered x0,x4,x1,x5,x2,x6,x3,x7.
struct PreparedX {
    const uint16_t* x;
    const int* xexp;
};
// prepare_x writes that layout for m rows of x (input row rows[r] for output
// row r when rows is set) into the device's operand workspace.
// workspace (optional): prepared_x_bytes(m, Kp) bytes to use instead.
PreparedX prepare_x(th_device* dev, const void* x, bool xf32, size_t m, size_t ldx, size_t K, size_t Kp,
                    hipStream_t s, const int* rows = nullptr, void* workspace = nullptr);
size_t prepared_x_bytes(size_t m, size_t Kp);
// The MFMA GEMM on prepared activations, for producers that write the layout
// directly.  accumulate: y += x.W^T (a fused residual add) instead of y = x.W^T.
void launch_q4_linear_prepared(const th_qweight* w, PreparedX xp, size_t m, float* y, size_t ldy, hipStream_t s,
                               th_device* dev, bool accumulate = false);
// ws / ws_bytes (optional): a workspace for the MFMA path (prepared
// activations, then split-K partials) instead of the device's grow-only one.
void launch_q4_linear(const th_qweight* w, const void* x, th_dtype xdt, size_t m, size_t ldx, float* y,
                      size_t ldy, hipStream_t stream, th_device* dev, void* ws = nullptr, size_t ws_bytes = 0);
void launch_q8_linear(const th_qweight* w, const void* x, th_dtype xdt, size_t m, size_t ldx, float* y,
                      size_t ldy, hipStream_t stream);

}  // namespace th
