// Shared host/device definitions for the gfx950 backend.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <tuple>

#include "../../include/tang_hip.h"

namespace th {

// Error raised inside the library; the C ABI layer turns it into a status
// code plus th_last_error() text.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const std::string& msg);

#define TH_REQUIRE(cond, msg)                                                      \
    do {                                                                            \
        if (!(cond)) throw ::th::Error(TH_ERR_INVALID, std::string(__func__) + ": " + (msg)); \
    } while (0)

#define TH_HIP(expr)                                                                        \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            throw ::th::Error(e_ == hipErrorOutOfMemory ? TH_ERR_OOM : TH_ERR_HIP,          \
                              std::string(#expr) + ": " + hipGetErrorString(e_));           \
    } while (0)

// Check the launch that was just enqueued.
#define TH_LAUNCH_CHECK() TH_HIP(hipGetLastError())

// Kernel launches go through launch_kernel: a HIP launch on the stream, or,
// while this thread records an AQL sequence (aql.cpp), a packet of that
// sequence with the arguments laid out as the kernel's kernarg segment
// (each parameter at its natural alignment, in order).
struct AqlSeq;
AqlSeq* aql_recording();
void aql_record_launch(AqlSeq* seq, const void* kernel, dim3 grid, dim3 block, size_t shmem, const void* args,
                       size_t bytes);

constexpr size_t KERNARG_MAX = 1024;

template <typename P>
inline void kernarg_put(char* buf, size_t& off, const P& v) {
    off = (off + alignof(P) - 1) / alignof(P) * alignof(P);
    if (off + sizeof(P) > KERNARG_MAX) throw Error(TH_ERR_INVALID, "kernel arguments exceed the kernarg buffer");
    std::memcpy(buf + off, &v, sizeof(P));
    off += sizeof(P);
}

template <typename... P, typename... A>
inline void launch_kernel(void (*kernel)(P...), dim3 grid, dim3 block, size_t shmem, hipStream_t stream,
                          A&&... args) {
    static_assert(sizeof...(P) == sizeof...(A), "argument count does not match the kernel");
    if (AqlSeq* seq = aql_recording()) {
        alignas(16) char buf[KERNARG_MAX];
        size_t off = 0;
        (kernarg_put<P>(buf, off, static_cast<P>(args)), ...);
        aql_record_launch(seq, (const void*)kernel, grid, block, shmem, buf, off);
        return;
    }
    std::tuple<P...> vals(static_cast<P>(args)...);
    void* ptrs[sizeof...(P) + 1];
    std::apply([&](auto&... v) {
        size_t i = 0;
        ((ptrs[i++] = (void*)&v), ...);
    }, vals);
    (void)hipLaunchKernel((const void*)kernel, grid, block, ptrs, shmem, stream);
}

#define TH_LAUNCH(...) ::th::launch_kernel(__VA_ARGS__)

inline size_t dtype_size(th_dtype t) {
    switch (t) {
        case TH_F32: case TH_U32: case TH_I32: return 4;
        case TH_BF16: case TH_F16: return 2;
        case TH_U8: case TH_I8: return 1;
    }
    return 0;
}

inline size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }
inline size_t round_up(size_t a, size_t b) { return ceil_div(a, b) * b; }

// ---------------------------------------------------------------------------
// Host-side scalar conversions (identical rounding to the device kernels).
// ---------------------------------------------------------------------------

// f32 -> bf16, round-to-nearest-even by bits + 0x7FFF + lsb
// (crates/tang-compute/src/cuda.rs:22-27).
inline uint16_t f32_to_bf16_host(float v) {
    uint32_t b; std::memcpy(&b, &v, 4);
    b += 0x7FFFu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}
inline float bf16_to_f32_host(uint16_t h) {
    uint32_t b = (uint32_t)h << 16; float f; std::memcpy(&f, &b, 4); return f;
}
inline float f16_to_f32_host(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
inline uint16_t f32_to_f16_host(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }

}  // namespace th

// ---------------------------------------------------------------------------
// Library objects behind the opaque C handles.
// ---------------------------------------------------------------------------

namespace th {
struct AqlDev;
struct ExprCache;
void aql_wait(th_device* d);
void aql_release(th_device* d);
}  // namespace th

struct th_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    int num_cus = 0;
    void* scratch = nullptr;  // stream-ordered workspace (split-K and attention partials)
    size_t scratch_bytes = 0;
    void* scratch_x = nullptr;  // stream-ordered workspace for GEMM operands prepared in f16
    size_t scratch_x_bytes = 0;
    int* counters = nullptr;  // see device_counters
    void* noalloc_scratch = nullptr;  // this device's address of the th_gemm_q4_noalloc workspace
    size_t n_counters = 0;
    int live = 0;          // buffers, weights and engines that hold this device
    bool closed = false;   // th_device_destroy ran; the struct waits for live == 0
    th::AqlDev* aql = nullptr;  // HSA queue for recorded sequences (created on first use)
    th::ExprCache* expr = nullptr;  // compiled element-wise graphs (expr.cpp), by source
};

// Objects holding a th_device keep the struct alive: th_device_destroy
// drains and releases the stream and workspaces at once, and the struct
// itself goes with the last object freed after it (so such a free never
// reads a deleted device).
inline void device_retain(th_device* d) { d->live++; }
inline void device_release(th_device* d) {
    if (--d->live == 0 && d->closed) delete d;
}
// Drain the device's stream before freeing memory it may still use (nothing
// is in flight once the device is closed).
inline void device_drain(th_device* d) {
    if (d->closed) return;
    try {
        th::aql_wait(d);
    } catch (...) {
    }
    (void)hipStreamSynchronize(d->stream);
}

// A captured sequence of library calls (th_capture_begin / th_capture_end).
struct th_graph {
    th_device* dev = nullptr;
    hipGraphExec_t exec = nullptr;
};

struct th_buffer {
    th_device* dev = nullptr;
    th_dtype dtype = TH_F32;
    size_t n = 0;
    void* ptr = nullptr;
};

// Device layout of a quantized matrix.  Rows are padded to a multiple of 16
// (Np) and K to a multiple of 128 (Kp); padding carries a zero weight.
//
// q4: tiles of 16 rows x 128 k (four groups of 32).  Tile (t, gq) occupies
//     1024 bytes at (t*GQ + gq)*1024; inside it lane L = q*16 + r (q = 0..3,
//     r = 0..15) owns 16 bytes = four 32-bit words, word j holding bytes
//     [4q, 4q+4) of the reference block (row 16t+r, group 4gq+j), i.e.
//     elements 8q..8q+7 of that group with Q4Block nibble packing.
//     Scales: [NT][GQ][16 r][4 j] of f16 or f32.
// q8: tiles of 16 rows x 64 k.  Tile (t, c) occupies 1024 bytes; lane
//     L = q*16 + r holds elements 16q..16q+15 of chunk c of row 16t+r.
//     Scales: f32, one per row ([Np]) or one per 32-group ([Np][Kp/32]).
struct th_qweight {
    th_device* dev = nullptr;
    int bits = 4;            // 4 or 8
    size_t rows = 0, cols = 0;
    size_t Np = 0, Kp = 0;
    th_dtype scale_dtype = TH_F16;
    bool per_row = false;    // q8 only: one scale per row
    void* data = nullptr;    // packed tiles
    void* scales = nullptr;
    size_t data_bytes = 0, scale_bytes = 0;
    int* row_exp = nullptr;  // q4: [Np] power-of-two exponent of each row's largest scale (MFMA GEMM)
};
