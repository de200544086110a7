// Device helpers shared by the row-wise op kernels and the decode engine.
#pragma once

#include <cmath>
#include <vector>

#include "common.hpp"

namespace th {

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float v) {
    // crates/tang-compute/src/cuda.rs:22-27
    uint32_t b = __float_as_uint(v);
    b += 0x7FFFu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

__device__ __forceinline__ float load_w(const void* w, int bf16, size_t i) {
    return bf16 ? __uint_as_float((uint32_t)((const uint16_t*)w)[i] << 16) : ((const float*)w)[i];
}

// Cross-workgroup hand-off without cache flushes: values another workgroup
// (possibly on another XCD, whose L2 is not coherent with ours) will read are
// stored and loaded as relaxed device-scope atomics, which go to the
// coherence point; an agent-scope fence would instead write back or
// invalidate the whole L2.  wait_stores() drains this thread's stores before
// it publishes an arrival count.
__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(uint16_t* p, uint16_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(_Float16* p, _Float16 v) {
    __hip_atomic_store((uint16_t*)p, __builtin_bit_cast(uint16_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

// Cache-policy bit of a gfx950 vector memory access that makes it coherent
// across XCDs (the bit the relaxed agent-scope atomics above carry).
constexpr int CPOL_SC1 = 16;
// Non-temporal (streaming) bit of the same cache-policy field.
constexpr int CPOL_NT = 2;
// dword 3 of a raw (untyped) buffer resource.
constexpr int BUFFER_RSRC_W3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, BUFFER_RSRC_W3);
}

// Copy n floats that other workgroups stored with st_coherent into LDS.
// Same coherence as a relaxed agent-scope atomic load, but plain buffer
// loads, which the compiler does not serialise (atomic loads each wait for
// the previous one): sixteen per thread are in flight per round.  Call with
// the whole NT-thread block.
template <int NT = 256>
__device__ __forceinline__ void ld_coherent_to_lds(const float* src, int n, float* dst, int tid) {
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(src, (uint32_t)n * 4u);
    for (int base = 0; base < n; base += 16 * NT) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; u++)  // past n: out of the resource, reads 0
            v[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (base + tid + u * NT) * 4, 0, CPOL_SC1));
#pragma unroll
        for (int u = 0; u < 16; u++)
            if (base + tid + u * NT < n) dst[base + tid + u * NT] = v[u];
    }
}
// Count this workgroup's arrival; true in the last of `total` to arrive
// (which also resets the counter).  Call with the whole block after every
// thread's st_coherent stores.
__device__ __forceinline__ bool last_arrival(int* counter, int total, int* s_flag) {
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = prev == total - 1;
        if (*s_flag) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return *s_flag != 0;
}

// One DPP move inside rows of 16 lanes (CTRL: the dpp_ctrl encoding).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over aligned groups of N lanes (N a power of two up to 64) on the VALU:
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror,
// then cross-row shuffles.  Every lane of a group gets the same value.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (N >= 2) v += dpp_move<0xB1>(v);
    if constexpr (N >= 4) v += dpp_move<0x4E>(v);
    if constexpr (N >= 8) v += dpp_move<0x141>(v);
    if constexpr (N >= 16) v += dpp_move<0x140>(v);
    if constexpr (N >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (N >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

template <int N>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (N >= 2) v = fmaxf(v, dpp_move<0xB1>(v));
    if constexpr (N >= 4) v = fmaxf(v, dpp_move<0x4E>(v));
    if constexpr (N >= 8) v = fmaxf(v, dpp_move<0x141>(v));
    if constexpr (N >= 16) v = fmaxf(v, dpp_move<0x140>(v));
    if constexpr (N >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    if constexpr (N >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// Wave-level sum: row-local DPP-free butterfly over 64 lanes.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Pairwise sum of n (a power of two) values: ((r0+r1)+(r2+r3))+...
template <int N>
__device__ __forceinline__ float tree_sum(const float* r) {
    if constexpr (N == 1) return r[0];
    else return tree_sum<N / 2>(r) + tree_sum<N / 2>(r + N / 2);
}

// Sum over a 256-thread block; every thread gets the result.
__device__ __forceinline__ float block_sum_256(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = (red[0] + red[1]) + (red[2] + red[3]);
    return s;
}
__device__ __forceinline__ float block_max_256(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// out = g * sigmoid(g) * u evaluated in f64 and stored as f32, as the
// reference's elementwise closure (device.rs:727-736 via cpu.rs:68-97).
__device__ __forceinline__ float swiglu_f64(float g, float u) {
    const double gd = (double)g;
    const double sig = 1.0 / (1.0 + exp(-gd));
    return (float)(gd * sig * (double)u);
}

// bf16 (cuda.rs:22 rule) of swiglu_f64(g, u), the rounding every consumer of
// a SwiGLU output applies (it is a linear input).  Evaluated in f32 -- expf,
// one division and two products stay within a few f32 ulps of the f64 value
// -- and the f32 result decides the bf16 rounding unless it lies within 64
// ulps of a bf16 rounding midpoint (or is tiny or not finite), where the f64
// evaluation decides.  So the bits are always those of
// f32_to_bf16_rne(swiglu_f64(g, u)); the f64 path runs for ~0.2% of inputs.
__device__ __forceinline__ uint16_t swiglu_bf16(float g, float u) {
    const float s = 1.0f / (1.0f + expf(-g));
    const float y = g * s * u;
    const uint32_t lo = __float_as_uint(y) & 0xFFFFu;
    const float ay = fabsf(y);
    if (ay >= 0x1p-100f && ay <= 0x1p+100f && (lo + 64u < 0x8000u || lo > 0x8000u + 64u))
        return f32_to_bf16_rne(y);
    return f32_to_bf16_rne(swiglu_f64(g, u));
}

// First-maximum argmax over one row with a 256-thread block
// (crates/tang-infer/src/sampling.rs:184-194: strict '>' keeps the lowest index).
__device__ __forceinline__ void argmax_block_256(const float* x, int n, float* rv, int* ri, float& bv_out, int& bi_out) {
    float bv = -INFINITY;
    int bi = n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = x[i];
        if (v > bv) { bv = v; bi = i; }
    }
    rv[threadIdx.x] = bv;
    ri[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const float ov = rv[threadIdx.x + s];
            const int oi = ri[threadIdx.x + s];
            const float mv = rv[threadIdx.x];
            const int mi = ri[threadIdx.x];
            if (ov > mv || (ov == mv && oi < mi)) { rv[threadIdx.x] = ov; ri[threadIdx.x] = oi; }
        }
        __syncthreads();
    }
    bv_out = rv[0];
    bi_out = ri[0] == n ? 0 : ri[0];
}

// InterleavedRoPE::new tables (crates/tang-compute/src/modules.rs:495-511):
// freq = 1/base^(i/half), angle = pos*freq in f64, stored f32.
inline void rope_tables_host(size_t head_dim, size_t max_seq, double base, float* cs, float* sn) {
    const size_t half = head_dim / 2;
    for (size_t pos = 0; pos < max_seq; pos++) {
        for (size_t i = 0; i < half; i++) {
            const double freq = 1.0 / std::pow(base, (double)i / (double)half);
            const double angle = (double)pos * freq;
            cs[pos * half + i] = (float)std::cos(angle);
            sn[pos * half + i] = (float)std::sin(angle);
        }
    }
}

}  // namespace th
