// Dequant-fused weight-only quantized linear kernels for gfx950.
//
// Arithmetic spec: q4_matvec / q8_matvec (crates/tang-infer/src/quantize.rs:227-289):
//   y[m][n] = sum_b scale[n][b] * sum_i (q[n][32b+i]) * x[m][32b+i]
// with q = nibble-8 (int4) or the int8 value.  The device sums in f32.
//
// Weight layouts are described next to th_qweight in common.hpp.
#pragma once

#include "common.hpp"

namespace th {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float v) {
    // bits + 0x7FFF + lsb (crates/tang-compute/src/cuda.rs:22-27)
    uint32_t b = __float_as_uint(v);
    b += 0x7FFFu + ((b >> 16) & 1u);
    return b >> 16;
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// a.lo*b.lo + a.hi*b.hi + c with bf16 pairs, f32 accumulate (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Four nibble pairs of one packed word as bf16 pairs holding 128+nibble:
// pair k = (element k, element k+4) of the word's eight elements.  bf16 with
// exponent 2^7 has unit spacing, so 0x4300|n is exactly 128+n.
__device__ __forceinline__ void nib_pairs_bf16(uint32_t w, uint32_t p[4]) {
    p[0] = (w & 0x000F000Fu) | 0x43004300u;
    p[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
    p[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
    p[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
}

// Eight x values x[0..8) as the matching bf16 pairs (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ __forceinline__ uint4 pack_perm_bf16(const uint32_t h[8]) {
    uint4 o;
    o.x = h[0] | (h[4] << 16);
    o.y = h[1] | (h[5] << 16);
    o.z = h[2] | (h[6] << 16);
    o.w = h[3] | (h[7] << 16);
    return o;
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Streaming 128-bit load of packed weights (read once: non-temporal hint).
__device__ __forceinline__ uint4 ldg_stream(const uint4* p) {
    const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float wave_sum_xor16_32(float v) {
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// ---------------------------------------------------------------------------
// Epilogues: receive (batch row m, output column n, f32 value).
// ---------------------------------------------------------------------------

struct EpiStore {
    float* y; int ldy;
    __device__ __forceinline__ void operator()(int m, int n, float v) const { y[(size_t)m * ldy + n] = v; }
};

// ---------------------------------------------------------------------------
// int4 GEMV, VALU path (small m).  One workgroup = one 16-row tile; its four
// waves take group-quads gq = wave, wave+4, ...  x is staged once per
// workgroup in LDS as bf16 pairs in nibble-pair order together with
// bias[m][gq][q][j] = -136 * sum of the eight x values lane q multiplies in
// group 4gq+j, so that dot(128+n, x) + bias = dot(n-8, x).
// f32 activations are split as x = hi + lo (two bf16, 16 significant bits)
// and both halves are dotted.
// ---------------------------------------------------------------------------

template <int M, bool XF32>
struct Q4GemvSmem {
    static constexpr int XR = XF32 ? 2 * M : M;
    static size_t bytes(int Kp) {
        return (size_t)XR * (Kp / 8) * 16 + (size_t)M * (Kp / 8) * 4 + 4 * 16 * M * 4;
    }
};

template <int U, typename ST>
struct ScaleVec;
template <int U>
struct ScaleVec<U, _Float16> {
    uint2 v[U];
    __device__ __forceinline__ void load(const _Float16* p, int u) { v[u] = *(const uint2*)p; }
    __device__ __forceinline__ float get(int u, int j) const {
        uint32_t w = (j < 2) ? v[u].x : v[u].y;
        uint16_t h = (j & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xFFFF);
        return (float)__builtin_bit_cast(_Float16, h);
    }
};
template <int U>
struct ScaleVec<U, float> {
    float4 v[U];
    __device__ __forceinline__ void load(const float* p, int u) { v[u] = *(const float4*)p; }
    __device__ __forceinline__ float get(int u, int j) const {
        return j == 0 ? v[u].x : j == 1 ? v[u].y : j == 2 ? v[u].z : v[u].w;
    }
};

template <int M, bool XF32, typename ST, typename Epi>
__global__ __launch_bounds__(256) void q4_gemv_kernel(const uint4* __restrict__ wt,
                                                      const ST* __restrict__ sc,
                                                      const void* __restrict__ xin, int K, int Kp,
                                                      int N, int ldx, Epi epi) {
    constexpr int XR = XF32 ? 2 * M : M;
    constexpr int U = 4;  // group-quads in flight per wave
    extern __shared__ uint4 smem[];
    const int GQ = Kp >> 7;
    const int NC = Kp >> 3;  // 8-element chunks per x row
    uint4* xl = smem;                                        // [XR][NC]
    float* bias = (float*)(xl + (size_t)XR * NC);            // [M][NC]
    float* red = bias + (size_t)M * NC;                      // [4][M][16]

    const int t = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int nmine = (GQ - wave + 3) >> 2;  // group-quads of this wave
    const uint4* wp = wt + (size_t)t * GQ * 64 + lane;
    const ST* sp = sc + (size_t)t * GQ * 64 + r * 4;

    // First batch of weights in flight before x is staged.
    uint4 wcur[U];
    ScaleVec<U, ST> scur;
#pragma unroll
    for (int u = 0; u < U; u++) {
        int gq = wave + 4 * u;
        if (u < nmine) {
            wcur[u] = ldg_stream(wp + (size_t)gq * 64);
            scur.load(sp + (size_t)gq * 64, u);
        }
    }

    // Stage x (vector loads only when every row start is 16-byte aligned).
    const bool vec = (ldx & 7) == 0 && (((uintptr_t)xin) & 15) == 0;
    for (int c = tid; c < M * NC; c += 256) {
        const int m = c / NC, cc = c - m * NC;
        const int k0 = cc * 8;
        float xv[8];
        if (XF32) {
            const float* xr = (const float*)xin + (size_t)m * ldx;
            if (vec && k0 + 8 <= K) {
                float4 a = *(const float4*)(xr + k0), b = *(const float4*)(xr + k0 + 4);
                xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
                xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) xv[i] = (k0 + i < K) ? xr[k0 + i] : 0.0f;
            }
        } else {
            const uint16_t* xr = (const uint16_t*)xin + (size_t)m * ldx;
            if (vec && k0 + 8 <= K) {
                uint4 a = *(const uint4*)(xr + k0);
                uint32_t w4[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    xv[2 * i] = bf16_bits_to_f32(w4[i] & 0xFFFF);
                    xv[2 * i + 1] = bf16_bits_to_f32(w4[i] >> 16);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) xv[i] = (k0 + i < K) ? bf16_bits_to_f32(xr[k0 + i]) : 0.0f;
            }
        }
        uint32_t hi[8], lo[8];
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            hi[i] = XF32 ? f32_to_bf16_bits(xv[i]) : f32_to_bf16_bits(xv[i]);
            float fh = bf16_bits_to_f32(hi[i]);
            s += fh;
            if (XF32) {
                lo[i] = f32_to_bf16_bits(xv[i] - fh);
                s += bf16_bits_to_f32(lo[i]);
            }
        }
        if (XF32) {
            xl[(size_t)(2 * m) * NC + cc] = pack_perm_bf16(hi);
            xl[(size_t)(2 * m + 1) * NC + cc] = pack_perm_bf16(lo);
        } else {
            xl[(size_t)m * NC + cc] = pack_perm_bf16(hi);
        }
        // chunk cc = group g (= 4gq + j), lane-quad qq; bias index (gq*4 + qq)*4 + j
        const int g = cc >> 2, qq = cc & 3, gq = g >> 2, j = g & 3;
        bias[(size_t)m * NC + (gq * 4 + qq) * 4 + j] = -136.0f * s;
    }
    __syncthreads();

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.0f;

    for (int base = 0; base < nmine; base += U) {
        uint4 wnxt[U];
        ScaleVec<U, ST> snxt;
#pragma unroll
        for (int u = 0; u < U; u++) {
            int i = base + U + u;
            if (i < nmine) {
                int gq = wave + 4 * i;
                wnxt[u] = ldg_stream(wp + (size_t)gq * 64);
                snxt.load(sp + (size_t)gq * 64, u);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            int i = base + u;
            if (i < nmine) {
                const int gq = wave + 4 * i;
                const uint32_t wv[4] = {wcur[u].x, wcur[u].y, wcur[u].z, wcur[u].w};
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const float4 b4 = *(const float4*)(bias + (size_t)m * NC + (gq * 4 + q) * 4);
                    const float bj[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        uint32_t p[4];
                        nib_pairs_bf16(wv[j], p);
                        const int cidx = (4 * gq + j) * 4 + q;
                        float d = bj[j];
                        const uint4 xa = xl[(size_t)(XF32 ? 2 * m : m) * NC + cidx];
                        d = dot2_bf16(p[0], xa.x, d);
                        d = dot2_bf16(p[1], xa.y, d);
                        d = dot2_bf16(p[2], xa.z, d);
                        d = dot2_bf16(p[3], xa.w, d);
                        if (XF32) {
                            const uint4 xb = xl[(size_t)(2 * m + 1) * NC + cidx];
                            d = dot2_bf16(p[0], xb.x, d);
                            d = dot2_bf16(p[1], xb.y, d);
                            d = dot2_bf16(p[2], xb.z, d);
                            d = dot2_bf16(p[3], xb.w, d);
                        }
                        acc[m] = __builtin_fmaf(scur.get(u, j), d, acc[m]);
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) wcur[u] = wnxt[u];
        scur = snxt;
    }

#pragma unroll
    for (int m = 0; m < M; m++) {
        float v = wave_sum_xor16_32(acc[m]);
        if (q == 0) red[(wave * M + m) * 16 + r] = v;
    }
    __syncthreads();
    if (tid < 16 * M) {
        const int m = tid >> 4, rr = tid & 15;
        float v = red[(0 * M + m) * 16 + rr] + red[(1 * M + m) * 16 + rr];
        v += red[(2 * M + m) * 16 + rr];
        v += red[(3 * M + m) * 16 + rr];
        const int n = t * 16 + rr;
        if (n < N) epi(m, n, v);
    }
}

// ---------------------------------------------------------------------------
// int8 GEMV, VALU path.  One workgroup = one 16-row tile; waves take chunks
// c = wave, wave+4, ...  x is staged in LDS as f32 with
// bias[m][c][q] = -128 * sum of the 16 x values of lane-quad q, so that
// sum((q8 ^ 0x80) * x) + bias = sum(q8 * x).
// ---------------------------------------------------------------------------

template <int M>
struct Q8GemvSmem {
    static size_t bytes(int Kp) { return (size_t)M * Kp * 4 + (size_t)M * (Kp / 16) * 4 + 4 * 16 * M * 4; }
};

template <int M, bool XF32, bool PER_ROW, typename Epi>
__global__ __launch_bounds__(256) void q8_gemv_kernel(const uint4* __restrict__ wt,
                                                      const float* __restrict__ sc,
                                                      const void* __restrict__ xin, int K, int Kp,
                                                      int N, int ldx, Epi epi) {
    constexpr int U = 4;
    extern __shared__ uint4 smem[];
    const int NCH = Kp >> 6;  // 64-element chunks
    float* xl = (float*)smem;                 // [M][Kp]
    float* bias = xl + (size_t)M * Kp;        // [M][Kp/16]
    float* red = bias + (size_t)M * (Kp / 16);

    const int t = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int nmine = (NCH - wave + 3) >> 2;
    const uint4* wp = wt + (size_t)t * NCH * 64 + lane;
    const int row = t * 16 + r;
    const int GPR = Kp >> 5;  // groups per row (per-group scales)

    uint4 wcur[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if (u < nmine) wcur[u] = ldg_stream(wp + (size_t)(wave + 4 * u) * 64);

    for (int c = tid; c < M * (Kp / 16); c += 256) {
        const int m = c / (Kp / 16), cc = c - m * (Kp / 16);
        const int k0 = cc * 16;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float v;
            int k = k0 + i;
            if (XF32) v = (k < K) ? ((const float*)xin)[(size_t)m * ldx + k] : 0.0f;
            else v = (k < K) ? bf16_bits_to_f32(((const uint16_t*)xin)[(size_t)m * ldx + k]) : 0.0f;
            xl[(size_t)m * Kp + k] = v;
            s += v;
        }
        bias[(size_t)m * (Kp / 16) + cc] = -128.0f * s;
    }
    __syncthreads();

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.0f;

    for (int base = 0; base < nmine; base += U) {
        uint4 wnxt[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            int i = base + U + u;
            if (i < nmine) wnxt[u] = ldg_stream(wp + (size_t)(wave + 4 * i) * 64);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            int i = base + u;
            if (i < nmine) {
                const int c = wave + 4 * i;
                const uint32_t wv[4] = {wcur[u].x ^ 0x80808080u, wcur[u].y ^ 0x80808080u,
                                        wcur[u].z ^ 0x80808080u, wcur[u].w ^ 0x80808080u};
                const int k0 = c * 64 + q * 16;
                float s = 1.0f;
                if (!PER_ROW) s = sc[(size_t)row * GPR + (k0 >> 5)];
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const float4* xp = (const float4*)(xl + (size_t)m * Kp + k0);
                    float d = bias[(size_t)m * (Kp / 16) + (k0 >> 4)];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float4 xv = xp[j];
                        const uint32_t w = wv[j];
                        d = __builtin_fmaf((float)(w & 0xFF), xv.x, d);
                        d = __builtin_fmaf((float)((w >> 8) & 0xFF), xv.y, d);
                        d = __builtin_fmaf((float)((w >> 16) & 0xFF), xv.z, d);
                        d = __builtin_fmaf((float)(w >> 24), xv.w, d);
                    }
                    if (PER_ROW) acc[m] += d;
                    else acc[m] = __builtin_fmaf(s, d, acc[m]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) wcur[u] = wnxt[u];
    }

#pragma unroll
    for (int m = 0; m < M; m++) {
        float v = wave_sum_xor16_32(acc[m]);
        if (q == 0) red[(wave * M + m) * 16 + r] = v;
    }
    __syncthreads();
    if (tid < 16 * M) {
        const int m = tid >> 4, rr = tid & 15;
        float v = red[(0 * M + m) * 16 + rr] + red[(1 * M + m) * 16 + rr];
        v += red[(2 * M + m) * 16 + rr];
        v += red[(3 * M + m) * 16 + rr];
        const int n = t * 16 + rr;
        if (n < N) {
            if (PER_ROW) v *= sc[n];
            epi(m, n, v);
        }
    }
}

// ---------------------------------------------------------------------------
// int4 GEMM on MFMA (v_mfma_f32_16x16x32_f16), for larger m.
// Workgroup: 4 waves stacked along n, each owning RT 16-row tiles; CB blocks
// of 16 activation rows.  Per group (K = 32 = one MFMA) a lane dequantises its
// eight weights to f16 as (n-8)*scale (exact n-8 via the 1024+n magic, one f16
// rounding of the product) and the activations are rounded to f16.  B tiles
// (activations for one group-quad, permuted to the nibble-pair order) are
// staged in LDS.  With KS > 1 each workgroup covers a K slice and writes f32
// partials [KS][m][n] that q4_splitk_reduce sums in a fixed order.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void nib_pairs_f16(uint32_t w, half2_t s2, half2_t out[4]) {
    const half2_t off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t p = ((w >> (4 * k)) & 0x000F000Fu) | 0x64006400u;
        half2_t h = __builtin_bit_cast(half2_t, p);
        out[k] = (h + off) * s2;
    }
}

__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
    half2_t h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
}

template <int RT, int CB, bool XF32, typename ST>
__global__ __launch_bounds__(256) void q4_gemm_mfma_kernel(const uint4* __restrict__ wt,
                                                           const ST* __restrict__ sc,
                                                           const void* __restrict__ xin, float* __restrict__ y,
                                                           int M, int N, int K, int Kp, int ldx, int ldy,
                                                           int gq_per_split) {
    // LDS B tile: [CB][4 j][4 q][16 col] uint4 (8 f16 each)
    __shared__ uint4 bt[CB * 4 * 4 * 16];
    const int GQ = Kp >> 7;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int tile0 = (blockIdx.x * 4 + wave) * RT;  // first 16-row tile of this wave
    const int NT = (N + 15) >> 4;
    const int m0 = blockIdx.y * CB * 16;
    const int gq0 = blockIdx.z * gq_per_split;
    const int gq1 = min(GQ, gq0 + gq_per_split);

    const bool vec = (ldx & 7) == 0 && (((uintptr_t)xin) & 15) == 0;
    float4_t acc[RT][CB];
#pragma unroll
    for (int a = 0; a < RT; a++)
#pragma unroll
        for (int b = 0; b < CB; b++) acc[a][b] = (float4_t){0.f, 0.f, 0.f, 0.f};

    // staging assignment: CB*16 cols * 16 chunks (4 groups x 4 quads) = CB*256 chunks
    auto load_x = [&](int gq, uint4 regs[CB]) {
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int idx = tid + i * 256;        // chunk id
            const int col = idx & 15;
            const int qq = (idx >> 4) & 3;
            const int j = (idx >> 6) & 3;
            const int cb = idx >> 8;
            const int m = m0 + cb * 16 + col;
            const int k0 = gq * 128 + j * 32 + qq * 8;
            float xv[8];
#pragma unroll
            for (int e = 0; e < 8; e++) xv[e] = 0.0f;
            if (m < M) {
                if (XF32) {
                    const float* xr = (const float*)xin + (size_t)m * ldx;
                    if (vec && k0 + 8 <= K) {
                        float4 a = *(const float4*)(xr + k0), b = *(const float4*)(xr + k0 + 4);
                        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
                        xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
                    } else {
                        for (int e = 0; e < 8; e++) if (k0 + e < K) xv[e] = xr[k0 + e];
                    }
                } else {
                    const uint16_t* xr = (const uint16_t*)xin + (size_t)m * ldx;
                    if (vec && k0 + 8 <= K) {
                        uint4 a = *(const uint4*)(xr + k0);
                        uint32_t w4[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            xv[2 * e] = bf16_bits_to_f32(w4[e] & 0xFFFF);
                            xv[2 * e + 1] = bf16_bits_to_f32(w4[e] >> 16);
                        }
                    } else {
                        for (int e = 0; e < 8; e++) if (k0 + e < K) xv[e] = bf16_bits_to_f32(xr[k0 + e]);
                    }
                }
            }
            uint4 o;
            o.x = pack_half2(xv[0], xv[4]);
            o.y = pack_half2(xv[1], xv[5]);
            o.z = pack_half2(xv[2], xv[6]);
            o.w = pack_half2(xv[3], xv[7]);
            regs[i] = o;
        }
    };
    auto store_x = [&](const uint4 regs[CB]) {
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int idx = tid + i * 256;
            const int col = idx & 15, qq = (idx >> 4) & 3, j = (idx >> 6) & 3, cb = idx >> 8;
            bt[((cb * 4 + j) * 4 + qq) * 16 + col] = regs[i];
        }
    };

    uint4 xr[CB];
    uint4 wcur[RT], wnxt[RT];
    ScaleVec<RT, ST> scur, snxt;
    auto load_w = [&](int gq, uint4 w[RT], ScaleVec<RT, ST>& s) {
#pragma unroll
        for (int a = 0; a < RT; a++) {
            int tt = min(tile0 + a, NT - 1);
            w[a] = ldg_stream(wt + ((size_t)tt * GQ + gq) * 64 + lane);
            s.load(sc + ((size_t)tt * GQ + gq) * 64 + r * 4, a);
        }
    };
    if (gq0 < gq1) {
        load_x(gq0, xr);
        load_w(gq0, wcur, scur);
    }
    for (int gq = gq0; gq < gq1; gq++) {
        __syncthreads();
        store_x(xr);
        __syncthreads();
        if (gq + 1 < gq1) {
            load_x(gq + 1, xr);
            load_w(gq + 1, wnxt, snxt);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            half8_t bfrag[CB];
#pragma unroll
            for (int b = 0; b < CB; b++)
                bfrag[b] = __builtin_bit_cast(half8_t, bt[((b * 4 + j) * 4 + q) * 16 + r]);
#pragma unroll
            for (int a = 0; a < RT; a++) {
                const uint32_t w = j == 0 ? wcur[a].x : j == 1 ? wcur[a].y : j == 2 ? wcur[a].z : wcur[a].w;
                const _Float16 s = (_Float16)scur.get(a, j);
                const half2_t s2 = {s, s};
                half2_t p[4];
                nib_pairs_f16(w, s2, p);
                half8_t afrag = {p[0].x, p[0].y, p[1].x, p[1].y, p[2].x, p[2].y, p[3].x, p[3].y};
#pragma unroll
                for (int b = 0; b < CB; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag, bfrag[b], acc[a][b], 0, 0, 0);
            }
        }
#pragma unroll
        for (int a = 0; a < RT; a++) wcur[a] = wnxt[a];
        scur = snxt;
    }

    // D layout: lane holds rows 4*(lane/16)+i (weight rows) of column lane%16.
    float* yb = y + (size_t)blockIdx.z * M * ldy;
#pragma unroll
    for (int a = 0; a < RT; a++) {
        const int n0 = (tile0 + a) * 16 + 4 * q;
#pragma unroll
        for (int b = 0; b < CB; b++) {
            const int m = m0 + b * 16 + r;
            if (m < M && tile0 + a < NT) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (n0 + i < N) yb[(size_t)m * ldy + n0 + i] = acc[a][b][i];
            }
        }
    }
}

}  // namespace th
