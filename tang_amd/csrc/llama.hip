// Device-resident Llama-style decode engine with int4 group-32 weights.
//
// One decode step restates crates/tang-train/examples/smollm.rs:215-300
// (pre-norm -> attention -> +residual -> pre-norm -> SwiGLU MLP -> +residual,
// final norm, LM head) with the ComputeDevice ops of the reference
// (rms_norm cpu.rs:126, rope device.rs:582, kv_attention cpu.rs:257,
// swiglu device.rs:727) and greedy sampling (sampling.rs:184).  Rounding
// points: every linear reads its input as bf16 (cuda.rs:22 rounding), K/V are
// stored f16, the residual stream and all other values are f32.
//
// Per layer the step is five kernels:
//   QKV GEMV (prologue: RMSNorm; epilogue: RoPE, f16 K/V append)
//   -> split attention (last chunk per head merges, bf16 out)
//   -> O GEMV (epilogue: +residual, tile sums of squares)
//   -> gate/up GEMV (prologue: RMSNorm; epilogue: SwiGLU, bf16)
//   -> down GEMV (epilogue: +residual, tile sums of squares)
// plus an LM-head GEMV (epilogue: tile maxima) and the argmax, which also
// writes the next token's embedding.  The whole step reads the position and
// token from device memory, so it is recorded once and replayed per token
// with no host round trip: on the library's own AQL queue (aql.cpp; every
// kernel stores what later kernels read write-through, so the packets carry
// no release fences), or as a HIP graph (TANG_HIP_DISPATCH=graph, or inside
// a caller's stream capture).
#include <algorithm>
#include <cstdlib>
#include <vector>

#include "aql.hpp"
#include "attention.hpp"
#include "capi_util.hpp"
#include "ops.hpp"
#include "qlinear.hpp"

namespace th {

// Tensor ids for th_synth_seed(seed, layer, id).
enum : int { T_WQ = 0, T_WK, T_WV, T_WO, T_WG, T_WU, T_WD, T_ATTN_NORM, T_FFN_NORM,
             T_EMBED = 10, T_FINAL_NORM, T_LM_HEAD, T_KCACHE = 20, T_VCACHE };

constexpr float Q4_SMIN = 0.002f, Q4_SMAX = 0.01f, NORM_STD = 0.02f;
constexpr int ATTN_SPLIT_ENGINE = 256;  // cache positions per attention workgroup (fixed-chunk mode)
// Even mode: the attended length shared over n_heads * n_splits workgroups,
// n_splits = CUs / n_heads (one round of the chip), at most ATTN_EVEN_MAX
// positions per workgroup; ATTN_EVEN_MAX is the largest instantiated bound.
constexpr int ATTN_EVEN_SPLS[] = {128, 192, 256, 288, 384, 512};

// state[0] = position, state[1] = current token, state[2] = steps taken
struct LlamaState { int pos, token, step, pad; };

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------

// Embedding row copy (cpu.rs:151-168) into the f32 residual, plus the
// per-16-element sums of squares the next RMSNorm prologue consumes.
__global__ void llama_embed_kernel(const uint16_t* __restrict__ embed, const LlamaState* __restrict__ st, int d,
                                   float* __restrict__ x, float* __restrict__ ssq) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t * 16 >= d) return;
    const uint16_t* src = embed + (size_t)st->token * d + t * 16;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float v = __uint_as_float((uint32_t)src[i] << 16);
        x[t * 16 + i] = v;
        s += v * v;
    }
    ssq[t] = s;
}

// QKV epilogue: rows [0,qd) are q, [qd,qd+kvd) k, then v.  q and k get the
// interleaved RoPE of device.rs:582-610 at the device-side position; k and v
// are appended to the f16 cache row `pos`.
struct EpiQKV : EpiNoFinish {
    float* q; _Float16* kc; _Float16* vc;
    const float* cs; const float* sn; const LlamaState* st;
    int qd, kvd, hd;
    __device__ __forceinline__ void operator()(int, int n, float v, const float* tile, float*) const {
        const int pos = st->pos;
        const int rr = n & 15;
        float out = v;
        if (n < qd + kvd) {
            const int half = hd / 2;
            const int i = (n % hd) >> 1;
            const float c = cs[(size_t)pos * half + i], s = sn[(size_t)pos * half + i];
            if ((rr & 1) == 0) {
                const float x0 = v, x1 = tile[rr + 1];
                out = x0 * c - x1 * s;
            } else {
                const float x0 = tile[rr - 1], x1 = v;
                out = x0 * s + x1 * c;
            }
        }
        if (n < qd) st_coherent(&q[n], out);
        else if (n < qd + kvd) st_coherent(&kc[(size_t)pos * kvd + (n - qd)], (_Float16)out);
        else st_coherent(&vc[(size_t)pos * kvd + (n - qd - kvd)], (_Float16)out);
    }
};

// x += linear (residual add, device.rs:721, on the f32 stream) and the tile's
// sum of squares of the new x for the next RMSNorm prologue.
struct EpiAddToSsq {
    static constexpr bool HAS_FINISH = true;
    float* x; float* ssq;
    __device__ __forceinline__ void operator()(int, int n, float v, const float*, float* aux) const {
        const float xn = x[n] + v;
        st_coherent(&x[n], xn);
        aux[n & 15] = xn;
    }
    __device__ __forceinline__ void finish(int t, int, const float* aux, int tid) const {
        if (tid == 0) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) s += aux[i] * aux[i];
            st_coherent(&ssq[t], s);
        }
    }
};

// Gate/up tiles hold gate rows 8b..8b+7 then up rows 8b..8b+7: the first
// eight lanes emit bf16(swiglu(g, u)) for intermediate index 8b + rr.
struct EpiSwiGLU : EpiNoFinish {
    uint16_t* out;
    __device__ __forceinline__ void operator()(int, int n, float v, const float* tile, float*) const {
        const int rr = n & 15;
        if (rr < 8) st_coherent(&out[(n >> 4) * 8 + rr], swiglu_bf16(v, tile[rr + 8]));
    }
};

// LM-head epilogue: logits, and each 16-row tile's maximum (first maximum
// within the tile) for llama_argmax_embed_kernel.  (Taking the final argmax
// in the last workgroup to finish was measured slower: its arrival counter
// sees one atomic per tile, 2000 at the 7B shape, and they serialise.)
struct EpiTileMax {
    static constexpr bool HAS_FINISH = true;
    float* logits; float* part_v; int* part_i; int vocab;
    __device__ __forceinline__ void operator()(int, int n, float v, const float*, float* aux) const {
        st_coherent(&logits[n], v);
        aux[n & 15] = v;
    }
    __device__ __forceinline__ void finish(int t, int, const float* aux, int tid) const {
        if (tid == 0) {
            const int cnt = min(16, vocab - t * 16);
            float bv = -INFINITY;
            int bi = t * 16;
            for (int i = 0; i < cnt; i++)
                if (aux[i] > bv) { bv = aux[i]; bi = t * 16 + i; }
            st_coherent(&part_v[t], bv);
            st_coherent(&part_i[t], bi);
        }
    }
};

// Greedy argmax over the tile maxima (value descending, then index
// ascending: the first maximum wins, sampling.rs:184-194); records the
// token, advances the position and writes the next step's input: the
// token's embedding row into x and its per-16-element sums of squares into
// ssq (cpu.rs:151-168, as llama_embed_kernel), so a step needs no embedding
// launch of its own.  One 1024-thread workgroup; d <= 16384.
__global__ __launch_bounds__(1024) void llama_argmax_embed_kernel(const float* __restrict__ part_v,
                                                                  const int* __restrict__ part_i, int ntile,
                                                                  LlamaState* st, int32_t* __restrict__ history,
                                                                  const uint16_t* __restrict__ embed, int d,
                                                                  float* __restrict__ x, float* __restrict__ ssq) {
    __shared__ float wv[16];
    __shared__ int wi[16], s_tok;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = tid; i < ntile; i += 1024) {  // ascending i: strict > keeps the first
        const float pv = part_v[i];
        if (pv > bv) { bv = pv; bi = part_i[i]; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { wv[wave] = bv; wi[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; w++)
            if (wv[w] > bv || (wv[w] == bv && wi[w] < bi)) { bv = wv[w]; bi = wi[w]; }
        const int tok = bi == 0x7fffffff ? 0 : bi;
        const int step = st->step, pos = st->pos;
        st_coherent(&history[step], tok);
        st_coherent(&st->token, tok);
        st_coherent(&st->step, step + 1);
        st_coherent(&st->pos, pos + 1);
        s_tok = tok;
    }
    __syncthreads();
    const uint16_t* src = embed + (size_t)s_tok * d;
    for (int c = tid; c * 16 < d; c += 1024) {
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float v = __uint_as_float((uint32_t)src[c * 16 + i] << 16);
            st_coherent(&x[c * 16 + i], v);
            sq += v * v;
        }
        st_coherent(&ssq[c], sq);
    }
}

// ---- prefill (a prompt chunk of n tokens at positions pos0..pos0+n-1) ----

// Embedding rows (cpu.rs:151-168) into the f32 residual [n][d].
__global__ void prefill_embed_kernel(const uint16_t* __restrict__ embed, const int32_t* __restrict__ tok, int d,
                                     float* __restrict__ x) {
    const int row = blockIdx.y;
    const uint16_t* src = embed + (size_t)tok[row] * d;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x)
        x[(size_t)row * d + i] = __uint_as_float((uint32_t)src[i] << 16);
}

// RMSNorm of one row to the linear input, with the decode engine's rounding
// and summation order: per-16-element sums of squares, four per lane, a fixed
// butterfly, then x * inv_rms * w (cpu.rs:126-149) rounded to bf16
// (cuda.rs:22).  One wave per row; d <= 4096, d % 8 == 0.  XP: the values go
// out in the MFMA GEMM's prepared layout (f16 of value * 2^-xexp[row], the
// row maximum brought to [2^12, 2^13), exact for a bf16 value within 2^26 of
// it; 8-value chunks as x0,x4,x1,x5,x2,x6,x3,x7; rows of ldo >= d, zero past
// d); otherwise as bf16 rows of ldo.
template <bool XP>
__global__ __launch_bounds__(64) void prefill_rmsnorm_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                            int d, float eps, uint16_t* __restrict__ out, int ldo,
                                                            int* __restrict__ xexp) {
    const int row = blockIdx.x, lane = threadIdx.x;
    const float* xr = x + (size_t)row * d;
    float part = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int t = lane + 64 * u;
        float sq = 0.0f;
        if (t * 16 < d) {
            float v[16];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4 f = *(const float4*)(xr + t * 16 + 4 * c);
                v[4 * c] = f.x; v[4 * c + 1] = f.y; v[4 * c + 2] = f.z; v[4 * c + 3] = f.w;
            }
#pragma unroll
            for (int i = 0; i < 16; i++) sq += v[i] * v[i];
        }
        part += sq;
    }
    const float tot = wave_sum(part);
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
    // the eight bf16-rounded outputs of chunk k0 (zero past d)
    auto chunk = [&](int k0, float y[8]) {
        if (k0 < d) {
            const float4 a = *(const float4*)(xr + k0), b = *(const float4*)(xr + k0 + 4);
            const uint4 wb = *(const uint4*)(w + k0);
            const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            const uint32_t ww[4] = {wb.x, wb.y, wb.z, wb.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t wbits = (i & 1) ? (ww[i >> 1] >> 16) : (ww[i >> 1] & 0xFFFFu);
                y[i] = bf16_bits_to_f32(f32_to_bf16_rne(xv[i] * inv * __uint_as_float(wbits << 16)));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) y[i] = 0.0f;
        }
    };
    uint16_t* orow = out + (size_t)row * ldo;
    if (XP) {
        float mx = 0.0f;
        for (int c = lane; c * 8 < d; c += 64) {
            float y[8];
            chunk(c * 8, y);
#pragma unroll
            for (int i = 0; i < 8; i++) mx = fmaxf(mx, fabsf(y[i]));
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        const int e = range_exp(mx, XPREP_TOP);
        if (lane == 0) xexp[row] = e;
        for (int c = lane; c * 8 < ldo; c += 64) {
            float y[8];
            chunk(c * 8, y);
#pragma unroll
            for (int i = 0; i < 8; i++) y[i] = __builtin_amdgcn_ldexpf(y[i], -e);
            *(uint4*)(orow + c * 8) = make_uint4(pack_half2(y[0], y[4]), pack_half2(y[1], y[5]),
                                                 pack_half2(y[2], y[6]), pack_half2(y[3], y[7]));
        }
    } else {
        for (int c = lane; c * 8 < d; c += 64) {
            float y[8];
            chunk(c * 8, y);
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                o[i] = (uint32_t)f32_to_bf16_rne(y[2 * i]) | ((uint32_t)f32_to_bf16_rne(y[2 * i + 1]) << 16);
            *(uint4*)(orow + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// RoPE of q and k (device.rs:582-610, as EpiQKV) at position pos0 + row; q to
// f32 [n][qd], k and v appended to the f16 cache rows.  A thread takes eight
// consecutive columns (four rotation pairs of one head, never straddling q,
// k and v) with 16-byte loads and stores; per pair (x0 c - x1 s, x0 s + x1 c).
__global__ __launch_bounds__(256) void prefill_rope_kv_kernel(const float* __restrict__ qkv, int pos0,
                                                              const float* __restrict__ cs,
                                                              const float* __restrict__ sn, int qd, int kvd, int hd,
                                                              float* __restrict__ q, _Float16* __restrict__ kc,
                                                              _Float16* __restrict__ vc) {
    const int row = blockIdx.y, W = qd + 2 * kvd, pos = pos0 + row;
    const int n = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (n >= W) return;
    const float* src = qkv + (size_t)row * W + n;
    const float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if (n < qd + kvd) {
        const int half = hd / 2, i0 = (n % hd) >> 1;
        const float4 c4 = *(const float4*)(cs + (size_t)pos * half + i0);
        const float4 s4 = *(const float4*)(sn + (size_t)pos * half + i0);
        const float c[4] = {c4.x, c4.y, c4.z, c4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float x0 = v[2 * p], x1 = v[2 * p + 1];
            v[2 * p] = x0 * c[p] - x1 * sv[p];
            v[2 * p + 1] = x0 * sv[p] + x1 * c[p];
        }
    }
    if (n < qd) {
        float* dst = q + (size_t)row * qd + n;
        *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
        *(float4*)(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        _Float16* dst = n < qd + kvd ? kc + (size_t)pos * kvd + (n - qd) : vc + (size_t)pos * kvd + (n - qd - kvd);
        uint32_t h[4];
#pragma unroll
        for (int p = 0; p < 4; p++)
            h[p] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * p]) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * p + 1]) << 16);
        *(uint4*)dst = make_uint4(h[0], h[1], h[2], h[3]);
    }
}

// x += y (device.rs:721, f32 residual).
__global__ void prefill_add_kernel(float* __restrict__ x, const float* __restrict__ y, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        x[i] = x[i] + y[i];
}

// SwiGLU of the interleaved gate/up rows (tile b: gate 8b..8b+7, up
// 8b..8b+7) to the down-projection input, rounded to bf16 as bf16 rows of
// ldo.  One thread per value (f64 math, as cpu.rs:68).
__global__ void prefill_swiglu_kernel(const float* __restrict__ gu, int ff, uint16_t* __restrict__ out, int ldo) {
    const int row = blockIdx.y;
    const float* g = gu + (size_t)row * 2 * ff;
    uint16_t* orow = out + (size_t)row * ldo;
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < ff; j += gridDim.x * blockDim.x) {
        const int b = j >> 3, rr = j & 7;
        orow[j] = swiglu_bf16(g[16 * b + rr], g[16 * b + 8 + rr]);
    }
}

// The same values in the MFMA GEMM's prepared layout (as the XP RMSNorm
// above): one 256-thread workgroup per row stages the row's bf16 values in
// LDS (dynamic, ldo halves), takes their largest magnitude, then writes the
// scaled f16 chunks (zero past ff) and the row exponent.
// RMSNorm into the prepared GEMM layout with the row held in registers:
// 256 threads per row, U chunks of 8 elements per thread (d <= 2048 * U), so
// the row is read once (one wave re-reading it per pass was latency-bound:
// 10 us per 512 rows).  Same arithmetic per element as prefill_rmsnorm_kernel
// (x * inv * w rounded to bf16, then the row exponent and f16), the sum of
// squares in a fixed order: per thread over its chunks, then across the block.
template <int U>
__global__ __launch_bounds__(256) void prefill_rmsnorm_xp_kernel(const float* __restrict__ x,
                                                                 const uint16_t* __restrict__ w, int d, float eps,
                                                                 uint16_t* __restrict__ out, int ldo,
                                                                 int* __restrict__ xexp) {
    __shared__ float red_sum[4], red_max[4];
    const int row = blockIdx.x, t = threadIdx.x;
    const float* xr = x + (size_t)row * d;
    float y[U][8];
    uint4 wv[U];
#pragma unroll
    for (int u = 0; u < U; u++) {  // every load first
        const int k0 = (t + 256 * u) * 8;
        if (k0 < d) {
            const float4 a = *(const float4*)(xr + k0), b = *(const float4*)(xr + k0 + 4);
            y[u][0] = a.x; y[u][1] = a.y; y[u][2] = a.z; y[u][3] = a.w;
            y[u][4] = b.x; y[u][5] = b.y; y[u][6] = b.z; y[u][7] = b.w;
            wv[u] = *(const uint4*)(w + k0);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) y[u][i] = 0.0f;
            wv[u] = make_uint4(0, 0, 0, 0);
        }
    }
    float sq = 0.0f;
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
        for (int i = 0; i < 8; i++) sq += y[u][i] * y[u][i];
    sq = wave_sum(sq);
    if ((t & 63) == 0) red_sum[t >> 6] = sq;
    __syncthreads();
    const float tot = (red_sum[0] + red_sum[1]) + (red_sum[2] + red_sum[3]);
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
        for (int i = 0; i < 8; i++) {  // cpu.rs:146: x * inv_rms * w, then the bf16 linear input
            const uint32_t wbits = (i & 1) ? (ww[i >> 1] >> 16) : (ww[i >> 1] & 0xFFFFu);
            y[u][i] = bf16_bits_to_f32(f32_to_bf16_rne(y[u][i] * inv * __uint_as_float(wbits << 16)));
            mx = fmaxf(mx, fabsf(y[u][i]));
        }
    }
    const int e = range_exp(block_absmax256(mx, red_max), XPREP_TOP);
    if (t == 0) xexp[row] = e;
    uint16_t* orow = out + (size_t)row * ldo;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int c = t + 256 * u;
        if (c * 8 >= ldo) continue;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = __builtin_amdgcn_ldexpf(y[u][i], -e);  // zero past d
        *(uint4*)(orow + c * 8) = make_uint4(pack_half2(v[0], v[4]), pack_half2(v[1], v[5]), pack_half2(v[2], v[6]),
                                             pack_half2(v[3], v[7]));
    }
}

// Gate/up GEMM epilogue of the prefill: the fused weight's 16-row tiles hold
// 8 gate rows then their 8 up rows, so a gate row's partner is in lane + 32
// (D rows 4q..4q+3 per lane).  Writes bf16(swiglu(g, u)) (f64 SwiGLU, as the
// decode epilogue and device.rs:727 via cpu.rs:68) into h[row][ff].
struct EpiGemmSwiGLU {
    uint16_t* h;
    int ff;
    __device__ __forceinline__ void operator()(int row, int n0, int, bool live, const float4_t& v) const {
        float up[4];
#pragma unroll
        for (int i = 0; i < 4; i++) up[i] = __shfl_xor(v[i], 32, 64);
        const int rr = n0 & 15;
        if (!live || rr >= 8) return;
        uint16_t o[4];
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = swiglu_bf16(v[i], up[i]);
        *(uint2*)(h + (size_t)row * ff + (n0 >> 4) * 8 + rr) =
            make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
    }
};

__global__ __launch_bounds__(256) void prefill_swiglu_xp_kernel(const float* __restrict__ gu, int ff,
                                                               uint16_t* __restrict__ out, int ldo,
                                                               int* __restrict__ xexp) {
    extern __shared__ uint16_t hrow[];
    __shared__ float red4[4];
    const int row = blockIdx.x;
    const float* g = gu + (size_t)row * 2 * ff;
    float mx = 0.0f;
    for (int j = threadIdx.x; j < ldo; j += 256) {
        uint16_t hb = 0;
        if (j < ff) {
            const int b = j >> 3, rr = j & 7;
            hb = swiglu_bf16(g[16 * b + rr], g[16 * b + 8 + rr]);
            mx = fmaxf(mx, fabsf(bf16_bits_to_f32(hb)));
        }
        hrow[j] = hb;
    }
    const int e = range_exp(block_absmax256(mx, red4), XPREP_TOP);  // its barrier also orders hrow
    if (threadIdx.x == 0) xexp[row] = e;
    uint16_t* orow = out + (size_t)row * ldo;
    for (int c = threadIdx.x; c * 8 < ldo; c += 256) {
        const uint4 hv = *(const uint4*)&hrow[c * 8];
        const uint32_t w4[4] = {hv.x, hv.y, hv.z, hv.w};
        float y[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            y[2 * i] = __builtin_amdgcn_ldexpf(bf16_bits_to_f32(w4[i] & 0xFFFF), -e);
            y[2 * i + 1] = __builtin_amdgcn_ldexpf(bf16_bits_to_f32(w4[i] >> 16), -e);
        }
        *(uint4*)(orow + c * 8) = make_uint4(pack_half2(y[0], y[4]), pack_half2(y[1], y[5]), pack_half2(y[2], y[6]),
                                             pack_half2(y[3], y[7]));
    }
}

// The last prompt row into the decode engine's residual, with the
// per-16-element sums of squares its RMSNorm prologue reads.
__global__ void prefill_last_row_kernel(const float* __restrict__ xrow, int d, float* __restrict__ x,
                                        float* __restrict__ ssq) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t * 16 >= d) return;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float v = xrow[t * 16 + i];
        x[t * 16 + i] = v;
        s += v * v;
    }
    ssq[t] = s;
}

// One M=1 int4 GEMV of the engine: bf16 input (or the f32 residual through
// the RMSNorm prologue when norm.ssq is set).  Small matrices split K over
// eight waves per tile to keep enough weight bytes in flight.
template <bool NORM, typename Epi>
static void gemv_engine(const th_qweight* w, const void* x, NormArgs norm, Epi epi, hipStream_t s) {
    TH_REQUIRE(w->bits == 4 && w->scale_dtype == TH_F16, "engine weights must be q4 with f16 scales");
    TH_REQUIRE(!NORM || (w->cols % 16 == 0 && w->cols / 16 <= 256), "RMSNorm prologue supports K <= 4096");
    const bool small = w->Np / 16 < 512;
    if (small && w->Kp / 128 >= 64) {  // few tiles, long K (down projection): sixteen waves per tile
        const size_t smem = Q4GemvSmem<1, 16>::bytes((int)(w->Kp / 128));
        TH_REQUIRE(smem <= 64 * 1024, "engine GEMV LDS above 64 KiB");
        TH_LAUNCH((q4_gemv_kernel<1, false, true, _Float16, Epi, 2, 4, 16, NORM>), dim3((unsigned)(w->Np / 16)),
                           dim3(1024), smem, s, (const uint4*)w->data, (const _Float16*)w->scales, x, (int)w->cols,
                           (int)w->Kp, (int)w->rows, (int)w->cols, epi, norm, SingleMatrix{});
    } else if (small) {
        const size_t smem = Q4GemvSmem<1, 8>::bytes((int)(w->Kp / 128));
        TH_REQUIRE(smem <= 64 * 1024, "engine GEMV LDS above 64 KiB");
        TH_LAUNCH((q4_gemv_kernel<1, false, true, _Float16, Epi, 2, 4, 8, NORM>), dim3((unsigned)(w->Np / 16)),
                           dim3(512), smem, s, (const uint4*)w->data, (const _Float16*)w->scales, x, (int)w->cols,
                           (int)w->Kp, (int)w->rows, (int)w->cols, epi, norm, SingleMatrix{});
    } else if (NORM && w->Np / 16 >= 1376) {  // many tiles (gate/up, LM head): two per workgroup, one staging
        // (QKV's 768 tiles run faster one per workgroup: 709 against 723 tok/s)
        const size_t smem = Q4GemvSmem<1, 4, 2>::bytes((int)(w->Kp / 128));
        TH_REQUIRE(smem <= 64 * 1024, "engine GEMV LDS above 64 KiB");
        SingleMatrixTiles<2> src;
        src.tiles = (int)(w->Np / 16);
        // the two tiles streamed side by side, one reduction (+1% decode)
        TH_LAUNCH((q4_gemv_kernel<1, false, true, _Float16, Epi, 2, 4, 4, NORM, SingleMatrixTiles<2>, 2>),
                           dim3((unsigned)ceil_div(w->Np / 16, (size_t)2)), dim3(256), smem, s, (const uint4*)w->data,
                           (const _Float16*)w->scales, x, (int)w->cols, (int)w->Kp, (int)w->rows, (int)w->cols, epi,
                           norm, src);
    } else {
        const size_t smem = Q4GemvSmem<1, 4>::bytes((int)(w->Kp / 128));
        TH_REQUIRE(smem <= 64 * 1024, "engine GEMV LDS above 64 KiB");
        TH_LAUNCH((q4_gemv_kernel<1, false, true, _Float16, Epi, 2, 4, 4, NORM>), dim3((unsigned)(w->Np / 16)),
                           dim3(256), smem, s, (const uint4*)w->data, (const _Float16*)w->scales, x, (int)w->cols,
                           (int)w->Kp, (int)w->rows, (int)w->cols, epi, norm, SingleMatrix{});
    }
    TH_LAUNCH_CHECK();
}

}  // namespace th

using namespace th;

struct th_llama {
    th_device* dev = nullptr;
    th_llama_config cfg{};
    int qd = 0, kvd = 0, max_steps = 0, n_splits = 0;
    bool attn_even = true;  // decode attention splits: even shares of the attended length
    int attn_spl = 0;       // even mode: positions per workgroup at most (an ATTN_EVEN_SPLS entry)
    std::vector<th_qweight*> wqkv, wo, wgu, wd;
    th_qweight* lm = nullptr;
    uint16_t *embed = nullptr, *attn_norm = nullptr, *ffn_norm = nullptr, *final_norm = nullptr;
    _Float16 *kcache = nullptr, *vcache = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    float *x = nullptr, *q = nullptr, *logits = nullptr, *part = nullptr, *ssq = nullptr, *amax_v = nullptr;
    uint16_t *att = nullptr, *sg = nullptr;
    int *counters = nullptr, *amax_i = nullptr;  // counters: [n_heads] attention, [n_heads] argmax
    LlamaState* st = nullptr;
    int32_t* history = nullptr;
    hipGraphExec_t graph = nullptr;
    AqlSeq* aql_step = nullptr;  // the step as a write-through AQL sequence
    bool weights_ready = false;
    // prefill workspace (rows = prompt chunk), grown on demand
    size_t pf_rows = 0;
    float *pf_x = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_y = nullptr, *pf_gu = nullptr;
    uint16_t *pf_xb = nullptr, *pf_att = nullptr, *pf_sg = nullptr;
    int* pf_xe = nullptr;  // row exponents of prepared pf_xb, pf_att, pf_sg ([3][rows])
    int32_t* pf_tok = nullptr;
};

namespace th {

static void llama_free(th_llama* m) {
    if (!m) return;
    device_drain(m->dev);
    for (auto* v : {&m->wqkv, &m->wo, &m->wgu, &m->wd})
        for (th_qweight* w : *v) th_qweight_free(w);
    if (m->lm) th_qweight_free(m->lm);
    void* ptrs[] = {m->embed, m->attn_norm, m->ffn_norm, m->final_norm, m->kcache, m->vcache, m->rope_cos,
                    m->rope_sin, m->x, m->q, m->logits, m->part, m->ssq, m->amax_v, m->att, m->sg, m->counters,
                    m->amax_i, m->st, m->history, m->pf_x, m->pf_qkv, m->pf_q, m->pf_y, m->pf_gu, m->pf_xb,
                    m->pf_att, m->pf_sg, m->pf_tok, m->pf_xe};
    aql_free(m->aql_step);
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    if (m->graph) (void)hipGraphExecDestroy(m->graph);
    th_device* d = m->dev;
    delete m;
    device_release(d);
}

template <typename T>
static T* dalloc(size_t n) {
    void* p = nullptr;
    TH_HIP(hipMalloc(&p, n * sizeof(T)));
    return (T*)p;
}

// Enqueue one decode step (all layers) on the device stream.

// Final RMSNorm and LM head (tile maxima), then the greedy argmax, which
// also writes the next token's embedding.
static void llama_lm_head_argmax(th_llama* m, hipStream_t s) {
    const th_llama_config& c = m->cfg;
    const int d = c.d_model;
    NormArgs fin;
    fin.ssq = m->ssq; fin.nssq = d / 16; fin.w = m->final_norm; fin.eps = c.eps;
    gemv_engine<true>(m->lm, m->x, fin, EpiTileMax{m->logits, m->amax_v, m->amax_i, c.vocab}, s);
    TH_LAUNCH(llama_argmax_embed_kernel, dim3(1), dim3(1024), 0, s, m->amax_v, m->amax_i,
                       (int)ceil_div((size_t)c.vocab, 16), m->st, m->history, m->embed, d, m->x, m->ssq);
    TH_LAUNCH_CHECK();
}

// x / ssq <- the embedding of the state's current token (after the host
// sets the token; decode steps chain it themselves).
static void llama_embed_current(th_llama* m, hipStream_t s) {
    const int d = m->cfg.d_model;
    TH_LAUNCH(llama_embed_kernel, dim3((unsigned)ceil_div((size_t)d / 16, (size_t)256)), dim3(256), 0, s,
                       m->embed, m->st, d, m->x, m->ssq);
    TH_LAUNCH_CHECK();
}

// The engine's decode attention: even splits (attn_spl positions at most per
// workgroup) or fixed ATTN_SPLIT_ENGINE-position chunks.
static void launch_engine_attention(th_llama* m, const _Float16* kc, const _Float16* vc, hipStream_t s) {
    const th_llama_config& c = m->cfg;
    const int hd = c.head_dim;
    const int* pos = (const int*)&m->st->pos;
    if (!m->attn_even) {
        launch_attn_decode<ATTN_SPLIT_ENGINE, true>(m->q, kc, vc, c.n_heads, c.n_kv_heads, hd, m->n_splits, m->part,
                                                    m->counters, (void*)m->att, pos, s);
        return;
    }
// 512 threads (two waves per SIMD, half the keys per thread) where the split
// shape allows: 7B decode +1.8% against 256 (722.4 / 709.5 tok/s, same
// tokens; 1024 threads: 702.5)
#define TH_ATT_EVEN(S)                                                                                                \
    case S:                                                                                                           \
        launch_attn_decode<S, true, 512, true>(m->q, kc, vc, c.n_heads, c.n_kv_heads, hd, m->n_splits, m->part,       \
                                               m->counters, (void*)m->att, pos, s);                                   \
        break;
    switch (m->attn_spl) {
        TH_ATT_EVEN(128) TH_ATT_EVEN(192) TH_ATT_EVEN(256) TH_ATT_EVEN(288) TH_ATT_EVEN(384) TH_ATT_EVEN(512)
        default: throw Error(TH_ERR_INVALID, "attention split size not instantiated");
    }
#undef TH_ATT_EVEN
}

static void llama_enqueue_step(th_llama* m) {
    const th_llama_config& c = m->cfg;
    hipStream_t s = m->dev->stream;
    const int d = c.d_model, hd = c.head_dim;
    const int nssq = d / 16;
    // x and ssq hold the current token's embedding: written by the previous
    // step's argmax (llama_argmax_embed_kernel) or by llama_embed_current
    const size_t cache_layer = (size_t)c.max_seq * m->kvd;
    for (int l = 0; l < c.n_layers; l++) {
        _Float16* kc = m->kcache + l * cache_layer;
        _Float16* vc = m->vcache + l * cache_layer;
        NormArgs an;
        an.ssq = m->ssq; an.nssq = nssq; an.w = m->attn_norm + (size_t)l * d; an.eps = c.eps;
        gemv_engine<true>(m->wqkv[l], m->x, an,
                          EpiQKV{{}, m->q, kc, vc, m->rope_cos, m->rope_sin, m->st, m->qd, m->kvd, hd}, s);
        launch_engine_attention(m, kc, vc, s);
        gemv_engine<false>(m->wo[l], m->att, NormArgs{}, EpiAddToSsq{m->x, m->ssq}, s);
        NormArgs fn;
        fn.ssq = m->ssq; fn.nssq = nssq; fn.w = m->ffn_norm + (size_t)l * d; fn.eps = c.eps;
        gemv_engine<true>(m->wgu[l], m->x, fn, EpiSwiGLU{{}, m->sg}, s);
        gemv_engine<false>(m->wd[l], m->sg, NormArgs{}, EpiAddToSsq{m->x, m->ssq}, s);
    }
    llama_lm_head_argmax(m, s);
}

static void llama_build_graph(th_llama* m) {
    if (m->graph) return;
    hipStream_t s = m->dev->stream;
    hipGraph_t g;
    TH_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    try {
        llama_enqueue_step(m);
    } catch (...) {
        hipGraph_t dummy;
        (void)hipStreamEndCapture(s, &dummy);
        throw;
    }
    TH_HIP(hipStreamEndCapture(s, &g));
    TH_HIP(hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0));
    TH_HIP(hipGraphDestroy(g));
}

// One decode step: graph replay, or (TANG_HIP_EAGER=1, for kernel tracers
// that do not follow graph launches) the same kernels enqueued directly.
static bool llama_eager() {
    static const bool eager = [] {
        const char* e = std::getenv("TANG_HIP_EAGER");
        return e && e[0] == '1';
    }();
    return eager;
}

static bool stream_capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// Every kernel of the step stores what later kernels read with write-through
// stores (the epilogues, the attention merge, the argmax), so its AQL
// sequence needs no release fences between kernels.
static bool llama_use_aql(th_llama* m) {
    return !llama_eager() && aql_enabled() && !stream_capturing(m->dev->stream);
}

static void llama_prepare_step(th_llama* m) {
    if (llama_use_aql(m)) {
        if (!m->aql_step) m->aql_step = aql_record(m->dev, true, [&] { llama_enqueue_step(m); });
    } else if (!llama_eager()) {
        llama_build_graph(m);
    }
}

// Enqueue one step: a replay on the device's AQL queue (the caller waits
// with aql_wait / device_sync before further stream work), or a HIP graph
// launch when TANG_HIP_DISPATCH=graph or inside a caller's stream capture.
static void llama_launch_steps(th_llama* m, size_t n) {
    if (llama_eager()) {
        for (size_t i = 0; i < n; i++) llama_enqueue_step(m);
        return;
    }
    llama_prepare_step(m);
    if (llama_use_aql(m)) {
        // n steps with no host work between them: one submission, so the
        // token boundaries carry the sequence's own fences (every kernel of
        // the step stores write-through) rather than system-scope ones
        aql_submit(*m->aql_step, n);
        return;
    }
    for (size_t i = 0; i < n; i++) TH_HIP(hipGraphLaunch(m->graph, m->dev->stream));
}

static void llama_launch_step(th_llama* m) { llama_launch_steps(m, 1); }

constexpr size_t PREFILL_CHUNK = 512;  // prompt rows per pass (workspace ~100 MB at the 7B shape)

static void prefill_reserve(th_llama* m, size_t rows) {
    if (rows <= m->pf_rows) return;
    device_sync(m->dev);
    void* old[] = {m->pf_x, m->pf_qkv, m->pf_q, m->pf_y, m->pf_gu, m->pf_xb, m->pf_att, m->pf_sg, m->pf_tok, m->pf_xe};
    for (void* p : old)
        if (p) (void)hipFree(p);
    const th_llama_config& c = m->cfg;
    const size_t d = c.d_model, ff = c.d_ff;
    m->pf_x = dalloc<float>(rows * d);
    m->pf_y = dalloc<float>(rows * d);
    m->pf_qkv = dalloc<float>(rows * (m->qd + 2 * m->kvd));
    m->pf_q = dalloc<float>(rows * m->qd);
    m->pf_gu = dalloc<float>(rows * 2 * ff);
    m->pf_xb = dalloc<uint16_t>(rows * round_up(d, 128));  // bf16 rows, or prepared rows of Kp
    m->pf_att = dalloc<uint16_t>(rows * round_up((size_t)m->qd, 128));
    m->pf_sg = dalloc<uint16_t>(rows * round_up(ff, 128));
    m->pf_xe = dalloc<int>(3 * rows);
    m->pf_tok = dalloc<int32_t>(rows);
    m->pf_rows = rows;
}

// One chunk of n prompt tokens at positions pos0.. through every layer; the
// residual of its rows ends in pf_x.
// QKV GEMM epilogue of the prefill: RoPE on the q and k columns (each lane
// holds four consecutive columns, i.e. two rotation pairs, of one row), q to
// f32 [n][qd], k and v appended to the f16 cache at pos0 + row -- the
// arithmetic of prefill_rope_kv_kernel, without the f32 qkv round trip.
struct EpiGemmQKVRope {
    float* q;
    _Float16 *kc, *vc;
    const float *cs, *sn;
    int pos0, qd, kvd, hd;
    __device__ __forceinline__ void operator()(int row, int n0, int N, bool live, const float4_t& v) const {
        if (!live || n0 >= N) return;
        const int pos = pos0 + row;
        float o[4] = {v[0], v[1], v[2], v[3]};
        if (n0 < qd + kvd) {
            const int half = hd / 2, i0 = (n0 % hd) >> 1;
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const float c = cs[(size_t)pos * half + i0 + p], sv = sn[(size_t)pos * half + i0 + p];
                const float x0 = o[2 * p], x1 = o[2 * p + 1];
                o[2 * p] = x0 * c - x1 * sv;
                o[2 * p + 1] = x0 * sv + x1 * c;
            }
        }
        if (n0 < qd) {
            *(float4*)(q + (size_t)row * qd + n0) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
            _Float16* dst = n0 < qd + kvd ? kc + (size_t)pos * kvd + (n0 - qd) : vc + (size_t)pos * kvd + (n0 - qd - kvd);
            const uint32_t h0 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)o[0]) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)o[1]) << 16);
            const uint32_t h1 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)o[2]) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)o[3]) << 16);
            *(uint2*)dst = make_uint2(h0, h1);
        }
    }
};

// Prepared-layout RMSNorm of n rows of the residual (d <= 8192).
static void prefill_rmsnorm_xp(const float* x, const uint16_t* w, int d, float eps, uint16_t* out, int ldo,
                               int* xexp, size_t n, hipStream_t s) {
    const int chunks = std::max(d, ldo) / 8;
    if (chunks <= 512)
        TH_LAUNCH(prefill_rmsnorm_xp_kernel<2>, dim3((unsigned)n), dim3(256), 0, s, x, w, d, eps, out, ldo, xexp);
    else
        TH_LAUNCH(prefill_rmsnorm_xp_kernel<4>, dim3((unsigned)n), dim3(256), 0, s, x, w, d, eps, out, ldo, xexp);
    TH_LAUNCH_CHECK();
}

// A prefill linear with its epilogue fused (no split-K: used from
// PREFILL_FUSED_ROWS rows, where the grid covers the chip without it).
constexpr size_t PREFILL_FUSED_ROWS = 256;
template <typename Epi>
static void prefill_gemm_epi(const th_qweight* w, PreparedX xp, size_t n, const Epi& epi, hipStream_t s) {
    const size_t NT = w->Np / 16;
    const int GQ = (int)(w->Kp / 128);
    GemmDense src;
    src.M = (int)n;
    if (n <= 1024)
        TH_LAUNCH((q4_gemm_mfma_kernel<2, 4, _Float16, GemmDense, Epi>),
                  dim3((unsigned)ceil_div(NT, (size_t)8), (unsigned)ceil_div(n, (size_t)64), 1), dim3(256), 0, s,
                  (const uint4*)w->data, (const _Float16*)w->scales, (const int*)w->row_exp, xp.x, xp.xexp, epi, src,
                  (int)w->rows, (int)w->cols, (int)w->Kp, (int)w->Kp, GQ);
    else
        TH_LAUNCH((q4_gemm_mfma_kernel<2, 8, _Float16, GemmDense, Epi>),
                  dim3((unsigned)ceil_div(NT, (size_t)8), (unsigned)ceil_div(n, (size_t)128), 1), dim3(256), 0, s,
                  (const uint4*)w->data, (const _Float16*)w->scales, (const int*)w->row_exp, xp.x, xp.xexp, epi, src,
                  (int)w->rows, (int)w->cols, (int)w->Kp, (int)w->Kp, GQ);
    TH_LAUNCH_CHECK();
}

static void prefill_chunk(th_llama* m, const int32_t* tok_host, size_t n, size_t pos0) {
    const th_llama_config& c = m->cfg;
    th_device* dev = m->dev;
    hipStream_t s = dev->stream;
    const int d = c.d_model, ff = c.d_ff, hd = c.head_dim, W = m->qd + 2 * m->kvd;
    TH_HIP(hipMemcpyAsync(m->pf_tok, tok_host, n * 4, hipMemcpyHostToDevice, s));
    TH_LAUNCH(prefill_embed_kernel, dim3(4, (unsigned)n), dim3(256), 0, s, m->embed, m->pf_tok, d, m->pf_x);
    TH_LAUNCH_CHECK();
    const size_t cache_layer = (size_t)c.max_seq * m->kvd;
    // Above 16 rows the linears run on the MFMA GEMM, whose activation layout
    // the RMSNorm and SwiGLU kernels then write directly.
    const bool xp = n > 16;
    int* xe_xb = m->pf_xe;  // row exponents of the prepared pf_xb, pf_att, pf_sg
    int* xe_att = m->pf_xe + m->pf_rows;
    int* xe_sg = m->pf_xe + 2 * m->pf_rows;
    auto prefill_norm = [&](const uint16_t* w, const th_qweight* consumer) {
        if (xp && d <= 8192 && (int)consumer->Kp <= 8192)
            prefill_rmsnorm_xp(m->pf_x, w, d, c.eps, m->pf_xb, (int)consumer->Kp, xe_xb, n, s);
        else if (xp)
            TH_LAUNCH(prefill_rmsnorm_kernel<true>, dim3((unsigned)n), dim3(64), 0, s, m->pf_x, w, d, c.eps,
                               m->pf_xb, (int)consumer->Kp, xe_xb);
        else
            TH_LAUNCH(prefill_rmsnorm_kernel<false>, dim3((unsigned)n), dim3(64), 0, s, m->pf_x, w, d,
                               c.eps, m->pf_xb, d, (int*)nullptr);
        TH_LAUNCH_CHECK();
    };
    auto linear = [&](const th_qweight* w, const uint16_t* xin, const int* xe, int k, float* y, int ldy) {
        if (xp) launch_q4_linear_prepared(w, PreparedX{xin, xe}, n, y, ldy, s, dev);
        else launch_q4_linear(w, xin, TH_BF16, n, k, y, ldy, s, dev);
    };
    // split attention: few enough splits that q_len * heads * splits records fit the scratch
    const size_t attended = pos0 + n;
    const int subs = (int)std::max<size_t>(1, ceil_div(attended, (size_t)ATTN_SUB * 8));
    const int n_splits = (int)ceil_div(attended, (size_t)subs * ATTN_SUB);
    // From PREFILL_FUSED_ROWS rows: RoPE/KV append in the QKV GEMM epilogue,
    // SwiGLU in the gate/up GEMM epilogue (engine weights: f16 scales)
    const bool fused = xp && n >= PREFILL_FUSED_ROWS && m->wqkv[0]->scale_dtype == TH_F16 &&
                       m->wgu[0]->scale_dtype == TH_F16;
    for (int l = 0; l < c.n_layers; l++) {
        _Float16* kc = m->kcache + l * cache_layer;
        _Float16* vc = m->vcache + l * cache_layer;
        prefill_norm(m->attn_norm + (size_t)l * d, m->wqkv[l]);
        if (fused) {  // RoPE and the K/V append in the QKV GEMM's epilogue
            prefill_gemm_epi(m->wqkv[l], PreparedX{m->pf_xb, xe_xb}, n,
                             EpiGemmQKVRope{m->pf_q, kc, vc, m->rope_cos, m->rope_sin, (int)pos0, m->qd, m->kvd, hd},
                             s);
        } else {
        linear(m->wqkv[l], m->pf_xb, xe_xb, d, m->pf_qkv, W);
        TH_LAUNCH(prefill_rope_kv_kernel, dim3((unsigned)ceil_div((size_t)W / 8, (size_t)256), (unsigned)n), dim3(256),
                  0, s, m->pf_qkv, (int)pos0,
                           m->rope_cos, m->rope_sin, m->qd, m->kvd, hd, m->pf_q, kc, vc);
        TH_LAUNCH_CHECK();
        }
        const bool xp_att = xp && (hd == 64 || hd == 128);
        if (hd == 64 || hd == 128) {  // causal flash attention on MFMA
            launch_attn_prefill(m->pf_q, m->qd, kc, vc, c.n_heads, c.n_kv_heads, hd, (int)pos0, (int)n,
                                (uint16_t*)m->pf_att, xp ? (int)m->wo[l]->Kp : m->qd, xp, xe_att, s);
        } else {
            float* part = (float*)device_scratch(dev, n * c.n_heads * n_splits * (hd + 2) * sizeof(float));
            int* counters = device_counters(dev, n * c.n_heads);
            launch_attn_split<true>(m->pf_q, kc, vc, true, (int)pos0, (int)n, c.n_heads, c.n_kv_heads, hd, subs,
                                    n_splits, part, counters, (void*)m->pf_att, nullptr, s);
        }
        if (xp_att) {  // x += att.Wo^T in the GEMM's epilogue
            launch_q4_linear_prepared(m->wo[l], PreparedX{m->pf_att, xe_att}, n, m->pf_x, d, s, dev, true);
        } else {
            launch_q4_linear(m->wo[l], m->pf_att, TH_BF16, n, m->qd, m->pf_y, d, s, dev);
            TH_LAUNCH(prefill_add_kernel, dim3(1024), dim3(256), 0, s, m->pf_x, m->pf_y, n * d);
            TH_LAUNCH_CHECK();
        }
        prefill_norm(m->ffn_norm + (size_t)l * d, m->wgu[l]);
        if (fused) {
            // SwiGLU in the gate/up GEMM's epilogue (bf16 rows in pf_gu's
            // memory), prepared for the down GEMM by the activation pass, and
            // x += sg.Wd^T in the down GEMM's epilogue
            uint16_t* h = (uint16_t*)m->pf_gu;
            prefill_gemm_epi(m->wgu[l], PreparedX{m->pf_xb, xe_xb}, n, EpiGemmSwiGLU{h, ff}, s);
            const PreparedX sg = prepare_x(dev, h, false, n, ff, ff, m->wd[l]->Kp, s);
            launch_q4_linear_prepared(m->wd[l], sg, n, m->pf_x, d, s, dev, true);
            continue;
        }
        linear(m->wgu[l], m->pf_xb, xe_xb, d, m->pf_gu, 2 * ff);
        if (xp) {
            const int ldo = (int)m->wd[l]->Kp;
            TH_REQUIRE(ldo * 2 <= 64 * 1024, "prefill: d_ff above 32768");
            TH_LAUNCH(prefill_swiglu_xp_kernel, dim3((unsigned)n), dim3(256), (size_t)ldo * 2, s, m->pf_gu,
                               ff, m->pf_sg, ldo, xe_sg);
        } else {
            TH_LAUNCH(prefill_swiglu_kernel, dim3(8, (unsigned)n), dim3(256), 0, s, m->pf_gu, ff, m->pf_sg,
                               ff);
        }
        TH_LAUNCH_CHECK();
        if (xp) {  // x += sg.Wd^T in the GEMM's epilogue
            launch_q4_linear_prepared(m->wd[l], PreparedX{m->pf_sg, xe_sg}, n, m->pf_x, d, s, dev, true);
        } else {
            linear(m->wd[l], m->pf_sg, nullptr, ff, m->pf_y, d);
            TH_LAUNCH(prefill_add_kernel, dim3(1024), dim3(256), 0, s, m->pf_x, m->pf_y, n * d);
            TH_LAUNCH_CHECK();
        }
    }
}

// Concatenate rows of q4 matrices generated by th_synth_q4 (nib + f16 scales).
struct HostQ4 {
    std::vector<uint8_t> nib;
    std::vector<uint16_t> sc;
    size_t rows = 0, cols = 0;
};

static HostQ4 synth_q4_host(uint64_t seed, size_t rows, size_t cols) {
    HostQ4 h;
    h.rows = rows; h.cols = cols;
    const size_t bpr = ceil_div(cols, 32);
    h.nib.resize(rows * bpr * 16);
    h.sc.resize(rows * bpr);
    if (th_synth_q4(seed, rows, cols, Q4_SMIN, Q4_SMAX, h.nib.data(), h.sc.data()) != TH_OK)
        throw Error(TH_ERR_INVALID, "th_synth_q4 failed");
    return h;
}

// A row-major f32 matrix through quantize_matrix_q4 (quantize.rs:208-221),
// with each block's amax/7 scale then rounded to f16 (RNE), the engine's
// scale format: relative error <= 2^-11 for scales in f16's normal range.
// A smaller scale (a near-zero block, amax < 4.3e-4) becomes an f16
// subnormal or zero, off by at most 2^-25 absolute, which bounds each of its
// dequantized weights' error by 8 * 2^-25 = 2.4e-7, below what the rounding
// of a normal block's scale costs.  Scales above 65504 are rejected.
static HostQ4 quant_q4_host(const std::vector<float>& w, size_t rows, size_t cols, const std::string& name) {
    HostQ4 h;
    h.rows = rows; h.cols = cols;
    const size_t bpr = ceil_div(cols, (size_t)32);
    std::vector<th_q4_block> blocks(rows * bpr);
    check_status(th_quantize_q4(w.data(), rows, cols, blocks.data()));
    h.nib.resize(rows * bpr * 16);
    h.sc.resize(rows * bpr);
    for (size_t i = 0; i < blocks.size(); i++) {
        std::memcpy(&h.nib[i * 16], blocks[i].values, 16);
        const float sc = blocks[i].scale;
        TH_REQUIRE(sc >= 0.0f && sc <= 65504.0f, name + ": a block scale is above the f16 range");
        h.sc[i] = f32_to_f16_host(sc);
    }
    return h;
}

// Rows of several matrices with the same column count, in order.
static HostQ4 concat_rows(std::initializer_list<const HostQ4*> parts) {
    HostQ4 f;
    f.cols = (*parts.begin())->cols;
    for (const HostQ4* p : parts) {
        TH_REQUIRE(p->cols == f.cols, "concatenated matrices differ in width");
        f.rows += p->rows;
        f.nib.insert(f.nib.end(), p->nib.begin(), p->nib.end());
        f.sc.insert(f.sc.end(), p->sc.begin(), p->sc.end());
    }
    return f;
}

// The engine's gate/up matrix: 16-row tile b holds gate rows 8b..8b+7 then
// up rows 8b..8b+7 (the SwiGLU epilogue pairs them inside one tile).
static HostQ4 interleave_gate_up(const HostQ4& g, const HostQ4& u) {
    TH_REQUIRE(g.rows == u.rows && g.cols == u.cols && g.rows % 8 == 0, "gate/up shapes differ");
    const size_t bpr = ceil_div(g.cols, (size_t)32), ff = g.rows;
    HostQ4 gi;
    gi.rows = 2 * ff; gi.cols = g.cols;
    gi.nib.resize(2 * ff * bpr * 16);
    gi.sc.resize(2 * ff * bpr);
    for (size_t b = 0; b < ff / 8; b++) {
        for (size_t r = 0; r < 8; r++) {
            const size_t src = 8 * b + r, dg = 16 * b + r, du = 16 * b + 8 + r;
            std::memcpy(&gi.nib[dg * bpr * 16], &g.nib[src * bpr * 16], bpr * 16);
            std::memcpy(&gi.nib[du * bpr * 16], &u.nib[src * bpr * 16], bpr * 16);
            std::memcpy(&gi.sc[dg * bpr], &g.sc[src * bpr], bpr * 2);
            std::memcpy(&gi.sc[du * bpr], &u.sc[src * bpr], bpr * 2);
        }
    }
    return gi;
}

}  // namespace th

extern "C" {

int th_llama_create(th_device* dev, const th_llama_config* cfg, th_llama** out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && cfg && out, "null argument");
    const th_llama_config& c = *cfg;
    TH_REQUIRE(c.n_layers > 0 && c.d_model > 0 && c.vocab > 0 && c.max_seq > 0, "bad config");
    TH_REQUIRE(c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256, "head_dim must be 64, 128 or 256");
    TH_REQUIRE(c.n_kv_heads > 0 && c.n_heads % c.n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
    TH_REQUIRE(c.n_heads * c.head_dim == c.d_model, "n_heads*head_dim must equal d_model");
    TH_REQUIRE(c.d_ff % 8 == 0 && c.d_model % 16 == 0, "d_model must be a multiple of 16 and d_ff of 8");
    TH_REQUIRE(c.d_model <= 4096, "the RMSNorm prologue supports d_model <= 4096");
    TH_REQUIRE(ceil_div((size_t)c.max_seq, (size_t)ATTN_SPLIT_ENGINE) <= 256, "max_seq too long for the attention splits");
    th_llama* m = new th_llama();
    m->dev = dev;
    device_retain(dev);
    try {
        m->cfg = c;
        m->qd = c.n_heads * c.head_dim;
        m->kvd = c.n_kv_heads * c.head_dim;
        m->max_steps = c.max_seq;
        // even splits: one workgroup per CU (n_heads * n_splits ~ CUs), each
        // at most attn_spl positions; TANG_HIP_ATTN_FIXED=1 selects fixed
        // ATTN_SPLIT_ENGINE-position chunks instead
        const char* fixed = getenv("TANG_HIP_ATTN_FIXED");
        m->attn_even = !(fixed && fixed[0] == '1');
        if (m->attn_even) {
            const int want = std::max(1, dev->num_cus / c.n_heads);
            const int need = (int)ceil_div((size_t)c.max_seq, (size_t)want);
            m->attn_spl = ATTN_EVEN_SPLS[sizeof(ATTN_EVEN_SPLS) / sizeof(int) - 1];
            for (int v : ATTN_EVEN_SPLS)
                if (v >= need) { m->attn_spl = v; break; }
            m->n_splits = (int)ceil_div((size_t)c.max_seq, (size_t)m->attn_spl);
            // spread over the same split count as the request, or more when
            // the largest split size caps it
            m->n_splits = std::max(m->n_splits, std::min(want, (int)ceil_div((size_t)c.max_seq, (size_t)64)));
            TH_REQUIRE(m->n_splits <= 256, "max_seq too long for the attention splits");
        } else {
            m->n_splits = (int)ceil_div((size_t)c.max_seq, ATTN_SPLIT_ENGINE);
        }
        TH_HIP(hipSetDevice(dev->ordinal));
        const size_t L = c.n_layers, d = c.d_model;
        m->embed = dalloc<uint16_t>((size_t)c.vocab * d);
        m->attn_norm = dalloc<uint16_t>(L * d);
        m->ffn_norm = dalloc<uint16_t>(L * d);
        m->final_norm = dalloc<uint16_t>(d);
        m->kcache = dalloc<_Float16>(L * c.max_seq * m->kvd);
        m->vcache = dalloc<_Float16>(L * c.max_seq * m->kvd);
        m->rope_cos = dalloc<float>((size_t)c.max_seq * c.head_dim / 2);
        m->rope_sin = dalloc<float>((size_t)c.max_seq * c.head_dim / 2);
        m->x = dalloc<float>(d);
        m->q = dalloc<float>(m->qd);
        m->logits = dalloc<float>(c.vocab);
        m->part = dalloc<float>((size_t)c.n_heads * m->n_splits * (c.head_dim + 2));
        m->ssq = dalloc<float>(d / 16);
        m->amax_v = dalloc<float>(ceil_div((size_t)c.vocab, 16));
        m->amax_i = dalloc<int>(ceil_div((size_t)c.vocab, 16));
        m->counters = dalloc<int>(2 * (size_t)c.n_heads + 2);
        TH_HIP(hipMemset(m->counters, 0, (2 * (size_t)c.n_heads + 2) * sizeof(int)));
        m->att = dalloc<uint16_t>(m->qd);
        m->sg = dalloc<uint16_t>(c.d_ff);
        m->st = dalloc<LlamaState>(1);
        m->history = dalloc<int32_t>(m->max_steps);
        std::vector<float> cs((size_t)c.max_seq * c.head_dim / 2), sn(cs.size());
        rope_tables_host(c.head_dim, c.max_seq, c.rope_theta, cs.data(), sn.data());
        TH_HIP(hipMemcpy(m->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
        TH_HIP(hipMemcpy(m->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    } catch (...) {
        llama_free(m);
        throw;
    }
    *out = m;
    TH_API_END
}

int th_llama_destroy(th_llama* m) {
    TH_API_BEGIN
    llama_free(m);
    TH_API_END
}

int th_llama_init_synthetic(th_llama* m, uint64_t seed) {
    TH_API_BEGIN
    TH_REQUIRE(m, "null model");
    TH_REQUIRE(!m->weights_ready, "weights already initialised");
    const th_llama_config& c = m->cfg;
    const size_t d = c.d_model, ff = c.d_ff, L = c.n_layers;
    m->wqkv.assign(L, nullptr); m->wo.assign(L, nullptr); m->wgu.assign(L, nullptr); m->wd.assign(L, nullptr);
    // Host generation runs in parallel over layers; uploads stay serial.
    std::vector<HostQ4> qkv(L), wo(L), gu(L), dn(L);
    std::string err;
#pragma omp parallel for schedule(dynamic, 1)
    for (long l = 0; l < (long)L; l++) {
        try {
            const HostQ4 q = synth_q4_host(th_synth_seed(seed, l, T_WQ), m->qd, d);
            const HostQ4 k = synth_q4_host(th_synth_seed(seed, l, T_WK), m->kvd, d);
            const HostQ4 v = synth_q4_host(th_synth_seed(seed, l, T_WV), m->kvd, d);
            qkv[l] = concat_rows({&q, &k, &v});
            wo[l] = synth_q4_host(th_synth_seed(seed, l, T_WO), d, d);
            const HostQ4 g = synth_q4_host(th_synth_seed(seed, l, T_WG), ff, d);
            const HostQ4 u = synth_q4_host(th_synth_seed(seed, l, T_WU), ff, d);
            gu[l] = interleave_gate_up(g, u);
            dn[l] = synth_q4_host(th_synth_seed(seed, l, T_WD), d, ff);
        } catch (const std::exception& e) {
#pragma omp critical
            err = e.what();
        }
    }
    if (!err.empty()) throw Error(TH_ERR_INVALID, err);
    for (size_t l = 0; l < L; l++) {
        m->wqkv[l] = q4_pack(m->dev, qkv[l].nib.data(), qkv[l].sc.data(), TH_F16, qkv[l].rows, d);
        m->wo[l] = q4_pack(m->dev, wo[l].nib.data(), wo[l].sc.data(), TH_F16, d, d);
        m->wgu[l] = q4_pack(m->dev, gu[l].nib.data(), gu[l].sc.data(), TH_F16, 2 * ff, d);
        m->wd[l] = q4_pack(m->dev, dn[l].nib.data(), dn[l].sc.data(), TH_F16, d, ff);
        qkv[l] = HostQ4(); wo[l] = HostQ4(); gu[l] = HostQ4(); dn[l] = HostQ4();
    }
    {
        HostQ4 lm = synth_q4_host(th_synth_seed(seed, L, T_LM_HEAD), c.vocab, d);
        m->lm = q4_pack(m->dev, lm.nib.data(), lm.sc.data(), TH_F16, c.vocab, d);
    }
    std::vector<uint16_t> buf((size_t)c.vocab * d);
    check_status(th_synth_normal(th_synth_seed(seed, L, T_EMBED), buf.size(), NORM_STD, TH_BF16, buf.data()));
    TH_HIP(hipMemcpy(m->embed, buf.data(), buf.size() * 2, hipMemcpyHostToDevice));
    for (size_t l = 0; l < L; l++) {
        check_status(th_synth_normal(th_synth_seed(seed, l, T_ATTN_NORM), d, NORM_STD, TH_BF16, buf.data()));
        TH_HIP(hipMemcpy(m->attn_norm + l * d, buf.data(), d * 2, hipMemcpyHostToDevice));
        check_status(th_synth_normal(th_synth_seed(seed, l, T_FFN_NORM), d, NORM_STD, TH_BF16, buf.data()));
        TH_HIP(hipMemcpy(m->ffn_norm + l * d, buf.data(), d * 2, hipMemcpyHostToDevice));
    }
    check_status(th_synth_normal(th_synth_seed(seed, L, T_FINAL_NORM), d, NORM_STD, TH_BF16, buf.data()));
    TH_HIP(hipMemcpy(m->final_norm, buf.data(), d * 2, hipMemcpyHostToDevice));
    m->weights_ready = true;
    TH_API_END
}

int th_llama_load_safetensors(th_llama* m, const th_st_file* f) {
    TH_API_BEGIN
    TH_REQUIRE(m && f, "null argument");
    TH_REQUIRE(!m->weights_ready, "weights already initialised");
    const th_llama_config& c = m->cfg;
    const size_t d = c.d_model, ff = c.d_ff, L = c.n_layers, V = c.vocab;
    // smollm.rs:364-420 (load_model), with every tensor required except
    // lm_head.weight, which falls back to the embedding (weight tying)
    std::vector<HostQ4> qkv(L), wo(L), gu(L), dn(L);
    std::vector<uint16_t> attn_norm(L * d), ffn_norm(L * d);
    std::string err;
#pragma omp parallel for schedule(dynamic, 1)
    for (long l = 0; l < (long)L; l++) {
        try {
            const std::string pre = "model.layers." + std::to_string(l) + ".";
            auto lin = [&](const char* name, size_t rows, size_t cols) {
                const std::string n = pre + name;
                return quant_q4_host(st_read_shaped(f, n, {rows, cols}), rows, cols, n);
            };
            const HostQ4 q = lin("self_attn.q_proj.weight", m->qd, d);
            const HostQ4 k = lin("self_attn.k_proj.weight", m->kvd, d);
            const HostQ4 v = lin("self_attn.v_proj.weight", m->kvd, d);
            qkv[l] = concat_rows({&q, &k, &v});
            wo[l] = lin("self_attn.o_proj.weight", d, m->qd);
            const HostQ4 g = lin("mlp.gate_proj.weight", ff, d);
            const HostQ4 u = lin("mlp.up_proj.weight", ff, d);
            gu[l] = interleave_gate_up(g, u);
            dn[l] = lin("mlp.down_proj.weight", d, ff);
            const std::vector<float> an = st_read_shaped(f, pre + "input_layernorm.weight", {d});
            const std::vector<float> fn = st_read_shaped(f, pre + "post_attention_layernorm.weight", {d});
            for (size_t i = 0; i < d; i++) {
                attn_norm[l * d + i] = f32_to_bf16_host(an[i]);
                ffn_norm[l * d + i] = f32_to_bf16_host(fn[i]);
            }
        } catch (const std::exception& e) {
#pragma omp critical
            err = e.what();
        }
    }
    if (!err.empty()) throw Error(TH_ERR_INVALID, err);
    const std::vector<float> emb = st_read_shaped(f, "model.embed_tokens.weight", {V, d});
    const std::vector<float> fin = st_read_shaped(f, "model.norm.weight", {d});
    HostQ4 lm = st_has(f, "lm_head.weight")
                    ? quant_q4_host(st_read_shaped(f, "lm_head.weight", {V, d}), V, d, "lm_head.weight")
                    : quant_q4_host(emb, V, d, "model.embed_tokens.weight (tied lm_head)");
    m->wqkv.assign(L, nullptr); m->wo.assign(L, nullptr); m->wgu.assign(L, nullptr); m->wd.assign(L, nullptr);
    for (size_t l = 0; l < L; l++) {
        m->wqkv[l] = q4_pack(m->dev, qkv[l].nib.data(), qkv[l].sc.data(), TH_F16, qkv[l].rows, d);
        m->wo[l] = q4_pack(m->dev, wo[l].nib.data(), wo[l].sc.data(), TH_F16, d, m->qd);
        m->wgu[l] = q4_pack(m->dev, gu[l].nib.data(), gu[l].sc.data(), TH_F16, 2 * ff, d);
        m->wd[l] = q4_pack(m->dev, dn[l].nib.data(), dn[l].sc.data(), TH_F16, d, ff);
        qkv[l] = HostQ4(); wo[l] = HostQ4(); gu[l] = HostQ4(); dn[l] = HostQ4();
    }
    m->lm = q4_pack(m->dev, lm.nib.data(), lm.sc.data(), TH_F16, V, d);
    std::vector<uint16_t> buf(V * d);
    for (size_t i = 0; i < buf.size(); i++) buf[i] = f32_to_bf16_host(emb[i]);
    TH_HIP(hipMemcpy(m->embed, buf.data(), buf.size() * 2, hipMemcpyHostToDevice));
    TH_HIP(hipMemcpy(m->attn_norm, attn_norm.data(), L * d * 2, hipMemcpyHostToDevice));
    TH_HIP(hipMemcpy(m->ffn_norm, ffn_norm.data(), L * d * 2, hipMemcpyHostToDevice));
    for (size_t i = 0; i < d; i++) buf[i] = f32_to_bf16_host(fin[i]);
    TH_HIP(hipMemcpy(m->final_norm, buf.data(), d * 2, hipMemcpyHostToDevice));
    m->weights_ready = true;
    TH_API_END
}

int th_llama_fill_kv_synthetic(th_llama* m, size_t len, uint64_t seed) {
    TH_API_BEGIN
    TH_REQUIRE(m, "null model");
    TH_REQUIRE(len <= (size_t)m->cfg.max_seq, "len beyond max_seq");
    const size_t L = m->cfg.n_layers, n = len * m->kvd, layer = (size_t)m->cfg.max_seq * m->kvd;
    std::vector<std::vector<uint16_t>> k(L), v(L);
#pragma omp parallel for schedule(dynamic, 1)
    for (long l = 0; l < (long)L; l++) {
        k[l].resize(n); v[l].resize(n);
        th_synth_normal(th_synth_seed(seed, l, T_KCACHE), n, 1.0f, TH_F16, k[l].data());
        th_synth_normal(th_synth_seed(seed, l, T_VCACHE), n, 1.0f, TH_F16, v[l].data());
    }
    device_sync(m->dev);  // the engine stream is non-blocking: drain it first
    for (size_t l = 0; l < L; l++) {
        TH_HIP(hipMemcpy(m->kcache + l * layer, k[l].data(), n * 2, hipMemcpyHostToDevice));
        TH_HIP(hipMemcpy(m->vcache + l * layer, v[l].data(), n * 2, hipMemcpyHostToDevice));
    }
    TH_API_END
}

int th_llama_set_token(th_llama* m, int32_t token) {
    TH_API_BEGIN
    TH_REQUIRE(m, "null model");
    TH_REQUIRE(token >= 0 && token < m->cfg.vocab, "token out of range");
    device_sync(m->dev);
    LlamaState s{};
    TH_HIP(hipMemcpy(&s, m->st, sizeof s, hipMemcpyDeviceToHost));
    s.token = token;
    TH_HIP(hipMemcpy(m->st, &s, sizeof s, hipMemcpyHostToDevice));
    llama_embed_current(m, m->dev->stream);
    TH_API_END
}

int th_llama_step_device(th_llama* m, size_t pos) {
    TH_API_BEGIN
    TH_REQUIRE(m && m->weights_ready, "model not initialised");
    TH_REQUIRE(pos < (size_t)m->cfg.max_seq, "position beyond max_seq");
    LlamaState s{};
    device_sync(m->dev);
    TH_HIP(hipMemcpy(&s, m->st, sizeof s, hipMemcpyDeviceToHost));
    s.pos = (int)pos;
    s.step = 0;
    TH_HIP(hipMemcpy(m->st, &s, sizeof s, hipMemcpyHostToDevice));
    llama_embed_current(m, m->dev->stream);
    llama_launch_step(m);
    aql_wait(m->dev);
    TH_API_END
}

int th_llama_generate(th_llama* m, int32_t token, size_t pos, size_t n_steps, int32_t* tokens_out, float* last_logits) {
    TH_API_BEGIN
    TH_REQUIRE(m && m->weights_ready, "model not initialised");
    TH_REQUIRE(token >= 0 && token < m->cfg.vocab, "token out of range");
    TH_REQUIRE(pos + n_steps <= (size_t)m->cfg.max_seq, "generation runs past max_seq");
    TH_REQUIRE(n_steps <= (size_t)m->max_steps, "too many steps");
    if (n_steps == 0) return TH_OK;
    LlamaState s{(int)pos, token, 0, 0};
    device_sync(m->dev);
    TH_HIP(hipMemcpy(m->st, &s, sizeof s, hipMemcpyHostToDevice));
    llama_embed_current(m, m->dev->stream);
    llama_launch_steps(m, n_steps);
    device_sync(m->dev);
    if (tokens_out) TH_HIP(hipMemcpy(tokens_out, m->history, n_steps * 4, hipMemcpyDeviceToHost));
    if (last_logits) TH_HIP(hipMemcpy(last_logits, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost));
    TH_API_END
}

int th_llama_generate_sampled(th_llama* m, th_sampler* smp, const int32_t* prompt, size_t n_prompt, size_t pos,
                              int32_t* tokens_out, size_t* n_out) {
    TH_API_BEGIN
    TH_REQUIRE(m && m->weights_ready, "model not initialised");
    TH_REQUIRE(smp && prompt && n_prompt > 0 && tokens_out && n_out, "null argument");
    const th_sampling_config& c = sampler_config(smp);
    TH_REQUIRE(pos + c.max_tokens <= (size_t)m->cfg.max_seq, "generation runs past max_seq");
    TH_REQUIRE(c.max_tokens <= (size_t)m->max_steps, "too many steps");
    for (size_t i = 0; i < n_prompt; i++) TH_REQUIRE(prompt[i] >= 0 && prompt[i] < m->cfg.vocab, "token out of range");
    *n_out = 0;
    std::vector<int32_t> past(prompt, prompt + n_prompt);  // generate() passes every token so far
    std::vector<float> logits((size_t)m->cfg.vocab);
    LlamaState st{(int)pos, prompt[n_prompt - 1], 0, 0};
    device_sync(m->dev);
    TH_HIP(hipMemcpy(m->st, &st, sizeof st, hipMemcpyHostToDevice));
    hipStream_t s = m->dev->stream;  // non-blocking: every copy goes on it and is waited for
    llama_embed_current(m, s);
    for (size_t i = 0; i < c.max_tokens; i++) {
        llama_launch_step(m);  // advances the device position; its greedy token is replaced below
        aql_wait(m->dev);
        TH_HIP(hipMemcpyAsync(logits.data(), m->logits, logits.size() * 4, hipMemcpyDeviceToHost, s));
        device_sync(m->dev);
        int32_t next = 0;
        check_status(th_sampler_sample(smp, logits.data(), logits.size(), past.data(), past.size(), &next));
        if (c.stop_token >= 0 && next == c.stop_token) break;  // sampling.rs:246-250
        past.push_back(next);
        tokens_out[(*n_out)++] = next;
        TH_HIP(hipMemcpyAsync(&m->st->token, &next, sizeof next, hipMemcpyHostToDevice, s));
        llama_embed_current(m, s);  // the sampled token replaces the greedy one the step embedded
        device_sync(m->dev);
    }
    TH_API_END
}

int th_llama_prefill(th_llama* m, const int32_t* tokens, size_t n, size_t pos, int32_t* next_token, float* last_logits) {
    TH_API_BEGIN
    TH_REQUIRE(m && m->weights_ready, "model not initialised");
    TH_REQUIRE(tokens && n > 0, "empty prompt");
    TH_REQUIRE(pos + n <= (size_t)m->cfg.max_seq, "prompt runs past max_seq");
    for (size_t i = 0; i < n; i++) TH_REQUIRE(tokens[i] >= 0 && tokens[i] < m->cfg.vocab, "token out of range");
    hipStream_t s = m->dev->stream;
    prefill_reserve(m, std::min(n, PREFILL_CHUNK));
    size_t rows = 0;
    for (size_t c0 = 0; c0 < n; c0 += PREFILL_CHUNK) {
        rows = std::min(PREFILL_CHUNK, n - c0);
        prefill_chunk(m, tokens + c0, rows, pos + c0);
        device_sync(m->dev);  // the token chunk is copied from the caller's memory
    }
    // the last row: final norm, LM head and argmax as a decode step would
    const th_llama_config& c = m->cfg;
    const int d = c.d_model;
    LlamaState st{(int)(pos + n - 1), tokens[n - 1], 0, 0};
    TH_HIP(hipMemcpyAsync(m->st, &st, sizeof st, hipMemcpyHostToDevice, s));
    TH_LAUNCH(prefill_last_row_kernel, dim3((unsigned)ceil_div((size_t)d / 16, (size_t)256)), dim3(256), 0, s,
                       m->pf_x + (rows - 1) * (size_t)d, d, m->x, m->ssq);
    TH_LAUNCH_CHECK();
    llama_lm_head_argmax(m, s);
    device_sync(m->dev);
    if (next_token) TH_HIP(hipMemcpy(next_token, m->history, 4, hipMemcpyDeviceToHost));
    if (last_logits) TH_HIP(hipMemcpy(last_logits, m->logits, (size_t)c.vocab * 4, hipMemcpyDeviceToHost));
    TH_API_END
}

int th_llama_time_prefill(th_llama* m, const int32_t* tokens, size_t n, size_t pos, float* ms) {
    TH_API_BEGIN
    TH_REQUIRE(m && ms, "null argument");
    check_status(th_llama_prefill(m, tokens, n, pos, nullptr, nullptr));  // warm: workspace, scratch
    TH_HIP(hipEventRecord(m->dev->ev_start, m->dev->stream));
    check_status(th_llama_prefill(m, tokens, n, pos, nullptr, nullptr));
    TH_HIP(hipEventRecord(m->dev->ev_stop, m->dev->stream));
    TH_HIP(hipEventSynchronize(m->dev->ev_stop));
    TH_HIP(hipEventElapsedTime(ms, m->dev->ev_start, m->dev->ev_stop));
    TH_API_END
}

int th_llama_time_steps(th_llama* m, int32_t token, size_t pos, size_t n_steps, float* ms) {
    TH_API_BEGIN
    TH_REQUIRE(m && m->weights_ready && ms, "model not initialised");
    TH_REQUIRE(token >= 0 && token < m->cfg.vocab, "token out of range");
    TH_REQUIRE(pos + n_steps <= (size_t)m->cfg.max_seq, "generation runs past max_seq");
    LlamaState s{(int)pos, token, 0, 0};
    device_sync(m->dev);
    TH_HIP(hipMemcpy(m->st, &s, sizeof s, hipMemcpyHostToDevice));
    llama_embed_current(m, m->dev->stream);
    llama_prepare_step(m);
    if (llama_use_aql(m)) {  // device clock stamps around the replays
        aql_stamp(m->dev, 0);
        llama_launch_steps(m, n_steps);
        aql_stamp(m->dev, 1);
        *ms = aql_stamped_ms(m->dev);
    } else {
        TH_HIP(hipEventRecord(m->dev->ev_start, m->dev->stream));
        llama_launch_steps(m, n_steps);
        TH_HIP(hipEventRecord(m->dev->ev_stop, m->dev->stream));
        TH_HIP(hipEventSynchronize(m->dev->ev_stop));
        TH_HIP(hipEventElapsedTime(ms, m->dev->ev_start, m->dev->ev_stop));
    }
    TH_API_END
}

}  // extern "C"
