// Split-K decode attention kernels (shared by th_kv_attention and the decode
// engine).  See attention.hip for the contract.
#pragma once

#include "common.hpp"
#include "ops.hpp"

namespace th {

// Chunk of cache positions per workgroup: small enough that the grid covers
// the chip about twice.
inline int attn_chunk_for(size_t max_len, size_t n_rows, int num_cus) {
    int chunk = 256;
    while (chunk > 32 && n_rows * ((max_len + chunk - 1) / chunk) < (size_t)num_cus * 2) chunk >>= 1;
    return chunk;
}

template <typename CT>
__device__ __forceinline__ void load8(const CT* p, float v[8]);
template <>
__device__ __forceinline__ void load8<_Float16>(const _Float16* p, float v[8]) {
    const uint4 a = *(const uint4*)p;
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xFFFF));
        v[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
    }
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float v[8]) {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// One (head, query, chunk) per workgroup of 256 threads.  LPK = D/8 lanes
// share one key (eight elements each); the block walks 4*64/LPK keys per step.
// part[(qi*H + h)*n_splits + s] = {m, l, acc[D]}.
// cache_start_dev (optional): read cache_start from device memory instead, so
// one captured launch serves every decode position.
template <int D, typename CT>
__global__ __launch_bounds__(256) void attn_split_kernel(const float* __restrict__ q, const CT* __restrict__ kc,
                                                         const CT* __restrict__ vc, int cache_start, int n_heads,
                                                         int n_kv_heads, int chunk, int n_splits,
                                                         float* __restrict__ part, const int* cache_start_dev = nullptr) {
    constexpr int LPK = D / 8;
    constexpr int KPB = 256 / LPK;  // keys per block step
    __shared__ float sc[256];
    __shared__ float red[256];
    __shared__ float vacc[KPB][D + 1];
    const int h = blockIdx.x, qi = blockIdx.y, s = blockIdx.z;
    const int tid = threadIdx.x;
    const int slot = tid / LPK, e = tid % LPK;
    const int kv_dim = n_kv_heads * D;
    const int kv_h = h / (n_heads / n_kv_heads);
    if (cache_start_dev) cache_start = *cache_start_dev;
    const int attend = cache_start + qi + 1;
    const int j0 = s * chunk;
    const int len = max(0, min(chunk, attend - j0));
    float* rec = part + ((size_t)(qi * n_heads + h) * n_splits + s) * (D + 2);
    if (len == 0) {
        for (int i = tid; i < D + 2; i += 256) rec[i] = i == 0 ? -INFINITY : 0.0f;
        return;
    }
    const float scale = 1.0f / sqrtf((float)D);
    float qv[8];
    {
        const float* qp = q + ((size_t)qi * n_heads + h) * D + e * 8;
#pragma unroll
        for (int i = 0; i < 8; i++) qv[i] = qp[i];
    }
    const CT* kbase = kc + (size_t)j0 * kv_dim + kv_h * D + e * 8;
    const CT* vbase = vc + (size_t)j0 * kv_dim + kv_h * D + e * 8;
    // scores
    for (int jj = slot; jj < len; jj += KPB) {
        float kv[8];
        load8<CT>(kbase + (size_t)jj * kv_dim, kv);
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) d += qv[i] * kv[i];
#pragma unroll
        for (int o = LPK / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, 64);
        if (e == 0) sc[jj] = d * scale;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int i = tid; i < len; i += 256) mx = fmaxf(mx, sc[i]);
    mx = block_max_256(mx, red);
    float l = 0.0f;
    for (int i = tid; i < len; i += 256) {
        const float p = expf(sc[i] - mx);
        sc[i] = p;
        l += p;
    }
    l = block_sum_256(l, red);  // includes the barrier that publishes sc
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.0f;
    for (int jj = slot; jj < len; jj += KPB) {
        float vv[8];
        load8<CT>(vbase + (size_t)jj * kv_dim, vv);
        const float p = sc[jj];
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = __builtin_fmaf(p, vv[i], acc[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) vacc[slot][e * 8 + i] = acc[i];
    __syncthreads();
    for (int d = tid; d < D; d += 256) {
        float v = 0.0f;
        for (int k = 0; k < KPB; k++) v += vacc[k][d];
        rec[2 + d] = v;
    }
    if (tid == 0) { rec[0] = mx; rec[1] = l; }
}

// Merge the chunk records of one (head, query): out = sum acc_s e^{m_s-M} / sum l_s e^{m_s-M}.
template <bool OUT_BF16 = false>
__global__ void attn_combine_kernel(const float* __restrict__ part, int n_heads, int D, int n_splits,
                                    void* __restrict__ out) {
    const int h = blockIdx.x, qi = blockIdx.y;
    const float* recs = part + (size_t)(qi * n_heads + h) * n_splits * (D + 2);
    float M = -INFINITY;
    for (int s = 0; s < n_splits; s++) M = fmaxf(M, recs[(size_t)s * (D + 2)]);
    float L = 0.0f;
    for (int s = 0; s < n_splits; s++) {
        const float m = recs[(size_t)s * (D + 2)];
        if (m != -INFINITY) L += recs[(size_t)s * (D + 2) + 1] * expf(m - M);
    }
    const float inv = 1.0f / L;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float a = 0.0f;
        for (int s = 0; s < n_splits; s++) {
            const float m = recs[(size_t)s * (D + 2)];
            if (m != -INFINITY) a += recs[(size_t)s * (D + 2) + 2 + d] * expf(m - M);
        }
        const size_t o = ((size_t)qi * n_heads + h) * D + d;
        if (OUT_BF16) ((uint16_t*)out)[o] = f32_to_bf16_rne(a * inv);
        else ((float*)out)[o] = a * inv;
    }
}

template <int D>
inline void launch_attn_split_d(const float* q, const void* kc, const void* vc, bool f16, int cache_start, int q_len,
                                int n_heads, int n_kv_heads, int chunk, int n_splits, float* part, float* out,
                                hipStream_t s) {
    dim3 grid((unsigned)n_heads, (unsigned)q_len, (unsigned)n_splits);
    if (f16)
        hipLaunchKernelGGL((attn_split_kernel<D, _Float16>), grid, dim3(256), 0, s, q, (const _Float16*)kc,
                           (const _Float16*)vc, cache_start, n_heads, n_kv_heads, chunk, n_splits, part);
    else
        hipLaunchKernelGGL((attn_split_kernel<D, float>), grid, dim3(256), 0, s, q, (const float*)kc, (const float*)vc,
                           cache_start, n_heads, n_kv_heads, chunk, n_splits, part);
    TH_LAUNCH_CHECK();
    hipLaunchKernelGGL(attn_combine_kernel<false>, dim3((unsigned)n_heads, (unsigned)q_len), dim3(D < 256 ? D : 256), 0,
                       s, part, n_heads, D, n_splits, (void*)out);
    TH_LAUNCH_CHECK();
}

inline void launch_attn_split(const float* q, const void* kc, const void* vc, bool f16, int cache_start, int q_len,
                              int n_heads, int n_kv_heads, int head_dim, int chunk, int n_splits, float* part,
                              float* out, hipStream_t s) {
    TH_REQUIRE(chunk <= 256, "attention chunk above 256");
    switch (head_dim) {
        case 64: launch_attn_split_d<64>(q, kc, vc, f16, cache_start, q_len, n_heads, n_kv_heads, chunk, n_splits, part, out, s); break;
        case 128: launch_attn_split_d<128>(q, kc, vc, f16, cache_start, q_len, n_heads, n_kv_heads, chunk, n_splits, part, out, s); break;
        case 256: launch_attn_split_d<256>(q, kc, vc, f16, cache_start, q_len, n_heads, n_kv_heads, chunk, n_splits, part, out, s); break;
        default: throw Error(TH_ERR_INVALID, "launch_attn_split: unsupported head_dim");
    }
}

void launch_kv_attention(const float* q, const void* kc, const void* vc, bool f16, size_t cache_start, size_t q_len,
                         size_t n_heads, size_t n_kv_heads, size_t head_dim, float* out, hipStream_t s,
                         th_device* dev);

}  // namespace th
