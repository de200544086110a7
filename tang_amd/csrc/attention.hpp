// Split-K decode attention kernels (shared by th_kv_attention and the decode
// engine).  See attention.hip for the contract.
#pragma once

#include "common.hpp"
#include "ops.hpp"

namespace th {


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

// One (head, query, split) per workgroup of 256 threads; a split covers
// `subs` consecutive chunks of ATTN_SUB = 64 positions.  LPK = D/8 lanes share
// one key (eight elements each), so the block holds KPB = 256/LPK keys per
// pass and each thread KPT = 64/KPB keys of a chunk, whose K and V rows are
// all loaded before any arithmetic.  Chunks merge with the running max
// (online softmax).  Each split writes {m, l, acc[D]} to
// part[(qi*H + h)*n_splits + s]; the last split of a (query, head) to finish
// (counted on counters[qi*H + h], reset on exit) merges all splits in order:
//   out = sum_s acc_s e^{m_s-M} / sum_s l_s e^{m_s-M},  M = max_s m_s.
// cache_start_dev (optional): read cache_start from device memory, so one
// captured launch serves every decode position.
constexpr int ATTN_SUB = 64;

template <int D, typename CT, bool OUT_BF16>
__global__ __launch_bounds__(256) void attn_split_kernel(const float* __restrict__ q, const CT* __restrict__ kc,
                                                         const CT* __restrict__ vc, int cache_start, int n_heads,
                                                         int n_kv_heads, int subs, int n_splits,
                                                         float* __restrict__ part, int* __restrict__ counters,
                                                         void* __restrict__ out, const int* cache_start_dev) {
    constexpr int LPK = D / 8;
    constexpr int KPB = 256 / LPK;         // keys per block pass
    constexpr int KPT = ATTN_SUB / KPB;    // keys per thread per chunk
    static_assert(KPT >= 1 && KPT * KPB == ATTN_SUB, "chunk must be a multiple of the block pass");
    __shared__ float sc[ATTN_SUB];
    __shared__ float red[256];
    __shared__ float vacc[KPB][D + 1];
    __shared__ int s_last;
    const int h = blockIdx.x, qi = blockIdx.y, s = blockIdx.z;
    const int tid = threadIdx.x;
    const int slot = tid / LPK, e = tid % LPK;
    const int kv_dim = n_kv_heads * D;
    const int kv_h = h / (n_heads / n_kv_heads);
    if (cache_start_dev) cache_start = *cache_start_dev;
    const int attend = cache_start + qi + 1;
    const int split_len = subs * ATTN_SUB;
    const int j0 = s * split_len;
    const int len = max(0, min(split_len, attend - j0));
    float* recs = part + (size_t)(qi * n_heads + h) * n_splits * (D + 2);
    float* rec = recs + (size_t)s * (D + 2);
    if (len == 0) {
        for (int i = tid; i < D + 2; i += 256) st_coherent(&rec[i], i == 0 ? -INFINITY : 0.0f);
    } else {
        const float scale = 1.0f / sqrtf((float)D);
        float qv[8];
        {
            const float* qp = q + ((size_t)qi * n_heads + h) * D + e * 8;
#pragma unroll
            for (int i = 0; i < 8; i++) qv[i] = qp[i];
        }
        float m_run = -INFINITY, l_run = 0.0f;
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = 0.0f;
        const int nsub = (len + ATTN_SUB - 1) / ATTN_SUB;
        for (int c = 0; c < nsub; c++) {
            const int cj = j0 + c * ATTN_SUB;               // first position of the chunk
            const int clen = min(ATTN_SUB, len - c * ATTN_SUB);
            float kv[KPT][8], vv[KPT][8];
#pragma unroll
            for (int k = 0; k < KPT; k++) {
                const int jj = slot + k * KPB;
                const int row = cj + (jj < clen ? jj : 0);   // clamped: masked below
                load8<CT>(kc + (size_t)row * kv_dim + kv_h * D + e * 8, kv[k]);
                load8<CT>(vc + (size_t)row * kv_dim + kv_h * D + e * 8, vv[k]);
            }
#pragma unroll
            for (int k = 0; k < KPT; k++) {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) d += qv[i] * kv[k][i];
#pragma unroll
                for (int o = LPK / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, 64);
                const int jj = slot + k * KPB;
                if (e == 0) sc[jj] = jj < clen ? d * scale : -INFINITY;
            }
            __syncthreads();
            float mx = -INFINITY;
            if (tid < ATTN_SUB) mx = sc[tid];
            mx = block_max_256(mx, red);
            const float m_new = fmaxf(m_run, mx);
            const float rescale = expf(m_run - m_new);  // 0 on the first chunk
            float lsum = 0.0f;
            if (tid < ATTN_SUB) lsum = tid < clen ? expf(sc[tid] - m_new) : 0.0f;
            lsum = block_sum_256(lsum, red);
            l_run = l_run * rescale + lsum;
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i] *= rescale;
#pragma unroll
            for (int k = 0; k < KPT; k++) {
                const int jj = slot + k * KPB;
                const float p = jj < clen ? expf(sc[jj] - m_new) : 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) acc[i] = __builtin_fmaf(p, vv[k][i], acc[i]);
            }
            m_run = m_new;
            __syncthreads();  // sc is rewritten by the next chunk
        }
#pragma unroll
        for (int i = 0; i < 8; i++) vacc[slot][e * 8 + i] = acc[i];
        __syncthreads();
        for (int d = tid; d < D; d += 256) {
            float v = 0.0f;
            for (int k = 0; k < KPB; k++) v += vacc[k][d];
            st_coherent(&rec[2 + d], v);
        }
        if (tid == 0) { st_coherent(&rec[0], m_run); st_coherent(&rec[1], l_run); }
    }
    // publish this split; the last one to arrive merges
    if (!last_arrival(&counters[qi * n_heads + h], n_splits, &s_last)) return;
    // stage every split record into LDS: independent loads, one latency round
    extern __shared__ float recl[];  // [n_splits][D + 2]
    const int total = n_splits * (D + 2);
    ld_coherent_to_lds(recs, total, recl, tid);
    __syncthreads();
    float mloc = -INFINITY;
    for (int i = tid; i < n_splits; i += 256) mloc = fmaxf(mloc, recl[(size_t)i * (D + 2)]);
    const float M = block_max_256(mloc, red);
    float lloc = 0.0f;
    __shared__ float wts[256];
    for (int i = tid; i < n_splits; i += 256) {
        const float m = recl[(size_t)i * (D + 2)];
        const float w = m == -INFINITY ? 0.0f : expf(m - M);
        wts[i] = w;
        lloc += w * recl[(size_t)i * (D + 2) + 1];
    }
    const float L = block_sum_256(lloc, red);  // its barriers also publish wts
    const float inv = 1.0f / L;
    for (int d = tid; d < D; d += 256) {
        float a = 0.0f;
        for (int i = 0; i < n_splits; i++) a += recl[(size_t)i * (D + 2) + 2 + d] * wts[i];
        const size_t o = ((size_t)qi * n_heads + h) * D + d;
        if (OUT_BF16) ((uint16_t*)out)[o] = f32_to_bf16_rne(a * inv);
        else ((float*)out)[o] = a * inv;
    }
}

// Decode attention (one query, f16 cache), as attn_split_kernel with a single
// chunk of at most SPL positions per workgroup: every K and V row of the
// split is loaded in one round (raw 16-byte pieces, converted at use), then
// scores, one softmax pass and P.V; records and the last-arrival merge as
// above.  The attended length is read on the device (the launch is replayed
// for every position); splits past it only write an empty record.  (Sharing
// the length evenly over all n_splits workgroups was measured slower: more
// workgroups each paying the record and merge overhead.)
template <int D, int SPL, bool OUT_BF16>
__global__ __launch_bounds__(256) void attn_decode_kernel(const float* __restrict__ q, const _Float16* __restrict__ kc,
                                                          const _Float16* __restrict__ vc, int n_heads, int n_kv_heads,
                                                          int n_splits, float* __restrict__ part,
                                                          int* __restrict__ counters, void* __restrict__ out,
                                                          const int* __restrict__ cache_start_dev) {
    constexpr int LPK = D / 8;           // lanes per key (eight elements each)
    constexpr int KPB = 256 / LPK;       // keys per block pass
    constexpr int KPT = SPL / KPB;       // keys per thread
    static_assert(KPT >= 1 && KPT * KPB == SPL && LPK <= 64 && 64 % LPK == 0, "bad split shape");
    __shared__ float red[2][4];
    __shared__ float vacc[KPB][D + 1];
    __shared__ int s_last;
    const int h = blockIdx.x, s = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slot = tid / LPK, e = tid % LPK;
    const int kv_dim = n_kv_heads * D;
    const int kv_h = h / (n_heads / n_kv_heads);
    const int attend = *cache_start_dev + 1;  // <= n_splits * SPL (checked by the host)
    const int j0 = s * SPL;
    const int len = max(0, min(SPL, attend - j0));
    float* recs = part + (size_t)h * n_splits * (D + 2);
    float* rec = recs + (size_t)s * (D + 2);
    if (len == 0) {
        for (int i = tid; i < D + 2; i += 256) st_coherent(&rec[i], i == 0 ? -INFINITY : 0.0f);
    } else {
        // Issue order = use order (loads complete in order): q, every K row,
        // then every V row, so the scores start while V is still streaming.
        float qv[8];
        {
            const float4 a = *(const float4*)(q + (size_t)h * D + e * 8);
            const float4 b = *(const float4*)(q + (size_t)h * D + e * 8 + 4);
            qv[0] = a.x; qv[1] = a.y; qv[2] = a.z; qv[3] = a.w; qv[4] = b.x; qv[5] = b.y; qv[6] = b.z; qv[7] = b.w;
        }
        // Rows past the split re-read the last row (clamped: no branch around
        // the loads, which would make the first use wait for all of them;
        // masked below).  Buffer loads with an out-of-range resource instead
        // of the clamp measured slower.
        uint4 kr[KPT], vr[KPT];
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const int row = j0 + min(slot + k * KPB, len - 1);
            kr[k] = *(const uint4*)(kc + (size_t)row * kv_dim + kv_h * D + e * 8);
        }
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const int row = j0 + min(slot + k * KPB, len - 1);
            vr[k] = *(const uint4*)(vc + (size_t)row * kv_dim + kv_h * D + e * 8);
        }
        const float scale = 1.0f / sqrtf((float)D);
        float sc[KPT];
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const uint32_t w[4] = {kr[k].x, kr[k].y, kr[k].z, kr[k].w};
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                d += qv[2 * i] * (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xFFFF));
                d += qv[2 * i + 1] * (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
            }
#pragma unroll
            for (int o = LPK / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, 64);
            sc[k] = slot + k * KPB < len ? d * scale : -INFINITY;
            mx = fmaxf(mx, sc[k]);
        }
        // block max: the LPK lanes of a key hold equal values
#pragma unroll
        for (int o = LPK; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        if (lane == 0) red[0][wave] = mx;
        __syncthreads();
        const float M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = 0.0f;
        float lsum = 0.0f;
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const float p = expf(sc[k] - M);  // 0 for masked keys
            lsum += p;
            const uint32_t w[4] = {vr[k].x, vr[k].y, vr[k].z, vr[k].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[2 * i] = __builtin_fmaf(p, (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xFFFF)), acc[2 * i]);
                acc[2 * i + 1] = __builtin_fmaf(p, (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16)), acc[2 * i + 1]);
            }
        }
#pragma unroll
        for (int o = LPK; o < 64; o <<= 1) lsum += __shfl_xor(lsum, o, 64);
        if (lane == 0) red[1][wave] = lsum;
#pragma unroll
        for (int i = 0; i < 8; i++) vacc[slot][e * 8 + i] = acc[i];
        __syncthreads();
        for (int d = tid; d < D; d += 256) {
            float v = 0.0f;
#pragma unroll
            for (int k = 0; k < KPB; k++) v += vacc[k][d];
            st_coherent(&rec[2 + d], v);
        }
        if (tid == 0) {
            st_coherent(&rec[0], M);
            st_coherent(&rec[1], (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]));
        }
    }
    if (!last_arrival(&counters[h], n_splits, &s_last)) return;
    extern __shared__ float recl[];  // [n_splits][D + 2]
    __shared__ float redm[256];
    const int total = n_splits * (D + 2);
    ld_coherent_to_lds(recs, total, recl, tid);
    __syncthreads();
    float mloc = -INFINITY;
    for (int i = tid; i < n_splits; i += 256) mloc = fmaxf(mloc, recl[(size_t)i * (D + 2)]);
    const float Mx = block_max_256(mloc, redm);
    float lloc = 0.0f;
    __shared__ float wts[256];
    for (int i = tid; i < n_splits; i += 256) {
        const float m = recl[(size_t)i * (D + 2)];
        const float w = m == -INFINITY ? 0.0f : expf(m - Mx);
        wts[i] = w;
        lloc += w * recl[(size_t)i * (D + 2) + 1];
    }
    const float L = block_sum_256(lloc, redm);  // its barriers also publish wts
    const float inv = 1.0f / L;
    for (int d = tid; d < D; d += 256) {
        float a = 0.0f;
        for (int i = 0; i < n_splits; i++) a += recl[(size_t)i * (D + 2) + 2 + d] * wts[i];
        const size_t o = (size_t)h * D + d;
        if (OUT_BF16) ((uint16_t*)out)[o] = f32_to_bf16_rne(a * inv);
        else ((float*)out)[o] = a * inv;
    }
}

// Dynamic LDS of the split kernel: the merging split stages all records.
inline size_t attn_merge_lds(int n_splits, int head_dim) { return (size_t)n_splits * (head_dim + 2) * sizeof(float); }

// counters: q_len*n_heads ints, zero on entry and on return.
template <int D, bool OUT_BF16>
inline void launch_attn_split_d(const float* q, const void* kc, const void* vc, bool f16, int cache_start, int q_len,
                                int n_heads, int n_kv_heads, int subs, int n_splits, float* part, int* counters,
                                void* out, const int* cache_start_dev, hipStream_t s) {
    dim3 grid((unsigned)n_heads, (unsigned)q_len, (unsigned)n_splits);
    const size_t lds = attn_merge_lds(n_splits, D);
    TH_REQUIRE(lds <= 64 * 1024, "too many attention splits for the LDS merge");
    if (lds > 48 * 1024) {
        TH_HIP(hipFuncSetAttribute((const void*)attn_split_kernel<D, _Float16, OUT_BF16>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        TH_HIP(hipFuncSetAttribute((const void*)attn_split_kernel<D, float, OUT_BF16>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    }
    if (f16)
        hipLaunchKernelGGL((attn_split_kernel<D, _Float16, OUT_BF16>), grid, dim3(256), lds, s, q, (const _Float16*)kc,
                           (const _Float16*)vc, cache_start, n_heads, n_kv_heads, subs, n_splits, part, counters, out,
                           cache_start_dev);
    else
        hipLaunchKernelGGL((attn_split_kernel<D, float, OUT_BF16>), grid, dim3(256), lds, s, q, (const float*)kc,
                           (const float*)vc, cache_start, n_heads, n_kv_heads, subs, n_splits, part, counters, out,
                           cache_start_dev);
    TH_LAUNCH_CHECK();
}

// subs: 64-position chunks per split; n_splits*(head_dim+2) floats must fit
// the merge's LDS (64 KiB).
template <bool OUT_BF16>
inline void launch_attn_split(const float* q, const void* kc, const void* vc, bool f16, int cache_start, int q_len,
                              int n_heads, int n_kv_heads, int head_dim, int subs, int n_splits, float* part,
                              int* counters, void* out, const int* cache_start_dev, hipStream_t s) {
    TH_REQUIRE(subs >= 1 && n_splits >= 1 && n_splits <= 256, "attention split count out of range");
    switch (head_dim) {
        case 64: launch_attn_split_d<64, OUT_BF16>(q, kc, vc, f16, cache_start, q_len, n_heads, n_kv_heads, subs, n_splits, part, counters, out, cache_start_dev, s); break;
        case 128: launch_attn_split_d<128, OUT_BF16>(q, kc, vc, f16, cache_start, q_len, n_heads, n_kv_heads, subs, n_splits, part, counters, out, cache_start_dev, s); break;
        case 256: launch_attn_split_d<256, OUT_BF16>(q, kc, vc, f16, cache_start, q_len, n_heads, n_kv_heads, subs, n_splits, part, counters, out, cache_start_dev, s); break;
        default: throw Error(TH_ERR_INVALID, "launch_attn_split: unsupported head_dim");
    }
}

// Decode attention for the engine: one query, f16 cache, SPL positions per
// split; counters (n_heads ints) zero on entry and on return.
template <int SPL, bool OUT_BF16>
inline void launch_attn_decode(const float* q, const _Float16* kc, const _Float16* vc, int n_heads, int n_kv_heads,
                               int head_dim, int n_splits, float* part, int* counters, void* out,
                               const int* cache_start_dev, hipStream_t s) {
    TH_REQUIRE(n_splits >= 1 && n_splits <= 256, "attention split count out of range");
    const dim3 grid((unsigned)n_heads, 1, (unsigned)n_splits);
    const size_t lds = attn_merge_lds(n_splits, head_dim);
    TH_REQUIRE(lds <= 48 * 1024, "too many attention splits for the LDS merge");
    switch (head_dim) {
        case 64: hipLaunchKernelGGL((attn_decode_kernel<64, SPL, OUT_BF16>), grid, dim3(256), lds, s, q, kc, vc, n_heads, n_kv_heads, n_splits, part, counters, out, cache_start_dev); break;
        case 128: hipLaunchKernelGGL((attn_decode_kernel<128, SPL, OUT_BF16>), grid, dim3(256), lds, s, q, kc, vc, n_heads, n_kv_heads, n_splits, part, counters, out, cache_start_dev); break;
        case 256: hipLaunchKernelGGL((attn_decode_kernel<256, SPL, OUT_BF16>), grid, dim3(256), lds, s, q, kc, vc, n_heads, n_kv_heads, n_splits, part, counters, out, cache_start_dev); break;
        default: throw Error(TH_ERR_INVALID, "launch_attn_decode: unsupported head_dim");
    }
    TH_LAUNCH_CHECK();
}

void launch_kv_attention(const float* q, const void* kc, const void* vc, bool f16, size_t cache_start, size_t q_len,
                         size_t n_heads, size_t n_kv_heads, size_t head_dim, float* out, hipStream_t s,
                         th_device* dev);

}  // namespace th
