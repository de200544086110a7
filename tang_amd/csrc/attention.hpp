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

// Causal prefill attention on MFMA (f16 cache, bf16 output), flash style:
// one workgroup = 64 consecutive queries of one head, each wave 16 of them;
// key blocks of 64 stream through LDS (K row-major, V transposed), with
// online softmax in registers.  Both products run transposed so that no
// operand needs a cross-lane shuffle:
//   S^T = K . Q^T   (A = K rows from LDS, B = the wave's queries, kept in
//                    registers as f16, pre-scaled by 1/sqrt(D)); lane (g, r)
//                    then holds the scores of query r for keys 4g..4g+3 of
//                    each 16-key tile;
//   O^T += V^T . P^T (A = V^T rows from LDS, B = those scores as f16); the
//                    MFMA's k index j of lane group g stands for key 4g+j of
//                    the first tile of a 32-key chunk (j < 4) or 4g+j-4 of
//                    the second, the same order in A and B; lane (g, r)
//                    accumulates dims 4g..4g+3 of each 16-dim tile for query r,
//                    so the softmax rescale uses the lane's own query.
// Query i (0 <= i < n) sits at position pos0 + i and attends keys
// 0..pos0+i (kv_attention, cpu.rs:257-315).  K/V rows are read clamped to the
// last valid key so masked lanes only ever see finite values.
typedef _Float16 attn_f16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ uint32_t attn_pack_h2(float a, float b) {  // two f16, a in the low half
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}
typedef float attn_f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t attn_u32x4_t __attribute__((ext_vector_type(4)));  // (uint4 arrays captured by the
                                                                    // staging lambdas went to scratch)

template <int D, bool XP>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const float* __restrict__ q, int ldq,
                                                           const _Float16* __restrict__ kc,
                                                           const _Float16* __restrict__ vc, int n_heads,
                                                           int n_kv_heads, int pos0, int n,
                                                           uint16_t* __restrict__ out, int ldo,
                                                           int* __restrict__ xexp) {
    constexpr int KB = 64;          // keys per block
    constexpr int KS = D + 8;       // Ks row stride (halves)
    constexpr int VS = KB + 8;      // Vt row stride (halves)
    constexpr int NDC = D / 32;     // 32-dim k-steps of S
    constexpr int NDT = D / 16;     // 16-dim tiles of O
    constexpr int CPR = D / 8;      // 16-byte chunks per K/V row
    constexpr int KLD = KB * CPR / 256;        // K chunks per thread per block
    constexpr int VLD = (KB / 2) * CPR / 256;  // V chunk pairs per thread per block
    static_assert(KLD >= 1 && VLD >= 1 && NDC >= 1, "head_dim must be 64 or 128");
    __shared__ __align__(16) _Float16 Ks[KB * KS];
    __shared__ __align__(16) _Float16 Vt[D * VS];
    const int h = blockIdx.y, kv_h = h / (n_heads / n_kv_heads), kv_dim = n_kv_heads * D;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r = lane & 15;
    const int qi = blockIdx.x * 64 + wave * 16 + r;  // this lane's query
    const int qpos = pos0 + qi;
    const int last_key = pos0 + n - 1;
    const float scale = 1.0f / sqrtf((float)D);

    attn_f16x8_t qb[NDC];
    {
        const float* qp = q + (size_t)min(qi, n - 1) * ldq + h * D + 8 * g;
#pragma unroll
        for (int dc = 0; dc < NDC; dc++) {
            const float4 a = *(const float4*)(qp + dc * 32);
            const float4 b = *(const float4*)(qp + dc * 32 + 4);
            qb[dc] = attn_f16x8_t{(_Float16)(a.x * scale), (_Float16)(a.y * scale), (_Float16)(a.z * scale),
                                  (_Float16)(a.w * scale), (_Float16)(b.x * scale), (_Float16)(b.y * scale),
                                  (_Float16)(b.z * scale), (_Float16)(b.w * scale)};
        }
    }
    attn_f32x4_t o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) o[dt] = attn_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;
    const int qlast = min((int)blockIdx.x * 64 + 63, n - 1);
    const int nkb = (pos0 + qlast) / KB + 1;

    attn_u32x4_t kr[KLD], vr[VLD][2];
    auto gload = [&](int kb) {
        const int key0 = kb * KB;
#pragma unroll
        for (int p = 0; p < KLD; p++) {
            const int idx = tid + 256 * p, key = idx / CPR, c = idx % CPR;
            const size_t row = (size_t)min(key0 + key, last_key);
            kr[p] = *(const attn_u32x4_t*)(kc + row * kv_dim + kv_h * D + c * 8);
        }
#pragma unroll
        for (int p = 0; p < VLD; p++) {
            const int idx = tid + 256 * p, c = idx % CPR, kk = idx / CPR;
            const size_t r0 = (size_t)min(key0 + 2 * kk, last_key), r1 = (size_t)min(key0 + 2 * kk + 1, last_key);
            vr[p][0] = *(const attn_u32x4_t*)(vc + r0 * kv_dim + kv_h * D + c * 8);
            vr[p][1] = *(const attn_u32x4_t*)(vc + r1 * kv_dim + kv_h * D + c * 8);
        }
    };
    // Vt column swizzle: XOR of the key index's bits 2-4 with the dim's bits
    // 3-5 keeps 4-key groups contiguous and spreads the transposing writes
    // over the banks.
    auto vcol = [](int dim, int key) { return key ^ (((dim >> 3) & 7) << 2); };
    auto lstore = [&]() {
#pragma unroll
        for (int p = 0; p < KLD; p++) {
            const int idx = tid + 256 * p, key = idx / CPR, c = idx % CPR;
            *(attn_u32x4_t*)&Ks[key * KS + c * 8] = kr[p];
        }
#pragma unroll
        for (int p = 0; p < VLD; p++) {
            const int idx = tid + 256 * p, c = idx % CPR, kk = idx / CPR;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int dim = c * 8 + i;
                const uint32_t wa = vr[p][0][i >> 1], wb = vr[p][1][i >> 1];
                const uint32_t lo = (i & 1) ? (wa >> 16) : (wa & 0xFFFFu);
                const uint32_t hi = (i & 1) ? (wb >> 16) : (wb & 0xFFFFu);
                *(uint32_t*)&Vt[dim * VS + vcol(dim, 2 * kk)] = lo | (hi << 16);
            }
        }
    };

    gload(0);
    for (int kb = 0; kb < nkb; kb++) {
        __syncthreads();  // the previous block's LDS reads are done
        lstore();
        __syncthreads();
        if (kb + 1 < nkb) gload(kb + 1);  // next block in flight during this one's math
        attn_f32x4_t sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            sc[kt] = attn_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int dc = 0; dc < NDC; dc++) {
                const attn_f16x8_t a = *(const attn_f16x8_t*)&Ks[(kt * 16 + r) * KS + dc * 32 + 8 * g];
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qb[dc], sc[kt], 0, 0, 0);
            }
        }
        float bm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = kb * KB + kt * 16 + 4 * g + i;
                if (key > qpos) sc[kt][i] = -INFINITY;
                bm = fmaxf(bm, sc[kt][i]);
            }
        bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        const float mn = fmaxf(m_run, bm);  // finite: key 0 is in block 0 for every query
        const float alpha = expf(m_run - mn);
        float ps = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float p = expf(sc[kt][i] - mn);
                sc[kt][i] = p;
                ps += p;
            }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        l_run = l_run * alpha + ps;
        m_run = mn;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) o[dt] *= alpha;
#pragma unroll
        for (int kc2 = 0; kc2 < 2; kc2++) {
            const attn_f16x8_t pb = {(_Float16)sc[2 * kc2][0], (_Float16)sc[2 * kc2][1], (_Float16)sc[2 * kc2][2],
                                     (_Float16)sc[2 * kc2][3], (_Float16)sc[2 * kc2 + 1][0],
                                     (_Float16)sc[2 * kc2 + 1][1], (_Float16)sc[2 * kc2 + 1][2],
                                     (_Float16)sc[2 * kc2 + 1][3]};
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                const int dim = dt * 16 + r, c0 = kc2 * 32 + 4 * g;
                const uint2 lo = *(const uint2*)&Vt[dim * VS + vcol(dim, c0)];
                const uint2 hi = *(const uint2*)&Vt[dim * VS + vcol(dim, c0 + 16)];
                const attn_f16x8_t a = __builtin_bit_cast(attn_f16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, o[dt], 0, 0, 0);
            }
        }
    }
    const float inv = 1.0f / l_run;
    if constexpr (XP) {
        // the O projection's prepared layout: the 8-dim chunk of lane groups
        // g (even) and g+1 goes out from the even lane as (x0,x4,x1,x5,...).
        // Row exponent 0: an output row averages V rows of the f16 cache, so
        // it stays within f16's range.
        if (h == 0 && g == 0 && qi < n) xexp[qi] = 0;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            float y[4], z[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                y[i] = __uint_as_float((uint32_t)f32_to_bf16_rne(o[dt][i] * inv) << 16);
                z[i] = __shfl_xor(y[i], 16, 64);
            }
            if (qi < n && (g & 1) == 0) {
                uint16_t* op = out + (size_t)qi * ldo + h * D + dt * 16 + 4 * g;
                *(uint4*)op = make_uint4(attn_pack_h2(y[0], z[0]), attn_pack_h2(y[1], z[1]),
                                         attn_pack_h2(y[2], z[2]), attn_pack_h2(y[3], z[3]));
            }
        }
    } else if (qi < n) {
        uint16_t* op = out + (size_t)qi * ldo + h * D + 4 * g;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const uint32_t w0 = f32_to_bf16_rne(o[dt][0] * inv) | ((uint32_t)f32_to_bf16_rne(o[dt][1] * inv) << 16);
            const uint32_t w1 = f32_to_bf16_rne(o[dt][2] * inv) | ((uint32_t)f32_to_bf16_rne(o[dt][3] * inv) << 16);
            *(uint2*)(op + dt * 16) = make_uint2(w0, w1);
        }
    }
}

// out: bf16 rows of ldo, or (xp) the MFMA GEMM's prepared f16 layout (rows
// of ldo >= n_heads * head_dim, which must then be the consumer's Kp) with
// row exponents xexp.
inline void launch_attn_prefill(const float* q, int ldq, const _Float16* kc, const _Float16* vc, int n_heads,
                                int n_kv_heads, int head_dim, int pos0, int n, uint16_t* out, int ldo, bool xp,
                                int* xexp, hipStream_t s) {
    TH_REQUIRE(n >= 1 && n_kv_heads >= 1 && n_heads % n_kv_heads == 0, "prefill attention: bad shape");
    const dim3 grid((unsigned)ceil_div((size_t)n, (size_t)64), (unsigned)n_heads);
    switch (head_dim * 2 + (xp ? 1 : 0)) {
        case 128: TH_LAUNCH((attn_prefill_kernel<64, false>), grid, dim3(256), 0, s, q, ldq, kc, vc, n_heads, n_kv_heads, pos0, n, out, ldo, xexp); break;
        case 129: TH_LAUNCH((attn_prefill_kernel<64, true>), grid, dim3(256), 0, s, q, ldq, kc, vc, n_heads, n_kv_heads, pos0, n, out, ldo, xexp); break;
        case 256: TH_LAUNCH((attn_prefill_kernel<128, false>), grid, dim3(256), 0, s, q, ldq, kc, vc, n_heads, n_kv_heads, pos0, n, out, ldo, xexp); break;
        case 257: TH_LAUNCH((attn_prefill_kernel<128, true>), grid, dim3(256), 0, s, q, ldq, kc, vc, n_heads, n_kv_heads, pos0, n, out, ldo, xexp); break;
        default: throw Error(TH_ERR_INVALID, "prefill attention: head_dim must be 64 or 128");
    }
    TH_LAUNCH_CHECK();
}

// Decode attention (one query, f16 cache), as attn_split_kernel with a single
// chunk of at most SPL positions per workgroup: every K and V row of the
// split is loaded in one round (raw 16-byte pieces, converted at use), then
// scores, one softmax pass and P.V; records and the last-arrival merge as
// above.  The attended length is read on the device (the launch is replayed
// for every position); splits past it only write an empty record.  (Sharing
// the length evenly over all n_splits workgroups was measured slower: more
// workgroups each paying the record and merge overhead.)
// EVEN: the attended length is shared evenly over the n_splits workgroups
// (ceil(attend / n_splits) <= SPL positions each, so every workgroup of the
// launch streams the same bytes) instead of fixed SPL-position chunks.
template <int D, int SPL, bool OUT_BF16, int NT, bool EVEN = false>
__global__ __launch_bounds__(NT) void attn_decode_kernel(const float* __restrict__ q, const _Float16* __restrict__ kc,
                                                          const _Float16* __restrict__ vc, int n_heads, int n_kv_heads,
                                                          int n_splits, float* __restrict__ part,
                                                          int* __restrict__ counters, void* __restrict__ out,
                                                          const int* __restrict__ cache_start_dev) {
    constexpr int LPK = D / 8;           // lanes per key (eight elements each)
    constexpr int NWV = NT / 64;         // waves
    constexpr int KPB = NT / LPK;        // keys per block pass
    constexpr int KPT = SPL / KPB;       // keys per thread
    static_assert(KPT >= 1 && KPT * KPB == SPL && LPK <= 64 && 64 % LPK == 0, "bad split shape");
    __shared__ float red[2][NWV];
    __shared__ float vacc[KPB][D + 1];
    __shared__ int s_last;
    const int h = blockIdx.x, s = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slot = tid / LPK, e = tid % LPK;
    const int kv_dim = n_kv_heads * D;
    const int kv_h = h / (n_heads / n_kv_heads);
    const int attend = *cache_start_dev + 1;  // <= n_splits * SPL (checked by the host)
    const int per = EVEN ? (attend + n_splits - 1) / n_splits : SPL;  // <= SPL
    const int j0 = s * per;
    const int len = max(0, min(per, attend - j0));
    float* recs = part + (size_t)h * n_splits * (D + 2);
    float* rec = recs + (size_t)s * (D + 2);
    if (len == 0) {
        for (int i = tid; i < D + 2; i += NT) st_coherent(&rec[i], i == 0 ? -INFINITY : 0.0f);
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
            float d = 0.0f;  // mixed-precision FMAs: the f16 operand is read in place
#pragma unroll
            for (int i = 0; i < 4; i++) {
                d = __builtin_fmaf(qv[2 * i], (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xFFFF)), d);
                d = __builtin_fmaf(qv[2 * i + 1], (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16)), d);
            }
            d = group_sum<LPK>(d);
            sc[k] = slot + k * KPB < len ? d * scale : -INFINITY;
            mx = fmaxf(mx, sc[k]);
        }
        // block max: the LPK lanes of a key hold equal values
#pragma unroll
        for (int o = LPK; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        if (lane == 0) red[0][wave] = mx;
        __syncthreads();
        float M = red[0][0];
#pragma unroll
        for (int w = 1; w < NWV; w++) M = fmaxf(M, red[0][w]);
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
        for (int d = tid; d < D; d += NT) {
            float v = 0.0f;
#pragma unroll
            for (int k = 0; k < KPB; k++) v += vacc[k][d];
            st_coherent(&rec[2 + d], v);
        }
        if (tid == 0) {
            st_coherent(&rec[0], M);
            st_coherent(&rec[1], tree_sum<NWV>(red[1]));  // fixed pairwise order
        }
    }
    if (!last_arrival(&counters[h], n_splits, &s_last)) return;
    // Merge in the last split to arrive: thread d combines column d of the
    // splits that hold keys (the others wrote empty records), sixteen splits
    // per round of coherent loads, with a running max; every thread forms
    // the same M and L in the same order.
    const int ns = min(n_splits, (attend + per - 1) / per);
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(recs, (uint32_t)(ns * (D + 2)) * 4u);
    for (int d = tid; d < D; d += NT) {
        float M = -INFINITY, L = 0.0f, A = 0.0f;
        for (int c = 0; c < ns; c += 16) {
            float m[16], l[16], o[16];
#pragma unroll
            for (int u = 0; u < 16; u++) {  // past ns: outside the resource, reads 0 (masked below)
                const int off = ((c + u) * (D + 2)) * 4;
                m[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, CPOL_SC1));
                l[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off + 4, 0, CPOL_SC1));
                o[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off + 8 + 4 * d, 0, CPOL_SC1));
            }
            float cm = M;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (c + u < ns) cm = fmaxf(cm, m[u]);
            const float r = expf(M - cm);  // 0 on the first round (M = -inf)
            L *= r;
            A *= r;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (c + u < ns) {
                    const float w = expf(m[u] - cm);
                    L = __builtin_fmaf(w, l[u], L);
                    A = __builtin_fmaf(w, o[u], A);
                }
            M = cm;
        }
        const float v = A * (1.0f / L);
        const size_t oi = (size_t)h * D + d;
        if (OUT_BF16) st_coherent(&((uint16_t*)out)[oi], f32_to_bf16_rne(v));
        else st_coherent(&((float*)out)[oi], v);
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
        TH_LAUNCH((attn_split_kernel<D, _Float16, OUT_BF16>), grid, dim3(256), lds, s, q, (const _Float16*)kc,
                           (const _Float16*)vc, cache_start, n_heads, n_kv_heads, subs, n_splits, part, counters, out,
                           cache_start_dev);
    else
        TH_LAUNCH((attn_split_kernel<D, float, OUT_BF16>), grid, dim3(256), lds, s, q, (const float*)kc,
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

// Threads of a decode-attention workgroup: NT when the split's SPL positions
// divide into whole passes of NT / (D / 8) keys, else 256.
constexpr int attn_decode_nt(int D, int SPL, int NT) { return SPL % (NT / (D / 8)) == 0 ? NT : 256; }

// Decode attention for the engine: one query, f16 cache, SPL positions per
// split; counters (n_heads ints) zero on entry and on return.
template <int SPL, bool OUT_BF16, int NT = 256, bool EVEN = false>
inline void launch_attn_decode(const float* q, const _Float16* kc, const _Float16* vc, int n_heads, int n_kv_heads,
                               int head_dim, int n_splits, float* part, int* counters, void* out,
                               const int* cache_start_dev, hipStream_t s) {
    TH_REQUIRE(n_splits >= 1 && n_splits <= 256, "attention split count out of range");
    const dim3 grid((unsigned)n_heads, 1, (unsigned)n_splits);
    const size_t lds = 0;
    switch (head_dim) {
        case 64: TH_LAUNCH((attn_decode_kernel<64, SPL, OUT_BF16, attn_decode_nt(64, SPL, NT), EVEN>), grid, dim3(attn_decode_nt(64, SPL, NT)), lds, s, q, kc, vc, n_heads, n_kv_heads, n_splits, part, counters, out, cache_start_dev); break;
        case 128: TH_LAUNCH((attn_decode_kernel<128, SPL, OUT_BF16, attn_decode_nt(128, SPL, NT), EVEN>), grid, dim3(attn_decode_nt(128, SPL, NT)), lds, s, q, kc, vc, n_heads, n_kv_heads, n_splits, part, counters, out, cache_start_dev); break;
        case 256: TH_LAUNCH((attn_decode_kernel<256, SPL, OUT_BF16, attn_decode_nt(256, SPL, NT), EVEN>), grid, dim3(attn_decode_nt(256, SPL, NT)), lds, s, q, kc, vc, n_heads, n_kv_heads, n_splits, part, counters, out, cache_start_dev); break;
        default: throw Error(TH_ERR_INVALID, "launch_attn_decode: unsupported head_dim");
    }
    TH_LAUNCH_CHECK();
}

void launch_kv_attention(const float* q, const void* kc, const void* vc, bool f16, size_t cache_start, size_t q_len,
                         size_t n_heads, size_t n_kv_heads, size_t head_dim, float* out, hipStream_t s,
                         th_device* dev);

}  // namespace th
