// MLA (multi-head latent attention) decode, absorbed form.
// The reference has no MLA; this is the definition of DeepSeek-V2's absorbed
// decode with the reference's kv_attention semantics (cpu.rs:257: softmax of
// scaled scores over every cached position, f32 accumulation):
//   q_lat[b,h] = W_UK[h] . q_nope[b,h]                (int8, per-row scale)
//   s[b,h,t]   = (q_lat . c[b,t,:r] + q_rope . c[b,t,r:]) * sm_scale
//   o_lat[b,h] = sum_t softmax_t(s) c[b,t,:r]
//   out[b,h]   = W_UV[h] . o_lat[b,h]                 (int8, per-row scale)
// Three launches:
//   1. absorb: q_lat (f32) emitted as hi+mid+lo bf16 parts (24 significant
//      bits; scores reach ~1e2, so a 16-bit split would cost ~1e-3), with
//      q_rope appended, as the MFMA A operand [B][3][H][r+dr];
//   2. one workgroup per (sequence, split of 128 positions) serves all H
//      heads from one pass over the latent cache: the chunk is staged in LDS,
//      scores run on v_mfma_f32_16x16x32_bf16 (heads x positions), online
//      softmax per head, P.C on VALU; the last split of a sequence merges;
//   3. up-projection through W_UV.
// The cache dominates the traffic: B*L*(r+dr)*2 bytes.
#include "capi_util.hpp"
#include "ops.hpp"
#include "qlinear.hpp"

namespace th {

constexpr int MLA_H = 16;       // heads per MFMA row block (config 5: 16)
constexpr int MLA_CHUNK = 64;   // positions staged per pass
constexpr int MLA_SPLIT = 128;  // positions per workgroup

// Per-head batched int8 GEMV over the tiled q8 layout (16 rows x 64 k per
// tile, lane q*16+r holds k 16q..16q+15 of row r), per-row scales.
// y[b][h][n] = scale[h*rows+n] * sum_k q[h*rows+n][k] * x[b][h][k].
// One workgroup: head h, 16 output rows, all B inputs; thread (row, b).
template <int MODE>  // 0: absorb (write hi/mid/lo bf16 A operand), 1: plain f32 out
__global__ __launch_bounds__(256) void mla_q8_heads_kernel(const uint8_t* __restrict__ wq, const float* __restrict__ wsc,
                                                           int rows_per_head, int K, int Kp, int B, int H,
                                                           const float* __restrict__ x, int ldx_b, int ldx_h,
                                                           float* __restrict__ y, uint16_t* __restrict__ qa,
                                                           const float* __restrict__ q_rope, int dr) {
    extern __shared__ float xs[];  // [B][K]
    const int h = blockIdx.x, t_local = blockIdx.y, tid = threadIdx.x;
    for (int i = tid; i < B * K; i += blockDim.x) {
        const int b = i / K, k = i - b * K;
        xs[i] = x[(size_t)b * ldx_b + (size_t)h * ldx_h + k];
    }
    __syncthreads();
    const int r = tid & 15, b = tid >> 4;
    if (b >= B) return;
    const int row = h * rows_per_head + t_local * 16 + r;  // global row of the stacked matrix
    const int t = row >> 4;                                // its 16-row tile
    const int NCH = Kp >> 6;
    float acc = 0.0f;
    for (int c = 0; c < NCH; c++) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 w = *(const uint4*)(wq + (((size_t)t * NCH + c) * 64 + q * 16 + r) * 16);
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
            const int k0 = c * 64 + q * 16;
#pragma unroll
            for (int j = 0; j < 4; j++) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int k = k0 + j * 4 + e;
                    const float xv = k < K ? xs[b * K + k] : 0.0f;
                    acc = __builtin_fmaf((float)(int8_t)(ww[j] >> (8 * e)), xv, acc);
                }
            }
        }
    }
    const float v = acc * wsc[row];
    const int n = t_local * 16 + r;
    if (MODE == 0) {
        // A operand row (b, part, h): q_lat parts then q_rope parts
        const int R = rows_per_head, W = R + dr;
        const uint32_t hi = f32_to_bf16_bits(v);
        const float r1 = v - bf16_bits_to_f32(hi);
        const uint32_t mid = f32_to_bf16_bits(r1);
        const uint32_t lo = f32_to_bf16_bits(r1 - bf16_bits_to_f32(mid));
        qa[(((size_t)b * 3 + 0) * H + h) * W + n] = (uint16_t)hi;
        qa[(((size_t)b * 3 + 1) * H + h) * W + n] = (uint16_t)mid;
        qa[(((size_t)b * 3 + 2) * H + h) * W + n] = (uint16_t)lo;
        if (t_local == 0) {
            for (int i = r; i < dr; i += 16) {
                const float qr = q_rope[((size_t)b * H + h) * dr + i];
                const uint32_t h2 = f32_to_bf16_bits(qr);
                const float s1 = qr - bf16_bits_to_f32(h2);
                const uint32_t m2 = f32_to_bf16_bits(s1);
                const uint32_t l2 = f32_to_bf16_bits(s1 - bf16_bits_to_f32(m2));
                qa[(((size_t)b * 3 + 0) * H + h) * W + R + i] = (uint16_t)h2;
                qa[(((size_t)b * 3 + 1) * H + h) * W + R + i] = (uint16_t)m2;
                qa[(((size_t)b * 3 + 2) * H + h) * W + R + i] = (uint16_t)l2;
            }
        }
    } else {
        y[((size_t)b * H + h) * rows_per_head + n] = v;
    }
}

// Latent attention for one (sequence b, split s of MLA_SPLIT positions), all
// H = 16 heads.  W = r + dr (576) columns per cache row.  Each wave scores 16
// positions of a 64-position chunk: D[head][pos] = sum_k A[head][k] B[k][pos]
// over W/32 k-steps x 3 parts (hi, mid, lo).  Record per (b, s, h):
// {m, l, acc[r]} (coherent stores); the last split of b merges into o_lat.
__global__ __launch_bounds__(256) void mla_attn_kernel(const uint16_t* __restrict__ qa, const uint16_t* __restrict__ cache,
                                                       int L, int R, int dr, float sm_scale, int n_splits,
                                                       float* __restrict__ part, int* __restrict__ counters,
                                                       float* __restrict__ o_lat) {
    extern __shared__ uint4 lds_raw[];
    const int W = R + dr;
    uint16_t* cs = (uint16_t*)lds_raw;                           // [MLA_CHUNK][W] bf16
    float* ps = (float*)(cs + (size_t)MLA_CHUNK * W);            // [MLA_H][MLA_CHUNK] probabilities
    float* mrow = ps + MLA_H * MLA_CHUNK;                        // [4 waves][MLA_H] chunk maxima
    __shared__ float m_run[MLA_H], l_run[MLA_H], rescale[MLA_H];
    __shared__ int s_last;
    const int b = blockIdx.x, s = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int p0 = s * MLA_SPLIT;
    const int len = max(0, min(MLA_SPLIT, L - p0));
    const uint16_t* cb = cache + (size_t)b * L * W;
    // accumulators: thread owns latent dims d = tid, tid + 256 (R <= 512) for all heads
    constexpr int DPT = 2;
    float acc[MLA_H][DPT];
#pragma unroll
    for (int hh = 0; hh < MLA_H; hh++)
#pragma unroll
        for (int i = 0; i < DPT; i++) acc[hh][i] = 0.0f;
    if (tid < MLA_H) { m_run[tid] = -INFINITY; l_run[tid] = 0.0f; }
    const uint16_t* qab = qa + (size_t)b * 3 * MLA_H * W;
    for (int c0 = 0; c0 < len; c0 += MLA_CHUNK) {
        const int clen = min(MLA_CHUNK, len - c0);
        // stage the chunk (16-byte pieces; W*2 is a multiple of 16)
        const int pieces = MLA_CHUNK * W / 8;
        for (int i = tid; i < pieces; i += 256) {
            const int pos = i / (W / 8), col = (i - pos * (W / 8)) * 8;
            const int src = pos < clen ? p0 + c0 + pos : p0 + c0;  // clamp: masked below
            *(uint4*)(cs + (size_t)pos * W + col) = *(const uint4*)(cb + (size_t)src * W + col);
        }
        __syncthreads();
        // scores: wave handles positions 16*wave .. +15
        float4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
        const int pos_b = wave * 16 + r;  // B column owned by this lane
        for (int k0 = 0; k0 < W; k0 += 32) {
            const uint4 bq = *(const uint4*)(cs + (size_t)pos_b * W + k0 + q * 8);
#pragma unroll
            for (int part = 0; part < 3; part++) {
                const uint4 aq = *(const uint4*)(qab + ((size_t)part * MLA_H + r) * W + k0 + q * 8);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, aq),
                                                            __builtin_bit_cast(bf16x8_t, bq), d, 0, 0, 0);
            }
        }
        // lane (q, r) holds D[head 4q+i][position 16*wave + r]
        float sc4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) sc4[i] = (16 * wave + r < clen) ? d[i] * sm_scale : -INFINITY;
        // per-head max over this wave's 16 positions, then over the 4 waves
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float mx = sc4[i];
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            if (r == 0) mrow[wave * MLA_H + 4 * q + i] = mx;
        }
        __syncthreads();
        if (tid < MLA_H) {
            float mx = fmaxf(fmaxf(mrow[tid], mrow[MLA_H + tid]), fmaxf(mrow[2 * MLA_H + tid], mrow[3 * MLA_H + tid]));
            const float mn = fmaxf(m_run[tid], mx);
            rescale[tid] = expf(m_run[tid] - mn);
            m_run[tid] = mn;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int hh = 4 * q + i;
            ps[hh * MLA_CHUNK + 16 * wave + r] = (16 * wave + r < clen) ? expf(sc4[i] - m_run[hh]) : 0.0f;
        }
        __syncthreads();
        if (tid < MLA_H) {
            float l = 0.0f;
            for (int p = 0; p < clen; p++) l += ps[tid * MLA_CHUNK + p];
            l_run[tid] = l_run[tid] * rescale[tid] + l;
        }
        // P.C for this thread's latent dims
#pragma unroll
        for (int i = 0; i < DPT; i++) {
            const int dd = tid + 256 * i;
            if (dd < R) {
#pragma unroll
                for (int hh = 0; hh < MLA_H; hh++) acc[hh][i] *= rescale[hh];
                for (int p = 0; p < clen; p++) {
                    const float cv = __uint_as_float((uint32_t)cs[(size_t)p * W + dd] << 16);
#pragma unroll
                    for (int hh = 0; hh < MLA_H; hh++) acc[hh][i] = __builtin_fmaf(ps[hh * MLA_CHUNK + p], cv, acc[hh][i]);
                }
            }
        }
        __syncthreads();  // cs/ps reused by the next chunk
    }
    // record per head: {m, l, acc[R]}
    float* recs = part + (size_t)b * n_splits * MLA_H * (R + 2);
    float* rec = recs + (size_t)s * MLA_H * (R + 2);
#pragma unroll
    for (int i = 0; i < DPT; i++) {
        const int dd = tid + 256 * i;
        if (dd < R)
#pragma unroll
            for (int hh = 0; hh < MLA_H; hh++) st_coherent(&rec[(size_t)hh * (R + 2) + 2 + dd], acc[hh][i]);
    }
    if (tid < MLA_H) {
        st_coherent(&rec[(size_t)tid * (R + 2)], len > 0 ? m_run[tid] : -INFINITY);
        st_coherent(&rec[(size_t)tid * (R + 2) + 1], l_run[tid]);
    }
    if (!last_arrival(&counters[b], n_splits, &s_last)) return;
    // merge splits of sequence b (split order), per head
    __shared__ float wts[MLA_H][64];
    __shared__ float Ls[MLA_H];
    if (tid < MLA_H) {
        float M = -INFINITY;
        for (int sp = 0; sp < n_splits; sp++) M = fmaxf(M, ld_coherent(&recs[((size_t)sp * MLA_H + tid) * (R + 2)]));
        float Lsum = 0.0f;
        for (int sp = 0; sp < n_splits; sp++) {
            const float m = ld_coherent(&recs[((size_t)sp * MLA_H + tid) * (R + 2)]);
            const float w = m == -INFINITY ? 0.0f : expf(m - M);
            wts[tid][sp] = w;
            Lsum += w * ld_coherent(&recs[((size_t)sp * MLA_H + tid) * (R + 2) + 1]);
        }
        Ls[tid] = Lsum;
    }
    __syncthreads();
    for (int i = tid; i < MLA_H * R; i += 256) {
        const int hh = i / R, dd = i - hh * R;
        float a = 0.0f;
        for (int sp = 0; sp < n_splits; sp++) a += ld_coherent(&recs[((size_t)sp * MLA_H + hh) * (R + 2) + 2 + dd]) * wts[hh][sp];
        o_lat[((size_t)b * MLA_H + hh) * R + dd] = a / Ls[hh];
    }
}

}  // namespace th

using namespace th;

extern "C" int th_mla_decode(th_device* dev, const th_buffer* q_nope, const th_buffer* q_rope, const th_buffer* cache,
                             size_t B, size_t H, size_t L, size_t dn, size_t dr, size_t r, size_t dv,
                             const th_qweight* w_uk, const th_qweight* w_uv, float sm_scale, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && q_nope && q_rope && cache && w_uk && w_uv && out, "null argument");
    TH_REQUIRE(H == MLA_H, "this kernel serves 16 heads");
    TH_REQUIRE(r % 16 == 0 && r <= 512 && dr % 8 == 0 && (r + dr) % 32 == 0, "latent widths: r <= 512, (r+dr) % 32 == 0");
    TH_REQUIRE(L > 0 && B > 0 && B <= 16, "1 <= B <= 16 sequences");
    TH_REQUIRE(w_uk->bits == 8 && w_uk->per_row && w_uk->rows == H * r && w_uk->cols == dn, "w_uk must be q8 rowwise [H*r][dn]");
    TH_REQUIRE(w_uv->bits == 8 && w_uv->per_row && w_uv->rows == H * dv && w_uv->cols == r, "w_uv must be q8 rowwise [H*dv][r]");
    TH_REQUIRE(r % 16 == 0 && dv % 16 == 0, "r and dv must be multiples of 16");
    require_len(q_nope, TH_F32, B * H * dn, "q_nope");
    require_len(q_rope, TH_F32, B * H * dr, "q_rope");
    require_len(cache, TH_BF16, B * L * (r + dr), "cache");
    require_len(out, TH_F32, B * H * dv, "out");
    hipStream_t s = dev->stream;
    const size_t W = r + dr;
    const int n_splits = (int)ceil_div(L, (size_t)MLA_SPLIT);
    TH_REQUIRE(n_splits <= 64, "L above 8192 positions");
    // workspace: A operand, split records, o_lat
    const size_t qa_bytes = B * 3 * H * W * 2;
    const size_t part_bytes = B * (size_t)n_splits * H * (r + 2) * 4;
    const size_t olat_bytes = B * H * r * 4;
    char* ws = (char*)device_scratch(dev, round_up(qa_bytes, 256) + round_up(part_bytes, 256) + olat_bytes);
    uint16_t* qa = (uint16_t*)ws;
    float* part = (float*)(ws + round_up(qa_bytes, 256));
    float* olat = (float*)(ws + round_up(qa_bytes, 256) + round_up(part_bytes, 256));
    int* counters = device_counters(dev, B);
    // 1. absorb
    hipLaunchKernelGGL(mla_q8_heads_kernel<0>, dim3((unsigned)H, (unsigned)(r / 16)), dim3(256), B * dn * 4, s,
                       (const uint8_t*)w_uk->data, (const float*)w_uk->scales, (int)r, (int)dn, (int)w_uk->Kp, (int)B,
                       (int)H, (const float*)q_nope->ptr, (int)(H * dn), (int)dn, (float*)nullptr, qa,
                       (const float*)q_rope->ptr, (int)dr);
    TH_LAUNCH_CHECK();
    // 2. latent attention
    const size_t lds = (size_t)MLA_CHUNK * W * 2 + (size_t)MLA_H * MLA_CHUNK * 4 + 4 * MLA_H * 4;
    TH_REQUIRE(lds <= 150 * 1024, "latent chunk does not fit LDS");
    static size_t attr_lds = 0;  // largest dynamic LDS size granted so far
    if (lds > attr_lds) {
        TH_HIP(hipFuncSetAttribute((const void*)mla_attn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr_lds = lds;
    }
    hipLaunchKernelGGL(mla_attn_kernel, dim3((unsigned)B, (unsigned)n_splits), dim3(256), lds, s, qa,
                       (const uint16_t*)cache->ptr, (int)L, (int)r, (int)dr, sm_scale, n_splits, part, counters, olat);
    TH_LAUNCH_CHECK();
    // 3. up-projection
    hipLaunchKernelGGL(mla_q8_heads_kernel<1>, dim3((unsigned)H, (unsigned)(dv / 16)), dim3(256), B * r * 4, s,
                       (const uint8_t*)w_uv->data, (const float*)w_uv->scales, (int)dv, (int)r, (int)w_uv->Kp, (int)B,
                       (int)H, olat, (int)(H * r), (int)r, (float*)out->ptr, (uint16_t*)nullptr, (const float*)nullptr,
                       0);
    TH_LAUNCH_CHECK();
    TH_API_END
}
