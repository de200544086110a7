// MLA (multi-head latent attention) decode, absorbed form (DeepSeek-V2-Lite shape: 16 heads, latent 512, rope 64).
// The reference has no MLA; this is the definition of DeepSeek-V2's absorbed
// decode with the reference's kv_attention semantics (cpu.rs:257: softmax of
// scaled scores over every cached position, f32 accumulation):
//   q_lat[b,h] = W_UK[h] . q_nope[b,h]                (int8, per-row scale)
//   s[b,h,t]   = (q_lat . c[b,t,:r] + q_rope . c[b,t,r:]) * sm_scale
//   o_lat[b,h] = sum_t softmax_t(s) c[b,t,:r]
//   out[b,h]   = W_UV[h] . o_lat[b,h]                 (int8, per-row scale)
// Three launches:
//   1. absorb on MFMA (one wave per 16 W_UK rows, every sequence at once):
//      q = [q_lat ; q_rope] (f32) emitted as hi + lo bf16 parts (16
//      significant bits) as the attention's MFMA A operand [B][2][H][r+dr];
//   2. one workgroup per (sequence, split of 128 positions) serves all 16
//      heads from one pass over the latent cache, in chunks of 64 positions
//      staged in LDS (the next chunk is loaded into registers meanwhile):
//      scores on v_mfma_f32_16x16x32_bf16 (heads x positions; each wave owns
//      a quarter of the k-steps and keeps its A operand in registers; partial
//      scores are summed in LDS), online softmax per head, then P.C on the
//      same MFMA (P as hi + lo bf16, C exact bf16, read with transposing LDS
//      reads), one {max, sum, o_lat}
//      record per split;
//   3. per (head, sequence, 64 output rows): the split merge in LDS, then
//      the up-projection through W_UV on MFMA.
// The cache dominates the traffic: B*L*(r+dr)*2 bytes.
#include <mutex>
#include <utility>

#include "capi_util.hpp"
#include "ops.hpp"
#include "qlinear.hpp"

namespace th {

constexpr int MLA_H = 16;       // heads per MFMA row block (config 5: 16)
constexpr int MLA_CHUNK = 64;   // positions staged per pass
constexpr int MLA_SPLIT = 128;  // positions per workgroup

typedef __bf16 bf16x2_pk_t __attribute__((ext_vector_type(2)));
// Two f32 values as a bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32;
// the same bits as f32_to_bf16_bits for finite values).
__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    const bf16x2_pk_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}
// hi and lo bf16 pairs of (a, b): hi + lo carries 16 significant bits of each
__device__ __forceinline__ void bf16_pair_hilo(float a, float b, uint32_t& hi, uint32_t& lo) {
    hi = bf16_pair(a, b);
    lo = bf16_pair(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

// Absorb on MFMA: q_lat[b][h][n] = scale[h*R+n] * sum_k W_UK[h*R+n][k] x[b][h][k]
// for every sequence b at once.  One wave per 16-row tile of the stacked
// W_UK (q8 tiles: 16 rows x 64 k, lane q*16+r holding k 16q..16q+15 of row
// r): A = x (rows = sequences, at most 16, as hi + lo bf16 parts), B = the
// tile's int8 weights as bf16 (exact), v_mfma_f32_16x16x32_bf16 per half of
// a lane's 16 k (MFMA k index 8q + e of step (c, hh) = k c*64 + 16q + 8hh + e),
// so lane (q, r) ends with sequences 4q..4q+3 of row r.  Output: the
// attention's A operand [B][2][H][r+dr] (hi, lo bf16), q_rope copied in.
constexpr int MLA_ABS_CH = 4;  // 64-k chunks of W_UK: qk_nope width <= 256

__global__ __launch_bounds__(256) void mla_absorb_kernel(const uint8_t* __restrict__ wq, const float* __restrict__ wsc,
                                                         int R, int dn, int nch, int B, const float* __restrict__ x,
                                                         const float* __restrict__ q_rope, int dr,
                                                         uint16_t* __restrict__ qa) {
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int TT = MLA_H * R / 16, W = R + dr;
    const int t = min((int)blockIdx.x * 4 + wave, TT - 1);  // surplus waves redo the last tile, store nothing
    const int h = 16 * t / R;
    const float sc = wsc[16 * t + r];  // loaded now: a load in the store branch would end the kernel with a round trip
    uint4 w[MLA_ABS_CH];
#pragma unroll
    for (int c = 0; c < MLA_ABS_CH; c++) w[c] = *(const uint4*)(wq + (((size_t)t * nch + min(c, nch - 1)) * 64 + lane) * 16);
    // sequence r's activations (rows r >= B are zero): k = c*64 + 16q + 8hh + e
    float4 xv[MLA_ABS_CH][2][2];
    const float* xr = x + ((size_t)min(r, B - 1) * MLA_H + h) * dn;
#pragma unroll
    for (int c = 0; c < MLA_ABS_CH; c++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
#pragma unroll
            for (int f = 0; f < 2; f++) xv[c][hh][f] = *(const float4*)(xr + min(c * 64 + 16 * q + 8 * hh + 4 * f, dn - 4));
    float4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < MLA_ABS_CH; c++) {
        if (c >= nch) break;
        const uint32_t ww[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            uint32_t bw[4], ah[4], al[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t word = ww[2 * hh + (e >> 1)];
                const int sh = 16 * (e & 1);
                const float w0 = (float)(int8_t)(word >> sh), w1 = (float)(int8_t)(word >> (sh + 8));
                bw[e] = (__float_as_uint(w0) >> 16) | (__float_as_uint(w1) & 0xFFFF0000u);  // exact: |w| <= 127
                const float4 xf = xv[c][hh][e >> 1];
                const int k0 = c * 64 + 16 * q + 8 * hh + 2 * e;
                const bool live = r < B;
                const float x0 = live && k0 < dn ? ((e & 1) ? xf.z : xf.x) : 0.0f;
                const float x1 = live && k0 + 1 < dn ? ((e & 1) ? xf.w : xf.y) : 0.0f;
                bf16_pair_hilo(x0, x1, ah[e], al[e]);
            }
            const bf16x8_t B8 = __builtin_bit_cast(bf16x8_t, make_uint4(bw[0], bw[1], bw[2], bw[3]));
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, make_uint4(ah[0], ah[1], ah[2], ah[3])),
                                                        B8, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, make_uint4(al[0], al[1], al[2], al[3])),
                                                        B8, d, 0, 0, 0);
        }
    }
    if ((int)blockIdx.x * 4 + wave < TT) {
        const int row = 16 * t + r, n = row - h * R;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int b = 4 * q + j;
            if (b < B) {
                const float v = d[j] * sc;
                const uint32_t hi = f32_to_bf16_bits(v);
                qa[(((size_t)b * 2 + 0) * MLA_H + h) * W + n] = (uint16_t)hi;
                qa[(((size_t)b * 2 + 1) * MLA_H + h) * W + n] = (uint16_t)f32_to_bf16_bits(v - bf16_bits_to_f32(hi));
            }
        }
    }
    // q_rope, split over the grid
    for (int j = blockIdx.x * 256 + tid; j < B * MLA_H * dr; j += gridDim.x * 256) {
        const int bh = j / dr, i = j - bh * dr, b = bh / MLA_H, hh = bh - b * MLA_H;
        const float qr = q_rope[j];
        const uint32_t h2 = f32_to_bf16_bits(qr);
        qa[(((size_t)b * 2 + 0) * MLA_H + hh) * W + R + i] = (uint16_t)h2;
        qa[(((size_t)b * 2 + 1) * MLA_H + hh) * W + R + i] = (uint16_t)f32_to_bf16_bits(qr - bf16_bits_to_f32(h2));
    }
}

// Latent attention for one (sequence b, split s of MLA_SPLIT positions), all
// 16 heads.  W = r + dr columns per cache row (W % 32 == 0, W <= 576); cache
// rows sit in LDS at a stride of W + 8 bf16 so that the 16 rows one score
// MFMA reads start in different banks.  Record per (b, s, h): {m, l, acc[r]},
// with acc unnormalised (sum of p * c with p = exp(s - m)).
constexpr int MLA_WMAX = 576;
constexpr int MLA_WAVES = 8;                                 // 512 threads, two waves per SIMD
constexpr int MLA_THREADS = 64 * MLA_WAVES;
constexpr int MLA_NT = 512 / 16 / MLA_WAVES;                 // P.C output tiles of 16 latent dims per wave
constexpr int MLA_PS = MLA_CHUNK + 4;                        // P row stride: 16-byte rows, 8 heads in distinct banks

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// W = r + dr is a template parameter (a multiple of 32 up to 576) so that
// every index below is a constant expression.
template <int W>
__global__ __launch_bounds__(MLA_THREADS) void mla_attn_kernel(const uint16_t* __restrict__ qa,
                                                               const uint16_t* __restrict__ cache, int L, int R,
                                                               float sm_scale, int n_splits, float* __restrict__ part) {
    constexpr int WP = W + 8, KS = W / 32, PR = W / 8;  // PR: 16-byte pieces per row
    constexpr int KSW = (KS + MLA_WAVES - 1) / MLA_WAVES;  // k-steps per wave
    constexpr int pieces = MLA_CHUNK * PR;
    constexpr int PPT = (pieces + MLA_THREADS - 1) / MLA_THREADS;  // pieces per thread
    extern __shared__ uint4 lds_raw[];
    uint16_t* cs = (uint16_t*)lds_raw;                         // [MLA_CHUNK][WP]
    float* sred = (float*)(cs + (size_t)MLA_CHUNK * WP);        // [MLA_WAVES][MLA_H][MLA_CHUNK] partial scores
    float* ps = sred + MLA_WAVES * MLA_H * MLA_CHUNK;           // [MLA_H][MLA_PS] probabilities
    __shared__ float resc[MLA_H];
    const int b = blockIdx.x, s = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int p0 = s * MLA_SPLIT;
    const int len = min(MLA_SPLIT, L - p0);  // >= 1: the grid has ceil(L / MLA_SPLIT) splits
    const int nch = (len + MLA_CHUNK - 1) / MLA_CHUNK;
    const uint16_t* cb = cache + (size_t)b * L * W;

    // A operand of this wave's k-steps (ks = wave + 8 i), hi and lo parts;
    // k-steps past W read a valid row and are multiplied by zero.
    uint4 areg[KSW][2];
    const uint16_t* qab = qa + (size_t)b * 2 * MLA_H * W;
#pragma unroll
    for (int i = 0; i < KSW; i++) {
        const int ks = min(wave + MLA_WAVES * i, KS - 1);
        const bool live = wave + MLA_WAVES * i < KS;
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            const uint4 v = *(const uint4*)(qab + ((size_t)pp * MLA_H + r) * W + ks * 32 + q * 8);
            areg[i][pp] = make_uint4(live ? v.x : 0u, live ? v.y : 0u, live ? v.z : 0u, live ? v.w : 0u);
        }
    }
    // this thread's pieces: row offset within a chunk and column (fixed)
    int prow[PPT], pcol[PPT];
#pragma unroll
    for (int u = 0; u < PPT; u++) {
        const int i = min(tid + MLA_THREADS * u, pieces - 1);
        prow[u] = i / PR;
        pcol[u] = (i - prow[u] * PR) * 8;
    }
    const int last = p0 + len - 1;  // rows past the split are clamped here and masked below
    u32x4_t pre[PPT];  // native vectors: an array of uint4 structs stays in scratch memory
#pragma unroll
    for (int u = 0; u < PPT; u++) pre[u] = *(const u32x4_t*)(cb + (size_t)min(p0 + prow[u], last) * W + pcol[u]);
    float4_t acc[MLA_NT];
#pragma unroll
    for (int nt = 0; nt < MLA_NT; nt++) acc[nt] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
    // running max and sum of head tid >> 5, kept alike by its 32 softmax threads
    float m_run = -INFINITY, l_run = 0.0f;

    for (int c = 0; c < nch; c++) {
        const int clen = min(MLA_CHUNK, len - c * MLA_CHUNK);
        // branch-free (a load under a branch makes the compiler wait for
        // every load in flight): surplus pieces rewrite the last piece with
        // its own value, and the last chunk "prefetches" itself (L2 hits)
#pragma unroll
        for (int u = 0; u < PPT; u++) *(u32x4_t*)(cs + (size_t)prow[u] * WP + pcol[u]) = pre[u];
        lds_barrier();  // LDS only: the next chunk's loads stay in flight across it
        {
            const int cn = p0 + min(c + 1, nch - 1) * MLA_CHUNK;
#pragma unroll
            for (int u = 0; u < PPT; u++) pre[u] = *(const u32x4_t*)(cb + (size_t)min(cn + prow[u], last) * W + pcol[u]);
        }
        // partial scores over this wave's k-steps: D[head][position]
        float4_t d[4];
#pragma unroll
        for (int pt = 0; pt < 4; pt++) d[pt] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < KSW; i++) {
            const int ks = min(wave + MLA_WAVES * i, KS - 1);
            uint4 bs[4];
#pragma unroll
            for (int pt = 0; pt < 4; pt++) bs[pt] = *(const uint4*)(cs + (size_t)(pt * 16 + r) * WP + ks * 32 + q * 8);
#pragma unroll
            for (int pp = 0; pp < 2; pp++)
#pragma unroll
                for (int pt = 0; pt < 4; pt++)
                    d[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, areg[i][pp]),
                                                                    __builtin_bit_cast(bf16x8_t, bs[pt]), d[pt], 0, 0, 0);
        }
#pragma unroll
        for (int pt = 0; pt < 4; pt++)
#pragma unroll
            for (int j = 0; j < 4; j++) sred[(wave * MLA_H + 4 * q + j) * MLA_CHUNK + pt * 16 + r] = d[pt][j];
        lds_barrier();
        // softmax step: thread (head hh, positions 2 pg, 2 pg + 1); 32 threads per head
        {
            const int hh = tid >> 5, pg = tid & 31;
            float sv[2];
            float cmax = -INFINITY;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int p = 2 * pg + j;
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < MLA_WAVES; w++) v += sred[(w * MLA_H + hh) * MLA_CHUNK + p];
                sv[j] = p < clen ? v * sm_scale : -INFINITY;
                cmax = fmaxf(cmax, sv[j]);
            }
            cmax = group_max<32>(cmax);
            const float mold = m_run;
            const float mnew = fmaxf(mold, cmax);
            float lsum = 0.0f;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float e = 2 * pg + j < clen ? expf(sv[j] - mnew) : 0.0f;
                ps[hh * MLA_PS + 2 * pg + j] = e;
                lsum += e;
            }
            lsum = group_sum<32>(lsum);
            const float f = expf(mold - mnew);
            if (pg == 0) resc[hh] = f;
            l_run = l_run * f + lsum;
            m_run = mnew;
        }
        lds_barrier();
        // P.C: D[head][latent dim] += P[head][pos] C[pos][dim], MFMA k index
        // 8q + e of step kk = position 32 kk + 8q + e.  A: lane (q, r) holds
        // P[head r][32 kk + 8q ..+8); B: two transposing LDS reads, each
        // giving lane (q, r) C[32 kk + 8q + 4 hf ..+4][d0 + r] (the 16 lanes
        // of a row group address four rows of four dims each).
        uint4 ahi[2], alo[2];
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const float4 pa = *(const float4*)&ps[r * MLA_PS + 32 * kk + 8 * q];
            const float4 pb = *(const float4*)&ps[r * MLA_PS + 32 * kk + 8 * q + 4];
            const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
            uint32_t h2[4], l2[4];
#pragma unroll
            for (int e = 0; e < 4; e++) bf16_pair_hilo(pv[2 * e], pv[2 * e + 1], h2[e], l2[e]);
            ahi[kk] = make_uint4(h2[0], h2[1], h2[2], h2[3]);
            alo[kk] = make_uint4(l2[0], l2[1], l2[2], l2[3]);
        }
        float f4[4];
#pragma unroll
        for (int j = 0; j < 4; j++) f4[j] = resc[4 * q + j];
        uint4 bq[MLA_NT][2];
#pragma unroll
        for (int nt = 0; nt < MLA_NT; nt++) {
            const int d0 = min((wave * MLA_NT + nt) * 16, R - 16);  // tiles past r: computed, not stored
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                short4_t t[2];
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    const int row = 32 * kk + 8 * q + 4 * hf + (r >> 2);
                    t[hf] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_short4_t*)(cs + (size_t)row * WP + d0 + 4 * (r & 3)));
                }
                bq[nt][kk] = make_uint4((uint16_t)t[0][0] | ((uint32_t)(uint16_t)t[0][1] << 16),
                                        (uint16_t)t[0][2] | ((uint32_t)(uint16_t)t[0][3] << 16),
                                        (uint16_t)t[1][0] | ((uint32_t)(uint16_t)t[1][1] << 16),
                                        (uint16_t)t[1][2] | ((uint32_t)(uint16_t)t[1][3] << 16));
            }
        }
#pragma unroll
        for (int nt = 0; nt < MLA_NT; nt++) {
#pragma unroll
            for (int j = 0; j < 4; j++) acc[nt][j] *= f4[j];
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ahi[kk]),
                                                                  __builtin_bit_cast(bf16x8_t, bq[nt][kk]), acc[nt], 0, 0, 0);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, alo[kk]),
                                                                  __builtin_bit_cast(bf16x8_t, bq[nt][kk]), acc[nt], 0, 0, 0);
            }
        }
        lds_barrier();  // cs, sred and ps are rewritten by the next chunk
    }
    // record per head: {m, l, acc[R]}; lane (q, r) holds heads 4q..4q+3 of dim d0 + r
    // (plain stores: the merge is the next launch)
    float* rec = part + ((size_t)b * n_splits + s) * MLA_H * (R + 2);
#pragma unroll
    for (int nt = 0; nt < MLA_NT; nt++) {
        const int d0 = (wave * MLA_NT + nt) * 16;
        if (d0 < R)
#pragma unroll
            for (int j = 0; j < 4; j++) rec[(size_t)(4 * q + j) * (R + 2) + 2 + d0 + r] = acc[nt][j];
    }
    if ((tid & 31) == 0) {
        rec[(size_t)(tid >> 5) * (R + 2)] = m_run;
        rec[(size_t)(tid >> 5) * (R + 2) + 1] = l_run;
    }
}

// Split merge fused with the W_UV up-projection: workgroup (head h,
// sequence b, row group g).  o_lat[b][h] = sum_s w_s acc_s / sum_s w_s l_s
// (split order, w_s = exp(m_s - max m)) is built in LDS, then each wave
// takes one 16-row tile of the head's W_UV rows on v_mfma_f32_16x16x32_f16:
// A = o_lat (row 0; scaled by a power of two into f16 range, as hi + lo f16
// parts), B = the tile's int8 weights as f16 (exact), MFMA k index 8q + e of
// step (c, hh) = k c*64 + 16q + 8hh + e.  The W_UV
// and record loads are all issued at the start.  r <= 512, dv <= 128,
// n_splits <= 64.
constexpr int MLA_UP_THREADS = 256;
constexpr int MLA_UP_CH = 8;  // 64-k chunks of W_UV: r <= 512

__global__ __launch_bounds__(MLA_UP_THREADS) void mla_merge_up_kernel(const float* __restrict__ part, int n_splits,
                                                                     int R, const uint8_t* __restrict__ wq,
                                                                     const float* __restrict__ wsc, int dv, int nch,
                                                                     float* __restrict__ out) {
    __shared__ __align__(16) uint16_t olh[2][512];  // o_lat * 2^-oe as f16 hi, lo parts
    __shared__ float wts[64];
    __shared__ float Lsh;
    __shared__ float omax4[4];
    const int h = blockIdx.x, b = blockIdx.y, g = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), q = lane >> 4, r = lane & 15;
    const float* recs = part + (size_t)b * n_splits * MLA_H * (R + 2);
    constexpr int DPT = 2, SB = 32;  // dims per thread, splits per load round
    // this wave's W_UV tile first: it does not depend on the merge
    const int TV = dv / 16, tt = g * 4 + wave;
    const int trow = h * TV + min(tt, TV - 1);  // 16-row tile of the stacked W_UV
    const float usc = wsc[h * dv + min(tt, TV - 1) * 16 + r];  // loaded with the weights, not in the store branch
    uint4 w[MLA_UP_CH];
#pragma unroll
    for (int c = 0; c < MLA_UP_CH; c++) w[c] = *(const uint4*)(wq + (((size_t)trow * nch + min(c, nch - 1)) * 64 + lane) * 16);
    float v[SB][DPT];
#pragma unroll
    for (int i = 0; i < SB; i++)
#pragma unroll
        for (int j = 0; j < DPT; j++)
            v[i][j] = recs[((size_t)min(i, n_splits - 1) * MLA_H + h) * (R + 2) + 2 + min(tid + 256 * j, R - 1)];
    if (tid < 64) {
        const float* rec = recs + ((size_t)min(tid, n_splits - 1) * MLA_H + h) * (R + 2);
        const float m = tid < n_splits ? rec[0] : -INFINITY;
        const float l = tid < n_splits ? rec[1] : 0.0f;
        float M = m;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        const float wgt = tid < n_splits ? expf(m - M) : 0.0f;
        const float L = wave_sum(wgt * l);
        wts[tid] = wgt;
        if (tid == 0) Lsh = L;
    }
    __syncthreads();
    float a[DPT] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < SB; i++)
#pragma unroll
        for (int j = 0; j < DPT; j++) a[j] += i < n_splits ? v[i][j] * wts[i] : 0.0f;
    for (int s0 = SB; s0 < n_splits; s0 += SB) {  // beyond 32 splits: further rounds
#pragma unroll
        for (int i = 0; i < SB; i++)
#pragma unroll
            for (int j = 0; j < DPT; j++)
                v[i][j] = recs[((size_t)min(s0 + i, n_splits - 1) * MLA_H + h) * (R + 2) + 2 + min(tid + 256 * j, R - 1)];
#pragma unroll
        for (int i = 0; i < SB; i++)
#pragma unroll
            for (int j = 0; j < DPT; j++) a[j] += s0 + i < n_splits ? v[i][j] * wts[s0 + i] : 0.0f;
    }
    // o_lat in f16 range: scaled by 2^-oe so that its largest magnitude lies
    // in [2^12, 2^13), as hi + lo f16 parts (the result is scaled back exactly)
    float o[DPT], om = 0.0f;
#pragma unroll
    for (int j = 0; j < DPT; j++) {
        o[j] = tid + 256 * j < R ? a[j] / Lsh : 0.0f;
        om = fmaxf(om, fabsf(o[j]));
    }
    const int oe = range_exp(block_absmax256(om, omax4), XPREP_TOP);
#pragma unroll
    for (int j = 0; j < DPT; j++) {
        const float os = __builtin_amdgcn_ldexpf(o[j], -oe);
        const _Float16 hi = (_Float16)os;
        olh[0][tid + 256 * j] = __builtin_bit_cast(uint16_t, hi);
        olh[1][tid + 256 * j] = __builtin_bit_cast(uint16_t, (_Float16)(os - (float)hi));
    }
    __syncthreads();
    if (tt >= TV) return;  // wave-uniform: no barrier follows
    // A = o_lat (row 0; hi and lo f16 parts, the other rows zero), B = the
    // tile's int8 weights as f16, exact: bytes ^ 0x80 spliced under an f16
    // exponent of 2^10 give 1024 + w + 128, less 1152
    float4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
    const half2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
    for (int c = 0; c < MLA_UP_CH; c++) {
        if (c >= nch) break;
        const uint32_t ww[4] = {w[c].x ^ 0x80808080u, w[c].y ^ 0x80808080u, w[c].z ^ 0x80808080u, w[c].w ^ 0x80808080u};
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            uint32_t bw[4];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t word = ww[2 * hh + e];
                const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, word, 0x04010400u);
                const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, word, 0x04030402u);
                bw[2 * e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, p0) + off);
                bw[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, p1) + off);
            }
            const int k0 = min(c * 64 + 16 * q + 8 * hh, 504);  // k >= R: zero weight (padding)
            const uint4 ah = *(const uint4*)&olh[0][k0], al = *(const uint4*)&olh[1][k0];
            const uint4 z = make_uint4(0u, 0u, 0u, 0u);
            const half8_t B8 = __builtin_bit_cast(half8_t, make_uint4(bw[0], bw[1], bw[2], bw[3]));
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, r == 0 ? ah : z), B8, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, r == 0 ? al : z), B8, d, 0, 0, 0);
        }
    }
    if (q == 0) {  // D[row 0][col r]: lane (0, r), element 0
        const int n = tt * 16 + r;
        out[((size_t)b * MLA_H + h) * dv + n] = __builtin_amdgcn_ldexpf(d[0], oe) * usc;
    }
}

template <int W>
static void launch_mla_attn_w(dim3 grid, size_t lds, hipStream_t s, const uint16_t* qa, const uint16_t* cache, int L,
                              int R, float sm_scale, int n_splits, float* part) {
    static std::mutex mu;
    static size_t granted = 0;  // largest dynamic LDS size set so far
    {
        std::lock_guard<std::mutex> lock(mu);
        if (lds > granted) {
            TH_HIP(hipFuncSetAttribute((const void*)mla_attn_kernel<W>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds));
            granted = lds;
        }
    }
    TH_LAUNCH(mla_attn_kernel<W>, grid, dim3(MLA_THREADS), lds, s, qa, cache, L, R, sm_scale, n_splits, part);
}

template <int... Ks>
static void launch_mla_attn_any(std::integer_sequence<int, Ks...>, int W, dim3 grid, size_t lds, hipStream_t s,
                                const uint16_t* qa, const uint16_t* cache, int L, int R, float sm_scale, int n_splits,
                                float* part) {
    bool done = false;
    ((W == 32 * (Ks + 1) ? (launch_mla_attn_w<32 * (Ks + 1)>(grid, lds, s, qa, cache, L, R, sm_scale, n_splits, part),
                            done = true)
                         : false),
     ...);
    TH_REQUIRE(done, "latent row width must be a multiple of 32 up to 576");
}

static void launch_mla_attn(size_t W, dim3 grid, size_t lds, hipStream_t s, const uint16_t* qa, const uint16_t* cache,
                            int L, int R, float sm_scale, int n_splits, float* part) {
    launch_mla_attn_any(std::make_integer_sequence<int, MLA_WMAX / 32>{}, (int)W, grid, lds, s, qa, cache, L, R,
                        sm_scale, n_splits, part);
}

}  // namespace th

using namespace th;

extern "C" int th_mla_decode(th_device* dev, const th_buffer* q_nope, const th_buffer* q_rope, const th_buffer* cache,
                             size_t B, size_t H, size_t L, size_t dn, size_t dr, size_t r, size_t dv,
                             const th_qweight* w_uk, const th_qweight* w_uv, float sm_scale, th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && q_nope && q_rope && cache && w_uk && w_uv && out, "null argument");
    TH_REQUIRE(H == MLA_H, "this kernel serves 16 heads");
    TH_REQUIRE(r % 16 == 0 && r <= 512 && dr % 8 == 0 && (r + dr) % 32 == 0 && r + dr <= MLA_WMAX,
               "latent widths: r <= 512, r + dr <= 576, (r + dr) % 32 == 0");
    TH_REQUIRE(L > 0 && B > 0 && B <= 16, "1 <= B <= 16 sequences");
    TH_REQUIRE(w_uk->bits == 8 && w_uk->per_row && w_uk->rows == H * r && w_uk->cols == dn, "w_uk must be q8 rowwise [H*r][dn]");
    TH_REQUIRE(w_uv->bits == 8 && w_uv->per_row && w_uv->rows == H * dv && w_uv->cols == r, "w_uv must be q8 rowwise [H*dv][r]");
    TH_REQUIRE(r % 16 == 0 && dv % 16 == 0 && dv <= 128, "r and dv must be multiples of 16, dv <= 128");
    require_len(q_nope, TH_F32, B * H * dn, "q_nope");
    require_len(q_rope, TH_F32, B * H * dr, "q_rope");
    require_len(cache, TH_BF16, B * L * (r + dr), "cache");
    require_len(out, TH_F32, B * H * dv, "out");
    hipStream_t s = dev->stream;
    const size_t W = r + dr;
    const int n_splits = (int)ceil_div(L, (size_t)MLA_SPLIT);
    TH_REQUIRE(n_splits <= 64, "L above 8192 positions");
    TH_REQUIRE(dn % 4 == 0 && dn <= 64 * MLA_ABS_CH, "qk_nope width must be a multiple of 4, at most 256");
    // workspace: A operand, split records, o_lat
    const size_t qa_bytes = B * 2 * H * W * 2;
    const size_t part_bytes = B * (size_t)n_splits * H * (r + 2) * 4;
    char* ws = (char*)device_scratch(dev, round_up(qa_bytes, 256) + part_bytes);
    uint16_t* qa = (uint16_t*)ws;
    float* part = (float*)(ws + round_up(qa_bytes, 256));
    // 1. absorb
    TH_LAUNCH(mla_absorb_kernel, dim3((unsigned)ceil_div(H * r / 16, (size_t)4)), dim3(256), 0, s,
                       (const uint8_t*)w_uk->data, (const float*)w_uk->scales, (int)r, (int)dn, (int)(w_uk->Kp / 64),
                       (int)B, (const float*)q_nope->ptr, (const float*)q_rope->ptr, (int)dr, qa);
    TH_LAUNCH_CHECK();
    // 2. latent attention
    const size_t lds = (size_t)MLA_CHUNK * (W + 8) * 2 + (size_t)MLA_WAVES * MLA_H * MLA_CHUNK * 4 +
                       (size_t)MLA_H * MLA_PS * 4;
    TH_REQUIRE(lds <= 150 * 1024, "latent chunk does not fit LDS");
    launch_mla_attn(W, dim3((unsigned)B, (unsigned)n_splits), lds, s, qa, (const uint16_t*)cache->ptr, (int)L, (int)r,
                    sm_scale, n_splits, part);
    TH_LAUNCH_CHECK();
    // 3. merge + up-projection
    const unsigned groups = (unsigned)ceil_div(dv / 16, (size_t)4);  // four 16-row tiles per workgroup
    TH_LAUNCH(mla_merge_up_kernel, dim3((unsigned)H, (unsigned)B, groups), dim3(MLA_UP_THREADS), 0, s, part,
                       n_splits, (int)r, (const uint8_t*)w_uv->data, (const float*)w_uv->scales, (int)dv,
                       (int)(w_uv->Kp / 64), (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}
