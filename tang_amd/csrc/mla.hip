// MLA (multi-head latent attention) decode, absorbed form (DeepSeek-V2-Lite shape: 16 heads, latent 512, rope 64).
// The reference has no MLA; this is the definition of DeepSeek-V2's absorbed
// decode with the reference's kv_attention semantics (cpu.rs:257: softmax of
// scaled scores over every cached position, f32 accumulation):
//   q_lat[b,h] = W_UK[h] . q_nope[b,h]                (int8, per-row scale)
//   s[b,h,t]   = (q_lat . c[b,t,:r] + q_rope . c[b,t,r:]) * sm_scale
//   o_lat[b,h] = sum_t softmax_t(s) c[b,t,:r]
//   out[b,h]   = W_UV[h] . o_lat[b,h]                 (int8, per-row scale)
// Three launches:
//   1. absorb: q = [q_lat ; q_rope] (f32) emitted as hi + lo bf16 parts
//      (16 significant bits) as the MFMA A operand [B][2][H][r+dr];
//   2. one workgroup per (sequence, split of 128 positions) serves all 16
//      heads from one pass over the latent cache, in chunks of 64 positions
//      staged in LDS (the next chunk is loaded into registers meanwhile):
//      scores on v_mfma_f32_16x16x32_bf16 (heads x positions; each wave owns
//      a quarter of the k-steps and keeps its A operand in registers; partial
//      scores are summed in LDS), online softmax per head, then P.C on the
//      same MFMA (P as hi + lo bf16, C exact bf16), one {max, sum, o_lat}
//      record per split;
//   3. per (head, sequence): the split merge in LDS, then the up-projection
//      through W_UV.
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

// Per-head batched int8 GEMV over the tiled q8 layout (16 rows x 64 k per
// tile, lane q*16+r holds k 16q..16q+15 of row r), per-row scales:
// y[b][h][n] = scale[h*rows+n] * sum_k q[h*rows+n][k] * x[b][h][k].
// One workgroup: head h, 16 output rows, all B inputs.  Thread (row r,
// slice kq) owns the 16-value pieces kq, kq+16, ... of its row: every weight
// byte is loaded once, up front; partial sums meet in LDS.
constexpr int MLA_GEMV_PIECES = 4;  // pieces per thread: K <= 1024
constexpr int MLA_GEMV_X4 = 8;      // float4 activation loads per thread: B * K <= 8192

template <int MODE>  // 0: absorb (write the hi / lo bf16 A operand), 1: plain f32 out
__global__ __launch_bounds__(256) void mla_q8_heads_kernel(const uint8_t* __restrict__ wq, const float* __restrict__ wsc,
                                                           int rows_per_head, int K, int Kp, int B, int H,
                                                           const float* __restrict__ x, int ldx_b, int ldx_h,
                                                           float* __restrict__ y, uint16_t* __restrict__ qa,
                                                           const float* __restrict__ q_rope, int dr) {
    extern __shared__ float sm[];
    const int NP = Kp >> 4, NCH = Kp >> 6;
    float* xs = sm;                          // [B][NP][20]: piece-major; the pad puts a wave's 4 slices in different banks
    float* red = sm + (size_t)B * NP * 20;   // [B][16 slices][16 rows]
    const int h = blockIdx.x, t_local = blockIdx.y, tid = threadIdx.x;
    const int r = tid & 15, kq = tid >> 4;
    const int row = h * rows_per_head + t_local * 16 + r;  // row of the stacked matrix
    const int t = row >> 4;                                // its 16-row tile
    uint4 w[MLA_GEMV_PIECES];
#pragma unroll
    for (int j = 0; j < MLA_GEMV_PIECES; j++) {
        const int p = min(kq + 16 * j, NP - 1);  // surplus pieces: loaded, not used
        w[j] = *(const uint4*)(wq + (((size_t)t * NCH + (p >> 2)) * 64 + (p & 3) * 16 + r) * 16);
    }
    const float sc = wsc[row];
    // activations: float4 pieces, every load issued before any is used (a
    // loop of load-then-store would wait out one latency per iteration);
    // surplus threads repeat the last piece, k >= K is zero
    {
        const int K4 = Kp >> 2, n4 = B * K4;
        float4 xv[MLA_GEMV_X4];
#pragma unroll
        for (int u = 0; u < MLA_GEMV_X4; u++) {
            const int i = min(tid + 256 * u, n4 - 1);
            const int b = i / K4, k = (i - b * K4) * 4;
            xv[u] = *(const float4*)(x + (size_t)b * ldx_b + (size_t)h * ldx_h + min(k, K - 4));
            if (k >= K) xv[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < MLA_GEMV_X4; u++) {
            const int i = min(tid + 256 * u, n4 - 1);
            const int b = i / K4, k = (i - b * K4) * 4;
            *(float4*)(xs + (b * NP + (k >> 4)) * 20 + (k & 15)) = xv[u];
        }
    }
    // weights as f32 once (surplus pieces contribute zero)
    float wf[MLA_GEMV_PIECES][16];
#pragma unroll
    for (int j = 0; j < MLA_GEMV_PIECES; j++) {
        const bool live = kq + 16 * j < NP;
        const uint32_t wj[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
        for (int e = 0; e < 16; e++) wf[j][e] = live ? (float)(int8_t)(wj[e >> 2] >> (8 * (e & 3))) : 0.0f;
    }
    __syncthreads();
    for (int b = 0; b < B; b++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < MLA_GEMV_PIECES; j++) {
            const float4* xp = (const float4*)(xs + (b * NP + min(kq + 16 * j, NP - 1)) * 20);
#pragma unroll
            for (int e4 = 0; e4 < 4; e4++) {
                const float4 xv = xp[e4];
                acc = __builtin_fmaf(wf[j][4 * e4], xv.x, acc);
                acc = __builtin_fmaf(wf[j][4 * e4 + 1], xv.y, acc);
                acc = __builtin_fmaf(wf[j][4 * e4 + 2], xv.z, acc);
                acc = __builtin_fmaf(wf[j][4 * e4 + 3], xv.w, acc);
            }
        }
        red[(b * 16 + kq) * 16 + r] = acc;
    }
    __syncthreads();
    if (tid >= 16 * B) return;
    const int b = tid >> 4;  // r = tid & 15 as above
    float v = 0.0f;
#pragma unroll
    for (int k2 = 0; k2 < 16; k2++) v += red[(b * 16 + k2) * 16 + r];
    v *= sc;
    const int n = t_local * 16 + r;
    if (MODE == 0) {
        // A operand row (b, part, h): q_lat then q_rope, as hi / lo parts
        const int R = rows_per_head, W = R + dr;
        const uint32_t hi = f32_to_bf16_bits(v);
        const uint32_t lo = f32_to_bf16_bits(v - bf16_bits_to_f32(hi));
        qa[(((size_t)b * 2 + 0) * H + h) * W + n] = (uint16_t)hi;
        qa[(((size_t)b * 2 + 1) * H + h) * W + n] = (uint16_t)lo;
        if (t_local == 0) {
            for (int i = r; i < dr; i += 16) {
                const float qr = q_rope[((size_t)b * H + h) * dr + i];
                const uint32_t h2 = f32_to_bf16_bits(qr);
                const uint32_t l2 = f32_to_bf16_bits(qr - bf16_bits_to_f32(h2));
                qa[(((size_t)b * 2 + 0) * H + h) * W + R + i] = (uint16_t)h2;
                qa[(((size_t)b * 2 + 1) * H + h) * W + R + i] = (uint16_t)l2;
            }
        }
    } else {
        y[((size_t)b * H + h) * rows_per_head + n] = v;
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
    __shared__ float m_run[MLA_H], l_run[MLA_H], resc[MLA_H];
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
    if (tid < MLA_H) { m_run[tid] = -INFINITY; l_run[tid] = 0.0f; }

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
            uint4 bq[4];
#pragma unroll
            for (int pt = 0; pt < 4; pt++) bq[pt] = *(const uint4*)(cs + (size_t)(pt * 16 + r) * WP + ks * 32 + q * 8);
#pragma unroll
            for (int pp = 0; pp < 2; pp++)
#pragma unroll
                for (int pt = 0; pt < 4; pt++)
                    d[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, areg[i][pp]),
                                                                    __builtin_bit_cast(bf16x8_t, bq[pt]), d[pt], 0, 0, 0);
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
            const float mold = m_run[hh];
            const float mnew = fmaxf(mold, cmax);
            float lsum = 0.0f;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float e = 2 * pg + j < clen ? expf(sv[j] - mnew) : 0.0f;
                ps[hh * MLA_PS + 2 * pg + j] = e;
                lsum += e;
            }
            lsum = group_sum<32>(lsum);
            lds_barrier();  // every thread has read m_run
            if (pg == 0) {
                const float f = expf(mold - mnew);
                resc[hh] = f;
                l_run[hh] = l_run[hh] * f + lsum;
                m_run[hh] = mnew;
            }
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
            for (int e = 0; e < 4; e++) {
                const uint32_t ha = f32_to_bf16_bits(pv[2 * e]), hb = f32_to_bf16_bits(pv[2 * e + 1]);
                const uint32_t la = f32_to_bf16_bits(pv[2 * e] - bf16_bits_to_f32(ha));
                const uint32_t lb = f32_to_bf16_bits(pv[2 * e + 1] - bf16_bits_to_f32(hb));
                h2[e] = ha | (hb << 16);
                l2[e] = la | (lb << 16);
            }
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
    if (tid < MLA_H) {
        rec[(size_t)tid * (R + 2)] = m_run[tid];
        rec[(size_t)tid * (R + 2) + 1] = l_run[tid];
    }
}

// Split merge fused with the W_UV up-projection: workgroup (head h,
// sequence b).  o_lat[b][h] = sum_s w_s acc_s / sum_s w_s l_s (split order,
// w_s = exp(m_s - max m)) is built in LDS, then out[b][h][n] = scale_n *
// sum_k W_UV[h*dv + n][k] o_lat[k]: thread (row n, half of the 64-k chunks),
// halves summed in order; the W_UV and record loads are all issued at the
// start.  r <= 512, dv <= 128, n_splits <= 64.
constexpr int MLA_UP_THREADS = 256;

__global__ __launch_bounds__(MLA_UP_THREADS) void mla_merge_up_kernel(const float* __restrict__ part, int n_splits,
                                                                     int R, const uint8_t* __restrict__ wq,
                                                                     const float* __restrict__ wsc, int dv, int Kp,
                                                                     float* __restrict__ out) {
    __shared__ __align__(16) float olat[512];
    __shared__ float wts[64];
    __shared__ float Lsh;
    __shared__ float half_sum[2][128];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const float* recs = part + (size_t)b * n_splits * MLA_H * (R + 2);
    constexpr int DPT = 2, SB = 32;    // dims per thread, splits per load round
    constexpr int CPT = 4;             // 64-k chunks of W_UV per thread (r <= 512)
    // the up-projection's weights do not depend on the merge: load them first
    const int n = tid & 127, kh = tid >> 7, NCH = Kp >> 6;
    const int row = h * dv + min(n, dv - 1), t = row >> 4, r = row & 15;
    uint4 w4[CPT][4];
#pragma unroll
    for (int ci = 0; ci < CPT; ci++) {
        const int c = min(kh * CPT + ci, NCH - 1);  // chunks past K: loaded, multiplied by zero below
#pragma unroll
        for (int q = 0; q < 4; q++) w4[ci][q] = *(const uint4*)(wq + (((size_t)t * NCH + c) * 64 + q * 16 + r) * 16);
    }
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
        const float w = tid < n_splits ? expf(m - M) : 0.0f;
        const float L = wave_sum(w * l);
        wts[tid] = w;
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
#pragma unroll
    for (int j = 0; j < DPT; j++) olat[tid + 256 * j] = tid + 256 * j < R ? a[j] / Lsh : 0.0f;
    __syncthreads();
    // out[n] = scale_n * sum_k W_UV[n][k] o_lat[k]; thread (row n, half kh of the chunks)
    float acc = 0.0f;
#pragma unroll
    for (int ci = 0; ci < CPT; ci++) {
        const int c = kh * CPT + ci;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t ww[4] = {w4[ci][q].x, w4[ci][q].y, w4[ci][q].z, w4[ci][q].w};
#pragma unroll
            for (int e4 = 0; e4 < 4; e4++) {
                const int k0 = c * 64 + q * 16 + e4 * 4;  // olat is zero past R (cleared below), 512 entries
                const float4 o = (c < NCH) ? *(const float4*)&olat[min(k0, 508)] : make_float4(0.f, 0.f, 0.f, 0.f);
                const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                for (int e = 0; e < 4; e++)
                    acc = __builtin_fmaf((float)(int8_t)(ww[e4] >> (8 * e)), ov[e], acc);
            }
        }
    }
    half_sum[kh][n] = acc;
    __syncthreads();
    if (tid < dv) out[((size_t)b * MLA_H + h) * dv + tid] = (half_sum[0][tid] + half_sum[1][tid]) * wsc[h * dv + tid];
}

static size_t head_gemv_lds(size_t B, size_t Kp) { return (B * (Kp / 16) * 20 + B * 256) * 4; }

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
    hipLaunchKernelGGL(mla_attn_kernel<W>, grid, dim3(MLA_THREADS), lds, s, qa, cache, L, R, sm_scale, n_splits, part);
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
    TH_REQUIRE(dn % 4 == 0 && B * w_uk->Kp <= 8192 && B * w_uv->Kp <= 8192,
               "qk_nope width must be a multiple of 4, and B * width <= 8192 for both projections");
    // workspace: A operand, split records, o_lat
    const size_t qa_bytes = B * 2 * H * W * 2;
    const size_t part_bytes = B * (size_t)n_splits * H * (r + 2) * 4;
    char* ws = (char*)device_scratch(dev, round_up(qa_bytes, 256) + part_bytes);
    uint16_t* qa = (uint16_t*)ws;
    float* part = (float*)(ws + round_up(qa_bytes, 256));
    // 1. absorb
    hipLaunchKernelGGL(mla_q8_heads_kernel<0>, dim3((unsigned)H, (unsigned)(r / 16)), dim3(256), head_gemv_lds(B, w_uk->Kp), s,
                       (const uint8_t*)w_uk->data, (const float*)w_uk->scales, (int)r, (int)dn, (int)w_uk->Kp, (int)B,
                       (int)H, (const float*)q_nope->ptr, (int)(H * dn), (int)dn, (float*)nullptr, qa,
                       (const float*)q_rope->ptr, (int)dr);
    TH_LAUNCH_CHECK();
    // 2. latent attention
    const size_t lds = (size_t)MLA_CHUNK * (W + 8) * 2 + (size_t)MLA_WAVES * MLA_H * MLA_CHUNK * 4 +
                       (size_t)MLA_H * MLA_PS * 4;
    TH_REQUIRE(lds <= 150 * 1024, "latent chunk does not fit LDS");
    launch_mla_attn(W, dim3((unsigned)B, (unsigned)n_splits), lds, s, qa, (const uint16_t*)cache->ptr, (int)L, (int)r,
                    sm_scale, n_splits, part);
    TH_LAUNCH_CHECK();
    // 3. merge + up-projection
    hipLaunchKernelGGL(mla_merge_up_kernel, dim3((unsigned)H, (unsigned)B), dim3(MLA_UP_THREADS), 0, s, part, n_splits,
                       (int)r, (const uint8_t*)w_uv->data, (const float*)w_uv->scales, (int)dv, (int)w_uv->Kp,
                       (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}
