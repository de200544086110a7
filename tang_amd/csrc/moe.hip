// DeepSeek-style MoE FFN layer with int4 group-32 experts (benchmark shape: d 2048, ff 1408, 64 + 2 experts, top-6).
// The reference has no MoE; the layer is composed from its ops:
//   logits = h . W_r^T, p = softmax(logits) (cpu.rs:105-124), the top-k
//   experts by p (first maximum wins, as sampling.rs:184's argmax), weights
//   = p of the chosen experts (not renormalised); each expert is a SwiGLU
//   FFN of int4 linears (q4_matvec semantics, bf16 inputs); out = sum over the
//   token's experts in rank order of w * expert(h) + sum of the shared experts.
//
// Device flow, no host round trip:
//   router logits (token block x expert block)
//   -> top-k (one wave per token: softmax, k wave-wide argmaxes)
//   -> dispatch (one block: per-expert slots in token order and work items
//      of at most 8 rows for decode-sized batches, else 64; shared experts
//      take every token)
//   -> grouped gate/up GEMV (T <= 64) or MFMA GEMM (epilogue SwiGLU, bf16
//      per slot)
//   -> grouped down GEMV or MFMA GEMM (f32 per slot)
//   -> combine (per token, rank order, then shared).
// Grouped launches size the grid for the worst case; work items past the
// real ones return at once.
#include <mutex>
#include <type_traits>
#include <vector>

#include "capi_util.hpp"
#include "ops.hpp"
#include "qlinear.hpp"

namespace th {

constexpr int MOE_MAX_K = 16;
constexpr int MOE_MIN_ROWS = 8;     // rows per work item for decode-sized batches
constexpr int MOE_SMALL_T = 64;     // batches up to this use MOE_MIN_ROWS, larger ones 16
constexpr int MOE_MAX_E = 256;      // routed experts (top-k runs in one wave, 4 per lane)
constexpr int MOE_MAX_NE = 1024;    // routed + shared
constexpr int ROUTER_TOK = 4;       // tokens per router workgroup
constexpr int ROUTER_EXP = 4;       // experts per router workgroup (one per wave)

struct MoeWork { int expert, slot0, rows, pad; };

// Router logits: workgroup (token block, expert block); wave w takes expert
// w of the block for ROUTER_TOK tokens (decode-sized batches then spread over
// E * T / 16 workgroups instead of a handful); lane covers 8 consecutive
// elements of each 512-element stride of d (f32 products, f32 sums, in
// stride order).  The loads of ROUTER_ROUND elements of d are all issued
// before their first product, so the workgroup waits for memory once per
// round (once at d <= ROUTER_ROUND).
constexpr int ROUTER_ROUND = 2048;
__global__ __launch_bounds__(256) void moe_router_kernel(const uint16_t* __restrict__ h, const float* __restrict__ wr,
                                                         int T, int E, int d, float* __restrict__ logits) {
    constexpr int NS = ROUTER_ROUND / 512;
    constexpr int EPW = ROUTER_EXP / 4;  // experts per wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * ROUTER_TOK, e0 = blockIdx.y * ROUTER_EXP + wave * EPW;
    float acc[ROUTER_TOK][EPW];
#pragma unroll
    for (int a = 0; a < ROUTER_TOK; a++)
#pragma unroll
        for (int b = 0; b < EPW; b++) acc[a][b] = 0.0f;
    for (int base = 0; base < d; base += ROUTER_ROUND) {
    uint4 hx[NS][ROUTER_TOK];
    float4 wv[NS][EPW][2];
#pragma unroll
    for (int st = 0; st < NS; st++) {  // clamped addresses: pieces past d re-read the row start (not used)
        const int k0 = (base + st * 512 + lane * 8 < d) ? base + st * 512 + lane * 8 : 0;
#pragma unroll
        for (int a = 0; a < ROUTER_TOK; a++)
            hx[st][a] = *(const uint4*)(h + (size_t)min(t0 + a, T - 1) * d + k0);
#pragma unroll
        for (int b = 0; b < EPW; b++) {
            const float* wp = wr + (size_t)min(e0 + b, E - 1) * d + k0;
            wv[st][b][0] = *(const float4*)wp;
            wv[st][b][1] = *(const float4*)(wp + 4);
        }
    }
#pragma unroll
    for (int st = 0; st < NS; st++) {
        if (base + st * 512 + lane * 8 >= d) continue;
        float x[ROUTER_TOK][8];
#pragma unroll
        for (int a = 0; a < ROUTER_TOK; a++) {
            const uint32_t w4[4] = {hx[st][a].x, hx[st][a].y, hx[st][a].z, hx[st][a].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                x[a][2 * j] = __uint_as_float(w4[j] << 16);
                x[a][2 * j + 1] = __uint_as_float(w4[j] & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int b = 0; b < EPW; b++) {
            const float w8[8] = {wv[st][b][0].x, wv[st][b][0].y, wv[st][b][0].z, wv[st][b][0].w,
                                 wv[st][b][1].x, wv[st][b][1].y, wv[st][b][1].z, wv[st][b][1].w};
#pragma unroll
            for (int a = 0; a < ROUTER_TOK; a++)
#pragma unroll
                for (int j = 0; j < 8; j++) acc[a][b] = __builtin_fmaf(x[a][j], w8[j], acc[a][b]);
        }
    }
    }  // rounds
#pragma unroll
    for (int a = 0; a < ROUTER_TOK; a++)
#pragma unroll
        for (int b = 0; b < EPW; b++) {
            const float v = wave_sum(acc[a][b]);
            if (lane == 0 && t0 + a < T && e0 + b < E) logits[(size_t)(t0 + a) * E + e0 + b] = v;
        }
}

// Softmax over the E logits (max, exp, sum, scale by 1/sum, as cpu.rs:105-124)
// and top-k by probability, first maximum on ties (sampling.rs:184-194), for
// token t by one wave; lane holds experts lane, lane+64, ...  Repeated
// argmax picks experts in order of (probability descending, index
// ascending), so each expert's pick index is its rank in that order: the
// number of experts with a larger probability, or an equal one and a lower
// index.  Every lane counts its experts' ranks against the probabilities in
// the wave's LDS row sp[E] (no serial reductions); the expert of rank r < k
// writes entry r of the token to idx[r], w[r].
// PL: expert slots per lane, ceil(E / 64) (a compile-time count, so a
// 64-expert router runs one slot without per-slot guards)
template <int PL>
__device__ __forceinline__ void moe_topk_token(const float* __restrict__ logits, int t, int E, int k, int32_t* idx,
                                               float* w, float* sp) {
    const int lane = threadIdx.x & 63;
    static_assert(PL >= 1 && PL * 64 <= MOE_MAX_E, "slots per lane");
    float p[PL];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PL; i++) {
        const int e = lane + 64 * i;
        p[i] = e < E ? logits[(size_t)t * E + e] : -INFINITY;
        mx = fmaxf(mx, p[i]);
    }
    mx = group_max<64>(mx);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < PL; i++) {
        p[i] = lane + 64 * i < E ? expf(p[i] - mx) : 0.0f;
        sum += p[i];
    }
    sum = group_sum<64>(sum);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < PL; i++) p[i] = p[i] * inv;
    if constexpr (PL == 1) {
        // One expert per lane: k rounds of a wave argmax (DPP maximum, then
        // the lowest lane holding it), the same order as the ranks below at
        // a fifth of the instructions (the rank count compares every lane
        // with all 64 experts).
        float v = lane < E ? p[0] : -INFINITY;
        for (int r = 0; r < k; r++) {  // k <= E
            const float m = group_max<64>(v);
            const int win = (int)__builtin_ctzll(__ballot(v == m));
            if (lane == 0) {
                idx[r] = win;
                w[r] = m;
            }
            if (lane == win) v = -INFINITY;
        }
        return;
    }
    const int E16 = (E + 15) & ~15;  // sp is padded to whole 16-float rounds with -inf
#pragma unroll
    for (int i = 0; i < PL; i++) {
        const int e = lane + 64 * i;
        if (e < E16) sp[e] = e < E ? p[i] : -INFINITY;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    int rank[PL];
#pragma unroll
    for (int i = 0; i < PL; i++) rank[i] = 0;
    for (int j0 = 0; j0 < E16; j0 += 16) {
        float pj[16];  // same addresses in every lane: broadcast reads, all issued first
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float4 v = *(const float4*)(sp + j0 + 4 * u);
            pj[4 * u] = v.x; pj[4 * u + 1] = v.y; pj[4 * u + 2] = v.z; pj[4 * u + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < PL; i++) {
            const int e = lane + 64 * i;
#pragma unroll
            for (int u = 0; u < 16; u++) rank[i] += (pj[u] > p[i] || (pj[u] == p[i] && j0 + u < e)) ? 1 : 0;
        }
    }
#pragma unroll
    for (int i = 0; i < PL; i++)
        if (lane + 64 * i < E && rank[i] < k) {
            idx[rank[i]] = lane + 64 * i;
            w[rank[i]] = p[i];
        }
}

template <int PL>
__global__ __launch_bounds__(256) void moe_topk_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                       int32_t* __restrict__ topk_idx, float* __restrict__ topk_w) {
    __shared__ __align__(16) float sp[4][MOE_MAX_E];
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    moe_topk_token<PL>(logits, t, E, k, topk_idx + (size_t)t * k, topk_w + (size_t)t * k, sp[threadIdx.x >> 6]);
}

// Slot assignment, deterministic: slots are grouped by expert (routed
// experts 0..E-1, then the S shared experts with every token) and, within an
// expert, ordered by entry index t*k + r, i.e. by token.  16 waves each own a
// contiguous range of entries; a wave's 64 lanes find lanes of the same expert
// with eight ballots over the expert id bits, so ranks inside a batch come
// from popcounts, and per-(wave, expert) counts give each wave its first slot.
// Work items cover at most `rows` slots of one expert.
// With logits set (T * k <= MOE_FUSED_ENTRIES), the block first runs the
// top-k itself (wave w takes tokens w, w+16, ...), writes topk_idx/topk_w
// and keeps the indices in LDS for the slot passes: one launch instead of two
// for decode-sized batches.
constexpr int MOE_FUSED_ENTRIES = 1024;
// Inclusive prefix sum over the 64 lanes with DPP: row_shr 1, 2, 4, 8
// within each row of 16 (lanes without a source add 0), then row_bcast:15
// and row_bcast:31 carry each row's total into the rows above it.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
    return x;
}

template <int PL>
__global__ __launch_bounds__(1024) void moe_dispatch_kernel(const float* __restrict__ logits, int32_t* __restrict__ topk_idx_out,
                                                            float* __restrict__ topk_w_out,
                                                            const int32_t* __restrict__ topk_idx_in, int T, int k, int E,
                                                            int S, int rows, int* __restrict__ offsets,
                                                            int* __restrict__ slot_token, int* __restrict__ token_slot,
                                                            MoeWork* __restrict__ work, int max_work) {
    __shared__ __align__(16) int cnt[16][MOE_MAX_E];  // per-wave counts, then per-wave running slots
    __shared__ int tot[MOE_MAX_NE], base[MOE_MAX_NE + 1], wbase[MOE_MAX_NE + 1];
    __shared__ int32_t sidx[MOE_FUSED_ENTRIES];
    __shared__ float sw[MOE_FUSED_ENTRIES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, NE = E + S;
    const int32_t* topk_idx = topk_idx_in;
    if (logits) {
        // the wave's row of cnt (zeroed below) holds its probabilities
        for (int t = wave; t < T; t += 16)
            moe_topk_token<PL>(logits, t, E, k, sidx + t * k, sw + t * k, (float*)cnt[wave]);
        __syncthreads();
        for (int i = tid; i < T * k; i += 1024) {
            topk_idx_out[i] = sidx[i];
            topk_w_out[i] = sw[i];
        }
        topk_idx = sidx;
    }
    const int n = T * k, per = (n + 15) / 16;
    const int lo = wave * per, hi = min(n, lo + per);
    for (int i = tid; i < 16 * MOE_MAX_E; i += 1024) (&cnt[0][0])[i] = 0;
    __syncthreads();
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    auto same_expert = [&](int e, bool live) {
        uint64_t m = __ballot(live);
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const uint64_t bit = __ballot(live && ((e >> b) & 1));
            m &= ((e >> b) & 1) ? bit : ~bit;
        }
        return m;
    };
    for (int i0 = lo; i0 < hi; i0 += 64) {  // pass 1: counts
        const int i = i0 + lane;
        const bool live = i < hi;
        const int e = live ? topk_idx[i] : 0;
        const uint64_t m = same_expert(e, live);
        if (live && (m & below) == 0) cnt[wave][e] += __popcll(m);  // the expert's lowest lane
    }
    __syncthreads();
    for (int e = tid; e < NE; e += 1024) {
        int c = 0;
        if (e < E)
            for (int w = 0; w < 16; w++) c += cnt[w][e];
        else
            c = T;
        tot[e] = c;
    }
    __syncthreads();
    {  // exclusive scans of slots and of work items over experts (NE <= 1024: one per thread)
        __shared__ int wsum[2][16];
        const int tv = tid < NE ? tot[tid] : 0;
        const int wv = (tv + rows - 1) / rows;
        const int a = wave_incl_scan(tv), b = wave_incl_scan(wv);  // inclusive scans within the wave
        if (lane == 63) { wsum[0][wave] = a; wsum[1][wave] = b; }
        __syncthreads();
        int oa = 0, ob = 0;
        for (int w = 0; w < wave; w++) { oa += wsum[0][w]; ob += wsum[1][w]; }
        if (tid < NE) { base[tid] = oa + a - tv; wbase[tid] = ob + b - wv; }
        if (tid == NE - 1) { base[NE] = oa + a; wbase[NE] = ob + b; }
    }
    __syncthreads();
    for (int e = tid; e <= NE; e += 1024) offsets[e] = base[e];
    for (int e = tid; e < E; e += 1024) {  // per-wave first slots
        int o = base[e];
        for (int w = 0; w < 16; w++) {
            const int c = cnt[w][e];
            cnt[w][e] = o;
            o += c;
        }
    }
    __syncthreads();
    for (int i0 = lo; i0 < hi; i0 += 64) {  // pass 2: slots
        const int i = i0 + lane;
        const bool live = i < hi;
        const int e = live ? topk_idx[i] : 0;
        const uint64_t m = same_expert(e, live);
        if (live) {
            const int slot = cnt[wave][e] + __popcll(m & below);
            token_slot[i] = slot;
            slot_token[slot] = i / k;
        }
        __builtin_amdgcn_wave_barrier();
        if (live && (m & below) == 0) cnt[wave][e] += __popcll(m);
        __builtin_amdgcn_wave_barrier();
    }
    for (int s = 0; s < S; s++)
        for (int t = tid; t < T; t += 1024) slot_token[base[E + s] + t] = t;
    for (int e = tid; e < NE; e += 1024) {
        const int c = tot[e];
        for (int j = 0, w = wbase[e]; j < c; j += rows, w++)
            if (w < max_work) work[w] = MoeWork{e, base[e] + j, min(rows, c - j), 0};
    }
    for (int w = wbase[NE] + tid; w < max_work; w += 1024) work[w] = MoeWork{-1, 0, 0, 0};
}

// Grouped GEMV source: workgroup -> (work item, tile of that expert's matrix).
// A workgroup takes MOE_TPW consecutive tiles of one work item's expert, so
// the work item -> expert -> weights lookup and the activation staging are
// paid once per MOE_TPW tiles.
constexpr int MOE_TPW = 8;

struct MoeSrc {
    static constexpr bool GROUPED = true;
    static constexpr int TPW = MOE_TPW;
    const MoeWork* work;
    const uint4* const* wdata;
    const _Float16* const* wscales;
    const int* slot_token;  // null: activation rows are the slots themselves
    int tiles;              // 16-row tiles per expert matrix
    int wg_per_item;        // ceil(tiles / TPW)
    int slot0 = 0, nt = 1;
    template <typename ST>
    __device__ __forceinline__ bool select(int bid, const uint4*& wt, const ST*& sc, int& t, int& mrows) {
        const MoeWork w = work[bid / wg_per_item];
        if (w.expert < 0) return false;
        t = (bid % wg_per_item) * TPW;
        nt = min(TPW, tiles - t);
        wt = wdata[w.expert];
        sc = (const ST*)wscales[w.expert];
        mrows = w.rows;
        slot0 = w.slot0;
        return true;
    }
    __device__ __forceinline__ int tiles_here() const { return nt; }
    __device__ __forceinline__ int x_row(int m) const { return slot_token ? slot_token[slot0 + m] : slot0 + m; }
    __device__ __forceinline__ int out_row(int m) const { return slot0 + m; }
};

// Grouped MFMA GEMM source (prefill-sized batches): workgroup row block =
// one work item of at most 64 slots of one expert.
struct MoeGemmSrc {
    static constexpr bool GROUPED = true;
    const MoeWork* work;
    const uint4* const* wdata;
    const _Float16* const* wscales;
    const int* const* wexps;  // per-expert th_qweight::row_exp
    const int* slot_token;  // null: activation rows are the slots themselves
    int slot0 = 0;
    template <typename ST>
    __device__ __forceinline__ bool select(int by, int, const uint4*& wt, const ST*& sc, const int*& wexp,
                                           int& mrows) {
        const MoeWork w = work[by];
        if (w.expert < 0) return false;
        wt = wdata[w.expert];
        sc = (const ST*)wscales[w.expert];
        wexp = wexps[w.expert];
        mrows = w.rows;
        slot0 = w.slot0;
        return true;
    }
    __device__ __forceinline__ int x_row(int m) const { return slot_token ? slot_token[slot0 + m] : slot0 + m; }
    __device__ __forceinline__ int out_row(int m) const { return slot0 + m; }
};

// GEMM epilogues.  D fragment rows n0..n0+3 = 4q..4q+3 of a 16-row tile, so
// a gate row (tile rows 0..7, lanes q < 2) finds its up row (8 further) in
// lane + 32.
struct EpiGemmMoeSwiGLU {
    uint16_t* hbuf;
    int ff;
    __device__ __forceinline__ void operator()(int slot, int n0, int, bool live, const float4_t& v) const {
        float up[4];
#pragma unroll
        for (int i = 0; i < 4; i++) up[i] = __shfl_xor(v[i], 32, 64);
        const int rr = n0 & 15;
        if (!live || rr >= 8) return;
#pragma unroll
        for (int i = 0; i < 4; i++)
            hbuf[(size_t)slot * ff + (n0 >> 4) * 8 + rr + i] = f32_to_bf16_rne(swiglu_f64(v[i], up[i]));  // f64 here: the f32 form measured 2% slower in this GEMM
    }
};

struct EpiGemmMoeStore {
    float* y;
    int d;
    __device__ __forceinline__ void operator()(int slot, int n0, int N, bool live, const float4_t& v) const {
        if (!live) return;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (n0 + i < N) y[(size_t)slot * d + n0 + i] = v[i];
    }
};

// Gate/up tiles hold gate rows 8b..8b+7 then up rows 8b..8b+7 (as in the
// decode engine): bf16(swiglu(g, u)) per slot.
struct EpiMoeSwiGLU : EpiNoFinish {
    uint16_t* hbuf; int ff;
    __device__ __forceinline__ void operator()(int slot, int n, float v, const float* tile, float*) const {
        const int rr = n & 15;
        if (rr < 8) hbuf[(size_t)slot * ff + (n >> 4) * 8 + rr] = swiglu_bf16(v, tile[rr + 8]);
    }
};

struct EpiMoeStore : EpiNoFinish {
    float* y; int d;
    __device__ __forceinline__ void operator()(int slot, int n, float v, const float*, float*) const {
        y[(size_t)slot * d + n] = v;
    }
};

// out[tk][n..n+3] = sum_r w[tk][r] * y[slot(tk, r)] + sum_s y[shared slot]
// (rank order, then shared experts, f32).  Every slot row of a round of
// eight is loaded before the first FMA, so a token pays one memory latency
// per round rather than one per rank; any number of shared experts.
__device__ __forceinline__ float4 moe_combine4(const float* __restrict__ y, const int* __restrict__ token_slot,
                                               const float* __restrict__ topk_w, const int* __restrict__ offsets,
                                               int tk, int n, int k, int E, int S, int d) {
    auto load4 = [&](int slot) { return *(const float4*)(y + (size_t)slot * d + n); };
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int r0 = 0; r0 < k; r0 += 8) {
        float4 v[8];
        float w[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {  // past k: re-read the last rank (not used)
            const int r = min(r0 + u, k - 1);
            w[u] = topk_w[(size_t)tk * k + r];
            v[u] = load4(token_slot[tk * k + r]);
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (r0 + u < k) {
                acc.x = __builtin_fmaf(w[u], v[u].x, acc.x);
                acc.y = __builtin_fmaf(w[u], v[u].y, acc.y);
                acc.z = __builtin_fmaf(w[u], v[u].z, acc.z);
                acc.w = __builtin_fmaf(w[u], v[u].w, acc.w);
            }
    }
    for (int s0 = 0; s0 < S; s0 += 8) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = load4(offsets[E + min(s0 + u, S - 1)] + tk);
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (s0 + u < S) {
                acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
            }
    }
    return acc;
}

// Combine: workgroup (token, 1024 outputs), each thread four consecutive outputs
// (moe_combine4).
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y, const int* __restrict__ token_slot,
                                                          const float* __restrict__ topk_w, const int* __restrict__ offsets,
                                                          int k, int E, int S, int d, float* __restrict__ out) {
    const int t = blockIdx.x, n = (blockIdx.y * 256 + threadIdx.x) * 4;
    if (n < d) *(float4*)(out + (size_t)t * d + n) = moe_combine4(y, token_slot, topk_w, offsets, t, n, k, E, S, d);
}

}  // namespace th

using namespace th;

struct th_moe {
    th_device* dev = nullptr;
    size_t d = 0, ff = 0, E = 0, S = 0, k = 0;
    std::vector<th_qweight*> gu, dn;  // E + S each
    float* router = nullptr;
    const uint4** gu_data = nullptr;
    const _Float16** gu_scales = nullptr;
    const uint4** dn_data = nullptr;
    const _Float16** dn_scales = nullptr;
    const int** gu_exps = nullptr;
    const int** dn_exps = nullptr;
    size_t T_cap = 0;
    int *offsets = nullptr, *slot_token = nullptr, *token_slot = nullptr;
    MoeWork* work = nullptr;
    uint16_t* hbuf = nullptr;
    float* ybuf = nullptr;
    float* logits = nullptr;
    bool ready = false;
};

namespace th {

static void moe_free_work(th_moe* m) {
    void* ps[] = {m->offsets, m->slot_token, m->token_slot, m->work, m->hbuf, m->ybuf, m->logits};
    for (void* p : ps)
        if (p) (void)hipFree(p);
    m->offsets = m->slot_token = m->token_slot = nullptr;
    m->work = nullptr;
    m->hbuf = nullptr;
    m->ybuf = nullptr;
    m->logits = nullptr;
    m->T_cap = 0;
}

// Work items of `rows` slots: at most one partial item per expert.
static size_t moe_max_work(const th_moe* m, size_t T, size_t rows) {
    return ceil_div(T * m->k, rows) + m->E + m->S * ceil_div(T, rows);
}

static void moe_reserve(th_moe* m, size_t T) {
    if (T <= m->T_cap) return;
    TH_HIP(hipStreamSynchronize(m->dev->stream));
    moe_free_work(m);
    const size_t slots = T * m->k + m->S * T;
    TH_HIP(hipMalloc(&m->offsets, (m->E + m->S + 1) * sizeof(int)));
    TH_HIP(hipMalloc(&m->slot_token, slots * sizeof(int)));
    TH_HIP(hipMalloc(&m->token_slot, T * m->k * sizeof(int)));
    TH_HIP(hipMalloc(&m->work, moe_max_work(m, T, MOE_MIN_ROWS) * sizeof(MoeWork)));
    TH_HIP(hipMalloc(&m->logits, T * m->E * sizeof(float)));
    TH_HIP(hipMalloc(&m->hbuf, slots * m->ff * sizeof(uint16_t)));
    TH_HIP(hipMalloc(&m->ybuf, slots * m->d * sizeof(float)));
    m->T_cap = T;
}

static void moe_destroy(th_moe* m) {
    if (!m) return;
    device_drain(m->dev);
    for (auto* v : {&m->gu, &m->dn})
        for (th_qweight* w : *v)
            if (w) th_qweight_free(w);
    void* ps[] = {m->router,         (void*)m->gu_data, (void*)m->gu_scales, (void*)m->dn_data,
                  (void*)m->dn_scales, (void*)m->gu_exps, (void*)m->dn_exps};
    for (void* p : ps)
        if (p) (void)hipFree(p);
    moe_free_work(m);
    th_device* d = m->dev;
    delete m;
    device_release(d);
}

template <int MR, typename Epi, int NW>
static void moe_grouped_gemv(const th_moe* m, const th_qweight* w0, const uint4* const* data,
                             const _Float16* const* scales, const uint16_t* x, const int* slot_token, size_t max_work,
                             Epi epi) {
    const int tiles = (int)(w0->Np / 16);
    const int wg_per_item = (tiles + MOE_TPW - 1) / MOE_TPW;
    MoeSrc src{m->work, data, scales, slot_token, tiles, wg_per_item};
    const size_t smem = Q4GemvSmem<MR, NW>::bytes((int)(w0->Kp / 128));
    TH_REQUIRE(smem <= 160 * 1024, "MoE GEMV LDS above 160 KiB");
    // Expert matrices are short (K = 2048 is 16 items of 128): every item of
    // a wave in flight at once.
    auto k = q4_gemv_kernel<MR, false, true, _Float16, Epi, 4, (MR <= 8 ? 3 : 2), NW, false, MoeSrc>;
    static std::mutex mu;
    static size_t done = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (smem > 48 * 1024 && smem > done) {
            TH_HIP(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
            done = smem;
        }
    }
    TH_LAUNCH(k, dim3((unsigned)(max_work * wg_per_item)), dim3(64 * NW), smem, m->dev->stream, (const uint4*)nullptr,
                       (const _Float16*)nullptr, (const void*)x, (int)w0->cols, (int)w0->Kp, (int)w0->rows,
                       (int)w0->cols, epi, NormArgs{}, src);
    TH_LAUNCH_CHECK();
}

constexpr int MOE_GEMM_RT = 2;  // 16-row weight tiles per wave
constexpr int MOE_GEMM_CB = 4;  // 16-slot blocks per work item (64 slots)

template <typename Epi>
static void moe_grouped_gemm(const th_moe* m, const th_qweight* w0, const uint4* const* data,
                             const _Float16* const* scales, const int* const* wexps, const uint16_t* x, size_t x_rows,
                             const int* slot_token, size_t max_work, Epi epi) {
    // the x_rows activation rows (tokens, or slots) prepared once
    const PreparedX xp = prepare_x(m->dev, x, false, x_rows, w0->cols, w0->cols, w0->Kp, m->dev->stream);
    MoeGemmSrc src{m->work, data, scales, wexps, slot_token};
    const unsigned gx = (unsigned)ceil_div(w0->Np / 16, (size_t)(4 * MOE_GEMM_RT));
    TH_LAUNCH((q4_gemm_mfma_kernel<MOE_GEMM_RT, MOE_GEMM_CB, _Float16, MoeGemmSrc, Epi>),
                       dim3(gx, (unsigned)max_work, 1), dim3(256), 0, m->dev->stream, (const uint4*)nullptr,
                       (const _Float16*)nullptr, (const int*)nullptr, xp.x, xp.xexp, epi, src, (int)w0->rows,
                       (int)w0->cols, (int)w0->Kp, (int)w0->Kp, (int)(w0->Kp / 128));
    TH_LAUNCH_CHECK();
}

}  // namespace th

extern "C" {

int th_moe_create(th_device* dev, size_t d, size_t ff, size_t E, size_t S, size_t k, th_moe** out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && out, "null argument");
    TH_REQUIRE(d > 0 && ff > 0 && E > 0 && k > 0 && k <= E && k <= MOE_MAX_K, "bad MoE shape");
    TH_REQUIRE(E <= MOE_MAX_E && E + S <= MOE_MAX_NE, "at most 256 routed and 1024 total experts");
    TH_REQUIRE(ff % 8 == 0 && d % 8 == 0, "d and ff must be multiples of 8");
    th_moe* m = new th_moe();
    m->dev = dev; m->d = d; m->ff = ff; m->E = E; m->S = S; m->k = k;
    device_retain(dev);
    *out = m;
    TH_API_END
}

int th_moe_destroy(th_moe* m) {
    TH_API_BEGIN
    moe_destroy(m);
    TH_API_END
}

int th_moe_init_synthetic(th_moe* m, uint64_t seed) {
    TH_API_BEGIN
    TH_REQUIRE(m && !m->ready, "null or initialised MoE");
    const size_t NE = m->E + m->S, d = m->d, ff = m->ff;
    const size_t bpr_d = ceil_div(d, 32), bpr_ff = ceil_div(ff, 32);
    m->gu.assign(NE, nullptr);
    m->dn.assign(NE, nullptr);
    std::vector<uint8_t> gn(ff * bpr_d * 16), un(ff * bpr_d * 16), gun(2 * ff * bpr_d * 16), dnn(d * bpr_ff * 16);
    std::vector<uint16_t> gs(ff * bpr_d), us(ff * bpr_d), gus(2 * ff * bpr_d), dns(d * bpr_ff);
    for (size_t e = 0; e < NE; e++) {
        // tensor ids 4, 5, 6 = gate, up, down (as the decode engine), layer = expert
        check_status(th_synth_q4(th_synth_seed(seed, e, 4), ff, d, 0.002f, 0.01f, gn.data(), gs.data()));
        check_status(th_synth_q4(th_synth_seed(seed, e, 5), ff, d, 0.002f, 0.01f, un.data(), us.data()));
        for (size_t b = 0; b < ff / 8; b++) {
            for (size_t r = 0; r < 8; r++) {
                const size_t src = 8 * b + r, dg = 16 * b + r, du = 16 * b + 8 + r;
                std::memcpy(&gun[dg * bpr_d * 16], &gn[src * bpr_d * 16], bpr_d * 16);
                std::memcpy(&gun[du * bpr_d * 16], &un[src * bpr_d * 16], bpr_d * 16);
                std::memcpy(&gus[dg * bpr_d], &gs[src * bpr_d], bpr_d * 2);
                std::memcpy(&gus[du * bpr_d], &us[src * bpr_d], bpr_d * 2);
            }
        }
        m->gu[e] = q4_pack(m->dev, gun.data(), gus.data(), TH_F16, 2 * ff, d);
        check_status(th_synth_q4(th_synth_seed(seed, e, 6), d, ff, 0.002f, 0.01f, dnn.data(), dns.data()));
        m->dn[e] = q4_pack(m->dev, dnn.data(), dns.data(), TH_F16, d, ff);
    }
    std::vector<float> wr(m->E * d);
    check_status(th_synth_normal(th_synth_seed(seed, 1000, 0), wr.size(), 0.02f, TH_F32, wr.data()));
    TH_HIP(hipMalloc(&m->router, wr.size() * 4));
    TH_HIP(hipMemcpy(m->router, wr.data(), wr.size() * 4, hipMemcpyHostToDevice));
    std::vector<const void*> p(NE);
    auto table = [&](const void**& dst, auto get) {
        for (size_t e = 0; e < NE; e++) p[e] = get(e);
        TH_HIP(hipMalloc((void**)&dst, NE * sizeof(void*)));
        TH_HIP(hipMemcpy((void*)dst, p.data(), NE * sizeof(void*), hipMemcpyHostToDevice));
    };
    table((const void**&)m->gu_data, [&](size_t e) { return (const void*)m->gu[e]->data; });
    table((const void**&)m->gu_scales, [&](size_t e) { return (const void*)m->gu[e]->scales; });
    table((const void**&)m->dn_data, [&](size_t e) { return (const void*)m->dn[e]->data; });
    table((const void**&)m->dn_scales, [&](size_t e) { return (const void*)m->dn[e]->scales; });
    table((const void**&)m->gu_exps, [&](size_t e) { return (const void*)m->gu[e]->row_exp; });
    table((const void**&)m->dn_exps, [&](size_t e) { return (const void*)m->dn[e]->row_exp; });
    m->ready = true;
    TH_API_END
}

int th_moe_forward(th_moe* m, const th_buffer* h, size_t T, th_buffer* out, th_buffer* topk_idx, th_buffer* topk_w) {
    TH_API_BEGIN
    TH_REQUIRE(m && m->ready, "MoE not initialised");
    TH_REQUIRE(h && out && topk_idx && topk_w, "null argument");
    require_len(h, TH_BF16, T * m->d, "h");
    require_len(out, TH_F32, T * m->d, "out");
    TH_REQUIRE(topk_idx->dtype == TH_I32 || topk_idx->dtype == TH_U32, "topk_idx must be i32");
    require_len_any(topk_idx, T * m->k, "topk_idx");
    require_len(topk_w, TH_F32, T * m->k, "topk_w");
    if (T == 0) return TH_OK;
    moe_reserve(m, T);
    hipStream_t s = m->dev->stream;
    const bool gemm = T > (size_t)MOE_SMALL_T;  // prefill-sized: grouped MFMA GEMM, 64-slot work items
    const int rows = gemm ? MOE_GEMM_CB * 16 : MOE_MIN_ROWS;
    const size_t max_work = moe_max_work(m, T, rows);
    TH_LAUNCH(moe_router_kernel, dim3((unsigned)ceil_div(T, ROUTER_TOK), (unsigned)ceil_div(m->E, ROUTER_EXP)),
                       dim3(256), 0, s, (const uint16_t*)h->ptr, m->router, (int)T, (int)m->E, (int)m->d, m->logits);
    TH_LAUNCH_CHECK();
    const bool fused = T * m->k <= (size_t)MOE_FUSED_ENTRIES && T <= (size_t)MOE_SMALL_T;  // top-k inside dispatch
    auto route = [&](auto pl_tag) {  // top-k and dispatch with ceil(E / 64) expert slots per lane
        constexpr int PL = decltype(pl_tag)::value;
        if (!fused) {
            TH_LAUNCH(moe_topk_kernel<PL>, dim3((unsigned)ceil_div(T, 4)), dim3(256), 0, s, m->logits, (int)T,
                               (int)m->E, (int)m->k, (int32_t*)topk_idx->ptr, (float*)topk_w->ptr);
            TH_LAUNCH_CHECK();
        }
        TH_LAUNCH(moe_dispatch_kernel<PL>, dim3(1), dim3(1024), 0, s, fused ? (const float*)m->logits : nullptr,
                           (int32_t*)topk_idx->ptr, (float*)topk_w->ptr, (const int32_t*)topk_idx->ptr, (int)T, (int)m->k,
                           (int)m->E, (int)m->S, rows, m->offsets, m->slot_token, m->token_slot, m->work, (int)max_work);
        TH_LAUNCH_CHECK();
    };
    switch ((m->E + 63) / 64) {
        case 1: route(std::integral_constant<int, 1>{}); break;
        case 2: route(std::integral_constant<int, 2>{}); break;
        case 3: route(std::integral_constant<int, 3>{}); break;
        default: route(std::integral_constant<int, 4>{}); break;
    }
    const uint16_t* hx = (const uint16_t*)h->ptr;
    if (rows == MOE_MIN_ROWS) {
        moe_grouped_gemv<MOE_MIN_ROWS, EpiMoeSwiGLU, 4>(m, m->gu[0], m->gu_data, m->gu_scales, hx, m->slot_token,
                                                        max_work, EpiMoeSwiGLU{{}, m->hbuf, (int)m->ff});
        moe_grouped_gemv<MOE_MIN_ROWS, EpiMoeStore, 4>(m, m->dn[0], m->dn_data, m->dn_scales, m->hbuf, nullptr,
                                                       max_work, EpiMoeStore{{}, m->ybuf, (int)m->d});
    } else {
        moe_grouped_gemm(m, m->gu[0], m->gu_data, m->gu_scales, m->gu_exps, hx, T, m->slot_token, max_work,
                         EpiGemmMoeSwiGLU{m->hbuf, (int)m->ff});
        moe_grouped_gemm(m, m->dn[0], m->dn_data, m->dn_scales, m->dn_exps, m->hbuf, T * (m->k + m->S), nullptr,
                         max_work,
                         EpiGemmMoeStore{m->ybuf, (int)m->d});
    }
    TH_LAUNCH(moe_combine_kernel, dim3((unsigned)T, (unsigned)ceil_div(m->d, (size_t)1024)), dim3(256), 0, s, m->ybuf, m->token_slot,
                       (const float*)topk_w->ptr, m->offsets, (int)m->k, (int)m->E, (int)m->S, (int)m->d,
                       (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

}  // extern "C"
