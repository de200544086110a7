// DeepSeek-style MoE FFN layer with int4 group-32 experts.
// The reference has no MoE; the layer is composed from its ops:
//   logits = h . W_r^T, p = softmax(logits) (cpu.rs:105-124), the top-k
//   experts by p (first maximum wins, as sampling.rs:184's argmax), weights
//   = p of the chosen experts (not renormalised); each expert is a SwiGLU
//   FFN of int4 linears (q4_matvec semantics, bf16 inputs); out = sum over the
//   token's experts in rank order of w * expert(h) + sum of the shared experts.
//
// Device flow, no host round trip:
//   router (one block per token: logits, softmax, top-k)
//   -> dispatch (one block: per-expert slot lists in token order and work
//      items of at most 16 rows; shared experts take every token)
//   -> grouped gate/up GEMV (epilogue SwiGLU, bf16 per slot)
//   -> grouped down GEMV (f32 per slot)
//   -> combine (per token, rank order, then shared).
// Grouped launches size the grid for the worst case; work items past the
// real ones return at once.
#include <mutex>
#include <vector>

#include "capi_util.hpp"
#include "ops.hpp"
#include "qlinear.hpp"

namespace th {

constexpr int MOE_ROWS = 16;  // activation rows per work item (one MFMA row block)
constexpr int MOE_MAX_K = 16;

struct MoeWork { int expert, slot0, rows, pad; };

// One block per token: router logits (f32 dot over d), softmax, top-k.
__global__ __launch_bounds__(256) void moe_router_kernel(const uint16_t* __restrict__ h, const float* __restrict__ wr,
                                                         int E, int d, int k, int32_t* __restrict__ topk_idx,
                                                         float* __restrict__ topk_w) {
    __shared__ float logit[1024];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint16_t* hr = h + (size_t)t * d;
    for (int e = wave; e < E; e += 4) {
        const float* w = wr + (size_t)e * d;
        float s = 0.0f;
        for (int i = lane; i < d; i += 64) s += __uint_as_float((uint32_t)hr[i] << 16) * w[i];
        s = wave_sum(s);
        if (lane == 0) logit[e] = s;
    }
    __syncthreads();
    if (tid == 0) {
        // softmax, cpu.rs:105-124 order: max, exp, sequential sum, scale
        float mx = -INFINITY;
        for (int e = 0; e < E; e++) mx = fmaxf(mx, logit[e]);
        for (int e = 0; e < E; e++) logit[e] = expf(logit[e] - mx);
        float sum = 0.0f;
        for (int e = 0; e < E; e++) sum += logit[e];
        const float inv = 1.0f / sum;
        for (int e = 0; e < E; e++) logit[e] *= inv;
        uint32_t used[32] = {0};
        for (int r = 0; r < k; r++) {
            int best = -1;
            float bv = 0.0f;
            for (int e = 0; e < E; e++) {
                if (used[e >> 5] >> (e & 31) & 1u) continue;
                if (best < 0 || logit[e] > bv) { bv = logit[e]; best = e; }
            }
            used[best >> 5] |= 1u << (best & 31);
            topk_idx[(size_t)t * k + r] = best;
            topk_w[(size_t)t * k + r] = bv;
        }
    }
}

// Slots: experts 0..E-1 (routed, tokens ascending) then the S shared experts
// (every token).  offsets[e] = first slot of expert e; token_slot[t*k+r] =
// slot of the token's rank-r expert; work items cover <= MOE_ROWS slots.
__global__ __launch_bounds__(256) void moe_dispatch_kernel(const int32_t* __restrict__ topk_idx, int T, int k, int E,
                                                           int S, int* __restrict__ offsets,
                                                           int* __restrict__ slot_token, int* __restrict__ token_slot,
                                                           MoeWork* __restrict__ work, int max_work) {
    __shared__ int cnt[1024];
    const int tid = threadIdx.x, NE = E + S;
    for (int e = tid; e < NE; e += 256) {
        int c = 0;
        if (e < E) {
            for (int i = 0; i < T * k; i++) c += topk_idx[i] == e;
        } else {
            c = T;
        }
        cnt[e] = c;
    }
    __syncthreads();
    if (tid == 0) {
        int o = 0;
        for (int e = 0; e < NE; e++) { offsets[e] = o; o += cnt[e]; }
        offsets[NE] = o;
    }
    __syncthreads();
    for (int e = tid; e < NE; e += 256) {
        int pos = offsets[e];
        if (e < E) {
            for (int i = 0; i < T * k; i++) {
                if (topk_idx[i] == e) {
                    slot_token[pos] = i / k;
                    token_slot[i] = pos;
                    pos++;
                }
            }
        } else {
            for (int t = 0; t < T; t++) slot_token[pos + t] = t;
        }
    }
    if (tid == 0) {
        int w = 0;
        for (int e = 0; e < NE; e++)
            for (int m0 = 0; m0 < cnt[e]; m0 += MOE_ROWS)
                if (w < max_work) work[w++] = MoeWork{e, offsets[e] + m0, min(MOE_ROWS, cnt[e] - m0), 0};
        for (; w < max_work; w++) work[w] = MoeWork{-1, 0, 0, 0};
    }
}

// Grouped GEMV source: workgroup -> (work item, tile of that expert's matrix).
struct MoeSrc {
    static constexpr bool GROUPED = true;
    const MoeWork* work;
    const uint4* const* wdata;
    const _Float16* const* wscales;
    const int* slot_token;  // null: activation rows are the slots themselves
    int tiles;
    int slot0 = 0;
    template <typename ST>
    __device__ __forceinline__ bool select(int bid, const uint4*& wt, const ST*& sc, int& t, int& mrows) {
        const MoeWork w = work[bid / tiles];
        if (w.expert < 0) return false;
        t = bid % tiles;
        wt = wdata[w.expert];
        sc = (const ST*)wscales[w.expert];
        mrows = w.rows;
        slot0 = w.slot0;
        return true;
    }
    __device__ __forceinline__ int x_row(int m) const { return slot_token ? slot_token[slot0 + m] : slot0 + m; }
    __device__ __forceinline__ int out_row(int m) const { return slot0 + m; }
};

// Gate/up tiles hold gate rows 8b..8b+7 then up rows 8b..8b+7 (as in the
// decode engine): bf16(swiglu(g, u)) per slot.
struct EpiMoeSwiGLU : EpiNoFinish {
    uint16_t* hbuf; int ff;
    __device__ __forceinline__ void operator()(int slot, int n, float v, const float* tile, float*) const {
        const int rr = n & 15;
        if (rr < 8) hbuf[(size_t)slot * ff + (n >> 4) * 8 + rr] = f32_to_bf16_rne(swiglu_f64(v, tile[rr + 8]));
    }
};

struct EpiMoeStore : EpiNoFinish {
    float* y; int d;
    __device__ __forceinline__ void operator()(int slot, int n, float v, const float*, float*) const {
        y[(size_t)slot * d + n] = v;
    }
};

// out[t] = sum_r w[t][r] * y[slot(t, r)] + sum_s y[shared slot]: rank order,
// then shared experts (f32).
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y, const int* __restrict__ token_slot,
                                                          const float* __restrict__ topk_w, const int* __restrict__ offsets,
                                                          int k, int E, int S, int d, float* __restrict__ out) {
    const int t = blockIdx.x;
    for (int n = threadIdx.x; n < d; n += 256) {
        float acc = 0.0f;
        for (int r = 0; r < k; r++) acc = __builtin_fmaf(topk_w[(size_t)t * k + r], y[(size_t)token_slot[t * k + r] * d + n], acc);
        for (int s = 0; s < S; s++) acc += y[(size_t)(offsets[E + s] + t) * d + n];
        out[(size_t)t * d + n] = acc;
    }
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
    size_t T_cap = 0;
    int *offsets = nullptr, *slot_token = nullptr, *token_slot = nullptr;
    MoeWork* work = nullptr;
    uint16_t* hbuf = nullptr;
    float* ybuf = nullptr;
    bool ready = false;
};

namespace th {

static void moe_free_work(th_moe* m) {
    void* ps[] = {m->offsets, m->slot_token, m->token_slot, m->work, m->hbuf, m->ybuf};
    for (void* p : ps)
        if (p) (void)hipFree(p);
    m->offsets = m->slot_token = m->token_slot = nullptr;
    m->work = nullptr;
    m->hbuf = nullptr;
    m->ybuf = nullptr;
    m->T_cap = 0;
}

static size_t moe_max_work(const th_moe* m, size_t T) {
    return ceil_div(T * m->k, MOE_ROWS) + m->E + m->S * ceil_div(T, MOE_ROWS);
}

static void moe_reserve(th_moe* m, size_t T) {
    if (T <= m->T_cap) return;
    TH_HIP(hipStreamSynchronize(m->dev->stream));
    moe_free_work(m);
    const size_t slots = T * m->k + m->S * T;
    TH_HIP(hipMalloc(&m->offsets, (m->E + m->S + 1) * sizeof(int)));
    TH_HIP(hipMalloc(&m->slot_token, slots * sizeof(int)));
    TH_HIP(hipMalloc(&m->token_slot, T * m->k * sizeof(int)));
    TH_HIP(hipMalloc(&m->work, moe_max_work(m, T) * sizeof(MoeWork)));
    TH_HIP(hipMalloc(&m->hbuf, slots * m->ff * sizeof(uint16_t)));
    TH_HIP(hipMalloc(&m->ybuf, slots * m->d * sizeof(float)));
    m->T_cap = T;
}

static void moe_destroy(th_moe* m) {
    if (!m) return;
    (void)hipStreamSynchronize(m->dev->stream);
    for (auto* v : {&m->gu, &m->dn})
        for (th_qweight* w : *v)
            if (w) th_qweight_free(w);
    void* ps[] = {m->router, (void*)m->gu_data, (void*)m->gu_scales, (void*)m->dn_data, (void*)m->dn_scales};
    for (void* p : ps)
        if (p) (void)hipFree(p);
    moe_free_work(m);
    delete m;
}

template <typename Epi, int NW>
static void moe_grouped_gemv(const th_moe* m, const th_qweight* w0, const uint4* const* data,
                             const _Float16* const* scales, const uint16_t* x, const int* slot_token, size_t max_work,
                             Epi epi) {
    const int tiles = (int)(w0->Np / 16);
    MoeSrc src{m->work, data, scales, slot_token, tiles};
    const size_t smem = Q4GemvSmem<MOE_ROWS, NW>::bytes((int)(w0->Kp / 128));
    TH_REQUIRE(smem <= 160 * 1024, "MoE GEMV LDS above 160 KiB");
    auto k = q4_gemv_kernel<MOE_ROWS, false, true, _Float16, Epi, 2, 2, NW, false, MoeSrc>;
    static std::mutex mu;
    static size_t done = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (smem > 48 * 1024 && smem > done) {
            TH_HIP(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
            done = smem;
        }
    }
    hipLaunchKernelGGL(k, dim3((unsigned)(max_work * tiles)), dim3(64 * NW), smem, m->dev->stream, (const uint4*)nullptr,
                       (const _Float16*)nullptr, (const void*)x, (int)w0->cols, (int)w0->Kp, (int)w0->rows,
                       (int)w0->cols, epi, NormArgs{}, src);
    TH_LAUNCH_CHECK();
}

}  // namespace th

extern "C" {

int th_moe_create(th_device* dev, size_t d, size_t ff, size_t E, size_t S, size_t k, th_moe** out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && out, "null argument");
    TH_REQUIRE(d > 0 && ff > 0 && E > 0 && k > 0 && k <= E && k <= MOE_MAX_K, "bad MoE shape");
    TH_REQUIRE(E <= 1024 && E + S <= 1024, "at most 1024 experts");
    TH_REQUIRE(ff % 8 == 0 && d % 8 == 0, "d and ff must be multiples of 8");
    th_moe* m = new th_moe();
    m->dev = dev; m->d = d; m->ff = ff; m->E = E; m->S = S; m->k = k;
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
    const size_t max_work = moe_max_work(m, T);
    hipLaunchKernelGGL(moe_router_kernel, dim3((unsigned)T), dim3(256), 0, s, (const uint16_t*)h->ptr, m->router,
                       (int)m->E, (int)m->d, (int)m->k, (int32_t*)topk_idx->ptr, (float*)topk_w->ptr);
    TH_LAUNCH_CHECK();
    hipLaunchKernelGGL(moe_dispatch_kernel, dim3(1), dim3(256), 0, s, (const int32_t*)topk_idx->ptr, (int)T, (int)m->k,
                       (int)m->E, (int)m->S, m->offsets, m->slot_token, m->token_slot, m->work, (int)max_work);
    TH_LAUNCH_CHECK();
    moe_grouped_gemv<EpiMoeSwiGLU, 4>(m, m->gu[0], m->gu_data, m->gu_scales, (const uint16_t*)h->ptr, m->slot_token,
                                      max_work, EpiMoeSwiGLU{{}, m->hbuf, (int)m->ff});
    moe_grouped_gemv<EpiMoeStore, 4>(m, m->dn[0], m->dn_data, m->dn_scales, m->hbuf, nullptr, max_work,
                                     EpiMoeStore{{}, m->ybuf, (int)m->d});
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)T), dim3(256), 0, s, m->ybuf, m->token_slot,
                       (const float*)topk_w->ptr, m->offsets, (int)m->k, (int)m->E, (int)m->S, (int)m->d,
                       (float*)out->ptr);
    TH_LAUNCH_CHECK();
    TH_API_END
}

}  // extern "C"
