// KV-cached decode attention: ComputeDevice::kv_attention
// (crates/tang-compute/src/cpu.rs:257-315).  Query i of q_len attends to cache
// positions 0..cache_start+i; GQA maps head h to kv head h/(n_heads/n_kv_heads);
// scores are scaled by 1/sqrt(head_dim); f32 arithmetic throughout.
//
// Split-K ("flash-decoding") form: each workgroup scores one chunk of
// positions for one (query, head), keeps the chunk's max m, sum l and
// unnormalised weighted V, and the last chunk of each (query, head) to finish
// merges the chunks with exp(m_s - M) weights (one launch in all).  There is
// no length cap (the reference CUDA kernel holds scores in a fixed 2048-float
// array, attention_cuda.rs:85).
#include "attention.hpp"
#include "capi_util.hpp"
#include "ops.hpp"

namespace th {

// Generic path for head dims without a tuned kernel: one wave per
// (query, head), online softmax in the reference's own order.
template <typename CT>
__global__ __launch_bounds__(64) void attn_generic_kernel(const float* __restrict__ q, const CT* __restrict__ kc,
                                                          const CT* __restrict__ vc, int cache_start, int n_heads,
                                                          int n_kv_heads, int head_dim, float* __restrict__ out) {
    const int h = blockIdx.x, qi = blockIdx.y, lane = threadIdx.x;
    const int total_dim = n_heads * head_dim, kv_dim = n_kv_heads * head_dim;
    const int kv_h = h / (n_heads / n_kv_heads);
    const float scale = 1.0f / sqrtf((float)head_dim);
    const float* qp = q + (size_t)qi * total_dim + h * head_dim;
    float acc[8];
    for (int i = 0; i < 8; i++) acc[i] = 0.0f;
    float rmax = -INFINITY, rsum = 0.0f;
    const int attend = cache_start + qi + 1;
    for (int j = 0; j < attend; j++) {
        const CT* kr = kc + (size_t)j * kv_dim + kv_h * head_dim;
        float part = 0.0f;
        for (int i = 0, d = lane; d < head_dim; i++, d += 64) part += qp[d] * (float)kr[d];
        const float score = wave_sum(part) * scale;
        const float nmax = fmaxf(rmax, score);
        const float es = expf(score - nmax), rs = expf(rmax - nmax);
        rsum = rsum * rs + es;
        const CT* vr = vc + (size_t)j * kv_dim + kv_h * head_dim;
        for (int i = 0, d = lane; d < head_dim; i++, d += 64) acc[i] = acc[i] * rs + es * (float)vr[d];
        rmax = nmax;
    }
    const float inv = 1.0f / rsum;
    for (int i = 0, d = lane; d < head_dim; i++, d += 64) out[(size_t)qi * total_dim + h * head_dim + d] = acc[i] * inv;
}

void launch_kv_attention(const float* q, const void* kc, const void* vc, bool f16, size_t cache_start, size_t q_len,
                         size_t n_heads, size_t n_kv_heads, size_t head_dim, float* out, hipStream_t s,
                         th_device* dev) {
    if (q_len == 0 || n_heads == 0) return;
    const bool tuned = head_dim == 64 || head_dim == 128 || head_dim == 256;
    if (!tuned) {
        TH_REQUIRE(head_dim <= 512, "head_dim above 512 is not supported");
        if (f16)
            TH_LAUNCH(attn_generic_kernel<_Float16>, dim3((unsigned)n_heads, (unsigned)q_len), dim3(64), 0, s, q,
                               (const _Float16*)kc, (const _Float16*)vc, (int)cache_start, (int)n_heads,
                               (int)n_kv_heads, (int)head_dim, out);
        else
            TH_LAUNCH(attn_generic_kernel<float>, dim3((unsigned)n_heads, (unsigned)q_len), dim3(64), 0, s, q,
                               (const float*)kc, (const float*)vc, (int)cache_start, (int)n_heads, (int)n_kv_heads,
                               (int)head_dim, out);
        TH_LAUNCH_CHECK();
        return;
    }
    const size_t max_len = cache_start + q_len;
    // enough 64-position chunks per split that the merge fits in LDS
    const size_t max_splits = 64 * 1024 / ((head_dim + 2) * sizeof(float));
    const int subs = (int)std::max<size_t>(1, ceil_div(ceil_div(max_len, (size_t)ATTN_SUB), max_splits));
    const int n_splits = (int)ceil_div(max_len, (size_t)subs * ATTN_SUB);
    float* part = (float*)device_scratch(dev, q_len * n_heads * n_splits * (head_dim + 2) * sizeof(float));
    int* counters = device_counters(dev, q_len * n_heads);
    launch_attn_split<false>(q, kc, vc, f16, (int)cache_start, (int)q_len, (int)n_heads, (int)n_kv_heads,
                             (int)head_dim, subs, n_splits, part, counters, (void*)out, nullptr, s);
}

}  // namespace th

using namespace th;

extern "C" int th_kv_attention(th_device* dev, const th_buffer* q, const th_buffer* k, const th_buffer* v,
                               size_t cache_start, size_t q_len, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                               th_buffer* out) {
    TH_API_BEGIN
    TH_REQUIRE(dev && q && k && v && out, "null argument");
    TH_REQUIRE(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
    TH_REQUIRE(k->dtype == v->dtype && (k->dtype == TH_F32 || k->dtype == TH_F16), "caches must both be f32 or f16");
    require_len(q, TH_F32, q_len * n_heads * head_dim, "q");
    require_len(out, TH_F32, q_len * n_heads * head_dim, "out");
    require_len_any(k, (cache_start + q_len) * n_kv_heads * head_dim, "k_cache");
    require_len_any(v, (cache_start + q_len) * n_kv_heads * head_dim, "v_cache");
    launch_kv_attention((const float*)q->ptr, k->ptr, v->ptr, k->dtype == TH_F16, cache_start, q_len, n_heads, n_kv_heads,
                        head_dim, (float*)out->ptr, dev->stream, dev);
    TH_API_END
}
