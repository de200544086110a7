// Token sampling on the host, as the reference does it
// (crates/tang-infer/src/sampling.rs): repetition penalty, temperature,
// softmax, top-k, normalisation, top-p, then a categorical draw from the
// reference's LCG.  All arithmetic is f64 like the reference; the logits come
// from the device as f32 (exact in f64).
#include <algorithm>
#include <cmath>
#include <numeric>
#include <vector>

#include "capi_util.hpp"

struct th_sampler {
    th_sampling_config cfg;
    uint64_t state;
    std::vector<double> p;
    std::vector<size_t> order;
};

namespace th {

// sampling.rs:77-80
static double lcg_unit(uint64_t& s) {
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    return (double)(s >> 11) / 9007199254740992.0;  // 2^53
}

// sampling.rs:184-194: strictly greater wins, so ties keep the lowest index.
static size_t first_max(const std::vector<double>& v) {
    size_t best = 0;
    double bv = -INFINITY;
    for (size_t i = 0; i < v.size(); i++)
        if (v[i] > bv) bv = v[i], best = i;
    return best;
}

// Indices by descending value; equal values keep index order (Rust's
// sort_by is stable).
static void order_desc(const std::vector<double>& v, std::vector<size_t>& idx) {
    idx.resize(v.size());
    std::iota(idx.begin(), idx.end(), size_t(0));
    std::stable_sort(idx.begin(), idx.end(), [&](size_t a, size_t b) { return v[a] > v[b]; });
}

size_t sample_one(th_sampler* s, const float* logits, size_t n, const int32_t* past, size_t n_past) {
    const th_sampling_config& c = s->cfg;
    std::vector<double>& p = s->p;
    p.assign(logits, logits + n);
    if (c.repetition_penalty != 1.0)  // sampling.rs:93-104
        for (size_t j = 0; j < n_past; j++) {
            const size_t t = (size_t)past[j];
            if (t >= n) continue;
            p[t] = p[t] > 0.0 ? p[t] / c.repetition_penalty : p[t] * c.repetition_penalty;
        }
    if (c.temperature == 0.0) return first_max(p);  // :107-109
    if (c.temperature != 1.0) {                      // :112-117
        const double inv_t = 1.0 / c.temperature;
        for (double& v : p) v *= inv_t;
    }
    double mx = -INFINITY;  // :120-123, f64::max skips NaN like fmax
    for (double v : p) mx = std::fmax(mx, v);
    for (double& v : p) v = std::exp(v - mx);
    if (c.top_k > 0 && c.top_k < n) {  // :126-133 with kth_largest :172-178
        order_desc(p, s->order);
        const double thr = p[s->order[c.top_k - 1]];
        for (double& v : p)
            if (v < thr) v = 0.0;
    }
    double sum = 0.0;  // :136-142
    for (double v : p) sum += v;
    if (sum <= 0.0) return first_max(p);
    for (double& v : p) v /= sum;
    if (c.top_p < 1.0) {  // :145-154 with top_p_filter :197-215
        order_desc(p, s->order);
        double cum = 0.0;
        size_t cut = n;
        for (size_t r = 0; r < n; r++) {
            cum += p[s->order[r]];
            if (cum >= c.top_p) {
                cut = r + 1;
                break;
            }
        }
        for (size_t r = cut; r < n; r++) p[s->order[r]] = 0.0;
        double s2 = 0.0;
        for (double v : p) s2 += v;
        if (s2 > 0.0)
            for (double& v : p) v /= s2;
    }
    const double r = lcg_unit(s->state);  // categorical_sample :163-175
    double cum = 0.0;
    for (size_t i = 0; i < n; i++) {
        cum += p[i];
        if (r < cum) return i;
    }
    return n - 1;
}

const th_sampling_config& sampler_config(const th_sampler* s) { return s->cfg; }

}  // namespace th

using namespace th;

extern "C" {

int th_sampler_create(const th_sampling_config* cfg, uint64_t seed, th_sampler** out) {
    TH_API_BEGIN
    TH_REQUIRE(cfg && out, "null argument");
    TH_REQUIRE(cfg->temperature >= 0.0 && cfg->top_p > 0.0 && cfg->repetition_penalty > 0.0, "bad sampling config");
    th_sampler* s = new th_sampler();
    s->cfg = *cfg;
    s->state = seed;
    *out = s;
    TH_API_END
}

int th_sampler_destroy(th_sampler* s) {
    TH_API_BEGIN
    delete s;
    TH_API_END
}

int th_sampler_sample(th_sampler* s, const float* logits, size_t vocab, const int32_t* past, size_t n_past,
                      int32_t* token) {
    TH_API_BEGIN
    TH_REQUIRE(s && logits && token && vocab > 0 && (past || n_past == 0), "null argument");
    *token = (int32_t)sample_one(s, logits, vocab, past, n_past);
    TH_API_END
}

}  // extern "C"
