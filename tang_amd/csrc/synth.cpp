// Seeded synthetic data for benchmarks and tests (host side).
//
// Generator: xoshiro256** seeded through SplitMix64, the reference bench RNG
// (crates/tang-bench/src/lib.rs:7-46).  uniform(a,b) uses the reference's
// [-1,1] map f64() = next/u64::MAX*2-1 as a + (b-a)*(f64()+1)/2.  Normals are
// Box-Muller on two 53-bit uniforms (one normal per pair of draws).
#include <cmath>
#include <cstring>

#include "capi_util.hpp"

namespace th {

struct Xoshiro {
    uint64_t s[4];
    explicit Xoshiro(uint64_t seed) {
        uint64_t z = seed;
        for (int i = 0; i < 4; i++) {
            z += 0x9e3779b97f4a7c15ull;
            uint64_t x = z;
            x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
            x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
            s[i] = x ^ (x >> 31);
        }
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        const uint64_t result = rotl(s[1] * 5, 7) * 9;
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return result;
    }
    double f64() { return (double)next() / (double)UINT64_MAX * 2.0 - 1.0; }
    double uniform(double a, double b) { return a + (b - a) * (f64() + 1.0) * 0.5; }
    double normal() {
        const double u1 = ((double)(next() >> 11) + 1.0) * 0x1.0p-53;
        const double u2 = (double)(next() >> 11) * 0x1.0p-53;
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

}  // namespace th

using namespace th;

extern "C" {

uint64_t th_synth_seed(uint64_t base, uint64_t layer, uint64_t tensor) {
    uint64_t z = base ^ (layer * 0x9E3779B97F4A7C15ull) ^ (tensor * 0xC2B2AE3D27D4EB4Full);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

int th_synth_q4(uint64_t seed, size_t rows, size_t cols, float smin, float smax, uint8_t* nib, uint16_t* sc) {
    TH_API_BEGIN
    TH_REQUIRE(nib && sc, "null output");
    Xoshiro rng(seed);
    const size_t bpr = ceil_div(cols, 32);
    const size_t nbytes = rows * bpr * 16;
    size_t i = 0;
    for (; i + 8 <= nbytes; i += 8) {
        const uint64_t v = rng.next();
        std::memcpy(nib + i, &v, 8);
    }
    if (i < nbytes) {
        const uint64_t v = rng.next();
        std::memcpy(nib + i, &v, nbytes - i);
    }
    // Elements past `cols` in a ragged last block carry value 0 (nibble 8),
    // as quantize_q4 packs them (quantize.rs:100-109).
    if (cols % 32) {
        for (size_t r = 0; r < rows; r++) {
            uint8_t* blk = nib + (r * bpr + bpr - 1) * 16;
            for (size_t e = cols % 32; e < 32; e++) {
                if (e & 1) blk[e / 2] = (uint8_t)((blk[e / 2] & 0x0F) | 0x80);
                else blk[e / 2] = (uint8_t)((blk[e / 2] & 0xF0) | 0x08);
            }
        }
    }
    for (size_t b = 0; b < rows * bpr; b++) sc[b] = f32_to_f16_host((float)rng.uniform(smin, smax));
    TH_API_END
}

int th_synth_q8_rowwise(uint64_t seed, size_t rows, size_t cols, float smin, float smax, int8_t* q, float* rs) {
    TH_API_BEGIN
    TH_REQUIRE(q && rs, "null output");
    Xoshiro rng(seed);
    for (size_t i = 0; i < rows * cols; i++) q[i] = (int8_t)((int)(rng.next() % 255) - 127);
    for (size_t r = 0; r < rows; r++) rs[r] = (float)rng.uniform(smin, smax);
    TH_API_END
}

int th_synth_normal(uint64_t seed, size_t n, float std_, th_dtype dt, void* out) {
    TH_API_BEGIN
    TH_REQUIRE(out || n == 0, "null output");
    Xoshiro rng(seed);
    for (size_t i = 0; i < n; i++) {
        const float v = (float)(rng.normal() * (double)std_);
        if (dt == TH_F32) ((float*)out)[i] = v;
        else if (dt == TH_BF16) ((uint16_t*)out)[i] = f32_to_bf16_host(v);
        else if (dt == TH_F16) ((uint16_t*)out)[i] = f32_to_f16_host(v);
        else throw Error(TH_ERR_INVALID, "th_synth_normal: dtype must be f32, bf16 or f16");
    }
    TH_API_END
}

}  // extern "C"
