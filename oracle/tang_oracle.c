/*
 * tang_oracle.c -- CPU restatement of ecto/tang's reference arithmetic for the
 * quantized-inference decode path.  TEST INFRASTRUCTURE ONLY: this file is the
 * parity checker.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Every function states the reference file:line it follows (paths relative to
 * the ecto/tang repository root).  Loop order, accumulation type and rounding
 * points follow the reference exactly; the file is compiled with
 * -ffp-contract=off so that no multiply-add is fused where Rust would not fuse.
 *
 * Functions whose only pin is the mathematics (MoE, MLA: no reference
 * implementation exists) are marked "from definition" below.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32 /* BLOCK_SIZE, crates/tang-infer/src/quantize.rs:11 */

/* crates/tang-infer/src/quantize.rs:15-19 (Q8Block) as a C struct. */
typedef struct { float scale; int8_t values[QK]; } or_q8_block;
/* crates/tang-infer/src/quantize.rs:25-29 (Q4Block). */
typedef struct { float scale; uint8_t values[QK / 2]; } or_q4_block;

static void set_threads(int t) {
#ifdef _OPENMP
    if (t > 0) omp_set_num_threads(t);
#else
    (void)t;
#endif
}

/* ---------------------------------------------------------------------- */
/* dtype conversions                                                       */
/* ---------------------------------------------------------------------- */

/* crates/tang-compute/src/cuda.rs:22-27 f32_to_bf16: bits + 0x7FFF + lsb. */
uint16_t or_f32_to_bf16(float v) {
    uint32_t bits; memcpy(&bits, &v, 4);
    uint32_t lsb = (bits >> 16) & 1u;
    uint32_t r = bits + 0x7FFFu + lsb;
    return (uint16_t)(r >> 16);
}

/* crates/tang-compute/src/cuda.rs:29-31 bf16_to_f32. */
float or_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16; float f; memcpy(&f, &bits, 4); return f;
}

/* crates/tang-safetensors/src/lib.rs:262 f16_to_f32 (IEEE half: sign, 5-bit
 * exponent, 10-bit mantissa, subnormals, inf/nan). */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t exp = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t mant = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else { /* subnormal: value = mant * 2^-24 */
            float f = (float)mant * 5.9604644775390625e-08f;
            if (sign) f = -f;
            return f;
        }
    } else if (exp == 31) {
        bits = (sign << 31) | 0x7F800000u | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 112u) << 23) | (mant << 13);
    }
    float f; memcpy(&f, &bits, 4); return f;
}

/* f32 -> f16 round-to-nearest-even.  The reference has no f32->f16 writer
 * (safetensors only reads f16); this is IEEE 754 RNE, pinned against numpy's
 * astype(float16) in the tests. */
uint16_t or_f32_to_f16(float v) {
    uint32_t x; memcpy(&x, &v, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* overflow -> inf */
    if (ax < 0x38800000u) { /* result subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;          /* 14 + (113 - e) - 1 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

void or_f32_to_bf16_array(const float* x, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_bf16(x[i]);
}
void or_bf16_to_f32_array(const uint16_t* x, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = or_bf16_to_f32(x[i]);
}
void or_f16_to_f32_array(const uint16_t* x, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(x[i]);
}
void or_f32_to_f16_array(const float* x, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_f16(x[i]);
}

/* ---------------------------------------------------------------------- */
/* quantize.rs                                                             */
/* ---------------------------------------------------------------------- */

/* Rust `f32::round`: half away from zero == C roundf.  `as i8` after clamp. */

/* crates/tang-infer/src/quantize.rs:47-70 quantize_q8. */
size_t or_quantize_q8(const float* data, size_t n, or_q8_block* out) {
    size_t nb = (n + QK - 1) / QK;
    for (size_t b = 0; b < nb; b++) {
        size_t start = b * QK, end = start + QK < n ? start + QK : n;
        float amax = 0.0f;
        for (size_t i = start; i < end; i++) amax = fmaxf(amax, fabsf(data[i]));
        float scale = amax == 0.0f ? 1.0f : amax / 127.0f;
        float inv = 1.0f / scale;
        or_q8_block* blk = &out[b];
        memset(blk->values, 0, QK);
        for (size_t i = start; i < end; i++) {
            float q = roundf(data[i] * inv);
            if (q < -128.0f) q = -128.0f;
            if (q > 127.0f) q = 127.0f;
            blk->values[i - start] = (int8_t)q;
        }
        blk->scale = scale;
    }
    return nb;
}

/* crates/tang-infer/src/quantize.rs:73-82 dequantize_q8. */
void or_dequantize_q8(const or_q8_block* blocks, size_t nb, float* out) {
    for (size_t b = 0; b < nb; b++)
        for (int i = 0; i < QK; i++) out[b * QK + i] = (float)blocks[b].values[i] * blocks[b].scale;
}

/* crates/tang-infer/src/quantize.rs:84-118 quantize_q4. */
size_t or_quantize_q4(const float* data, size_t n, or_q4_block* out) {
    size_t nb = (n + QK - 1) / QK;
    for (size_t b = 0; b < nb; b++) {
        size_t start = b * QK, len = (start + QK < n ? QK : n - start);
        const float* chunk = data + start;
        float amax = 0.0f;
        for (size_t i = 0; i < len; i++) amax = fmaxf(amax, fabsf(chunk[i]));
        float scale = amax == 0.0f ? 1.0f : amax / 7.0f;
        float inv = 1.0f / scale;
        for (int i = 0; i < QK / 2; i++) {
            size_t idx = (size_t)i * 2;
            int v0 = 0, v1 = 0;
            if (idx < len) {
                float q = roundf(chunk[idx] * inv);
                if (q < -8.0f) q = -8.0f;
                if (q > 7.0f) q = 7.0f;
                v0 = (int)q;
            }
            if (idx + 1 < len) {
                float q = roundf(chunk[idx + 1] * inv);
                if (q < -8.0f) q = -8.0f;
                if (q > 7.0f) q = 7.0f;
                v1 = (int)q;
            }
            out[b].values[i] = (uint8_t)((uint8_t)(v0 + 8) | (uint8_t)((v1 + 8) << 4));
        }
        out[b].scale = scale;
    }
    return nb;
}

/* crates/tang-infer/src/quantize.rs:121-132 dequantize_q4. */
void or_dequantize_q4(const or_q4_block* blocks, size_t nb, float* out) {
    for (size_t b = 0; b < nb; b++) {
        for (int i = 0; i < QK / 2; i++) {
            uint8_t byte = blocks[b].values[i];
            int v0 = (int)(byte & 0x0F) - 8;
            int v1 = (int)((byte >> 4) & 0x0F) - 8;
            out[b * QK + 2 * i] = (float)v0 * blocks[b].scale;
            out[b * QK + 2 * i + 1] = (float)v1 * blocks[b].scale;
        }
    }
}

/* crates/tang-infer/src/quantize.rs:193-206 quantize_matrix_q8 (row by row). */
size_t or_quantize_matrix_q8(const float* data, size_t rows, size_t cols, or_q8_block* out) {
    size_t bpr = (cols + QK - 1) / QK;
    for (size_t r = 0; r < rows; r++) or_quantize_q8(data + r * cols, cols, out + r * bpr);
    return rows * bpr;
}

/* crates/tang-infer/src/quantize.rs:208-221 quantize_matrix_q4. */
size_t or_quantize_matrix_q4(const float* data, size_t rows, size_t cols, or_q4_block* out) {
    size_t bpr = (cols + QK - 1) / QK;
    for (size_t r = 0; r < rows; r++) or_quantize_q4(data + r * cols, cols, out + r * bpr);
    return rows * bpr;
}

/* crates/tang-infer/src/quantize.rs:227-254 q8_matvec: f64 accumulate, sequential
 * element order, `xi < in_dim` guard. */
void or_q8_matvec(const or_q8_block* w, size_t out_dim, size_t in_dim, const double* x, double* y) {
    size_t bpr = (in_dim + QK - 1) / QK;
    for (size_t row = 0; row < out_dim; row++) {
        double sum = 0.0;
        for (size_t b = 0; b < bpr; b++) {
            const or_q8_block* blk = &w[row * bpr + b];
            size_t xs = b * QK;
            double scale = (double)blk->scale;
            for (int i = 0; i < QK; i++) {
                size_t xi = xs + (size_t)i;
                if (xi < in_dim) sum += ((double)blk->values[i]) * scale * x[xi];
            }
        }
        y[row] = sum;
    }
}

/* crates/tang-infer/src/quantize.rs:256-289 q4_matvec. */
void or_q4_matvec(const or_q4_block* w, size_t out_dim, size_t in_dim, const double* x, double* y) {
    size_t bpr = (in_dim + QK - 1) / QK;
    for (size_t row = 0; row < out_dim; row++) {
        double sum = 0.0;
        for (size_t b = 0; b < bpr; b++) {
            const or_q4_block* blk = &w[row * bpr + b];
            size_t xs = b * QK;
            double scale = (double)blk->scale;
            for (int i = 0; i < QK / 2; i++) {
                uint8_t byte = blk->values[i];
                double v0 = (double)((int)(byte & 0x0F) - 8);
                double v1 = (double)((int)((byte >> 4) & 0x0F) - 8);
                size_t xi0 = xs + (size_t)i * 2, xi1 = xi0 + 1;
                if (xi0 < in_dim) sum += v0 * scale * x[xi0];
                if (xi1 < in_dim) sum += v1 * scale * x[xi1];
            }
        }
        y[row] = sum;
    }
}

/* The same two routines over a struct-of-arrays view of the identical blocks:
 * block (row, b) is {scales[row*bpr+b], nib[(row*bpr+b)*16 .. +16]} for q4 and
 * {scales[row*bpr+b], q[row*bpr*32 + b*32 .. +32]} for q8.  Arithmetic and loop
 * order are those of quantize.rs:227-289; rows run in parallel (each row's sum
 * is still the reference's sequential f64 sum, so the result is bit-identical
 * to the single-threaded routine for any thread count). */
void or_q4_matvec_soa(const uint8_t* nib, const float* scales, size_t out_dim, size_t in_dim,
                      const double* x, double* y, int threads) {
    size_t bpr = (in_dim + QK - 1) / QK;
    set_threads(threads);
#pragma omp parallel for schedule(static) if (threads != 1)
    for (size_t row = 0; row < out_dim; row++) {
        double sum = 0.0;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t* vals = nib + (row * bpr + b) * (QK / 2);
            size_t xs = b * QK;
            double scale = (double)scales[row * bpr + b];
            for (int i = 0; i < QK / 2; i++) {
                uint8_t byte = vals[i];
                double v0 = (double)((int)(byte & 0x0F) - 8);
                double v1 = (double)((int)((byte >> 4) & 0x0F) - 8);
                size_t xi0 = xs + (size_t)i * 2, xi1 = xi0 + 1;
                if (xi0 < in_dim) sum += v0 * scale * x[xi0];
                if (xi1 < in_dim) sum += v1 * scale * x[xi1];
            }
        }
        y[row] = sum;
    }
}

void or_q8_matvec_soa(const int8_t* q, const float* scales, size_t out_dim, size_t in_dim,
                      const double* x, double* y, int threads) {
    size_t bpr = (in_dim + QK - 1) / QK;
    set_threads(threads);
#pragma omp parallel for schedule(static) if (threads != 1)
    for (size_t row = 0; row < out_dim; row++) {
        double sum = 0.0;
        for (size_t b = 0; b < bpr; b++) {
            const int8_t* vals = q + row * bpr * QK + b * QK;
            size_t xs = b * QK;
            double scale = (double)scales[row * bpr + b];
            for (int i = 0; i < QK; i++) {
                size_t xi = xs + (size_t)i;
                if (xi < in_dim) sum += ((double)vals[i]) * scale * x[xi];
            }
        }
        y[row] = sum;
    }
}

/* ---------------------------------------------------------------------- */
/* CpuDevice ops (crates/tang-compute/src/cpu.rs, device.rs defaults)      */
/* ---------------------------------------------------------------------- */

/* crates/tang-compute/src/cpu.rs:126-149 rms_norm: f32, sequential sum of x*x,
 * rms = sqrt(sum/dim + eps), out = x * (1/rms) * w. */
void or_rms_norm(const float* x, const float* w, size_t groups, size_t dim, float eps, float* out) {
    for (size_t g = 0; g < groups; g++) {
        const float* s = x + g * dim;
        float sq = 0.0f;
        for (size_t d = 0; d < dim; d++) sq += s[d] * s[d];
        float rms = sqrtf(sq / (float)dim + eps);
        float inv = 1.0f / rms;
        for (size_t d = 0; d < dim; d++) out[g * dim + d] = s[d] * inv * w[d];
    }
}

/* crates/tang-compute/src/device.rs:546-575 rms_norm_residual (default impl):
 * v = input + residual (kept as sum_out), normalised like rms_norm. */
void or_rms_norm_residual(const float* in, const float* res, const float* w, size_t groups,
                          size_t dim, float eps, float* out, float* sum_out) {
    for (size_t g = 0; g < groups; g++) {
        size_t base = g * dim;
        float sq = 0.0f;
        for (size_t i = 0; i < dim; i++) {
            float v = in[base + i] + res[base + i];
            sum_out[base + i] = v;
            sq += v * v;
        }
        float inv = 1.0f / sqrtf(sq / (float)dim + eps);
        for (size_t i = 0; i < dim; i++) out[base + i] = sum_out[base + i] * inv * w[i];
    }
}

/* crates/tang-compute/src/modules.rs:495-511 InterleavedRoPE::new tables:
 * freq = 1 / base^(i/half) and angle = pos*freq in f64, stored as f32. */
void or_rope_tables(size_t head_dim, size_t max_seq, double base, float* cos_t, float* sin_t) {
    size_t half = head_dim / 2;
    for (size_t pos = 0; pos < max_seq; pos++) {
        for (size_t i = 0; i < half; i++) {
            double freq = 1.0 / pow(base, (double)i / (double)half);
            double angle = (double)pos * freq;
            cos_t[pos * half + i] = (float)cos(angle);
            sin_t[pos * half + i] = (float)sin(angle);
        }
    }
}

/* crates/tang-compute/src/device.rs:582-610 rope_forward (interleaved pairs). */
void or_rope_forward(const float* in, const float* cos_t, const float* sin_t, size_t seq_len,
                     size_t n_heads, size_t head_dim, size_t start_pos, float* out) {
    size_t half = head_dim / 2;
    for (size_t s = 0; s < seq_len; s++) {
        size_t pos = start_pos + s;
        for (size_t h = 0; h < n_heads; h++) {
            size_t base = (s * n_heads + h) * head_dim;
            for (size_t i = 0; i < half; i++) {
                float c = cos_t[pos * half + i], sn = sin_t[pos * half + i];
                float x0 = in[base + 2 * i], x1 = in[base + 2 * i + 1];
                out[base + 2 * i] = x0 * c - x1 * sn;
                out[base + 2 * i + 1] = x0 * sn + x1 * c;
            }
        }
    }
}

/* crates/tang-compute/src/cpu.rs:257-315 kv_attention: per (qi, head) online
 * softmax in f32, scale 1/sqrt(head_dim), attends 0..cache_start+qi+1,
 * GQA head mapping kv_h = h / (n_heads/n_kv_heads). */
void or_kv_attention(const float* q, const float* k_cache, const float* v_cache, size_t cache_start,
                     size_t q_len, size_t n_heads, size_t n_kv_heads, size_t head_dim, float* out,
                     int threads) {
    size_t total_dim = n_heads * head_dim, kv_dim = n_kv_heads * head_dim;
    size_t hpk = n_heads / n_kv_heads;
    float scale = 1.0f / sqrtf((float)head_dim);
    set_threads(threads);
#pragma omp parallel for collapse(2) schedule(static) if (threads != 1)
    for (size_t qi = 0; qi < q_len; qi++) {
        for (size_t h = 0; h < n_heads; h++) {
            size_t attend = cache_start + qi + 1;
            size_t kv_h = h / hpk;
            size_t q_off = qi * total_dim + h * head_dim, kv_off = kv_h * head_dim;
            float rmax = -INFINITY, rsum = 0.0f;
            float* acc = (float*)calloc(head_dim, sizeof(float));
            for (size_t j = 0; j < attend; j++) {
                float dot = 0.0f;
                for (size_t d = 0; d < head_dim; d++) dot += q[q_off + d] * k_cache[j * kv_dim + kv_off + d];
                float score = dot * scale;
                float nmax = fmaxf(rmax, score);
                float es = expf(score - nmax);
                float rs = expf(rmax - nmax);
                rsum = rsum * rs + es;
                for (size_t d = 0; d < head_dim; d++)
                    acc[d] = acc[d] * rs + es * v_cache[j * kv_dim + kv_off + d];
                rmax = nmax;
            }
            float inv = 1.0f / rsum;
            for (size_t d = 0; d < head_dim; d++) out[q_off + d] = acc[d] * inv;
            free(acc);
        }
    }
}

/* crates/tang-compute/src/device.rs:727-736 swiglu_fused_buf: the elementwise
 * closure g * (1/(1+exp(-g))) * u, evaluated in f64 on f32 inputs and stored
 * as f32 (crates/tang-compute/src/cpu.rs:68-97). */
void or_swiglu(const float* gate, const float* up, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) {
        double g = (double)gate[i], u = (double)up[i];
        double sig = 1.0 / (1.0 + exp(-g));
        out[i] = (float)(g * sig * u);
    }
}

/* crates/tang-compute/src/device.rs:721-724 add_tensors_buf (f64 a+b -> f32,
 * which equals the f32 sum). */
void or_add(const float* a, const float* b, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = (float)((double)a[i] + (double)b[i]);
}

/* crates/tang-compute/src/cpu.rs:151-168 embedding: row copy by u32 id. */
void or_embedding(const float* weight, const uint32_t* ids, size_t seq_len, size_t dim, float* out) {
    for (size_t i = 0; i < seq_len; i++) memcpy(out + i * dim, weight + (size_t)ids[i] * dim, dim * sizeof(float));
}

/* crates/tang-compute/src/cpu.rs:105-124 softmax (f32, max-subtracted). */
void or_softmax(const float* x, size_t rows, size_t len, float* out) {
    for (size_t r = 0; r < rows; r++) {
        const float* s = x + r * len;
        float* o = out + r * len;
        float mx = -INFINITY;
        for (size_t i = 0; i < len; i++) mx = fmaxf(mx, s[i]);
        for (size_t i = 0; i < len; i++) o[i] = expf(s[i] - mx);
        float sum = 0.0f;
        for (size_t i = 0; i < len; i++) sum += o[i];
        float inv = 1.0f / sum;
        for (size_t i = 0; i < len; i++) o[i] *= inv;
    }
}

/* crates/tang-compute/src/cpu.rs:760-770 naive_matmul (the non-macOS
 * matmul_impl): C[m][n] = sum_p A[m][p] * B[p][n], one f32 sum per output in
 * p order. */
void or_matmul(const float* a, const float* b, size_t m, size_t k, size_t n, float* c) {
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            float sum = 0.0f;
            for (size_t p = 0; p < k; p++) sum += a[i * k + p] * b[p * n + j];
            c[i * n + j] = sum;
        }
}

/* crates/tang-compute/src/cpu.rs:317-326 transpose_2d: out[c][r] = in[r][c]. */
void or_transpose_2d(const float* in, size_t rows, size_t cols, float* out) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) out[c * rows + r] = in[r * cols + c];
}

/* crates/tang-compute/src/cpu.rs:169-199 reduce_sum over `axis` of a
 * row-major tensor: outputs start at 0 and add in (o, a, i) loop order. */
void or_reduce_sum(const float* in, const size_t* shape, size_t ndim, size_t axis, float* out) {
    size_t outer = 1, inner = 1;
    for (size_t d = 0; d < axis; d++) outer *= shape[d];
    for (size_t d = axis + 1; d < ndim; d++) inner *= shape[d];
    size_t len = shape[axis];
    for (size_t i = 0; i < outer * inner; i++) out[i] = 0.0f;
    for (size_t o = 0; o < outer; o++)
        for (size_t a = 0; a < len; a++)
            for (size_t i = 0; i < inner; i++) out[o * inner + i] += in[(o * len + a) * inner + i];
}

/* crates/tang-compute/src/device.rs:378-386 bias_add: out[i] = m[i] + bias[i % dim]. */
void or_bias_add(const float* m, const float* bias, size_t numel, size_t dim, float* out) {
    for (size_t i = 0; i < numel; i++) out[i] = m[i] + bias[i % dim];
}

/* crates/tang-infer/src/sampling.rs:184-194 argmax: first strictly greater
 * value wins (ties resolve to the lowest index). */
size_t or_argmax_f32(const float* v, size_t n) {
    size_t best = 0; double bv = -INFINITY;
    for (size_t i = 0; i < n; i++) if ((double)v[i] > bv) { bv = (double)v[i]; best = i; }
    return best;
}

/* ---------------------------------------------------------------------- */
/* Decode-step composition                                                 */
/* ---------------------------------------------------------------------- */

/* One Llama-style decode step for one token, composed as in
 * crates/tang-train/examples/smollm.rs:215-300 (pre-norm -> attention ->
 * +residual -> pre-norm -> SwiGLU MLP -> +residual; final norm; LM head)
 * from the CpuDevice ops above and q4_matvec.  Rounding points (shared with
 * the device engine): every linear consumes its input rounded to bf16 (the
 * f32_to_bf16 of crates/tang-compute/src/cuda.rs:22) and produces f32 from the
 * f64 sum; K/V are stored to the cache as f16.
 *
 * Weights are q4 struct-of-arrays views (see or_q4_matvec_soa); q/k/v are
 * three separate matrices.  The caches are f16, [layer][max_seq][kv_dim].
 * logits receives the f32 logits; returns the argmax token. */
typedef struct {
    int n_layers, d_model, n_heads, n_kv_heads, head_dim, d_ff, vocab, max_seq;
    float eps;
} or_llama_cfg;

typedef struct {
    const uint8_t* nib; const float* scales;
} or_q4_view;

typedef struct {
    const uint16_t* embed;        /* bf16 [vocab][d] */
    const uint16_t* attn_norm;    /* bf16 [L][d] */
    const uint16_t* ffn_norm;     /* bf16 [L][d] */
    const uint16_t* final_norm;   /* bf16 [d] */
    const or_q4_view* wq; const or_q4_view* wk; const or_q4_view* wv; const or_q4_view* wo;
    const or_q4_view* wg; const or_q4_view* wu; const or_q4_view* wd;
    or_q4_view lm_head;
    const float* rope_cos; const float* rope_sin; /* [max_seq][head_dim/2] */
} or_llama_weights;

static void linear_bf16in(const or_q4_view* w, size_t out_dim, size_t in_dim, const float* x,
                          float* y, double* xd, double* yd, int threads) {
    for (size_t i = 0; i < in_dim; i++) xd[i] = (double)or_bf16_to_f32(or_f32_to_bf16(x[i]));
    or_q4_matvec_soa(w->nib, w->scales, out_dim, in_dim, xd, yd, threads);
    for (size_t i = 0; i < out_dim; i++) y[i] = (float)yd[i];
}

int or_llama_decode_step(const or_llama_cfg* c, const or_llama_weights* W, uint16_t* k_cache,
                         uint16_t* v_cache, int token, int pos, float* logits, int threads) {
    size_t d = (size_t)c->d_model, kvd = (size_t)c->n_kv_heads * c->head_dim;
    size_t ff = (size_t)c->d_ff, ms = (size_t)c->max_seq;
    size_t big = ff > d ? ff : d;
    if ((size_t)c->vocab > big) big = (size_t)c->vocab;
    float* x = malloc(d * 4); float* h = malloc(d * 4); float* w = malloc(d * 4);
    float* q = malloc(d * 4); float* k = malloc(kvd * 4); float* v = malloc(kvd * 4);
    float* qr = malloc(d * 4); float* kr = malloc(kvd * 4); float* att = malloc(d * 4);
    float* o = malloc(d * 4); float* g = malloc(ff * 4); float* u = malloc(ff * 4);
    float* sgl = malloc(ff * 4);
    double* xd = malloc(big * 8); double* yd = malloc(big * 8);
    size_t T = (size_t)pos + 1;
    float* kf = malloc(T * kvd * 4); float* vf = malloc(T * kvd * 4);

    for (size_t i = 0; i < d; i++) x[i] = or_bf16_to_f32(W->embed[(size_t)token * d + i]);
    for (int l = 0; l < c->n_layers; l++) {
        for (size_t i = 0; i < d; i++) w[i] = or_bf16_to_f32(W->attn_norm[(size_t)l * d + i]);
        or_rms_norm(x, w, 1, d, c->eps, h);
        linear_bf16in(&W->wq[l], d, d, h, q, xd, yd, threads);
        linear_bf16in(&W->wk[l], kvd, d, h, k, xd, yd, threads);
        linear_bf16in(&W->wv[l], kvd, d, h, v, xd, yd, threads);
        or_rope_forward(q, W->rope_cos, W->rope_sin, 1, c->n_heads, c->head_dim, pos, qr);
        or_rope_forward(k, W->rope_cos, W->rope_sin, 1, c->n_kv_heads, c->head_dim, pos, kr);
        uint16_t* kc = k_cache + (size_t)l * ms * kvd;
        uint16_t* vc = v_cache + (size_t)l * ms * kvd;
        for (size_t i = 0; i < kvd; i++) {
            kc[(size_t)pos * kvd + i] = or_f32_to_f16(kr[i]);
            vc[(size_t)pos * kvd + i] = or_f32_to_f16(v[i]);
        }
        for (size_t i = 0; i < T * kvd; i++) { kf[i] = or_f16_to_f32(kc[i]); vf[i] = or_f16_to_f32(vc[i]); }
        or_kv_attention(qr, kf, vf, (size_t)pos, 1, c->n_heads, c->n_kv_heads, c->head_dim, att, threads);
        linear_bf16in(&W->wo[l], d, d, att, o, xd, yd, threads);
        or_add(x, o, d, x);
        for (size_t i = 0; i < d; i++) w[i] = or_bf16_to_f32(W->ffn_norm[(size_t)l * d + i]);
        or_rms_norm(x, w, 1, d, c->eps, h);
        linear_bf16in(&W->wg[l], ff, d, h, g, xd, yd, threads);
        linear_bf16in(&W->wu[l], ff, d, h, u, xd, yd, threads);
        or_swiglu(g, u, ff, sgl);
        linear_bf16in(&W->wd[l], d, ff, sgl, o, xd, yd, threads);
        or_add(x, o, d, x);
    }
    for (size_t i = 0; i < d; i++) w[i] = or_bf16_to_f32(W->final_norm[i]);
    or_rms_norm(x, w, 1, d, c->eps, h);
    linear_bf16in(&W->lm_head, (size_t)c->vocab, d, h, logits, xd, yd, threads);
    int tok = (int)or_argmax_f32(logits, (size_t)c->vocab);
    free(x); free(h); free(w); free(q); free(k); free(v); free(qr); free(kr); free(att); free(o);
    free(g); free(u); free(sgl); free(xd); free(yd); free(kf); free(vf);
    return tok;
}

/* ---------------------------------------------------------------------- */
/* MoE layer -- from definition (no reference implementation exists)      */
/* ---------------------------------------------------------------------- */

/* DeepSeek-style MoE FFN for T tokens (parity unpinned against the reference,
 * which has none; pinned by the invariants in tests/test_oracle.py):
 *   logits = h . W_r^T (f32, sequential), p = softmax(logits) (cpu.rs:105),
 *   top-k experts by p (ties -> lower expert index), weights = p of the chosen
 *   experts (not renormalised), expert e: down_e(swiglu(gate_e(hb), up_e(hb)))
 *   with the linears as q4_matvec on bf16-rounded inputs,
 *   out = sum_k w_k * expert_k(h) + sum_s shared_s(h), accumulated in f64 in
 *   the order (routed by rank, then shared), stored f32.
 * h: bf16 [T][d]; router: f32 [E][d]; experts: arrays of 3*E q4 views
 * (gate,up,down per expert), shared: 3*S views. */
void or_moe_forward(const uint16_t* h, size_t T, size_t d, size_t ff, size_t E, size_t S, size_t topk,
                    const float* router, const or_q4_view* experts, const or_q4_view* shared,
                    float* out, int32_t* topk_idx, float* topk_w, int threads) {
    size_t big = ff > d ? ff : d;
    float* lg = malloc(E * 4); float* p = malloc(E * 4);
    float* xf = malloc(d * 4); float* g = malloc(ff * 4); float* u = malloc(ff * 4);
    float* sg = malloc(ff * 4); float* y = malloc(d * 4);
    double* xd = malloc(big * 8); double* yd = malloc(big * 8); double* acc = malloc(d * 8);
    int* used = malloc(E * sizeof(int));
    for (size_t t = 0; t < T; t++) {
        for (size_t i = 0; i < d; i++) xf[i] = or_bf16_to_f32(h[t * d + i]);
        for (size_t e = 0; e < E; e++) {
            float s = 0.0f;
            for (size_t i = 0; i < d; i++) s += xf[i] * router[e * d + i];
            lg[e] = s;
        }
        or_softmax(lg, 1, E, p);
        memset(used, 0, E * sizeof(int));
        for (size_t k = 0; k < topk; k++) {
            size_t best = 0; float bv = -INFINITY; int found = 0;
            for (size_t e = 0; e < E; e++) if (!used[e] && (!found || p[e] > bv)) { bv = p[e]; best = e; found = 1; }
            used[best] = 1;
            topk_idx[t * topk + k] = (int32_t)best;
            topk_w[t * topk + k] = bv;
        }
        for (size_t i = 0; i < d; i++) acc[i] = 0.0;
        for (size_t k = 0; k < topk + S; k++) {
            const or_q4_view* ex;
            double wk;
            if (k < topk) { ex = &experts[3 * (size_t)topk_idx[t * topk + k]]; wk = topk_w[t * topk + k]; }
            else { ex = &shared[3 * (k - topk)]; wk = 1.0; }
            linear_bf16in(&ex[0], ff, d, xf, g, xd, yd, threads);
            linear_bf16in(&ex[1], ff, d, xf, u, xd, yd, threads);
            or_swiglu(g, u, ff, sg);
            linear_bf16in(&ex[2], d, ff, sg, y, xd, yd, threads);
            for (size_t i = 0; i < d; i++) acc[i] += wk * (double)y[i];
        }
        for (size_t i = 0; i < d; i++) out[t * d + i] = (float)acc[i];
    }
    free(lg); free(p); free(xf); free(g); free(u); free(sg); free(y); free(xd); free(yd); free(acc); free(used);
}

/* ---------------------------------------------------------------------- */
/* MLA decode attention -- from definition (no reference implementation)  */
/* ---------------------------------------------------------------------- */

/* Absorbed multi-head latent attention, one query token per sequence:
 *   q_lat[h]  = W_UK[h] . q_nope[b,h]         (W_UK int8 [H][r][dn], per-row scale)
 *   s[h,t]    = (q_lat[h] . c[b,t] + q_rope[b,h] . kr[b,t]) * sm_scale
 *   p         = softmax_t(s)                   (two-pass, f64)
 *   o_lat[h]  = sum_t p[h,t] c[b,t]
 *   out[b,h]  = W_UV[h] . o_lat[h]             (W_UV int8 [H][dv][r], per-row scale)
 * All sums in f64 (parity unpinned against the reference, which has none;
 * pinned by the explicit-decompression invariant in tests/test_oracle.py).
 * q_nope f32 [B][H][dn], q_rope f32 [B][H][dr], cache bf16 [B][L][r+dr]. */
void or_mla_decode(const float* q_nope, const float* q_rope, const uint16_t* cache, size_t B, size_t H,
                   size_t L, size_t dn, size_t dr, size_t r, size_t dv, const int8_t* wuk,
                   const float* wuk_scale, const int8_t* wuv, const float* wuv_scale, double sm_scale,
                   float* out, int threads) {
    set_threads(threads);
#pragma omp parallel for collapse(2) schedule(static) if (threads != 1)
    for (size_t b = 0; b < B; b++) {
        for (size_t hh = 0; hh < H; hh++) {
            double* ql = malloc(r * 8); double* s = malloc(L * 8); double* ol = malloc(r * 8);
            const float* qn = q_nope + (b * H + hh) * dn;
            const float* qr = q_rope + (b * H + hh) * dr;
            for (size_t i = 0; i < r; i++) {
                double acc = 0.0;
                const int8_t* wr = wuk + (hh * r + i) * dn;
                for (size_t j = 0; j < dn; j++) acc += (double)wr[j] * (double)qn[j];
                ql[i] = acc * (double)wuk_scale[hh * r + i];
            }
            double mx = -INFINITY;
            for (size_t t = 0; t < L; t++) {
                const uint16_t* row = cache + (b * L + t) * (r + dr);
                double acc = 0.0;
                for (size_t i = 0; i < r; i++) acc += ql[i] * (double)or_bf16_to_f32(row[i]);
                for (size_t i = 0; i < dr; i++) acc += (double)qr[i] * (double)or_bf16_to_f32(row[r + i]);
                s[t] = acc * sm_scale;
                if (s[t] > mx) mx = s[t];
            }
            double sum = 0.0;
            for (size_t t = 0; t < L; t++) { s[t] = exp(s[t] - mx); sum += s[t]; }
            for (size_t i = 0; i < r; i++) ol[i] = 0.0;
            for (size_t t = 0; t < L; t++) {
                const uint16_t* row = cache + (b * L + t) * (r + dr);
                double pt = s[t] / sum;
                for (size_t i = 0; i < r; i++) ol[i] += pt * (double)or_bf16_to_f32(row[i]);
            }
            for (size_t i = 0; i < dv; i++) {
                double acc = 0.0;
                const int8_t* wr = wuv + (hh * dv + i) * r;
                for (size_t j = 0; j < r; j++) acc += (double)wr[j] * ol[j];
                out[(b * H + hh) * dv + i] = (float)(acc * (double)wuv_scale[hh * dv + i]);
            }
            free(ql); free(s); free(ol);
        }
    }
}

/* ---------------------------------------------------------------------- */
/* Sampling (crates/tang-infer/src/sampling.rs)                            */
/* ---------------------------------------------------------------------- */

/* sampling.rs:6-20 SamplingConfig; stop_token < 0 means None. */
typedef struct {
    double temperature, top_p, repetition_penalty;
    size_t top_k, max_tokens;
    int64_t stop_token;
} or_sampling_cfg;

/* sampling.rs:77-80: LCG step, 53 high bits as [0, 1). */
static double or_rand_f64(uint64_t* state) {
    *state = *state * 6364136223846793005ULL + 1442695040888963407ULL;
    return (double)(*state >> 11) / (double)(1ULL << 53);
}

/* sampling.rs:184-194: first index with a strictly greater value. */
static size_t or_argmax_f64(const double* v, size_t n) {
    size_t best = 0;
    double bv = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

/* Stable descending order of indices by value (Rust's sort_by is a stable
 * merge sort; partial_cmp of NaN is treated as Equal).  Insertion-based merge
 * sort on index arrays. */
static void or_sort_desc_stable(const double* v, size_t* idx, size_t* tmp, size_t n) {
    for (size_t w = 1; w < n; w *= 2) {
        for (size_t lo = 0; lo < n; lo += 2 * w) {
            size_t mid = lo + w < n ? lo + w : n, hi = lo + 2 * w < n ? lo + 2 * w : n;
            size_t a = lo, b = mid, o = lo;
            while (a < mid && b < hi) {
                /* take from the right run only when it is strictly greater */
                if (v[idx[b]] > v[idx[a]]) tmp[o++] = idx[b++];
                else tmp[o++] = idx[a++];
            }
            while (a < mid) tmp[o++] = idx[a++];
            while (b < hi) tmp[o++] = idx[b++];
        }
        memcpy(idx, tmp, n * sizeof(size_t));
    }
}

/* sampling.rs:86-160 Sampler::sample, including kth_largest (:172-178) and
 * top_p_filter (:197-215), categorical_sample (:163-175).  logits: n values
 * (the Scalar -> f64 conversion of :91 is exact from f32). */
size_t or_sample(const or_sampling_cfg* c, uint64_t* state, const float* logits, size_t n, const int32_t* past,
                 size_t n_past) {
    double* p = malloc(n * sizeof(double));
    size_t* idx = malloc(n * sizeof(size_t));
    size_t* tmp = malloc(n * sizeof(size_t));
    size_t result;
    for (size_t i = 0; i < n; i++) p[i] = (double)logits[i];
    if (c->repetition_penalty != 1.0) {
        for (size_t j = 0; j < n_past; j++) {
            size_t t = (size_t)past[j];
            if (t < n) {
                if (p[t] > 0.0) p[t] /= c->repetition_penalty;
                else p[t] *= c->repetition_penalty;
            }
        }
    }
    if (c->temperature == 0.0) { result = or_argmax_f64(p, n); goto done; }
    if (c->temperature != 1.0) {
        double inv_t = 1.0 / c->temperature;
        for (size_t i = 0; i < n; i++) p[i] *= inv_t;
    }
    {
        double mx = -INFINITY;
        for (size_t i = 0; i < n; i++) mx = fmax(mx, p[i]);
        for (size_t i = 0; i < n; i++) p[i] = exp(p[i] - mx);
    }
    if (c->top_k > 0 && c->top_k < n) {
        for (size_t i = 0; i < n; i++) idx[i] = i;
        or_sort_desc_stable(p, idx, tmp, n);
        double thr = p[idx[c->top_k - 1]];
        for (size_t i = 0; i < n; i++) if (p[i] < thr) p[i] = 0.0;
    }
    {
        double sum = 0.0;
        for (size_t i = 0; i < n; i++) sum += p[i];
        if (sum <= 0.0) { result = or_argmax_f64(p, n); goto done; }
        for (size_t i = 0; i < n; i++) p[i] /= sum;
    }
    if (c->top_p < 1.0) {
        for (size_t i = 0; i < n; i++) idx[i] = i;
        or_sort_desc_stable(p, idx, tmp, n);
        double cum = 0.0;
        size_t cutoff = n;
        for (size_t r = 0; r < n; r++) {
            cum += p[idx[r]];
            if (cum >= c->top_p) { cutoff = r + 1; break; }
        }
        for (size_t r = cutoff; r < n; r++) p[idx[r]] = 0.0;
        double sum = 0.0;
        for (size_t i = 0; i < n; i++) sum += p[i];
        if (sum > 0.0) for (size_t i = 0; i < n; i++) p[i] /= sum;
    }
    {
        double r = or_rand_f64(state), cum = 0.0;
        result = n - 1;
        for (size_t i = 0; i < n; i++) {
            cum += p[i];
            if (r < cum) { result = i; break; }
        }
    }
done:
    free(p); free(idx); free(tmp);
    return result;
}
