// Dequant-fused weight-only quantized linear kernels for gfx950.
//
// Arithmetic spec: q4_matvec / q8_matvec (crates/tang-infer/src/quantize.rs:227-289):
//   y[m][n] = sum_b scale[n][b] * sum_i (q[n][32b+i]) * x[m][32b+i]
// with q = nibble-8 (int4) or the int8 value.  The device sums in f32.
//
// Weight layouts are described next to th_qweight in common.hpp.
#pragma once

#include <type_traits>

#include "common.hpp"
#include "ops.hpp"

namespace th {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float v) {
    // bits + 0x7FFF + lsb (crates/tang-compute/src/cuda.rs:22-27)
    uint32_t b = __float_as_uint(v);
    b += 0x7FFFu + ((b >> 16) & 1u);
    return b >> 16;
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// a.lo*b.lo + a.hi*b.hi + c with bf16 pairs, f32 accumulate (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Four nibble pairs of one packed word as bf16 pairs holding 128+nibble:
// pair k = (element k, element k+4) of the word's eight elements.  bf16 with
// exponent 2^7 has unit spacing, so 0x4300|n is exactly 128+n.
// The eight nibbles of one packed word (reference order: byte b holds
// elements 2b (low nibble) and 2b+1 (high nibble)) as four bf16 pairs of
// 128+nibble, built with byte permutes: lo/hi = the low/high nibbles of the
// four bytes, then v_perm_b32 splices in the 0x43 high bytes.
// Pair order: (e0,e2), (e4,e6), (e1,e3), (e5,e7); pack_x_q4 matches it.
__device__ __forceinline__ void nib_pairs_perm(uint32_t w, uint32_t p[4]) {
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    const uint32_t c43 = 0x43434343u;
    p[0] = __builtin_amdgcn_perm(c43, lo, 0x04010400u);
    p[1] = __builtin_amdgcn_perm(c43, lo, 0x04030402u);
    p[2] = __builtin_amdgcn_perm(c43, hi, 0x04010400u);
    p[3] = __builtin_amdgcn_perm(c43, hi, 0x04030402u);
}

// Eight bf16 x values as the pairs nib_pairs_perm produces.
__device__ __forceinline__ uint4 pack_x_q4(const uint32_t h[8]) {
    return make_uint4(h[0] | (h[2] << 16), h[4] | (h[6] << 16), h[1] | (h[3] << 16), h[5] | (h[7] << 16));
}

// Eight x values x[0..8) as the matching bf16 pairs (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ __forceinline__ uint4 pack_perm_bf16(const uint32_t h[8]) {
    uint4 o;
    o.x = h[0] | (h[4] << 16);
    o.y = h[1] | (h[5] << 16);
    o.z = h[2] | (h[6] << 16);
    o.w = h[3] | (h[7] << 16);
    return o;
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Streaming 128-bit load of packed weights (read once: non-temporal hint).
__device__ __forceinline__ uint4 ldg_stream(const uint4* p) {
    const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// A non-temporal load of a 16- or 8-byte record (the scale records of the
// single-tile GEMV: streamed once, like the weights).
template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) {
    if constexpr (sizeof(T) == 16) {
        const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
        return __builtin_bit_cast(T, v);
    } else {
        static_assert(sizeof(T) == 8, "16- or 8-byte records");
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t v = __builtin_nontemporal_load((const u32x2_t*)p);
        return __builtin_bit_cast(T, v);
    }
}

// Workgroup barrier that orders LDS accesses only: unlike __syncthreads()
// (a workgroup fence over all memory), it does not wait for this wave's
// outstanding global loads, so weights prefetched before it stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum over the 64 lanes in a fixed butterfly order (every lane gets it).
__device__ __forceinline__ float wave_sum_fixed(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_sum_xor16_32(float v) {
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// ---------------------------------------------------------------------------
// Epilogues: receive (batch row m, output column n, f32 value).
// ---------------------------------------------------------------------------

// `tile` points at the 16 finished values of the current 16-row tile for
// batch row m (tile[n % 16] == v), so an epilogue can combine neighbouring
// output rows (RoPE pairs, gate/up halves).
struct EpiStore {
    static constexpr bool HAS_FINISH = false;
    float* y; int ldy;
    __device__ __forceinline__ void operator()(int m, int n, float v, const float* tile, float*) const {
        st_coherent(&y[(size_t)m * ldy + n], v);
    }
    __device__ __forceinline__ void finish(int, int, const float*, int) const {}
};

// ---------------------------------------------------------------------------
// int4 GEMV, VALU path (small m).  One workgroup = one 16-row tile; its four
// waves take group-quads gq = wave, wave+4, ...  x is staged once per
// workgroup in LDS as bf16 pairs in nibble-pair order together with
// bias[m][gq][q][j] = -136 * sum of the eight x values lane q multiplies in
// group 4gq+j, so that dot(128+n, x) + bias = dot(n-8, x).
// f32 activations are split as x = hi + lo (two bf16, 16 significant bits)
// and both halves are dotted.
// ---------------------------------------------------------------------------

template <int U, typename ST>
struct ScaleVec;
template <int U>
struct ScaleVec<U, _Float16> {
    uint2 v[U];
    __device__ __forceinline__ void load(const _Float16* p, int u) { v[u] = *(const uint2*)p; }
    __device__ __forceinline__ float get(int u, int j) const { return (float)geth(u, j); }
    __device__ __forceinline__ _Float16 geth(int u, int j) const {
        uint32_t w = (j < 2) ? v[u].x : v[u].y;
        uint16_t h = (j & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xFFFF);
        return __builtin_bit_cast(_Float16, h);
    }
    // the scale times 2^e as f16 (one v_ldexp_f16; subnormal results exact
    // to f16's spacing)
    __device__ __forceinline__ _Float16 get_ldexp(int u, int j, int e) const {
        return __builtin_amdgcn_ldexph(geth(u, j), e);
    }
};
template <int U>
struct ScaleVec<U, float> {
    float4 v[U];
    __device__ __forceinline__ void load(const float* p, int u) { v[u] = *(const float4*)p; }
    __device__ __forceinline__ float get(int u, int j) const {
        return j == 0 ? v[u].x : j == 1 ? v[u].y : j == 2 ? v[u].z : v[u].w;
    }
    // scaled in f32, then rounded to f16 once
    __device__ __forceinline__ _Float16 get_ldexp(int u, int j, int e) const {
        return (_Float16)__builtin_amdgcn_ldexpf(get(u, j), e);
    }
};

// Eight consecutive activations x[m][k0..k0+8) of one row, raw: bf16 in
// a.xyzw, or f32 in a (elements 0-3) and b (4-7).  Elements at k >= K read as
// zero (VEC: finite values whose weights are zero).  Branch-free, so the
// loads stay in flight alongside the weight stream.  VEC requires K % 8 == 0,
// ldx % 8 == 0 and a 16-byte aligned base.
template <bool XF32, bool VEC>
__device__ __forceinline__ void load_x8(const void* xin, int m, int ldx, int K, int k0, uint4& a, uint4& b) {
    if (VEC) {
        // Chunks past K re-read the row start: the weights there are exact
        // zeros (packing forces elements >= K to the zero code), so any
        // finite value contributes nothing.
        const int kk = k0 < K ? k0 : 0;
        if (XF32) {
            const float* xr = (const float*)xin + (size_t)m * ldx + kk;
            a = *(const uint4*)xr;
            b = *(const uint4*)(xr + 4);
        } else {
            const uint16_t* xr = (const uint16_t*)xin + (size_t)m * ldx + kk;
            a = *(const uint4*)xr;
            b = make_uint4(0, 0, 0, 0);
        }
    } else {
        uint32_t v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int k = k0 + i;
            const int kk = k < K ? k : 0;
            uint32_t t = XF32 ? __float_as_uint(((const float*)xin)[(size_t)m * ldx + kk])
                              : (uint32_t)((const uint16_t*)xin)[(size_t)m * ldx + kk];
            v[i] = k < K ? t : 0u;
        }
        if (XF32) {
            a = make_uint4(v[0], v[1], v[2], v[3]);
            b = make_uint4(v[4], v[5], v[6], v[7]);
        } else {
            a = make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
            b = make_uint4(0, 0, 0, 0);
        }
    }
}

// Index of scale (row-tile t, group-quad gq, row r, group-in-quad j) in the
// q4 scale array.  f16: pairs of group-quads gq, gq+4 that one wave streams
// back to back sit in one 16-byte record per row:
//   [t][gq/8][gq%4][r][(gq%8)/4][j]   (GQ8 = ceil(GQ/8) octets per tile)
// f32: [t][gq][r][j].
__host__ __device__ inline size_t q4_scale_index(bool f16, size_t t, size_t gq, size_t r, size_t j, size_t GQ) {
    if (f16) {
        const size_t GQ8 = (GQ + 7) / 8;
        return ((((t * GQ8 + gq / 8) * 4 + gq % 4) * 16 + r) * 2 + (gq % 8) / 4) * 4 + j;
    }
    return ((t * GQ + gq) * 16 + r) * 4 + j;
}
inline size_t q4_scale_count(bool f16, size_t NT, size_t GQ) {
    return f16 ? NT * ((GQ + 7) / 8) * 512 : NT * GQ * 64;
}

// LDS bytes of the MFMA GEMV: per wave, x as [item][j][MR][q] 16-byte
// chunks plus a zero chunk and the bias as [item][j][8] floats; then the
// cross-wave reduction [NW][8][16], the finished tile [M][16] and 16 floats
// of epilogue scratch.  PAR > 1 (tiles streamed side by side): each wave's
// region also holds its partials of the PAR tiles once its items are done
// ([PAR][RS][16] floats, so the region is at least that large), and the
// finished values of all PAR tiles ([PAR][M][16]) follow the scratch.
template <int MR, int NW = 4, int PAR = 1>
struct Q4GemvSmem {
    static constexpr int BS = MR <= 8 ? 8 : 16;  // bias floats per (item, group)
    static constexpr int RS = MR <= 8 ? 8 : 16;  // reduction rows
    __host__ __device__ static size_t per_wave(int items) {
        const size_t staging = (size_t)items * 4 * (MR * 64 + BS * 4) + 16;
        const size_t partials = PAR > 1 ? (size_t)PAR * RS * 16 * 4 : 0;
        return staging > partials ? staging : partials;
    }
    static size_t bytes(int GQ) {
        const int items = (GQ + NW - 1) / NW;
        const size_t tiles = PAR > 1 ? (size_t)PAR * 16 * RS * 4 : 0;
        return NW * per_wave(items) + NW * RS * 16 * 4 + 16 * 16 * 4 + 16 * 4 + tiles;
    }
};

// Default source of a GEMV workgroup: one weight matrix, tile = blockIdx.x,
// activation rows 0..M-1.  A grouped launch (MoE experts) supplies a policy
// with the same members that picks the expert's weights, the tile, the
// number of live rows and the gathered activation / output rows.
struct SingleMatrix {
    static constexpr bool GROUPED = false;
    static constexpr int TPW = 1;  // tiles per workgroup
    template <typename ST>
    __device__ __forceinline__ bool select(int bid, const uint4*& wt, const ST*& sc, int& t, int& mrows) {
        t = bid;
        return true;
    }
    __device__ __forceinline__ int x_row(int m) const { return m; }
    __device__ __forceinline__ int out_row(int m) const { return m; }
};

// One matrix, TPW consecutive tiles per workgroup (activations staged once).
template <int TPWv>
struct SingleMatrixTiles : SingleMatrix {
    static constexpr int TPW = TPWv;
    int tiles;  // 16-row tiles of the matrix
    int nt = 1;
    template <typename ST>
    __device__ __forceinline__ bool select(int bid, const uint4*& wt, const ST*& sc, int& t, int& mrows) {
        t = bid * TPW;
        nt = min(TPW, tiles - t);
        return true;
    }
    __device__ __forceinline__ int tiles_here() const { return nt; }
};

// One matrix, `per` consecutive tiles per workgroup (chosen so that the grid
// is one round of the chip: a staged 8/16-row activation block is then read
// from HBM once per CU, not once per tile), with `rows` live activation rows
// when RT_ROWS (otherwise the kernel's constant row count).
template <bool RT_ROWS>
struct SingleMatrixSpan : SingleMatrix {
    static constexpr int TPW = 2;  // > 1: the kernel runs its multi-tile loop
    int tiles, per, rows = 0;
    int nt = 1;
    template <typename ST>
    __device__ __forceinline__ bool select(int bid, const uint4*& wt, const ST*& sc, int& t, int& mrows) {
        t = bid * per;
        nt = min(per, tiles - t);
        if constexpr (RT_ROWS) mrows = rows;
        return true;
    }
    __device__ __forceinline__ int tiles_here() const { return nt; }
};

// Scale access: f16 scales of the items (gq, gq+4) share one 16-byte record,
// so with four waves per tile one load serves two consecutive items; with
// any other wave count each item loads its own 8-byte half.
template <typename ST, int NW>
struct ScaleRec;
template <>
struct ScaleRec<_Float16, 4> {
    static constexpr int ITEMS = 2;
    typedef uint4 Rec;
    __device__ __forceinline__ static float get(const Rec& v, int h, int j) {
        const uint32_t w = h ? (j < 2 ? v.z : v.w) : (j < 2 ? v.x : v.y);
        const uint16_t b = (j & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xFFFF);
        return (float)__builtin_bit_cast(_Float16, b);
    }
};
template <int NW>
struct ScaleRec<_Float16, NW> {
    static constexpr int ITEMS = 1;
    typedef uint2 Rec;
    __device__ __forceinline__ static float get(const Rec& v, int, int j) {
        const uint32_t w = j < 2 ? v.x : v.y;
        const uint16_t b = (j & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xFFFF);
        return (float)__builtin_bit_cast(_Float16, b);
    }
};
template <int NW>
struct ScaleRec<float, NW> {
    static constexpr int ITEMS = 1;
    typedef uint4 Rec;
    __device__ __forceinline__ static float get(const Rec& v, int, int j) {
        return __uint_as_float(j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w);
    }
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// Optional RMSNorm prologue (rms_norm, crates/tang-compute/src/cpu.rs:126):
// the activation is the f32 residual x; the kernel sums the producer's
// per-16-element partials ssq[0..nssq) in a fixed order, and stages
// bf16(x * (1/sqrt(sum/K + eps)) * w) as the linear's input.
struct NormArgs {
    const float* ssq = nullptr;
    int nssq = 0;
    const uint16_t* w = nullptr;
    float eps = 0.0f;
};

// Default epilogue hook run by every thread after the tile's epilogue calls.
struct EpiNoFinish {
    static constexpr bool HAS_FINISH = false;
    __device__ __forceinline__ void finish(int, int, const float*, int) const {}
};

// ---------------------------------------------------------------------------
// int4 GEMV for m <= 4 on MFMA, "transposed": A = activations (row m = batch
// row, MR rows used: m, or hi/lo bf16 halves 2m, 2m+1 for f32 input),
// B = the tile's weights (column n = weight row).  One
// v_mfma_f32_16x16x32_bf16 per group of 32: B holds 128+nibble as bf16
// (exact), C carries bias = -136 * sum(x over the group) so
// D[m][n] = sum (nibble-8) * x, and acc[m][n] += scale[n][g] * D[m][n].
// One workgroup = one 16-row tile; its NW waves take group-quads
// gq = w + NW*i ("items"), stage only the activations they need in their own
// LDS region (no workgroup barrier) and keep D items of weights in flight.
// ---------------------------------------------------------------------------
// PAR > 1 (multi-tile sources only): the workgroup's tiles (at most PAR)
// are streamed side by side rather than one after another, every staged
// activation fragment feeding PAR weight tiles, and one cross-wave
// reduction at the end serves them all.
template <int MR, bool XF32, bool VEC, typename ST, typename Epi, int D = 2, int WPE = 4, int NW = 4,
          bool NORM = false, typename Src = SingleMatrix, int PAR = 1>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE))) void q4_gemv_kernel(
    const uint4* __restrict__ wt, const ST* __restrict__ sc, const void* __restrict__ xin, int K, int Kp, int N,
    int ldx, Epi epi, NormArgs norm, Src src = Src{}) {
    using SR = ScaleRec<ST, NW>;
    constexpr int SI = SR::ITEMS;
    constexpr int NS = D / SI;             // scale records in flight
    constexpr int M = XF32 ? MR / 2 : MR;  // activation rows
    constexpr bool F16S = std::is_same<ST, _Float16>::value;
    constexpr bool LOADF32 = XF32 || NORM;
    static_assert(!NORM || (MR == 1 && !XF32), "the RMSNorm prologue serves one bf16 row");
    static_assert(D % SI == 0, "prefetch depth must cover whole scale records");
    using Smem = Q4GemvSmem<MR, NW, PAR>;
    constexpr int BS = Smem::BS, RS = Smem::RS;
    extern __shared__ uint4 smem[];
    const int GQ = Kp >> 7;
    const int items_max = (GQ + NW - 1) / NW;

    int t = 0, mrows = M;  // tile, live activation rows (<= M)
    {
        const uint4* wsel = wt;
        const ST* ssel = sc;
        if (!src.select((int)blockIdx.x, wsel, ssel, t, mrows)) return;
        wt = wsel;
        sc = ssel;
    }
    // wave index in a scalar register: item indices, validity tests and the
    // wave's weight / scale addresses then run on the scalar unit
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int nmine = (GQ - wave + NW - 1) / NW;  // items of this wave (wave-uniform)

    // per-wave LDS region
    char* wl = (char*)smem + (size_t)wave * Smem::per_wave(items_max);
    uint4* xw = (uint4*)wl;                                   // [item][j][MR][4]
    uint4* zero = xw + (size_t)items_max * 4 * MR * 4;        // one zero chunk
    float* bw = (float*)(zero + 1);                           // [item][j][BS]
    float* red = (float*)((char*)smem + NW * Smem::per_wave(items_max));  // [NW][RS][16]
    float* tilev = red + NW * RS * 16;                        // [M][16]
    float* aux = tilev + 16 * 16;                             // [16]

    const uint4* wp = wt + (size_t)t * GQ * 64 + lane;
    auto item_gq = [&](int i) { return i < nmine ? wave + NW * i : 0; };
    // The weight stream of the plain-output GEMV up to 8 rows as buffer loads
    // off one scalar base (the byte offset per lane in a VGPR) with the
    // non-temporal bit, else non-temporal global loads.  Same-box A/B of the
    // two forms (whatever the other cache bits): config 2 M=1 5.84 against
    // 5.95 us, M=8 7.80 against 8.19, M=4 equal, but M=16 9.1-9.3 against
    // 8.9 and the decode step's fused-epilogue GEMVs 0.3% slower.
    constexpr bool BUF_W = MR <= 8 && !NORM && std::is_same<Epi, EpiStore>::value;
    // based at the tile (t is uniform), so the offsets stay below GQ KiB for
    // any matrix size
    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(wt + (size_t)t * GQ * 64, 0xFFFFFFFFu);
    auto load_item = [&](int i) -> uint4 {
        if constexpr (BUF_W) {
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(
                wrs, (uint32_t)(lane + item_gq(i) * 64) * 16u, 0, CPOL_NT);
            return make_uint4(v.x, v.y, v.z, v.w);
        } else {
            return ldg_stream(wt + (size_t)t * GQ * 64 + lane + (size_t)item_gq(i) * 64);
        }
    };
    auto scale_ptr_t = [&](int i, int tile) -> const typename SR::Rec* {
        const int gq = item_gq(i);  // past the end: a valid record of this tile
        const int g0 = (F16S && NW == 4) ? (gq & ~4) : gq;
        return (const typename SR::Rec*)(sc + q4_scale_index(F16S, tile, g0, r, 0, GQ));
    };
    auto scale_ptr = [&](int i) { return scale_ptr_t(i, t); };
    // single-tile sources stream their scale records non-temporally, like the
    // weights (config 2, M=1: 6.07 -> 5.99 us; multi-tile spans keep plain loads)
    auto load_scale = [&](int i) -> typename SR::Rec {
        if constexpr (Src::TPW == 1) return ld_nt(scale_ptr(i));
        else return *scale_ptr(i);
    };
    // tiles of this workgroup: t, t+1, ... (one unless the source groups them)
    int ntl = 1;
    if constexpr (Src::TPW > 1) ntl = src.tiles_here();

    // 1. activations for this wave's groups.  Task (item i, group j, row m)
    //    covers the 32 values of one group; its four 8-value chunks go to
    //    four consecutive lanes, so one load instruction reads contiguous
    //    memory (16 lanes span a 128-value item of one row).  A lane takes
    //    chunk (task slot) lane + 64 * pass.
    constexpr int PRE = MR <= 1 ? 2 : (MR <= 4 ? 4 : 8);  // passes loaded before the weight stream
    constexpr int BATCH = 4;                                // passes per later load round
    const int ntask = nmine * 4 * mrows;
    const int nchunk = ntask * 4;
    auto chunk_src = [&](int ci, int& xr, int& k0) {
        const int task = ci >> 2, c = ci & 3;
        const int m = task % mrows, ij = task / mrows, i = ij >> 2, j = ij & 3;
        xr = src.x_row(m);
        k0 = (4 * (wave + NW * i) + j) * 32 + c * 8;
    };
    uint4 xa[PRE], xb[PRE], nw[PRE];
    // RMSNorm partials (at most 256 = 4 per lane): loaded now, summed after
    // the weight stream is issued.
    float ssq_raw[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (NORM) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = lane + 64 * u;
            ssq_raw[u] = norm.ssq[i < norm.nssq ? i : 0];
        }
    }
#pragma unroll
    for (int pp = 0; pp < PRE; pp++) {
        int ci = lane + pp * 64;
        ci = ci < nchunk ? ci : 0;
        int xr, k0;
        chunk_src(ci, xr, k0);
        load_x8<LOADF32, VEC>(xin, xr, ldx, K, k0, xa[pp], xb[pp]);
        if (NORM) {
            uint4 dummy;
            load_x8<false, VEC>(norm.w, 0, 0, K, k0, nw[pp], dummy);
        }
    }
    // 2. weights and scales in flight
    //    Issue order = consumption order (a record before the weights of its
    //    items): loads complete in order, so an item never waits for a load
    //    issued after its own.
    uint4 wbuf[D];
    typename SR::Rec sbuf[NS], scur;
    static_assert(PAR == 1 || Src::TPW > 1, "side-by-side tiles need a multi-tile source");
    constexpr int PX = PAR > 1 ? PAR - 1 : 1;
    uint4 wbx[PX][D];  // PAR > 1: items of tiles t+1 .. t+PAR-1
    typename SR::Rec sbx[PX][NS];
    // tile p of this workgroup (past its last tile: a duplicate of that tile, never stored)
    auto tile_p = [&](int p) { return t + (p < ntl ? p : ntl - 1); };
#pragma unroll
    for (int u = 0; u < D; u++) {
        if (u % SI == 0) sbuf[u / SI] = load_scale(u);
        wbuf[u] = load_item(u);
        if constexpr (PAR > 1) {
#pragma unroll
            for (int pp = 0; pp < PAR - 1; pp++) {
                const int tp = tile_p(pp + 1);
                if (u % SI == 0) sbx[pp][u / SI] = *scale_ptr_t(u, tp);
                wbx[pp][u] = ldg_stream(wt + (size_t)tp * GQ * 64 + lane + (size_t)item_gq(u) * 64);
            }
        }
    }
    float inv_rms = 1.0f;
    if (NORM) {
        float part = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++) part += (lane + 64 * u < norm.nssq) ? ssq_raw[u] : 0.0f;
        const float tot = wave_sum_fixed(part);
        inv_rms = 1.0f / sqrtf(tot / (float)K + norm.eps);
    }
    // 3. stage: bf16 pairs in nibble-pair order; f32 input as hi/lo rows.
    //    The group's bias needs the sum over its four chunks: partial sums
    //    meet across the four lanes (every lane of a pass takes part, so the
    //    shuffles see defined values; surplus lanes write nothing).
    auto stage = [&](int ci, bool live, const uint4& ra, const uint4& rb, const uint4& rw) {
        const int task = ci >> 2, c = ci & 3;
        const int m = task % mrows, ij = task / mrows;
        float xv[8];
        if (LOADF32) {
            xv[0] = __uint_as_float(ra.x); xv[1] = __uint_as_float(ra.y);
            xv[2] = __uint_as_float(ra.z); xv[3] = __uint_as_float(ra.w);
            xv[4] = __uint_as_float(rb.x); xv[5] = __uint_as_float(rb.y);
            xv[6] = __uint_as_float(rb.z); xv[7] = __uint_as_float(rb.w);
        } else {
            const uint32_t w4[4] = {ra.x, ra.y, ra.z, ra.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                xv[2 * e] = bf16_bits_to_f32(w4[e] & 0xFFFF);
                xv[2 * e + 1] = bf16_bits_to_f32(w4[e] >> 16);
            }
        }
        if (NORM) {
            const uint32_t w4[4] = {rw.x, rw.y, rw.z, rw.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                // cpu.rs:146: x * inv_rms * w
                xv[2 * e] = xv[2 * e] * inv_rms * bf16_bits_to_f32(w4[e] & 0xFFFF);
                xv[2 * e + 1] = xv[2 * e + 1] * inv_rms * bf16_bits_to_f32(w4[e] >> 16);
            }
        }
        uint32_t hi[8], lo[8];
        float s_hi = 0.0f, s_lo = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            hi[e] = f32_to_bf16_bits(xv[e]);
            const float fh = bf16_bits_to_f32(hi[e]);
            s_hi += fh;
            if (XF32) {
                lo[e] = f32_to_bf16_bits(xv[e] - fh);
                s_lo += bf16_bits_to_f32(lo[e]);
            }
        }
        // group sum over the four chunk lanes: (c0 + c1) + (c2 + c3)
        s_hi += __shfl_xor(s_hi, 1, 64);
        s_hi += __shfl_xor(s_hi, 2, 64);
        if (XF32) {
            s_lo += __shfl_xor(s_lo, 1, 64);
            s_lo += __shfl_xor(s_lo, 2, 64);
        }
        if (!live) return;
        if (XF32) {
            xw[((size_t)ij * MR + 2 * m) * 4 + c] = pack_x_q4(hi);
            xw[((size_t)ij * MR + 2 * m + 1) * 4 + c] = pack_x_q4(lo);
        } else {
            xw[((size_t)ij * MR + m) * 4 + c] = pack_x_q4(hi);
        }
        if (c == 0) {
            if (XF32) {
                bw[ij * BS + 2 * m] = -136.0f * s_hi;
                bw[ij * BS + 2 * m + 1] = -136.0f * s_lo;
            } else {
                bw[ij * BS + m] = -136.0f * s_hi;
            }
        }
    };
    if (lane == 0) *zero = make_uint4(0, 0, 0, 0);
    const int mr_live = XF32 ? 2 * mrows : mrows;
    for (int ij = lane; ij < nmine * 4; ij += 64)
        for (int e = mr_live; e < BS; e++) bw[ij * BS + e] = 0.0f;
#pragma unroll
    for (int pp = 0; pp < PRE; pp++) {
        // no wave-uniform skip of whole passes: a load left unconsumed on one
        // path makes the compiler wait for every outstanding load (weights
        // included) where the paths join
        const int ci = lane + pp * 64;
        stage(ci < nchunk ? ci : 0, ci < nchunk, xa[pp], xb[pp], nw[pp]);
    }
    for (int base = PRE * 64; base < nchunk; base += BATCH * 64) {  // wave-uniform loop
        // every load of the round first, then the staging (one latency per round)
        uint4 ra[BATCH], rb[BATCH], rw[BATCH];
#pragma unroll
        for (int pp = 0; pp < BATCH; pp++) {
            const int ci = base + pp * 64 + lane;
            int xr, k0;
            chunk_src(ci < nchunk ? ci : 0, xr, k0);
            load_x8<LOADF32, VEC>(xin, xr, ldx, K, k0, ra[pp], rb[pp]);
            rw[pp] = make_uint4(0, 0, 0, 0);
            if (NORM) {
                uint4 dummy;
                load_x8<false, VEC>(norm.w, 0, 0, K, k0, rw[pp], dummy);
            }
        }
#pragma unroll
        for (int pp = 0; pp < BATCH; pp++) {
            const int ci = base + pp * 64 + lane;
            stage(ci < nchunk ? ci : 0, ci < nchunk, ra[pp], rb[pp], rw[pp]);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");

    constexpr int ACC = MR < 4 ? MR : 4;
    // A rows >= MR and C rows >= MR only feed D rows that are discarded, so
    // those lanes read real (finite) data of another row: no masking needed.
    const uint4* abase = xw + (size_t)(r < mr_live ? r : 0) * 4 + q;
    const float* cbase = bw + 4 * (q & (BS / 4 - 1));
    // one item (local index i) of the current tile: four MFMAs (one per
    // group, bias in C) and the scale FMAs into acc
    auto item_mfma = [&](int i, const uint4& wv, const float (&sj)[4], float (&acc)[4]) {
        const uint32_t wj[4] = {wv.x, wv.y, wv.z, wv.w};
        const uint4* ai = abase + (size_t)i * 4 * MR * 4;
        const float* ci = cbase + i * 4 * BS;
        uint4 aq[4];
        float4 cb[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            aq[j] = ai[j * MR * 4];
            cb[j] = *(const float4*)(ci + j * BS);
        }
        float4_t d[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t p[4];
            nib_pairs_perm(wj[j], p);
            const uint4 bq = make_uint4(p[0], p[1], p[2], p[3]);
            const float4_t c = {cb[j].x, cb[j].y, cb[j].z, cb[j].w};
            d[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, aq[j]),
                                                           __builtin_bit_cast(bf16x8_t, bq), c, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int e = 0; e < ACC; e++) acc[e] = __builtin_fmaf(sj[j], d[j][e], acc[e]);
        }
    };
    // cross-wave reduction of one tile's partial sums and its epilogue
    // trailing: a barrier after it (another tile follows in this workgroup)
    auto tile_end = [&](int tile, const float (&acc)[4], bool trailing) {
        // lane (q, r) holds D rows 4q..4q+3 of column r
        if (q * 4 < MR) {
#pragma unroll
            for (int e = 0; e < ACC; e++)
                if (4 * q + e < MR) red[(wave * RS + 4 * q + e) * 16 + r] = acc[e];
        }
        lds_barrier();
        float v = 0.0f;
        if (tid < 16 * M) {
            const int m = tid >> 4, rr = tid & 15;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                if (XF32) v += red[(w * RS + 2 * m) * 16 + rr] + red[(w * RS + 2 * m + 1) * 16 + rr];
                else v += red[(w * RS + m) * 16 + rr];
            }
            tilev[m * 16 + rr] = v;
        }
        lds_barrier();
        if (tid < 16 * M) {
            const int m = tid >> 4, rr = tid & 15;
            const int n = tile * 16 + rr;
            if (n < N && m < mrows) epi(src.out_row(m), n, v, tilev + m * 16, aux);
        }
        if constexpr (Epi::HAS_FINISH) {
            lds_barrier();
            epi.finish(tile, (int)gridDim.x, aux, tid);
        }
        if (trailing) lds_barrier();  // red and tilev are rewritten by the next tile
    };
    if constexpr (PAR > 1) {
        float accp[PAR][4];
#pragma unroll
        for (int pp = 0; pp < PAR; pp++)
#pragma unroll
            for (int e = 0; e < 4; e++) accp[pp][e] = 0.0f;
        typename SR::Rec scp[PAR];
        auto stepP = [&](auto refill_tag, int u, int i) {
#pragma unroll
            for (int pp = 0; pp < PAR; pp++) {
                const uint4 wv = pp == 0 ? wbuf[u] : wbx[pp - 1][u];
                if (u % SI == 0) scp[pp] = pp == 0 ? sbuf[u / SI] : sbx[pp - 1][u / SI];
                const typename SR::Rec sv = scp[pp];
                if constexpr (decltype(refill_tag)::value) {
                    const int tp = tile_p(pp);
                    typename SR::Rec& sdst = pp == 0 ? sbuf[u / SI] : sbx[pp - 1][u / SI];
                    uint4& wdst = pp == 0 ? wbuf[u] : wbx[pp - 1][u];
                    if (u % SI == 0) sdst = *scale_ptr_t(i + D, tp);
                    wdst = ldg_stream(wt + (size_t)tp * GQ * 64 + lane + (size_t)item_gq(i + D) * 64);
                }
                if (i >= nmine) continue;  // wave-uniform
                float sj[4];
#pragma unroll
                for (int j = 0; j < 4; j++) sj[j] = SR::get(sv, u % SI, j);
                item_mfma(i, wv, sj, accp[pp]);
            }
        };
        const int nbatch = (nmine + D - 1) / D;
        for (int bt = 0; bt + 1 < nbatch; bt++) {
#pragma unroll
            for (int u = 0; u < D; u++) stepP(std::true_type{}, u, bt * D + u);
        }
        if (nbatch > 0) {
#pragma unroll
            for (int u = 0; u < D; u++) stepP(std::false_type{}, u, (nbatch - 1) * D + u);
        }
        // One reduction for all PAR tiles: each wave's partials go to its
        // own staging region (its activations are no longer read), then
        // every output sums the waves in order, as tile_end does.
        float* mine = (float*)wl;  // [PAR][RS][16]
        if (q * 4 < MR) {
#pragma unroll
            for (int pp = 0; pp < PAR; pp++)
#pragma unroll
                for (int e = 0; e < ACC; e++)
                    if (4 * q + e < MR) mine[(pp * RS + 4 * q + e) * 16 + r] = accp[pp][e];
        }
        lds_barrier();
        // finished values of every tile: [PAR][M][16] after the epilogue scratch
        float* tv = aux + 16;
        for (int idx = tid; idx < PAR * 16 * M; idx += 64 * NW) {
            const int pp = idx / (16 * M), m = (idx >> 4) % M, rr = idx & 15;
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float* rw = (const float*)((const char*)smem + (size_t)w * Smem::per_wave(items_max)) +
                                  pp * RS * 16;
                if (XF32) v += rw[(2 * m) * 16 + rr] + rw[(2 * m + 1) * 16 + rr];
                else v += rw[m * 16 + rr];
            }
            tv[idx] = v;
        }
        lds_barrier();
        // epilogues tile by tile (they may read their tile's values and run
        // a per-tile finish hook)
#pragma unroll
        for (int pp = 0; pp < PAR; pp++) {
            if (pp >= ntl) break;  // workgroup-uniform
            if (tid < 16 * M) {
                const int m = tid >> 4, rr = tid & 15;
                const int n = (t + pp) * 16 + rr;
                if (n < N && m < mrows) epi(src.out_row(m), n, tv[(pp * M + m) * 16 + rr], tv + (pp * M + m) * 16, aux);
            }
            if constexpr (Epi::HAS_FINISH) {
                lds_barrier();
                epi.finish(t + pp, (int)gridDim.x, aux, tid);
                lds_barrier();  // aux is rewritten by the next tile's epilogue
            }
        }
        return;
    }
    // a 16-byte block of the activations (its allocation is 256-byte aligned)
    const void* xhot = (const void*)((uintptr_t)xin & ~(uintptr_t)15);
    for (int tt = 0; tt < ntl; tt++) {  // one trip unless the source groups tiles
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        // the next tile of a multi-tile source (branch-free: past the last
        // tile the loads read xhot, below)
        const int tn = tt + 1 < ntl ? t + 1 : t;
        const uint4* wpn = wt + (size_t)tn * GQ * 64 + lane;
        // refill: 1 = item i + D of this tile, 2 = item u of the next tile
        auto step = [&](auto refill_tag, int u, int i) {
            const uint4 wv = wbuf[u];
            if (u % SI == 0) scur = sbuf[u / SI];  // this record serves items i .. i+SI-1
            const typename SR::Rec sv = scur;
            if constexpr (decltype(refill_tag)::value == 1) {
                if (u % SI == 0) sbuf[u / SI] = load_scale(i + D);
                wbuf[u] = load_item(i + D);
            } else if constexpr (decltype(refill_tag)::value == 2) {
                // past the last tile the refill reads the activations (hot
                // in L2, never used): a re-read of this tile's own items
                // would stream from HBM again (the weights are loaded
                // non-temporally)
                const bool more = tt + 1 < ntl;
                if (u % SI == 0)
                    sbuf[u / SI] = more ? *scale_ptr_t(u, tn) : *(const typename SR::Rec*)xhot;
                wbuf[u] = ldg_stream(more ? wpn + (size_t)item_gq(u) * 64 : (const uint4*)xhot);
            }
            if (i >= nmine) return;  // past this wave's items (wave-uniform: a scalar branch)
            float sj[4];
#pragma unroll
            for (int j = 0; j < 4; j++) sj[j] = SR::get(sv, u % SI, j);
            item_mfma(i, wv, sj, acc);
        };
        const int nbatch = (nmine + D - 1) / D;
        for (int bt = 0; bt + 1 < nbatch; bt++) {
#pragma unroll
            for (int u = 0; u < D; u++) step(std::integral_constant<int, 1>{}, u, bt * D + u);
        }
        // last batch: a multi-tile source puts the next tile's first items in
        // flight as each buffer frees, so they stream in during this batch's
        // MFMAs, the reduction and the epilogue
        constexpr int LAST = Src::TPW > 1 ? 2 : 0;
        if (nbatch > 0) {
#pragma unroll
            for (int u = 0; u < D; u++) step(std::integral_constant<int, LAST>{}, u, (nbatch - 1) * D + u);
        } else if constexpr (LAST == 2) {
            const bool more = tt + 1 < ntl;
#pragma unroll
            for (int u = 0; u < D; u++) {
                if (u % SI == 0) sbuf[u / SI] = more ? *scale_ptr_t(u, tn) : *(const typename SR::Rec*)xhot;
                wbuf[u] = ldg_stream(more ? wpn + (size_t)item_gq(u) * 64 : (const uint4*)xhot);
            }
        }
        tile_end(t, acc, Src::TPW > 1);
        if constexpr (Src::TPW > 1) {
            t += 1;
            wp = wt + (size_t)t * GQ * 64 + lane;
        }
    }  // tiles
}

// ---------------------------------------------------------------------------
// int8 GEMV, VALU path.  One workgroup = one 16-row tile; its NW waves take
// chunks c = wave, wave+NW, ...  x is staged in LDS as f32 with
// bias[m][c][q] = -128 * sum of the 16 x values of lane-quad q, so that
// sum((q8 ^ 0x80) * x) + bias = sum(q8 * x).
// ---------------------------------------------------------------------------

template <int M, int NW = 4>
struct Q8GemvSmem {
    static size_t bytes(int Kp) { return (size_t)M * Kp * 4 + (size_t)M * (Kp / 16) * 4 + (NW + 1) * 16 * M * 4 + 64 * 4; }
};

template <int M, bool XF32, bool VEC, bool PER_ROW, typename Epi, int NW = 4, int DQ = 4>
__global__ __launch_bounds__(64 * NW) void q8_gemv_kernel(const uint4* __restrict__ wt,
                                                      const float* __restrict__ sc,
                                                      const void* __restrict__ xin, int K, int Kp,
                                                      int N, int ldx, Epi epi) {
    constexpr int D = DQ;  // weight chunks in flight per wave (4: best on config 1 with 4 or 8 waves)
    constexpr int XB = 4;  // 16-element x chunks per thread loaded ahead of the weights
    extern __shared__ uint4 smem[];
    const int NCH = Kp >> 6;  // 64-element chunks
    const int N16 = Kp >> 4;  // 16-element chunks per x row
    float* xl = (float*)smem;                 // [M][Kp]
    float* bias = xl + (size_t)M * Kp;        // [M][Kp/16]
    float* red = bias + (size_t)M * N16;

    const int t = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int nmine = (NCH - wave + NW - 1) / NW;
    const uint4* wp = wt + (size_t)t * NCH * 64 + lane;
    const int row = t * 16 + r;
    const int GPR = Kp >> 5;  // groups per row (per-group scales)
    const int nchunks = M * N16;
    auto item_off = [&](int i) { return (size_t)(i < nmine ? wave + NW * i : 0) * 64; };

    uint4 xa[XB][2], xb[XB][2];
#pragma unroll
    for (int b = 0; b < XB; b++) {
        int c = tid + b * 64 * NW;
        c = c < nchunks ? c : nchunks - 1;
        const int m = c / N16, k0 = (c - m * N16) * 16;
        load_x8<XF32, VEC>(xin, m, ldx, K, k0, xa[b][0], xb[b][0]);
        load_x8<XF32, VEC>(xin, m, ldx, K, k0 + 8, xa[b][1], xb[b][1]);
    }
    uint4 wbuf[D];
#pragma unroll
    for (int u = 0; u < D; u++) wbuf[u] = ldg_stream(wp + item_off(u));

    auto stage = [&](int c, const uint4 a[2], const uint4 b[2]) {
        const int m = c / N16, c16 = c - m * N16;
        float* dst = xl + (size_t)m * Kp + c16 * 16;
        float s = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float v[8];
            if (XF32) {
                v[0] = __uint_as_float(a[h].x); v[1] = __uint_as_float(a[h].y);
                v[2] = __uint_as_float(a[h].z); v[3] = __uint_as_float(a[h].w);
                v[4] = __uint_as_float(b[h].x); v[5] = __uint_as_float(b[h].y);
                v[6] = __uint_as_float(b[h].z); v[7] = __uint_as_float(b[h].w);
            } else {
                const uint32_t w4[4] = {a[h].x, a[h].y, a[h].z, a[h].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v[2 * i] = bf16_bits_to_f32(w4[i] & 0xFFFF);
                    v[2 * i + 1] = bf16_bits_to_f32(w4[i] >> 16);
                }
            }
#pragma unroll
            for (int i = 0; i < 8; i++) s += v[i];
            *(float4*)(dst + h * 8) = make_float4(v[0], v[1], v[2], v[3]);
            *(float4*)(dst + h * 8 + 4) = make_float4(v[4], v[5], v[6], v[7]);
        }
        bias[(size_t)m * N16 + c16] = -128.0f * s;
    };
#pragma unroll
    for (int b = 0; b < XB; b++) {
        const int c = tid + b * 64 * NW;
        if (c < nchunks) stage(c, xa[b], xb[b]);
    }
    for (int c = tid + XB * 64 * NW; c < nchunks; c += 64 * NW) {
        uint4 a[2], b2[2];
        const int m = c / N16, k0 = (c - m * N16) * 16;
        load_x8<XF32, VEC>(xin, m, ldx, K, k0, a[0], b2[0]);
        load_x8<XF32, VEC>(xin, m, ldx, K, k0 + 8, a[1], b2[1]);
        stage(c, a, b2);
    }
    __syncthreads();

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.0f;

    auto step = [&](auto refill_tag, int u, int i) {
        const bool valid = i < nmine;
        const int c = valid ? wave + NW * i : 0;
        const uint32_t wv[4] = {wbuf[u].x ^ 0x80808080u, wbuf[u].y ^ 0x80808080u,
                                wbuf[u].z ^ 0x80808080u, wbuf[u].w ^ 0x80808080u};
        if constexpr (decltype(refill_tag)::value) wbuf[u] = ldg_stream(wp + item_off(i + D));
        const int k0 = c * 64 + q * 16;
        float s = valid ? 1.0f : 0.0f;
        if (!PER_ROW) s = valid ? sc[(size_t)row * GPR + (k0 >> 5)] : 0.0f;
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float4* xp = (const float4*)(xl + (size_t)m * Kp + k0);
            float d = bias[(size_t)m * N16 + (k0 >> 4)];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 xv = xp[j];
                const uint32_t w = wv[j];
                d = __builtin_fmaf((float)(w & 0xFF), xv.x, d);
                d = __builtin_fmaf((float)((w >> 8) & 0xFF), xv.y, d);
                d = __builtin_fmaf((float)((w >> 16) & 0xFF), xv.z, d);
                d = __builtin_fmaf((float)(w >> 24), xv.w, d);
            }
            acc[m] = __builtin_fmaf(s, d, acc[m]);
        }
    };
    const int nbatch = (nmine + D - 1) / D;
    for (int bt = 0; bt + 1 < nbatch; bt++) {
#pragma unroll
        for (int u = 0; u < D; u++) step(std::true_type{}, u, bt * D + u);
    }
    if (nbatch > 0) {
#pragma unroll
        for (int u = 0; u < D; u++) step(std::false_type{}, u, (nbatch - 1) * D + u);
    }

#pragma unroll
    for (int m = 0; m < M; m++) {
        float v = wave_sum_xor16_32(acc[m]);
        if (q == 0) red[(wave * M + m) * 16 + r] = v;
    }
    __syncthreads();
    float* tilev = red + NW * 16 * M;  // [M][16]
    float v = 0.0f;
    if (tid < 16 * M) {
        const int m = tid >> 4, rr = tid & 15;
        v = red[(0 * M + m) * 16 + rr] + red[(1 * M + m) * 16 + rr];
#pragma unroll
        for (int w = 2; w < NW; w++) v += red[(w * M + m) * 16 + rr];
        const int n = t * 16 + rr;
        if (PER_ROW) v *= sc[n < N ? n : 0];
        tilev[m * 16 + rr] = v;
    }
    __syncthreads();
    if (tid < 16 * M) {
        const int m = tid >> 4, rr = tid & 15;
        const int n = t * 16 + rr;
        if (n < N) epi(m, n, v, tilev + m * 16, tilev + 4 * 16);
    }
}

// ---------------------------------------------------------------------------
// int4 GEMM on MFMA (v_mfma_f32_16x16x32_f16), for larger m.
// Workgroup: 4 waves stacked along n, each owning RT 16-row tiles; CB blocks
// of 16 activation rows.  Per group (K = 32 = one MFMA) a lane dequantises its
// eight weights to f16 as (n-8)*s' (exact n-8 via the 1024+n magic, one f16
// rounding of the product).  The activations come prepared (f16, permuted,
// see q4_gemm_xprep_kernel) and go through LDS.  With KS > 1 each workgroup
// covers a K slice and writes f32 partials [KS][m][n] that
// splitk_reduce_kernel sums in a fixed order.
//
// Range: f16 holds 2^-14..65504 at full precision, far less than the f32 /
// bf16 inputs of the reference's f64 q4_matvec (quantize.rs:256-289).  Both
// operands are therefore scaled by powers of two into f16's range and the
// result scaled back exactly: activation row m is stored as x * 2^-xexp[m]
// (its largest magnitude in [2^12, 2^13)), weight row n uses
// s' = s * 2^-wexp[n] (its largest scale in [2^8, 2^9), so |(q-8) s'| <=
// 2^12), and y[m][n] = ldexp(acc, xexp[m] + wexp[n]).  Values more than 2^26
// below their row's largest keep less than f16's 11 bits; their share of the
// sum is below f32 rounding of the large terms.
// ---------------------------------------------------------------------------

// out[k] = f16 pair (element k, element k+4) of the word, each (n-8)*scale.
// 0x6400|n is exactly 1024+n in f16; byte permutes splice the 0x64 high
// bytes onto the low / high nibbles of the four bytes (7 integer ops for the
// word instead of 11 with shifts, masks and ors per pair).
__device__ __forceinline__ void nib_pairs_f16(uint32_t w, half2_t s2, half2_t out[4]) {
    const half2_t off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const uint32_t lo = w & 0x0F0F0F0Fu;          // bytes: e0 e2 e4 e6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // bytes: e1 e3 e5 e7
    const uint32_t c64 = 0x64646464u;
    const uint32_t p[4] = {__builtin_amdgcn_perm(c64, lo, 0x04020400u), __builtin_amdgcn_perm(c64, hi, 0x04020400u),
                           __builtin_amdgcn_perm(c64, lo, 0x04030401u), __builtin_amdgcn_perm(c64, hi, 0x04030401u)};
#pragma unroll
    for (int k = 0; k < 4; k++) out[k] = (__builtin_bit_cast(half2_t, p[k]) + off) * s2;
}

__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
    half2_t h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
}

// Exponent that brings a row whose largest magnitude is mx to [2^(top-1),
// 2^top): mx * 2^-e lands there.  0 for an all-zero or non-finite row.
__host__ __device__ inline int range_exp(float mx, int top) {
    if (!(mx > 0.0f) || !(mx <= 3.402823466e38f)) return 0;
    int E;
    (void)frexpf(mx, &E);  // mx = f * 2^E, f in [0.5, 1)
    return E - top;
}
constexpr int XPREP_TOP = 13;  // prepared activations: row maximum in [2^12, 2^13)

// Largest magnitude over a 256-thread workgroup (every thread gets it).
__device__ __forceinline__ float block_absmax256(float v, float* red4) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
}
constexpr int WSCALE_TOP = 9;  // weight scales: row maximum in [2^8, 2^9)

// Sources of the MFMA GEMM: which weights a workgroup multiplies and which
// activation rows it takes.  Rows are local to the workgroup's block of
// CB*16 rows (0 <= m < mrows).
struct GemmDense {
    static constexpr bool GROUPED = false;
    int M;
    template <typename ST>
    __device__ __forceinline__ bool select(int by, int rows_per_block, const uint4*& wt, const ST*& sc,
                                           const int*& wexp, int& mrows) {
        m0 = by * rows_per_block;
        mrows = min(rows_per_block, M - m0);
        return true;
    }
    int m0 = 0;
    __device__ __forceinline__ int x_row(int m) const { return m0 + m; }
    __device__ __forceinline__ int out_row(int m) const { return m0 + m; }
};

// Epilogue of the MFMA GEMM: D fragment (weight rows n0..n0+3, activation
// row m) of one lane, already scaled back to the true result; `live` is false
// for rows past the block or the matrix.  Called by every lane (pairing
// epilogues shuffle).
struct EpiGemmStore {
    float* y;
    int ldy;
    size_t split_stride;  // split-K partials: y + split * split_stride
    int add = 0;          // y += v (a residual add, device.rs:721) instead of y = v
    int split = 0;        // this workgroup's K split (set by the kernel)
    __device__ __forceinline__ void operator()(int out_row, int n0, int N, bool live, const float4_t& v) const {
        if (!live) return;
        float* yb = y + (size_t)split * split_stride + (size_t)out_row * ldy;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (n0 + i < N) yb[n0 + i] = add ? yb[n0 + i] + v[i] : v[i];
    }
};

// Activations prepared for the MFMA GEMM: one wave per row.  Pass 1
// finds the row's largest magnitude, pass 2 writes x * 2^-xexp[row] as f16
// (RNE; exact for a bf16 input within 2^26 of the row maximum), each 8-value
// chunk in nibble-pair order (x0,x4,x1,x5,x2,x6,x3,x7), zero past K up to Kp.
// Row r of the output is input row rows[r] (rows == nullptr: row r).
template <bool XF32>
__device__ __forceinline__ void xprep_load8(const void* xin, size_t ldx, int row, int K, int k0, bool vec, float xv[8]) {
#pragma unroll
    for (int e = 0; e < 8; e++) xv[e] = 0.0f;
    if (XF32) {
        const float* xr = (const float*)xin + (size_t)row * ldx;
        if (vec && k0 + 8 <= K) {
            const float4 a = *(const float4*)(xr + k0), b = *(const float4*)(xr + k0 + 4);
            xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
            xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
        } else {
            for (int e = 0; e < 8; e++) if (k0 + e < K) xv[e] = xr[k0 + e];
        }
    } else {
        const uint16_t* xr = (const uint16_t*)xin + (size_t)row * ldx;
        if (vec && k0 + 8 <= K) {
            const uint4 a = *(const uint4*)(xr + k0);
            const uint32_t w4[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                xv[2 * e] = bf16_bits_to_f32(w4[e] & 0xFFFF);
                xv[2 * e + 1] = bf16_bits_to_f32(w4[e] >> 16);
            }
        } else {
            for (int e = 0; e < 8; e++) if (k0 + e < K) xv[e] = bf16_bits_to_f32(xr[k0 + e]);
        }
    }
}

template <bool XF32>
__global__ __launch_bounds__(256) void q4_gemm_xprep_kernel(const void* __restrict__ xin, int ldx, int K, int Kp,
                                                            int M, const int* __restrict__ rows,
                                                            uint4* __restrict__ out, int* __restrict__ xexp) {
    // one wave per row, four rows per workgroup
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= M) return;  // wave-uniform
    const int row = rows ? rows[r] : r;
    const int cpr = Kp >> 3;
    const bool vec = (ldx & 7) == 0 && (((uintptr_t)xin) & 15) == 0;
    float mx = 0.0f;
    for (int c = lane; c < cpr; c += 64) {
        float xv[8];
        xprep_load8<XF32>(xin, (size_t)ldx, row, K, c * 8, vec, xv);
#pragma unroll
        for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(xv[e]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const int e = range_exp(mx, XPREP_TOP);
    if (lane == 0) xexp[r] = e;
    for (int c = lane; c < cpr; c += 64) {  // second read: cache hits
        float xv[8];
        xprep_load8<XF32>(xin, (size_t)ldx, row, K, c * 8, vec, xv);
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = __builtin_amdgcn_ldexpf(xv[i], -e);
        out[(size_t)r * cpr + c] = make_uint4(pack_half2(xv[0], xv[4]), pack_half2(xv[1], xv[5]),
                                              pack_half2(xv[2], xv[6]), pack_half2(xv[3], xv[7]));
    }
}

// The same layout with one 256-thread workgroup per row and the row held in
// registers (U chunks of 8 per thread, Kp <= 2048 * U): one read of the row
// instead of two passes by one wave.  Identical output (the row maximum does
// not depend on the order).
template <bool XF32, int U>
__global__ __launch_bounds__(256) void q4_gemm_xprep_row_kernel(const void* __restrict__ xin, int ldx, int K, int Kp,
                                                                const int* __restrict__ rows, uint4* __restrict__ out,
                                                                int* __restrict__ xexp) {
    __shared__ float red4[4];
    const int r = blockIdx.x, t = threadIdx.x;
    const int row = rows ? rows[r] : r;
    const int cpr = Kp >> 3;
    const bool vec = (ldx & 7) == 0 && (((uintptr_t)xin) & 15) == 0;
    float xv[U][8];
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int c = t + 256 * u;
        if (c < cpr) {
            xprep_load8<XF32>(xin, (size_t)ldx, row, K, c * 8, vec, xv[u]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) xv[u][e] = 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(xv[u][e]));
    }
    const int e = range_exp(block_absmax256(mx, red4), XPREP_TOP);
    if (t == 0) xexp[r] = e;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int c = t + 256 * u;
        if (c >= cpr) continue;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = __builtin_amdgcn_ldexpf(xv[u][i], -e);
        out[(size_t)r * cpr + c] = make_uint4(pack_half2(v[0], v[4]), pack_half2(v[1], v[5]), pack_half2(v[2], v[6]),
                                              pack_half2(v[3], v[7]));
    }
}

// Workgroup -> (weight block, activation block, K split) of a dense GEMM
// grid.  Linear workgroup i runs on XCD i mod 8; this hands each XCD a
// contiguous range of tiles of the (x, y + gy * z) plane, walked in bands of
// 8 activation blocks, so the workgroups resident on one XCD share 8
// activation and 8 weight blocks in its L2.
__device__ __forceinline__ void gemm_xcd_tile(int& bx, int& by, int& bz) {
    const int gx = gridDim.x, gy = gridDim.y, gyz = gy * gridDim.z, W = gx * gyz;
    const int L = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const int k = L & 7;
    const int t = k * (W >> 3) + min(k, W & 7) + (L >> 3);
    constexpr int G = 8;
    const int band = t / (G * gx), rows = min(G, gyz - band * G);
    const int v = t - band * G * gx;
    bx = v / rows;
    const int yz = band * G + v % rows;
    bz = yz / gy;
    by = yz - bz * gy;
}

// xin: prepared rows (f16, ldx = Kp halves, row exponents xexp); wexp: the
// weight rows' scale exponents (th_qweight::row_exp).
template <int RT, int CB, typename ST, typename Src = GemmDense, typename Epi = EpiGemmStore>
__global__ __launch_bounds__(256) void q4_gemm_mfma_kernel(const uint4* __restrict__ wt,
                                                           const ST* __restrict__ sc, const int* __restrict__ wexp,
                                                           const uint16_t* __restrict__ xin,
                                                           const int* __restrict__ xexp, Epi epi, Src src,
                                                           int N, int K, int Kp, int ldx, int gq_per_split) {
    // LDS B tile: [CB][4 j][4 q][16 col] uint4 (8 f16 each)
    // two B tiles: the next group-quad's is written while this one is read,
    // so one barrier per step orders both
    __shared__ uint4 bt2[2][CB * 4 * 4 * 16];
    int mrows = 0, tile_blk = 0, split = blockIdx.z;
    {
        const uint4* wsel = wt;
        const ST* ssel = sc;
        const int* esel = wexp;
        int bx = blockIdx.x, by = blockIdx.y;
        if constexpr (!Src::GROUPED) gemm_xcd_tile(bx, by, split);
        tile_blk = bx;
        if (!src.select(by, CB * 16, wsel, ssel, esel, mrows)) return;
        wt = wsel;
        sc = ssel;
        wexp = esel;
    }
    const int GQ = Kp >> 7;
    // a scalar wave index pays off for the grouped (MoE) source and costs
    // the dense GEMM ~10% at M=2048 (measured), so only grouped launches use it
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = Src::GROUPED ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int tile0 = (tile_blk * 4 + wave) * RT;  // first 16-row tile of this wave
    const int NT = (N + 15) >> 4;
    const int gq0 = split * gq_per_split;
    if constexpr (std::is_same<Epi, EpiGemmStore>::value) epi.split = split;
    const int gq1 = min(GQ, gq0 + gq_per_split);

    float4_t acc[RT][CB];
#pragma unroll
    for (int a = 0; a < RT; a++)
#pragma unroll
        for (int b = 0; b < CB; b++) acc[a][b] = (float4_t){0.f, 0.f, 0.f, 0.f};
    // scale exponent of this lane's weight row (row r of each tile)
    int wneg[RT];
#pragma unroll
    for (int a = 0; a < RT; a++) wneg[a] = -wexp[min(tile0 + a, NT - 1) * 16 + r];

    const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(xin, 0x7FFFFFF0u);  // in-range offsets only
    // staging assignment: CB*16 cols * 16 chunks (4 groups x 4 quads) = CB*256 chunks.
    // A thread's chunks keep their row and their place in the group-quad
    // over the whole K loop: their offsets (for the grouped source, after the
    // slot -> token lookup) are formed once, so no step waits on that lookup.
    uint32_t xoff[CB];   // halves: row * ldx + j * 32 + qq * 8
    bool xlive[CB];
#pragma unroll
    for (int i = 0; i < CB; i++) {
        const int idx = tid + i * 256;  // chunk id
        const int col = idx & 15, qq = (idx >> 4) & 3, j = (idx >> 6) & 3, cb = idx >> 8;
        const int ml = cb * 16 + col;
        if constexpr (Src::GROUPED) {  // short work items: skip the loads of empty rows
            xlive[i] = ml < mrows;
            xoff[i] = (uint32_t)((xlive[i] ? src.x_row(ml) : 0) * ldx + j * 32 + qq * 8);
        } else {
            // branch-free: rows past mrows re-read the last live row (a finite
            // copy whose D columns are never stored)
            xlive[i] = true;
            xoff[i] = (uint32_t)(src.x_row(min(ml, mrows - 1)) * ldx + j * 32 + qq * 8);
        }
    }
    auto load_x = [&](int gq, uint4 (&regs)[CB]) {
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const uint32_t off = xoff[i] + (uint32_t)gq * 128u;
            if constexpr (Src::GROUPED) {
                regs[i] = xlive[i] ? *(const uint4*)(xin + off) : make_uint4(0, 0, 0, 0);
            } else {
                const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(xrs, off * 2u, 0, 0);
                regs[i] = make_uint4(v.x, v.y, v.z, v.w);
            }
        }
    };
    auto store_x = [&](uint4* bt, const uint4 (&regs)[CB]) {
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int idx = tid + i * 256;
            const int col = idx & 15, qq = (idx >> 4) & 3, j = (idx >> 6) & 3, cb = idx >> 8;
            bt[((cb * 4 + j) * 4 + qq) * 16 + col] = regs[i];
        }
    };

    uint4 xr[CB];
    uint4 wcur[RT], wnxt[RT];
    ScaleVec<RT, ST> scur, snxt;
    auto load_w = [&](int gq, uint4 (&w)[RT], ScaleVec<RT, ST>& s) {
#pragma unroll
        for (int a = 0; a < RT; a++) {
            int tt = min(tile0 + a, NT - 1);
            w[a] = ldg_stream(wt + ((size_t)tt * GQ + gq) * 64 + lane);
            s.load(sc + q4_scale_index(std::is_same<ST, _Float16>::value, tt, gq, r, 0, GQ), a);
        }
    };
    if (gq0 < gq1) {
        load_x(gq0, xr);
        load_w(gq0, wcur, scur);
        store_x(bt2[0], xr);
        __syncthreads();
    }
    for (int gq = gq0; gq < gq1; gq++) {
        const uint4* bt = bt2[(gq - gq0) & 1];
        const bool more = gq + 1 < gq1;
        if (more) {
            load_x(gq + 1, xr);
            load_w(gq + 1, wnxt, snxt);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            half8_t bfrag[CB];
#pragma unroll
            for (int b = 0; b < CB; b++)
                bfrag[b] = __builtin_bit_cast(half8_t, bt[((b * 4 + j) * 4 + q) * 16 + r]);
#pragma unroll
            for (int a = 0; a < RT; a++) {
                const uint32_t w = j == 0 ? wcur[a].x : j == 1 ? wcur[a].y : j == 2 ? wcur[a].z : wcur[a].w;
                const _Float16 s = scur.get_ldexp(a, j, wneg[a]);
                const half2_t s2 = {s, s};
                half2_t p[4];
                nib_pairs_f16(w, s2, p);
                half8_t afrag = {p[0].x, p[0].y, p[1].x, p[1].y, p[2].x, p[2].y, p[3].x, p[3].y};
#pragma unroll
                for (int b = 0; b < CB; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag, bfrag[b], acc[a][b], 0, 0, 0);
            }
        }
        // the other tile was last read in the previous step, before the
        // barrier that ended it
        if (more) store_x(bt2[(gq + 1 - gq0) & 1], xr);
        __syncthreads();
#pragma unroll
        for (int a = 0; a < RT; a++) wcur[a] = wnxt[a];
        scur = snxt;
    }

    // D layout: lane holds rows 4*(lane/16)+i (weight rows) of column lane%16.
    int xe[CB];
#pragma unroll
    for (int b = 0; b < CB; b++) {
        const int ml = b * 16 + r;
        xe[b] = xexp[src.x_row(ml < mrows ? ml : 0)];
    }
#pragma unroll
    for (int a = 0; a < RT; a++) {
        const int n0 = (tile0 + a) * 16 + 4 * q;
        const int4 we = *(const int4*)(wexp + min(tile0 + a, NT - 1) * 16 + 4 * q);
        const int wev[4] = {we.x, we.y, we.z, we.w};
#pragma unroll
        for (int b = 0; b < CB; b++) {
            const int ml = b * 16 + r;
            const bool live = ml < mrows && tile0 + a < NT;
            float4_t v;
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = __builtin_amdgcn_ldexpf(acc[a][b][i], xe[b] + wev[i]);
            epi(src.out_row(live ? ml : 0), n0, N, live, v);
        }
    }
}

}  // namespace th
