// Launchers and C entry points for the quantized linear kernels.
#include <cstdlib>
#include <map>
#include <mutex>

#include "aql.hpp"
#include "capi_util.hpp"
#include "qlinear.hpp"

namespace th {

// Raise a kernel's dynamic-LDS limit (once per kernel and size).
template <typename K>
static void set_smem(K kernel, size_t bytes) {
    static std::mutex mu;
    static std::map<const void*, size_t> done;
    if (bytes <= 48 * 1024) return;
    std::lock_guard<std::mutex> lock(mu);
    size_t& d = done[(const void*)kernel];
    if (bytes > d) {
        TH_HIP(hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
        d = bytes;
    }
}

// Vector activation loads need K, the row stride and the base 16-byte aligned.
static bool x_vec_ok(const void* x, size_t ldx, size_t K) {
    return K % 8 == 0 && ldx % 8 == 0 && ((uintptr_t)x & 15) == 0;
}

template <int M, bool XF32, typename ST, bool VEC, typename Src>
static void q4_gemv_launch_v(const th_qweight* w, const void* x, size_t ldx, float* y, size_t ldy, hipStream_t s,
                             Src src) {
    constexpr int MR = XF32 ? 2 * M : M;
    EpiStore epi{y, (int)ldy};
    if (M == 1 && w->Np / 16 < 512 && w->Kp / 128 >= 64) {  // few tiles, long K: sixteen waves per tile
        const size_t smem = Q4GemvSmem<MR, 16>::bytes((int)(w->Kp / 128));
        TH_REQUIRE(smem <= 160 * 1024, "activation too large for the LDS-staged GEMV");
        auto k = q4_gemv_kernel<MR, XF32, VEC, ST, EpiStore, 2, 4, 16, false, Src>;
        set_smem(k, smem);
        TH_LAUNCH(k, dim3((unsigned)(w->Np / 16)), dim3(1024), smem, s, (const uint4*)w->data,
                           (const ST*)w->scales, x, (int)w->cols, (int)w->Kp, (int)w->rows, (int)ldx, epi, NormArgs{}, src);
    } else if (MR >= 3 || w->Np / 16 < 512) {  // few tiles, or 3+ staged rows: split K over eight waves per tile
        const size_t smem = Q4GemvSmem<MR, 8>::bytes((int)(w->Kp / 128));
        TH_REQUIRE(smem <= 160 * 1024, "activation too large for the LDS-staged GEMV");
        auto k = q4_gemv_kernel<MR, XF32, VEC, ST, EpiStore, 2, 4, 8, false, Src>;
        set_smem(k, smem);
        TH_LAUNCH(k, dim3((unsigned)(w->Np / 16)), dim3(512), smem, s, (const uint4*)w->data,
                           (const ST*)w->scales, x, (int)w->cols, (int)w->Kp, (int)w->rows, (int)ldx, epi, NormArgs{}, src);
    } else {
        const size_t smem = Q4GemvSmem<MR, 4>::bytes((int)(w->Kp / 128));
        TH_REQUIRE(smem <= 160 * 1024, "activation too large for the LDS-staged GEMV");
        auto k = q4_gemv_kernel<MR, XF32, VEC, ST, EpiStore, 2, 4, 4, false, Src>;
        set_smem(k, smem);
        TH_LAUNCH(k, dim3((unsigned)(w->Np / 16)), dim3(256), smem, s, (const uint4*)w->data,
                           (const ST*)w->scales, x, (int)w->cols, (int)w->Kp, (int)w->rows, (int)ldx, epi, NormArgs{}, src);
    }
    TH_LAUNCH_CHECK();
}

template <int M, bool XF32, typename ST, typename Src = SingleMatrix>
static void q4_gemv_launch(const th_qweight* w, const void* x, size_t ldx, float* y, size_t ldy, hipStream_t s,
                           Src src = Src{}) {
    if (x_vec_ok(x, ldx, w->cols)) q4_gemv_launch_v<M, XF32, ST, true>(w, x, ldx, y, ldy, s, src);
    else q4_gemv_launch_v<M, XF32, ST, false>(w, x, ldx, y, ldy, s, src);
}

template <bool XF32, typename ST>
static void q4_gemv_dispatch(const th_qweight* w, const void* x, size_t m, size_t ldx, float* y,
                             size_t ldy, hipStream_t s) {
    switch (m) {
        case 1: q4_gemv_launch<1, XF32, ST>(w, x, ldx, y, ldy, s); break;
        case 2: q4_gemv_launch<2, XF32, ST>(w, x, ldx, y, ldy, s); break;
        default: throw Error(TH_ERR_INVALID, "q4 gemv: m out of range");
    }
}

// M block rows (4, 8 or 16; twice that staged after f32 hi/lo splitting), m
// of them live: NW waves split K, and each workgroup takes ceil(tiles / CUs)
// consecutive tiles so that the whole grid is resident at once and the
// staged activations are read once per workgroup.
template <int M, bool XF32, typename ST, bool VEC, bool RT>
static void q4_span_launch_v(const th_qweight* w, const void* x, size_t m, size_t ldx, float* y, size_t ldy,
                             hipStream_t s, int cus) {
    constexpr int MR = XF32 ? 2 * M : M;
    constexpr int NW = MR >= 16 ? 16 : 8, WPE = MR >= 16 ? 1 : 4;
    using Src = SingleMatrixSpan<RT>;
    const int tiles = (int)(w->Np / 16);
    Src src;
    src.tiles = tiles;
    src.per = (int)ceil_div((size_t)tiles, (size_t)cus);
    src.rows = (int)m;
    const unsigned grid = (unsigned)ceil_div((size_t)tiles, (size_t)src.per);
    const int GQ = (int)(w->Kp / 128);
    size_t smem = Q4GemvSmem<MR, NW>::bytes(GQ);
    auto k = q4_gemv_kernel<MR, XF32, VEC, ST, EpiStore, 2, WPE, NW, false, Src>;
    // two or three tiles per workgroup: streamed side by side (one reduction)
    if (src.per == 2) {
        k = q4_gemv_kernel<MR, XF32, VEC, ST, EpiStore, 2, WPE, NW, false, Src, 2>;
        smem = Q4GemvSmem<MR, NW, 2>::bytes(GQ);
    } else if (src.per == 3) {
        k = q4_gemv_kernel<MR, XF32, VEC, ST, EpiStore, 2, WPE, NW, false, Src, 3>;
        smem = Q4GemvSmem<MR, NW, 3>::bytes(GQ);
    }
    TH_REQUIRE(smem <= 160 * 1024, "activation too large for the LDS-staged GEMV");
    set_smem(k, smem);
    TH_LAUNCH(k, dim3(grid), dim3(64 * NW), smem, s, (const uint4*)w->data, (const ST*)w->scales, x,
                       (int)w->cols, (int)w->Kp, (int)w->rows, (int)ldx, EpiStore{y, (int)ldy}, NormArgs{}, src);
    TH_LAUNCH_CHECK();
}

template <int M, bool XF32, typename ST>
static void q4_span_launch(const th_qweight* w, const void* x, size_t m, size_t ldx, float* y, size_t ldy,
                           hipStream_t s, int cus) {
    const bool vec = x_vec_ok(x, ldx, w->cols);
    if (m == M) {  // all rows live: constant-folded staging
        if (vec) q4_span_launch_v<M, XF32, ST, true, false>(w, x, m, ldx, y, ldy, s, cus);
        else q4_span_launch_v<M, XF32, ST, false, false>(w, x, m, ldx, y, ldy, s, cus);
    } else {
        if (vec) q4_span_launch_v<M, XF32, ST, true, true>(w, x, m, ldx, y, ldy, s, cus);
        else q4_span_launch_v<M, XF32, ST, false, true>(w, x, m, ldx, y, ldy, s, cus);
    }
}

// Sum KS split-K partials [KS][m][N] in split order (then add it to y when
// add is set: the fused residual add).  VEC4: four consecutive columns per
// thread with 16-byte accesses (N and ldy multiples of 4); same sums.
template <bool VEC4>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, float* __restrict__ y,
                                                            int M, int N, int ldy, int KS, int add) {
    if (VEC4) {
        const int N4 = N >> 2;
        const int total = M * N4;
        for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
            const int m = i / N4, n = (i - m * N4) * 4;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            for (int s = 0; s < KS; s++) {
                const float4 p = *(const float4*)(part + ((size_t)s * M + m) * N + n);
                v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
            }
            float4* yp = (float4*)(y + (size_t)m * ldy + n);
            if (add) {
                const float4 o = *yp;
                v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
            }
            *yp = v;
        }
        return;
    }
    const size_t total = (size_t)M * N;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t m = i / N, n = i - m * N;
        float v = 0.0f;
        for (int s = 0; s < KS; s++) v += part[((size_t)s * M + m) * N + n];
        y[m * ldy + n] = add ? y[m * ldy + n] + v : v;
    }
}

// Convert m activation rows (f32 or bf16, rows of ldx) into the MFMA GEMM's
// prepared layout in the device's operand workspace.
size_t prepared_x_bytes(size_t m, size_t Kp) { return round_up(m * Kp * 2, 256) + round_up(m * sizeof(int), 256); }

PreparedX prepare_x(th_device* dev, const void* x, bool xf32, size_t m, size_t ldx, size_t K, size_t Kp,
                    hipStream_t s, const int* rows, void* workspace) {
    TH_REQUIRE(m * Kp * 2 < 0x7FFFFFF0u, "prepared activations above 2 GiB");  // 32-bit buffer offsets
    const size_t xbytes = round_up(m * Kp * 2, 256);
    char* ws = workspace ? (char*)workspace : (char*)device_scratch_x(dev, prepared_x_bytes(m, Kp));
    PreparedX p{(const uint16_t*)ws, (const int*)(ws + xbytes)};
    const size_t cpr = Kp / 8;
    if (cpr <= 8 * 256) {  // row per workgroup, in registers
        auto row_kernel = [&](auto xf, auto u) {
            constexpr bool XF = decltype(xf)::value;
            constexpr int UU = decltype(u)::value;
            TH_LAUNCH((q4_gemm_xprep_row_kernel<XF, UU>), dim3((unsigned)m), dim3(256), 0, s, x, (int)ldx, (int)K,
                      (int)Kp, rows, (uint4*)ws, (int*)(ws + xbytes));
        };
        auto by_u = [&](auto xf) {
            if (cpr <= 256) row_kernel(xf, std::integral_constant<int, 1>{});
            else if (cpr <= 512) row_kernel(xf, std::integral_constant<int, 2>{});
            else if (cpr <= 1024) row_kernel(xf, std::integral_constant<int, 4>{});
            else row_kernel(xf, std::integral_constant<int, 8>{});
        };
        if (xf32) by_u(std::true_type{});
        else by_u(std::false_type{});
        TH_LAUNCH_CHECK();
        return p;
    }
    const unsigned grid = (unsigned)ceil_div(m, (size_t)4);
    if (xf32)
        TH_LAUNCH((q4_gemm_xprep_kernel<true>), dim3(grid), dim3(256), 0, s, x, (int)ldx, (int)K, (int)Kp,
                           (int)m, rows, (uint4*)ws, (int*)(ws + xbytes));
    else
        TH_LAUNCH((q4_gemm_xprep_kernel<false>), dim3(grid), dim3(256), 0, s, x, (int)ldx, (int)K, (int)Kp,
                           (int)m, rows, (uint4*)ws, (int*)(ws + xbytes));
    TH_LAUNCH_CHECK();
    return p;
}

// A caller-provided workspace for the split-K partials (part_bytes of it);
// with none the device's grow-only workspace is used.
struct SplitWorkspace {
    float* part = nullptr;
    size_t part_bytes = 0;
};

template <int RT, int CB, typename ST>
static void q4_mfma_launch(const th_qweight* w, PreparedX xp, size_t m, float* y, size_t ldy, hipStream_t s,
                           th_device* dev, bool accumulate, SplitWorkspace sw) {
    const size_t NT = w->Np / 16, GQ = w->Kp / 128;
    const unsigned gx = (unsigned)ceil_div(NT, 4 * RT);
    const unsigned gy = (unsigned)ceil_div(m, 16 * CB);
    // Split K so that the grid covers the chip at least twice (and, with a
    // caller's workspace, only as far as its partials fit).
    const size_t target = 2 * (size_t)(dev ? dev->num_cus : 256);
    const size_t part_row = m * w->rows * sizeof(float);
    size_t ks = 1;
    while ((size_t)gx * gy * ks < target && ks * 2 <= GQ && ks < 16 &&
           (!sw.part || ks * 2 * part_row <= sw.part_bytes))
        ks *= 2;
    const int gps = (int)ceil_div(GQ, ks);
    ks = ceil_div(GQ, (size_t)gps);
    float* out = y;
    int ldo = (int)ldy;
    if (ks > 1) {
        out = sw.part ? sw.part : (float*)device_scratch(dev, ks * part_row);
        ldo = (int)w->rows;
    }
    GemmDense src;
    src.M = (int)m;
    EpiGemmStore epi{out, ldo, (size_t)m * (size_t)ldo, ks > 1 ? 0 : (int)accumulate};
    TH_LAUNCH((q4_gemm_mfma_kernel<RT, CB, ST, GemmDense, EpiGemmStore>), dim3(gx, gy, (unsigned)ks),
                       dim3(256), 0, s, (const uint4*)w->data, (const ST*)w->scales, (const int*)w->row_exp, xp.x,
                       xp.xexp, epi, src, (int)w->rows, (int)w->cols, (int)w->Kp, (int)w->Kp, gps);
    TH_LAUNCH_CHECK();
    if (ks > 1) {
        const size_t total = m * w->rows;
        const bool vec4 = w->rows % 4 == 0 && ldy % 4 == 0 && ((uintptr_t)y & 15) == 0 && total < (1u << 31);
        if (vec4)
            TH_LAUNCH(splitk_reduce_kernel<true>, dim3((unsigned)std::min<size_t>(ceil_div(total / 4, 256), 4096)),
                      dim3(256), 0, s, out, y, (int)m, (int)w->rows, (int)ldy, (int)ks, (int)accumulate);
        else
            TH_LAUNCH(splitk_reduce_kernel<false>, dim3((unsigned)std::min<size_t>(ceil_div(total, 256), 4096)),
                      dim3(256), 0, s, out, y, (int)m, (int)w->rows, (int)ldy, (int)ks, (int)accumulate);
        TH_LAUNCH_CHECK();
    }
}

// Tile shape by batch size: one 16-row block up to 16 rows; 64-row column
// blocks up to M=1024, 128-row blocks beyond (measured best of 2x4, 1x8, 2x6,
// 2x8, 4x4, 4x8).
template <typename ST>
static void q4_mfma_dispatch(const th_qweight* w, PreparedX xp, size_t m, float* y, size_t ldy, hipStream_t s,
                             th_device* dev, bool accumulate, SplitWorkspace sw = SplitWorkspace{}) {
    if (m <= 16) q4_mfma_launch<1, 1, ST>(w, xp, m, y, ldy, s, dev, accumulate, sw);
    else if (m <= 1024) q4_mfma_launch<2, 4, ST>(w, xp, m, y, ldy, s, dev, accumulate, sw);
    else q4_mfma_launch<2, 8, ST>(w, xp, m, y, ldy, s, dev, accumulate, sw);
}

// ws (optional, ws_bytes long): the caller's workspace for the MFMA path's
// prepared activations followed by its split-K partials.
template <bool XF32, typename ST>
static void q4_linear_t(const th_qweight* w, const void* x, size_t m, size_t ldx, float* y, size_t ldy,
                        hipStream_t s, th_device* dev, void* ws = nullptr, size_t ws_bytes = 0) {
    const int GQ = (int)(w->Kp / 128), cus = dev && dev->num_cus > 0 ? dev->num_cus : 256;
    // staged rows fit LDS (with the side-by-side tiles' extra, the largest case)
    const bool fits8 = Q4GemvSmem<8, 8, 3>::bytes(GQ) <= 160 * 1024;
    const bool fits16 = Q4GemvSmem<16, 16, 3>::bytes(GQ) <= 160 * 1024;
    const bool fits4 = Q4GemvSmem<XF32 ? 8 : 4, 8, 3>::bytes(GQ) <= 160 * 1024;
    // m <= 2: one tile per workgroup; 3..16: a 4-, 8- or 16-row block staged
    // once per workgroup over ceil(tiles / CUs) tiles (config 2, M=4: 8.3 ->
    // 7.6 us; M=1 is faster with one tile per workgroup, 6.7 against 7.0)
    if (m <= 2 && fits4) q4_gemv_dispatch<XF32, ST>(w, x, m, ldx, y, ldy, s);
    else if (m <= 4 && fits4) q4_span_launch<4, XF32, ST>(w, x, m, ldx, y, ldy, s, cus);
    else if (XF32 && m <= 8 && fits16) q4_span_launch<8, true, ST>(w, x, m, ldx, y, ldy, s, cus);
    else if (!XF32 && m <= 8 && fits8) q4_span_launch<8, false, ST>(w, x, m, ldx, y, ldy, s, cus);
    else if (!XF32 && m <= 16 && fits16) q4_span_launch<16, false, ST>(w, x, m, ldx, y, ldy, s, cus);
    else {  // activations prepared once per call, then the MFMA GEMM
        SplitWorkspace sw;
        void* xws = nullptr;
        if (ws) {
            const size_t xb = prepared_x_bytes(m, w->Kp);
            TH_REQUIRE(xb <= ws_bytes, "workspace too small for the prepared activations (m x K too large)");
            xws = ws;
            sw.part = (float*)((char*)ws + xb);
            sw.part_bytes = ws_bytes - xb;
        }
        const PreparedX xp = prepare_x(dev, x, XF32, m, ldx, w->cols, w->Kp, s, nullptr, xws);
        q4_mfma_dispatch<ST>(w, xp, m, y, ldy, s, dev, false, sw);
    }
}

void launch_q4_linear_prepared(const th_qweight* w, PreparedX xp, size_t m, float* y, size_t ldy, hipStream_t s,
                               th_device* dev, bool accumulate) {
    TH_REQUIRE(w && w->bits == 4, "not a q4 weight");
    if (m == 0) return;
    if (w->scale_dtype == TH_F16) q4_mfma_dispatch<_Float16>(w, xp, m, y, ldy, s, dev, accumulate);
    else q4_mfma_dispatch<float>(w, xp, m, y, ldy, s, dev, accumulate);
}

void launch_q4_linear(const th_qweight* w, const void* x, th_dtype xdt, size_t m, size_t ldx, float* y,
                      size_t ldy, hipStream_t s, th_device* dev, void* ws, size_t ws_bytes) {
    TH_REQUIRE(w && w->bits == 4, "not a q4 weight");
    TH_REQUIRE(xdt == TH_F32 || xdt == TH_BF16, "activations must be f32 or bf16");
    if (m == 0) return;
    const bool f32 = xdt == TH_F32;
    if (w->scale_dtype == TH_F16) {
        if (f32) q4_linear_t<true, _Float16>(w, x, m, ldx, y, ldy, s, dev, ws, ws_bytes);
        else q4_linear_t<false, _Float16>(w, x, m, ldx, y, ldy, s, dev, ws, ws_bytes);
    } else {
        if (f32) q4_linear_t<true, float>(w, x, m, ldx, y, ldy, s, dev, ws, ws_bytes);
        else q4_linear_t<false, float>(w, x, m, ldx, y, ldy, s, dev, ws, ws_bytes);
    }
}

template <int M, bool XF32, bool PR, bool VEC>
static void q8_launch_v(const th_qweight* w, const void* x, size_t ldx, float* y, size_t ldy, hipStream_t s) {
    // eight waves split each tile's K (config 1: 5.33 us; four waves 5.88,
    // sixteen 6.2-6.3; 2, 6 or 8 chunks in flight per wave instead of 4 were
    // slower)
    constexpr int NW = 8;
    const size_t smem = Q8GemvSmem<M, NW>::bytes((int)w->Kp);
    TH_REQUIRE(smem <= 160 * 1024, "activation too large for the LDS-staged GEMV");
    auto k = q8_gemv_kernel<M, XF32, VEC, PR, EpiStore, NW>;
    set_smem(k, smem);
    EpiStore epi{y, (int)ldy};
    TH_LAUNCH(k, dim3((unsigned)(w->Np / 16)), dim3(64 * NW), smem, s, (const uint4*)w->data,
                       (const float*)w->scales, x, (int)w->cols, (int)w->Kp, (int)w->rows, (int)ldx, epi);
    TH_LAUNCH_CHECK();
}

template <int M, bool XF32, bool PR>
static void q8_launch(const th_qweight* w, const void* x, size_t ldx, float* y, size_t ldy, hipStream_t s) {
    if (x_vec_ok(x, ldx, w->cols)) q8_launch_v<M, XF32, PR, true>(w, x, ldx, y, ldy, s);
    else q8_launch_v<M, XF32, PR, false>(w, x, ldx, y, ldy, s);
}

template <bool XF32, bool PR>
static void q8_dispatch(const th_qweight* w, const void* x, size_t m, size_t ldx, float* y, size_t ldy,
                        hipStream_t s) {
    // Process up to 4 activation rows per launch.
    for (size_t m0 = 0; m0 < m; m0 += 4) {
        const size_t mm = std::min<size_t>(4, m - m0);
        const void* xo = (const char*)x + m0 * ldx * (XF32 ? 4 : 2);
        float* yo = y + m0 * ldy;
        switch (mm) {
            case 1: q8_launch<1, XF32, PR>(w, xo, ldx, yo, ldy, s); break;
            case 2: q8_launch<2, XF32, PR>(w, xo, ldx, yo, ldy, s); break;
            case 3: q8_launch<3, XF32, PR>(w, xo, ldx, yo, ldy, s); break;
            default: q8_launch<4, XF32, PR>(w, xo, ldx, yo, ldy, s); break;
        }
    }
}

void launch_q8_linear(const th_qweight* w, const void* x, th_dtype xdt, size_t m, size_t ldx, float* y,
                      size_t ldy, hipStream_t s) {
    TH_REQUIRE(w && w->bits == 8, "not a q8 weight");
    TH_REQUIRE(xdt == TH_F32 || xdt == TH_BF16, "activations must be f32 or bf16");
    if (m == 0) return;
    if (xdt == TH_F32) {
        if (w->per_row) q8_dispatch<true, true>(w, x, m, ldx, y, ldy, s);
        else q8_dispatch<true, false>(w, x, m, ldx, y, ldy, s);
    } else {
        if (w->per_row) q8_dispatch<false, true>(w, x, m, ldx, y, ldy, s);
        else q8_dispatch<false, false>(w, x, m, ldx, y, ldy, s);
    }
}

}  // namespace th

using namespace th;

extern "C" {

int th_gemm_q4(th_device* dev, const th_buffer* x, size_t m, const th_qweight* w, th_buffer* y) {
    TH_API_BEGIN
    TH_REQUIRE(dev && x && w && y, "null argument");
    TH_REQUIRE(w->bits == 4, "weight is not q4");
    require_len_any(x, m * w->cols, "x");
    require_len(y, TH_F32, m * w->rows, "y");
    launch_q4_linear(w, x->ptr, x->dtype, m, w->cols, (float*)y->ptr, w->rows, dev->stream, dev);
    TH_API_END
}

int th_gemm_q4_noalloc(th_device* dev, const th_buffer* x, size_t m, const th_qweight* w, th_buffer* y) {
    TH_API_BEGIN
    TH_REQUIRE(dev && x && w && y, "null argument");
    TH_REQUIRE(w->bits == 4, "weight is not q4");
    TH_REQUIRE(dev->noalloc_scratch, "no workspace address for this device");
    require_len_any(x, m * w->cols, "x");
    require_len(y, TH_F32, m * w->rows, "y");
    launch_q4_linear(w, x->ptr, x->dtype, m, w->cols, (float*)y->ptr, w->rows, dev->stream, dev, dev->noalloc_scratch,
                     TH_NOALLOC_SCRATCH_BYTES);
    TH_API_END
}

int th_gemv_q8(th_device* dev, const th_buffer* x, size_t m, const th_qweight* w, th_buffer* y) {
    TH_API_BEGIN
    TH_REQUIRE(dev && x && w && y, "null argument");
    TH_REQUIRE(w->bits == 8, "weight is not q8");
    require_len_any(x, m * w->cols, "x");
    require_len(y, TH_F32, m * w->rows, "y");
    launch_q8_linear(w, x->ptr, x->dtype, m, w->cols, (float*)y->ptr, w->rows, dev->stream);
    TH_API_END
}

int th_bench_linear(th_device* dev, const th_buffer* x, size_t m, th_qweight* const* ws, size_t n_w, th_buffer* y,
                    size_t iters, int use_graph, float* ms) {
    TH_API_BEGIN
    TH_REQUIRE(dev && x && ws && n_w > 0 && y && ms, "null argument");
    const th_qweight* w0 = ws[0];
    for (size_t i = 0; i < n_w; i++)
        TH_REQUIRE(ws[i] && ws[i]->bits == w0->bits && ws[i]->rows == w0->rows && ws[i]->cols == w0->cols,
                   "weights must share one shape");
    require_len_any(x, m * w0->cols, "x");
    require_len(y, TH_F32, m * w0->rows, "y");
    auto call = [&](size_t i) {
        const th_qweight* w = ws[i % n_w];
        if (w->bits == 4) launch_q4_linear(w, x->ptr, x->dtype, m, w->cols, (float*)y->ptr, w->rows, dev->stream, dev);
        else launch_q8_linear(w, x->ptr, x->dtype, m, w->cols, (float*)y->ptr, w->rows, dev->stream);
    };
    call(0);  // sizes the workspace before any capture
    TH_HIP(hipStreamSynchronize(dev->stream));
    if (use_graph == 2) {
        // The GEMVs (q8, and q4 at m <= 16) store their output write-through:
        // no release fences between the launches.
        const bool wt = w0->bits == 8 || m <= 16;
        // Every call reads x and its weights and writes y: no call reads what
        // another writes (independent).
        // One sequence: whole passes over the copies (at least 240 launches,
        // so the timed launches run in the steady state of a busy queue and
        // every copy was last read n_w launches earlier), two clock stamps
        // back to back (the span of a stamp kernel and its dispatch), one
        // more pass, a clock stamp, the `iters` timed launches from copy 0,
        // a last stamp.  The time is the last interval less the stamps' own
        // span.  The sequence's system-scope acquire and release sit on its
        // first and last packets, outside both intervals.  It is replayed
        // twice; the second replay is timed.
        const size_t pre = ceil_div(std::max<size_t>(240, n_w), n_w) * n_w;
        AqlSeq* seq = aql_record(dev, wt, [&] {
            for (size_t i = 0; i < pre; i++) call(i);
            aql_stamp_launch(dev, 2);
            aql_stamp_launch(dev, 3);
            for (size_t i = 0; i < n_w; i++) call(i);
            aql_stamp_launch(dev, 0);
            for (size_t i = 0; i < iters; i++) call(i);
            aql_stamp_launch(dev, 1);
        }, true);
        try {
            aql_submit(*seq);  // warm replay
            aql_wait(dev);
            aql_submit(*seq);
            *ms = aql_stamped_ms(dev) - aql_stamp_span_ms(dev);
        } catch (...) {
            aql_free(seq);
            throw;
        }
        aql_free(seq);
    } else if (use_graph) {
        hipGraph_t g;
        hipGraphExec_t ge;
        TH_HIP(hipStreamBeginCapture(dev->stream, hipStreamCaptureModeThreadLocal));
        for (size_t i = 0; i < iters; i++) call(i);
        TH_HIP(hipStreamEndCapture(dev->stream, &g));
        TH_HIP(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        TH_HIP(hipGraphLaunch(ge, dev->stream));  // warm replay
        // then one stream-launched pass over the copies in cycle order, so
        // that the timed replay continues the cycle: every launch's weights
        // were last read n_w launches earlier (beyond the last-level cache
        // when n_w copies exceed it), whatever the number of launches
        for (size_t i = 0; i < n_w; i++) call(i);
        TH_HIP(hipEventRecord(dev->ev_start, dev->stream));
        TH_HIP(hipGraphLaunch(ge, dev->stream));
        TH_HIP(hipEventRecord(dev->ev_stop, dev->stream));
        TH_HIP(hipEventSynchronize(dev->ev_stop));
        TH_HIP(hipGraphExecDestroy(ge));
        TH_HIP(hipGraphDestroy(g));
    } else {
        for (size_t i = 0; i < n_w; i++) call(i);
        TH_HIP(hipEventRecord(dev->ev_start, dev->stream));
        for (size_t i = 0; i < iters; i++) call(i);
        TH_HIP(hipEventRecord(dev->ev_stop, dev->stream));
        TH_HIP(hipEventSynchronize(dev->ev_stop));
    }
    if (use_graph != 2) TH_HIP(hipEventElapsedTime(ms, dev->ev_start, dev->ev_stop));
    TH_API_END
}

}  // extern "C"
