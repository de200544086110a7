"""Dense ComputeDevice operators on the device against the oracle
(crates/tang-compute/src/cpu.rs naive_matmul :760, transpose_2d :317,
reduce_sum :169, add_assign :650; device.rs bias_add :378) and the
run-time compiled element-wise kernels of ComputeDevice::elementwise
(device.rs:93) against numpy.

Bars: transpose, reduce_sum (same summation order), bias_add and
add_assign bit-exact; matmul within 1e-5 max-abs-rel of the oracle's f32
sums (f32 MFMA products, f32 accumulation in another order; the north-star
bar for f32 is 1e-3); element-wise kernels within 1e-6 max-abs-rel of
numpy's float32 evaluation (the device's sin/exp2/log2/atan2/sqrt differ
from numpy's in the last bits)."""
import numpy as np
import pytest

import oracle
from conftest import max_abs_rel
from tang_amd import capi

pytestmark = pytest.mark.gpu


def _bf16_round(x):
    return oracle.bf16_to_f32(oracle.f32_to_bf16(x))


@pytest.mark.parametrize("m,k,n", [(1, 2, 1), (2, 3, 2), (37, 100, 71), (64, 64, 64), (256, 1024, 384),
                                   (5, 4096, 11)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_matmul_variants(dev, m, k, n, ta, tb):
    print(f"matmul m={m} k={k} n={n} ta={ta} tb={tb}", flush=True)
    rng = np.random.default_rng(m * 7 + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    ref = oracle.matmul(a, b, m, k, n)
    da = dev.upload((a.T if ta else a).reshape(-1).copy())
    db = dev.upload((b.T if tb else b).reshape(-1).copy())
    c = dev.matmul(da, db, m, k, n, trans_a=ta, trans_b=tb).to_numpy().reshape(m, n)
    err = max_abs_rel(c, ref)
    print("max_abs_rel", err)
    assert err < 1e-5


def test_matmul_kats_and_accumulate(dev):
    """cpu.rs:785-822 known answers; matmul_accumulate (device.rs:391) adds."""
    c = dev.matmul(dev.upload(np.array([1, 0, 0, 1], np.float32)), dev.upload(np.array([1, 2, 3, 4], np.float32)),
                   2, 2, 2)
    assert c.to_numpy().tolist() == [1, 2, 3, 4]
    c = dev.matmul(dev.upload(np.array([1, 2, 3, 4, 5, 6], np.float32)),
                   dev.upload(np.array([7, 8, 9, 10, 11, 12], np.float32)), 2, 3, 2)
    assert c.to_numpy().tolist() == [58, 64, 139, 154]
    dev.matmul(dev.upload(np.array([1, 2, 3, 4, 5, 6], np.float32)),
               dev.upload(np.array([7, 8, 9, 10, 11, 12], np.float32)), 2, 3, 2, accumulate_into=c)
    assert c.to_numpy().tolist() == [116, 128, 278, 308]


def test_linear_forward_2d_bf16_weight(dev):
    """Linear::forward_2d (modules.rs:56) on the device: x . W^T with W
    [out][in] in bf16, then bias_add."""
    rng = np.random.default_rng(9)
    m, k, n = 48, 320, 200
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = _bf16_round(rng.standard_normal((n, k)).astype(np.float32) * 0.05)
    bias = rng.standard_normal(n).astype(np.float32)
    y = dev.matmul_b_transposed(dev.upload(x.reshape(-1)), dev.upload(oracle.f32_to_bf16(w).reshape(-1), capi.BF16),
                                m, k, n)
    y = dev.bias_add(y, dev.upload(bias), m * n, n).to_numpy().reshape(m, n)
    ref = oracle.bias_add(oracle.matmul(x, w.T.copy(), m, k, n), bias, m * n, n).reshape(m, n)
    assert max_abs_rel(y, ref) < 1e-5


@pytest.mark.parametrize("rows,cols", [(2, 3), (1, 1000), (33, 65), (1024, 700)])
def test_transpose_exact(dev, rows, cols):
    x = np.random.default_rng(rows).standard_normal(rows * cols).astype(np.float32)
    got = dev.transpose_2d(dev.upload(x), rows, cols).to_numpy()
    assert np.array_equal(got, oracle.transpose_2d(x, rows, cols))


@pytest.mark.parametrize("shape", [[2, 3], [7, 300, 5], [4096, 3], [3, 1, 9], [1000]])
def test_reduce_sum_bit_exact(dev, shape):
    x = np.random.default_rng(len(shape)).standard_normal(int(np.prod(shape))).astype(np.float32)
    dx = dev.upload(x)
    for axis in range(len(shape)):
        got = dev.reduce_sum(dx, shape, axis).to_numpy()
        assert np.array_equal(got, oracle.reduce_sum(x, shape, axis)), axis
    # reduce_sum_accumulate (device.rs:451): dst + reduce_sum
    acc = dev.upload(np.ones(int(np.prod(shape[1:])), np.float32))
    dev.reduce_sum(dx, shape, 0, accumulate_into=acc)
    assert np.array_equal(acc.to_numpy(), (np.float32(1) + oracle.reduce_sum(x, shape, 0)).astype(np.float32))


def test_bias_add_and_add_assign_exact(dev):
    rng = np.random.default_rng(5)
    m = rng.standard_normal(30 * 17).astype(np.float32)
    b = rng.standard_normal(17).astype(np.float32)
    got = dev.bias_add(dev.upload(m), dev.upload(b), m.size, 17).to_numpy()
    assert np.array_equal(got, oracle.bias_add(m, b, m.size, 17))
    a = dev.upload(np.array([1.0, 2.0, 3.0], np.float32))  # cpu.rs:1152-1158
    dev.add_assign(a, dev.upload(np.array([0.5, 1.0, 1.5], np.float32)))
    assert a.to_numpy().tolist() == [1.5, 3.0, 4.5]
    with pytest.raises(capi.TangHipError):
        dev.add_assign(a, dev.upload(np.zeros(4, np.float32)))


def _expr_kernel(n_inputs, body, result):
    """A kernel in the form tang-expr generates for ComputeDevice::elementwise:
    inputs in0.., output `outputs`, element count, one thread per element,
    inputs loaded as x<i>, SSA temporaries, one output."""
    params = "".join("const float* __restrict__ in%d,\n    " % i for i in range(n_inputs))
    loads = "".join("    float x%d = in%d[gid];\n" % (i, i) for i in range(n_inputs))
    return ('extern "C" __global__ void k0(' + params + "float* __restrict__ outputs,\n"
            "    const unsigned int count) {\n"
            "    unsigned int gid = blockIdx.x * blockDim.x + threadIdx.x;\n"
            "    if (gid >= count) { return; }\n\n" + loads + "\n" +
            "".join("    float %s;\n" % line for line in body) + "\n"
            "    outputs[gid * 1 + 0] = %s;\n}\n" % result)


def test_elementwise_runtime_kernels(dev):
    rng = np.random.default_rng(8)
    n = 100003
    x = rng.uniform(0.1, 3.0, n).astype(np.float32)
    y = rng.standard_normal(n).astype(np.float32)
    dx, dy = dev.upload(x), dev.upload(y)
    cases = [
        # (x*y) + sin(x)
        (2, ["t2 = (x0 * x1)", "t3 = sin(x0)", "t4 = (t2 + t3)"], "t4",
         lambda: (x * y + np.sin(x)).astype(np.float32)),
        # select(y, sqrt(x), -1/x), exp2, log2
        (2, ["t2 = sqrt(x0)", "t3 = (1.0f / x0)", "t4 = (-t3)", "t5 = (x1 > 0.0f ? t2 : t4)",
             "t6 = exp2(x1)", "t7 = log2(x0)", "t8 = (t5 + t6)", "t9 = (t8 * t7)"], "t9",
         lambda: ((np.where(y > 0, np.sqrt(x), -1 / x) + np.exp2(y)) * np.log2(x)).astype(np.float32)),
        # atan2(y, x) with one input only used twice
        (2, ["t2 = atan2(x1, x0)"], "t2", lambda: np.arctan2(y, x).astype(np.float32)),
    ]
    for n_in, body, res, ref in cases:
        k = dev.compile_kernel(_expr_kernel(n_in, body, res))
        try:
            got = dev.run_kernel(k, [dx, dy][:n_in], n).to_numpy()
        finally:
            capi.lib().th_kernel_free(k)
        want = ref()
        err = max_abs_rel(got, want)
        print(res, "max_abs_rel", err)
        assert err < 1e-6


def test_elementwise_compile_error_reported(dev):
    with pytest.raises(capi.TangHipError) as e:
        dev.compile_kernel('extern "C" __global__ void k0(float* outputs, const unsigned int count) { oops; }')
    assert "compile" in str(e.value)


def _graphs():
    """(n_inputs, builder, exact): graphs over x in [0.1, 3) and y ~ N(0, 1).
    exact: only +, *, neg, 1/x, sqrt, select and literals, whose f64 results
    are IEEE-determined, so the device must give the CPU backend's bits."""
    def hypot_sel(g, v):
        x, y = v
        return g.select(y, g.sqrt(g.add(g.mul(x, x), g.mul(y, y))), g.neg(g.recip(x)))

    def poly(g, v):
        x, y = v
        t = g.add(g.mul(g.lit(0.1), x), g.lit(-2.5))
        return g.add(g.mul(t, t), g.mul(g.lit(1.0 / 3.0), g.mul(x, y)))

    def sigmoid_ish(g, v):  # the reference's softplus/sigmoid shapes go through exp2 and recip
        x, y = v
        e = g.exp2(g.mul(g.lit(-1.4426950408889634), y))
        return g.mul(x, g.recip(g.add(g.lit(1.0), e)))

    def trig(g, v):
        x, y = v
        return g.add(g.mul(g.sin(x), g.atan2(y, x)), g.log2(x))

    def one_input(g, v):
        (x,) = v
        return g.mul(g.add(x, g.lit(1.0)), g.add(x, g.lit(1.0)))

    return [(2, hypot_sel, True), (2, poly, True), (2, sigmoid_ish, False), (2, trig, False), (1, one_input, True)]


@pytest.mark.parametrize("n", [1, 3, 4, 1027, 100003])
def test_elementwise_graph_matches_cpu_backend(dev, n):
    """ComputeDevice::elementwise from a tang-expr graph: bit-identical to the
    CPU backend's f64 evaluation (oracle.expr_eval) for the IEEE-exact ops;
    within one f32 rounding step for sin/atan2/exp2/log2 (device math
    library against the host's libm, both f64).  n covers the 4-wide tail."""
    import oracle
    rng = np.random.default_rng(n)
    x = rng.uniform(0.1, 3.0, n).astype(np.float32)
    y = rng.standard_normal(n).astype(np.float32)
    dx, dy = dev.upload(x), dev.upload(y)
    for n_in, build, exact in _graphs():
        print("expr", build.__name__, n, flush=True)
        got = dev.elementwise([dx, dy][:n_in], n, build).to_numpy()
        g = capi.ExprGraph()
        out = build(g, [g.var(i) for i in range(n_in)])
        want = oracle.expr_eval(g.array(), out, [x, y][:n_in])
        if exact:
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), build.__name__
        else:
            ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
            assert ulp.max() <= 1, (build.__name__, ulp.max())


def test_elementwise_graph_cache_and_special_values(dev):
    """The same graph twice (second call from the device's compiled cache),
    and IEEE special values: 1/0 = inf, sqrt(-1) = NaN, select on NaN takes
    the else branch, as the CPU backend's closure does."""
    x = np.array([0.0, -1.0, np.nan, 4.0, -0.0], np.float32)
    dx = dev.upload(x)
    build = lambda g, v: g.add(g.recip(v[0]), g.select(v[0], g.sqrt(v[0]), g.lit(7.0)))
    a = dev.elementwise([dx], len(x), build).to_numpy()
    b = dev.elementwise([dx], len(x), build).to_numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.isposinf(a[0]) and a[1] == 6.0 and np.isnan(a[2]) and a[3] == 2.25 and np.isneginf(a[4])
