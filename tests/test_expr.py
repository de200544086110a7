"""Element-wise kernels generated from tang-expr graphs (tang_amd/csrc/expr.cpp),
host side: the generated HIP source and the graph checks, and the oracle's
evaluator (oracle.expr_eval, a restatement of crates/tang-expr/src/compile.rs:99-118
under cpu.rs:68-97) pinned against closed-form numpy expressions."""
import re
import struct

import numpy as np
import pytest

import oracle
from tang_amd import capi


def graph_hypot_sel():
    g = capi.ExprGraph()
    x, y = g.var(0), g.var(1)
    h = g.sqrt(g.add(g.mul(x, x), g.mul(y, y)))
    return g, g.select(y, h, g.neg(g.recip(x)))


def test_builder_shares_identical_nodes_and_preloads_literals():
    g = capi.ExprGraph()
    assert [g.lit(0.0), g.lit(1.0), g.lit(2.0)] == [0, 1, 2]
    x = g.var(0)
    assert g.mul(x, x) == g.mul(x, x)
    assert g.lit(0.5) == g.lit(0.5) != g.lit(0.25)
    assert len(g.nodes) == 7


def test_source_is_the_live_graph_in_f64():
    g, out = graph_hypot_sel()
    g.sin(g.var(0))  # dead: not an input of the output
    src = g.source(out, 2)
    assert "sin(" not in src
    for op in ("sqrt(", " > 0.0 ? ", "1.0 / ", " * ", " + "):
        assert op in src, op
    assert "th_expr_v4" in src and "th_expr_s1" in src
    assert "const double x0, const double x1" in src
    assert "float4" in src


def test_literals_are_exact_bits():
    g = capi.ExprGraph()
    v = 0.1  # not representable in f32: must reach the kernel as the f64 bits
    out = g.mul(g.var(0), g.lit(v))
    src = g.source(out, 1)
    bits = struct.unpack("<Q", struct.pack("<d", v))[0]
    assert "0x%016xll" % bits in src


def test_graph_errors():
    g = capi.ExprGraph()
    out = g.add(g.var(0), g.var(1))
    with pytest.raises(capi.TangHipError, match="variable index"):
        g.source(out, 1)
    nodes = g.array()
    bad = nodes.copy()
    bad[out]["a"] = out  # operand does not precede its node
    n = capi.ctypes.c_size_t()
    with pytest.raises(capi.TangHipError, match="precede"):
        capi.check(capi.lib().th_expr_source(capi.ptr(bad), len(bad), out, 2, None, 0, capi.ctypes.byref(n)))
    bad = nodes.copy()
    bad[out]["op"] = 99
    with pytest.raises(capi.TangHipError, match="unknown"):
        capi.check(capi.lib().th_expr_source(capi.ptr(bad), len(bad), out, 2, None, 0, capi.ctypes.byref(n)))
    with pytest.raises(capi.TangHipError, match="output"):
        capi.check(capi.lib().th_expr_source(capi.ptr(nodes), len(nodes), len(nodes), 2, None, 0,
                                             capi.ctypes.byref(n)))


def test_oracle_eval_matches_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.uniform(0.1, 3.0, 1000).astype(np.float32)
    y = rng.standard_normal(1000).astype(np.float32)
    xd, yd = x.astype(np.float64), y.astype(np.float64)
    g, out = graph_hypot_sel()
    want = np.where(yd > 0, np.sqrt(xd * xd + yd * yd), -(1.0 / xd)).astype(np.float32)
    assert np.array_equal(oracle.expr_eval(g.array(), out, [x, y]), want)
    g = capi.ExprGraph()
    a, b = g.var(0), g.var(1)
    out = g.mul(g.add(g.exp2(b), g.atan2(b, a)), g.log2(a))
    want = ((np.exp2(yd) + np.arctan2(yd, xd)) * np.log2(xd)).astype(np.float32)
    assert np.array_equal(oracle.expr_eval(g.array(), out, [x, y]), want)
    # f64 evaluation, one rounding: x*y - x*y computed in f32 with a
    # subtraction of the f32 products would not cancel the same way
    g = capi.ExprGraph()
    a, b = g.var(0), g.var(1)
    out = g.add(g.mul(a, b), g.mul(g.lit(-1.0), g.mul(g.lit(1.0 / 3.0), a)))
    want = (xd * yd - (1.0 / 3.0) * xd).astype(np.float32)
    assert np.array_equal(oracle.expr_eval(g.array(), out, [x, y]), want)
