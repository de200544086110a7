"""CPU oracle: ctypes binding of oracle/liboracle.so (oracle/tang_oracle.c).

TEST INFRASTRUCTURE ONLY -- the restatement of the reference's CPU
arithmetic that the HIP path is checked against.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q4_BLOCK = np.dtype([("scale", "<f4"), ("values", "u1", (16,))])
Q8_BLOCK = np.dtype([("scale", "<f4"), ("values", "i1", (32,))])

_P, _S, _I, _F, _D = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_double


class LlamaCfg(ctypes.Structure):
    _fields_ = [("n_layers", _I), ("d_model", _I), ("n_heads", _I), ("n_kv_heads", _I), ("head_dim", _I),
                ("d_ff", _I), ("vocab", _I), ("max_seq", _I), ("eps", _F)]


class Q4View(ctypes.Structure):
    _fields_ = [("nib", _P), ("scales", _P)]


class LlamaWeights(ctypes.Structure):
    _fields_ = [("embed", _P), ("attn_norm", _P), ("ffn_norm", _P), ("final_norm", _P),
                ("wq", _P), ("wk", _P), ("wv", _P), ("wo", _P), ("wg", _P), ("wu", _P), ("wd", _P),
                ("lm_head", Q4View), ("rope_cos", _P), ("rope_sin", _P)]


_SIG = {
    "or_f32_to_bf16": ([_F], ctypes.c_uint16),
    "or_bf16_to_f32": ([ctypes.c_uint16], _F),
    "or_f16_to_f32": ([ctypes.c_uint16], _F),
    "or_f32_to_f16": ([_F], ctypes.c_uint16),
    "or_f32_to_bf16_array": ([_P, _S, _P], None),
    "or_bf16_to_f32_array": ([_P, _S, _P], None),
    "or_f16_to_f32_array": ([_P, _S, _P], None),
    "or_f32_to_f16_array": ([_P, _S, _P], None),
    "or_quantize_q8": ([_P, _S, _P], _S),
    "or_dequantize_q8": ([_P, _S, _P], None),
    "or_quantize_q4": ([_P, _S, _P], _S),
    "or_dequantize_q4": ([_P, _S, _P], None),
    "or_quantize_matrix_q8": ([_P, _S, _S, _P], _S),
    "or_quantize_matrix_q4": ([_P, _S, _S, _P], _S),
    "or_q8_matvec": ([_P, _S, _S, _P, _P], None),
    "or_q4_matvec": ([_P, _S, _S, _P, _P], None),
    "or_q4_matvec_soa": ([_P, _P, _S, _S, _P, _P, _I], None),
    "or_q8_matvec_soa": ([_P, _P, _S, _S, _P, _P, _I], None),
    "or_rms_norm": ([_P, _P, _S, _S, _F, _P], None),
    "or_rms_norm_residual": ([_P, _P, _P, _S, _S, _F, _P, _P], None),
    "or_rope_tables": ([_S, _S, _D, _P, _P], None),
    "or_rope_forward": ([_P, _P, _P, _S, _S, _S, _S, _P], None),
    "or_kv_attention": ([_P, _P, _P, _S, _S, _S, _S, _S, _P, _I], None),
    "or_swiglu": ([_P, _P, _S, _P], None),
    "or_add": ([_P, _P, _S, _P], None),
    "or_embedding": ([_P, _P, _S, _S, _P], None),
    "or_softmax": ([_P, _S, _S, _P], None),
    "or_matmul": ([_P, _P, _S, _S, _S, _P], None),
    "or_transpose_2d": ([_P, _S, _S, _P], None),
    "or_reduce_sum": ([_P, _P, _S, _S, _P], None),
    "or_bias_add": ([_P, _P, _S, _S, _P], None),
    "or_argmax_f32": ([_P, _S], _S),
    "or_llama_decode_step": ([_P, _P, _P, _P, _I, _I, _P, _I], _I),
    "or_moe_forward": ([_P, _S, _S, _S, _S, _S, _S, _P, _P, _P, _P, _P, _P, _I], None),
    "or_sample": ([_P, _P, _P, _S, _P, _S], _S),
    "or_mla_decode": ([_P, _P, _P, _S, _S, _S, _S, _S, _S, _S, _P, _P, _P, _P, _D, _P, _I], None),
}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        for n, (a, r) in _SIG.items():
            f = getattr(L, n)
            f.argtypes = a
            f.restype = r
        _lib = L
    return _lib


def p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def f32_to_bf16(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_array(p(x), x.size, p(out))
    return out


def bf16_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_bf16_to_f32_array(p(h), h.size, p(out))
    return out


def f16_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_array(p(h), h.size, p(out))
    return out


def f32_to_f16(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_array(p(x), x.size, p(out))
    return out


def quantize_q4(data):
    data = np.ascontiguousarray(data, np.float32)
    out = np.zeros((data.size + 31) // 32, Q4_BLOCK)
    lib().or_quantize_q4(p(data), data.size, p(out))
    return out


def dequantize_q4(blocks):
    out = np.empty(blocks.size * 32, np.float32)
    lib().or_dequantize_q4(p(blocks), blocks.size, p(out))
    return out


def quantize_q8(data):
    data = np.ascontiguousarray(data, np.float32)
    out = np.zeros((data.size + 31) // 32, Q8_BLOCK)
    lib().or_quantize_q8(p(data), data.size, p(out))
    return out


def dequantize_q8(blocks):
    out = np.empty(blocks.size * 32, np.float32)
    lib().or_dequantize_q8(p(blocks), blocks.size, p(out))
    return out


def quantize_matrix_q4(data, rows, cols):
    data = np.ascontiguousarray(data, np.float32)
    out = np.zeros(rows * ((cols + 31) // 32), Q4_BLOCK)
    lib().or_quantize_matrix_q4(p(data), rows, cols, p(out))
    return out


def quantize_matrix_q8(data, rows, cols):
    data = np.ascontiguousarray(data, np.float32)
    out = np.zeros(rows * ((cols + 31) // 32), Q8_BLOCK)
    lib().or_quantize_matrix_q8(p(data), rows, cols, p(out))
    return out


def q4_matvec(blocks, rows, cols, x):
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty(rows, np.float64)
    lib().or_q4_matvec(p(np.ascontiguousarray(blocks)), rows, cols, p(x), p(y))
    return y


def q8_matvec(blocks, rows, cols, x):
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty(rows, np.float64)
    lib().or_q8_matvec(p(np.ascontiguousarray(blocks)), rows, cols, p(x), p(y))
    return y


def q4_matvec_soa(nib, scales_f32, rows, cols, x, threads=0):
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty(rows, np.float64)
    lib().or_q4_matvec_soa(p(np.ascontiguousarray(nib)), p(np.ascontiguousarray(scales_f32, np.float32)), rows,
                           cols, p(x), p(y), threads)
    return y


def q8_matvec_soa(q, scales_f32, rows, cols, x, threads=0):
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty(rows, np.float64)
    lib().or_q8_matvec_soa(p(np.ascontiguousarray(q, np.int8)), p(np.ascontiguousarray(scales_f32, np.float32)),
                           rows, cols, p(x), p(y), threads)
    return y


def rms_norm(x, w, groups, dim, eps):
    x = np.ascontiguousarray(x, np.float32); w = np.ascontiguousarray(w, np.float32)
    out = np.empty(groups * dim, np.float32)
    lib().or_rms_norm(p(x), p(w), groups, dim, eps, p(out))
    return out


def rms_norm_residual(inp, res, w, groups, dim, eps):
    a = np.ascontiguousarray(inp, np.float32); b = np.ascontiguousarray(res, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty(groups * dim, np.float32); s = np.empty(groups * dim, np.float32)
    lib().or_rms_norm_residual(p(a), p(b), p(w), groups, dim, eps, p(out), p(s))
    return out, s


def rope_tables(head_dim, max_seq, base):
    half = head_dim // 2
    c = np.empty(max_seq * half, np.float32); s = np.empty(max_seq * half, np.float32)
    lib().or_rope_tables(head_dim, max_seq, base, p(c), p(s))
    return c, s


def rope_forward(x, cos_t, sin_t, seq_len, n_heads, head_dim, start_pos):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().or_rope_forward(p(x), p(cos_t), p(sin_t), seq_len, n_heads, head_dim, start_pos, p(out))
    return out


def kv_attention(q, k, v, cache_start, q_len, n_heads, n_kv_heads, head_dim, threads=0):
    q = np.ascontiguousarray(q, np.float32); k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(q_len * n_heads * head_dim, np.float32)
    lib().or_kv_attention(p(q), p(k), p(v), cache_start, q_len, n_heads, n_kv_heads, head_dim, p(out), threads)
    return out


def swiglu(g, u):
    g = np.ascontiguousarray(g, np.float32); u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().or_swiglu(p(g), p(u), g.size, p(out))
    return out


def add(a, b):
    a = np.ascontiguousarray(a, np.float32); b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(a)
    lib().or_add(p(a), p(b), a.size, p(out))
    return out


def embedding(weight, ids, seq_len, dim):
    w = np.ascontiguousarray(weight, np.float32); i = np.ascontiguousarray(ids, np.uint32)
    out = np.empty(seq_len * dim, np.float32)
    lib().or_embedding(p(w), p(i), seq_len, dim, p(out))
    return out


def softmax(x, rows, length):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().or_softmax(p(x), rows, length, p(out))
    return out


def argmax(x):
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().or_argmax_f32(p(x), x.size))


def mla_decode(q_nope, q_rope, cache_bf16, B, H, L, dn, dr, r, dv, wuk, wuk_scale, wuv, wuv_scale, sm_scale,
               threads=0):
    """Absorbed MLA decode (f64 accumulation); out f32 [B][H][dv]."""
    q_nope = np.ascontiguousarray(q_nope, np.float32)
    q_rope = np.ascontiguousarray(q_rope, np.float32)
    cache_bf16 = np.ascontiguousarray(cache_bf16, np.uint16)
    wuk = np.ascontiguousarray(wuk, np.int8)
    wuv = np.ascontiguousarray(wuv, np.int8)
    wuk_scale = np.ascontiguousarray(wuk_scale, np.float32)
    wuv_scale = np.ascontiguousarray(wuv_scale, np.float32)
    out = np.empty(B * H * dv, np.float32)
    lib().or_mla_decode(p(q_nope), p(q_rope), p(cache_bf16), B, H, L, dn, dr, r, dv, p(wuk), p(wuk_scale), p(wuv),
                        p(wuv_scale), float(sm_scale), p(out), threads)
    return out


class SamplingCfg(ctypes.Structure):
    """or_sampling_cfg (sampling.rs:6-20); stop_token < 0 means None."""
    _fields_ = [("temperature", ctypes.c_double), ("top_p", ctypes.c_double),
                ("repetition_penalty", ctypes.c_double), ("top_k", ctypes.c_size_t),
                ("max_tokens", ctypes.c_size_t), ("stop_token", ctypes.c_int64)]


class OracleSampler:
    """Restated Sampler (sampling.rs:56-160): config, LCG state, sample()."""

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0, seed=42, stop_token=None,
                 max_tokens=256):
        self.cfg = SamplingCfg(temperature, top_p, repetition_penalty, top_k, max_tokens,
                               -1 if stop_token is None else stop_token)
        self.state = ctypes.c_uint64(seed)

    def sample(self, logits, past=()):
        lg = np.ascontiguousarray(logits, np.float32)
        pa = np.ascontiguousarray(past, np.int32)
        return int(lib().or_sample(ctypes.byref(self.cfg), ctypes.byref(self.state), p(lg), lg.size,
                                   p(pa) if pa.size else None, pa.size))


def matmul(a, b, m, k, n):
    """naive_matmul (cpu.rs:760): f32 sums in k order."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty(m * n, np.float32)
    lib().or_matmul(p(a), p(b), m, k, n, p(out))
    return out.reshape(m, n)


def transpose_2d(x, rows, cols):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(rows * cols, np.float32)
    lib().or_transpose_2d(p(x), rows, cols, p(out))
    return out


def reduce_sum(x, shape, axis):
    x = np.ascontiguousarray(x, np.float32)
    sh = np.ascontiguousarray(shape, np.uint64)
    n_out = int(np.prod([d for i, d in enumerate(shape) if i != axis], dtype=np.int64))
    out = np.empty(n_out, np.float32)
    lib().or_reduce_sum(p(x), p(sh), len(shape), axis, p(out))
    return out


def bias_add(m, bias, numel, dim):
    m = np.ascontiguousarray(m, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    out = np.empty(numel, np.float32)
    lib().or_bias_add(p(m), p(bias), numel, dim, p(out))
    return out


def expr_eval(nodes, output, inputs):
    """CpuDevice::elementwise (crates/tang-compute/src/cpu.rs:68-97) over a
    graph given as th_expr_node records: every input widened to f64, each
    live node evaluated in f64 as tang-expr's compiled closure does
    (crates/tang-expr/src/compile.rs:99-118; Select takes `a` when the
    condition is > 0, NaN included as false), the result rounded to f32.
    Numpy's f64 sin/arctan2/exp2/log2 stand for Rust's (the platform libm)."""
    ops = {0: "var", 1: "lit", 2: "add", 3: "mul", 4: "neg", 5: "recip", 6: "sqrt", 7: "sin", 8: "atan2",
           9: "exp2", 10: "log2", 11: "select"}
    xs = [np.asarray(v, np.float32).astype(np.float64) for v in inputs]
    vals = {}
    with np.errstate(all="ignore"):
        for i in range(output + 1):
            n = nodes[i]
            op, a, b, c = ops[int(n["op"])], int(n["a"]), int(n["b"]), int(n["c"])
            if op == "var":
                v = xs[a]
            elif op == "lit":
                v = np.float64(n["lit"])
            elif op == "add":
                v = vals[a] + vals[b]
            elif op == "mul":
                v = vals[a] * vals[b]
            elif op == "neg":
                v = -vals[a]
            elif op == "recip":
                v = 1.0 / vals[a]
            elif op == "sqrt":
                v = np.sqrt(vals[a])
            elif op == "sin":
                v = np.sin(vals[a])
            elif op == "atan2":
                v = np.arctan2(vals[a], vals[b])
            elif op == "exp2":
                v = np.exp2(vals[a])
            elif op == "log2":
                v = np.log2(vals[a])
            else:
                v = np.where(vals[a] > 0.0, vals[b], vals[c])
            vals[i] = v
    n = len(xs[0]) if xs else 1
    return np.broadcast_to(np.asarray(vals[output], np.float64), (n,)).astype(np.float32)
