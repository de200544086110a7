"""ctypes binding of the C ABI in include/tang_hip.h.

`HipComputeDevice` mirrors the method names and argument meaning of
`tang_compute::ComputeDevice` (crates/tang-compute/src/device.rs:19-869) for
the decode-path ops, plus the quantized extensions.  Errors raise
`TangHipError` carrying the C status code and th_last_error() text (the
reference panics instead).

The shared library must have been built (tang_amd/build.py); importing this
module without it raises, so no caller can silently fall back to CPU code.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtang_hip.so")

TH_OK, TH_ERR_INVALID, TH_ERR_HIP, TH_ERR_OOM, TH_ERR_UNSUPPORTED = 0, 1, 2, 3, 4
F32, BF16, F16, U8, I8, U32, I32 = range(7)

_NP = {F32: np.float32, BF16: np.uint16, F16: np.uint16, U8: np.uint8, I8: np.int8, U32: np.uint32, I32: np.int32}

Q4_BLOCK = np.dtype([("scale", "<f4"), ("values", "u1", (16,))])
Q8_BLOCK = np.dtype([("scale", "<f4"), ("values", "i1", (32,))])


class TangHipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("tang_hip error %d: %s" % (code, msg))
        self.code = code


class LlamaConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_int), ("d_model", ctypes.c_int), ("n_heads", ctypes.c_int),
        ("n_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("d_ff", ctypes.c_int),
        ("vocab", ctypes.c_int), ("max_seq", ctypes.c_int), ("eps", ctypes.c_float),
        ("rope_theta", ctypes.c_double),
    ]


# Every entry point declared in include/tang_hip.h, with its argument types.
_P, _S, _U64, _I, _F, _D = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int, ctypes.c_float, ctypes.c_double
SIGNATURES = {
    "th_last_error": ([], ctypes.c_char_p),
    "th_device_count": ([_P], _I),
    "th_device_create": ([_I, _P], _I),
    "th_device_destroy": ([_P], _I),
    "th_sync": ([_P], _I),
    "th_memory_info": ([_P, _P, _P], _I),
    "th_timer_start": ([_P], _I),
    "th_timer_stop": ([_P, _P], _I),
    "th_capture_begin": ([_P], _I),
    "th_capture_end": ([_P, _P], _I),
    "th_graph_launch": ([_P], _I),
    "th_graph_destroy": ([_P], _I),
    "th_buffer_alloc": ([_P, _I, _S, _P], _I),
    "th_buffer_free": ([_P], _I),
    "th_buffer_upload": ([_P, _P, _S], _I),
    "th_buffer_download": ([_P, _P, _S], _I),
    "th_buffer_info": ([_P, _P, _P], _I),
    "th_buffer_zero": ([_P], _I),
    "th_buffer_copy": ([_P, _P], _I),
    "th_buffer_copy_region": ([_P, _S, _P, _S, _S], _I),
    "th_convert": ([_P, _P, _P], _I),
    "th_q4_upload_blocks": ([_P, _P, _S, _S, _I, _P], _I),
    "th_q4_upload_packed": ([_P, _P, _P, _I, _S, _S, _P], _I),
    "th_q8_upload_blocks": ([_P, _P, _S, _S, _P], _I),
    "th_q8_upload_rowwise": ([_P, _P, _P, _S, _S, _P], _I),
    "th_q4_download_blocks": ([_P, _P], _I),
    "th_qweight_info": ([_P, _P, _P, _P], _I),
    "th_qweight_free": ([_P], _I),
    "th_gemm_q4": ([_P, _P, _S, _P, _P], _I),
    "th_gemv_q8": ([_P, _P, _S, _P, _P], _I),
    "th_gemm_q4_noalloc": ([_P, _P, _S, _P, _P], _I),
    "th_bench_linear": ([_P, _P, _S, _P, _S, _P, _S, _I, _P], _I),
    "th_rms_norm": ([_P, _P, _P, _S, _S, _F, _P], _I),
    "th_rms_norm_residual": ([_P, _P, _P, _P, _S, _S, _F, _P, _P], _I),
    "th_rope_tables": ([_S, _S, _D, _P, _P], _I),
    "th_rope_forward": ([_P, _P, _P, _P, _S, _S, _S, _S, _P], _I),
    "th_kv_attention": ([_P, _P, _P, _P, _S, _S, _S, _S, _S, _P], _I),
    "th_swiglu": ([_P, _P, _P, _S, _P], _I),
    "th_swiglu_bf16": ([_P, _P, _P, _S, _P], _I),
    "th_add": ([_P, _P, _P, _S, _P], _I),
    "th_embedding": ([_P, _P, _P, _S, _S, _P], _I),
    "th_softmax": ([_P, _P, _S, _S, _P], _I),
    "th_argmax": ([_P, _P, _S, _S, _P], _I),
    "th_llama_create": ([_P, _P, _P], _I),
    "th_llama_destroy": ([_P], _I),
    "th_llama_init_synthetic": ([_P, _U64], _I),
    "th_llama_load_safetensors": ([_P, _P], _I),
    "th_llama_fill_kv_synthetic": ([_P, _S, _U64], _I),
    "th_llama_generate": ([_P, ctypes.c_int32, _S, _S, _P, _P], _I),
    "th_llama_step_device": ([_P, _S], _I),
    "th_llama_set_token": ([_P, ctypes.c_int32], _I),
    "th_llama_time_steps": ([_P, ctypes.c_int32, _S, _S, _P], _I),
    "th_moe_create": ([_P, _S, _S, _S, _S, _S, _P], _I),
    "th_moe_destroy": ([_P], _I),
    "th_moe_init_synthetic": ([_P, _U64], _I),
    "th_moe_forward": ([_P, _P, _S, _P, _P, _P], _I),
    "th_sampler_create": ([_P, _U64, _P], _I),
    "th_sampler_destroy": ([_P], _I),
    "th_sampler_sample": ([_P, _P, _S, _P, _S, _P], _I),
    "th_llama_generate_sampled": ([_P, _P, _P, _S, _S, _P, _P], _I),
    "th_llama_prefill": ([_P, _P, _S, _S, _P, _P], _I),
    "th_llama_time_prefill": ([_P, _P, _S, _S, _P], _I),
    "th_quantize_q4": ([_P, _S, _S, _P], _I),
    "th_quantize_q8": ([_P, _S, _S, _P], _I),
    "th_st_open": ([ctypes.c_char_p, _P], _I),
    "th_st_close": ([_P], _I),
    "th_st_count": ([_P, _P], _I),
    "th_st_info": ([_P, _S, _P, _P, _P, _P, _S], _I),
    "th_st_read_f32": ([_P, ctypes.c_char_p, _P, _S], _I),
    "th_st_upload": ([_P, _P, ctypes.c_char_p, _I, _P], _I),
    "th_st_upload_q4": ([_P, _P, ctypes.c_char_p, _P], _I),
    "th_st_upload_q8": ([_P, _P, ctypes.c_char_p, _P], _I),
    "th_mla_decode": ([_P, _P, _P, _P, _S, _S, _S, _S, _S, _S, _S, _P, _P, _F, _P], _I),
    "th_matmul_ex": ([_P, _P, _P, _S, _S, _S, _I, _I, _I, _P], _I),
    "th_matmul": ([_P, _P, _P, _S, _S, _S, _P], _I),
    "th_matmul_b_transposed": ([_P, _P, _P, _S, _S, _S, _P], _I),
    "th_transpose_2d": ([_P, _P, _S, _S, _P], _I),
    "th_reduce_sum": ([_P, _P, _P, _S, _S, _I, _P], _I),
    "th_bias_add": ([_P, _P, _P, _S, _S, _P], _I),
    "th_add_assign": ([_P, _P, _P], _I),
    "th_expr_source": ([_P, _S, ctypes.c_uint32, _S, _P, _S, _P], _I),
    "th_elementwise_expr": ([_P, _P, _S, ctypes.c_uint32, _P, _S, _S, _P], _I),
    "th_kernel_compile": ([_P, ctypes.c_char_p, ctypes.c_char_p, _P], _I),
    "th_kernel_free": ([_P], _I),
    "th_elementwise": ([_P, _P, _S, _S, _P], _I),
    "th_synth_seed": ([_U64, _U64, _U64], _U64),
    "th_synth_q4": ([_U64, _S, _S, _F, _F, _P, _P], _I),
    "th_synth_q8_rowwise": ([_U64, _S, _S, _F, _F, _P, _P], _I),
    "th_synth_normal": ([_U64, _S, _F, _I, _P], _I),
}

_lib = None

# th_expr_node (include/tang_hip.h): op, three operand indices, a literal.
EXPR_NODE = np.dtype([("op", "<u4"), ("a", "<u4"), ("b", "<u4"), ("c", "<u4"), ("lit", "<f8")], align=True)
(EXPR_VAR, EXPR_LIT, EXPR_ADD, EXPR_MUL, EXPR_NEG, EXPR_RECIP, EXPR_SQRT, EXPR_SIN, EXPR_ATAN2, EXPR_EXP2, EXPR_LOG2,
 EXPR_SELECT) = range(12)


class ExprGraph:
    """A tang-expr expression graph (crates/tang-expr/src/graph.rs:12-143) in
    the form th_elementwise_expr takes: nodes in creation order, identical
    nodes shared (hash-consed), the literals 0, 1 and 2 at indices 0-2.  The
    builder methods return node indices."""

    def __init__(self):
        self.nodes = []
        self._index = {}
        for v in (0.0, 1.0, 2.0):
            self.lit(v)

    def _node(self, op, a=0, b=0, c=0, lit=0.0):
        key = (op, a, b, c, np.float64(lit).tobytes())
        if key not in self._index:
            self._index[key] = len(self.nodes)
            self.nodes.append((op, a, b, c, lit))
        return self._index[key]

    def var(self, i):
        return self._node(EXPR_VAR, i)

    def lit(self, v):
        return self._node(EXPR_LIT, lit=float(v))

    def add(self, a, b):
        return self._node(EXPR_ADD, a, b)

    def mul(self, a, b):
        return self._node(EXPR_MUL, a, b)

    def neg(self, a):
        return self._node(EXPR_NEG, a)

    def recip(self, a):
        return self._node(EXPR_RECIP, a)

    def sqrt(self, a):
        return self._node(EXPR_SQRT, a)

    def sin(self, a):
        return self._node(EXPR_SIN, a)

    def atan2(self, y, x):
        return self._node(EXPR_ATAN2, y, x)

    def exp2(self, a):
        return self._node(EXPR_EXP2, a)

    def log2(self, a):
        return self._node(EXPR_LOG2, a)

    def select(self, cond, a, b):
        return self._node(EXPR_SELECT, cond, a, b)

    def array(self):
        return np.array(self.nodes, EXPR_NODE)

    def source(self, output, n_inputs):
        """The HIP source th_elementwise_expr generates for this graph."""
        nodes = self.array()
        n = ctypes.c_size_t()
        check(lib().th_expr_source(ptr(nodes), len(nodes), output, n_inputs, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value + 1)
        check(lib().th_expr_source(ptr(nodes), len(nodes), output, n_inputs, buf, n.value + 1, ctypes.byref(n)))
        return buf.value.decode()


def lib():
    """Load libtang_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError("tang_amd: %s is missing; run __graft_entry__.build() first" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def check(rc):
    if rc != TH_OK:
        raise TangHipError(rc, lib().th_last_error().decode())


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def device_count():
    n = ctypes.c_int(0)
    check(lib().th_device_count(ctypes.byref(n)))
    return n.value


# --------------------------------------------------------------------------
# host-side generators (product code: the seeded synthetic data of benches)
# --------------------------------------------------------------------------

def synth_seed(base, layer, tensor):
    return lib().th_synth_seed(base, layer, tensor)


def synth_q4(seed, rows, cols, smin=0.002, smax=0.01):
    """Packed nibbles [rows][ceil(cols/32)*16] u8 and f16 scales (as u16) [rows][ceil(cols/32)]."""
    bpr = (cols + 31) // 32
    nib = np.empty((rows, bpr * 16), np.uint8)
    sc = np.empty((rows, bpr), np.uint16)
    check(lib().th_synth_q4(seed, rows, cols, smin, smax, ptr(nib), ptr(sc)))
    return nib, sc


def synth_q8_rowwise(seed, rows, cols, smin=0.005, smax=0.02):
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    check(lib().th_synth_q8_rowwise(seed, rows, cols, smin, smax, ptr(q), ptr(s)))
    return q, s


def synth_normal(seed, n, std=1.0, dtype=F32):
    out = np.empty(n, _NP[dtype])
    check(lib().th_synth_normal(seed, n, std, dtype, ptr(out)))
    return out


def rope_tables(head_dim, max_seq, base):
    half = head_dim // 2
    c = np.empty(max_seq * half, np.float32)
    s = np.empty(max_seq * half, np.float32)
    check(lib().th_rope_tables(head_dim, max_seq, base, ptr(c), ptr(s)))
    return c, s


# --------------------------------------------------------------------------
# device objects
# --------------------------------------------------------------------------

class Buffer:
    def __init__(self, dev, dtype, n, handle=None):
        """Allocate n elements of dtype, or adopt a buffer handle the library
        returned (which this object then frees)."""
        self.dev, self.dtype, self.n = dev, dtype, int(n)
        if handle is None:
            handle = ctypes.c_void_p()
            check(lib().th_buffer_alloc(dev.handle, dtype, self.n, ctypes.byref(handle)))
        self.handle = handle

    def __len__(self):
        return self.n

    def upload(self, arr):
        a = np.ascontiguousarray(arr, dtype=_NP[self.dtype]).reshape(-1)
        check(lib().th_buffer_upload(self.handle, ptr(a), a.size))

    def to_numpy(self, n=None):
        n = self.n if n is None else n
        out = np.empty(n, _NP[self.dtype])
        check(lib().th_buffer_download(self.handle, ptr(out), n))
        return out

    def free(self):
        if self.handle:
            check(lib().th_buffer_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.th_buffer_free(self.handle)
        except Exception:
            pass


class QWeight:
    def __init__(self, handle, rows, cols, bits):
        self.handle, self.rows, self.cols, self.bits = handle, rows, cols, bits

    def download_q4_blocks(self):
        bpr = (self.cols + 31) // 32
        out = np.zeros(self.rows * bpr, Q4_BLOCK)
        check(lib().th_q4_download_blocks(self.handle, ptr(out)))
        return out

    def free(self):
        if self.handle:
            check(lib().th_qweight_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.th_qweight_free(self.handle)
        except Exception:
            pass


ST_DTYPES = {0: "F64", 1: "F32", 2: "F16", 3: "BF16"}


def quantize_q4(data, rows, cols):
    """quantize_matrix_q4 (quantize.rs:208) -> Q4_BLOCK records."""
    a = np.ascontiguousarray(data, np.float32)
    out = np.empty(rows * ((cols + 31) // 32), Q4_BLOCK)
    check(lib().th_quantize_q4(ptr(a), rows, cols, ptr(out)))
    return out


def quantize_q8(data, rows, cols):
    """quantize_matrix_q8 (quantize.rs:193) -> Q8_BLOCK records."""
    a = np.ascontiguousarray(data, np.float32)
    out = np.empty(rows * ((cols + 31) // 32), Q8_BLOCK)
    check(lib().th_quantize_q8(ptr(a), rows, cols, ptr(out)))
    return out


class SafetensorsFile:
    """th_st_* over one file: names, dtypes and shapes, f32 reads, uploads."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(lib().th_st_open(str(path).encode(), ctypes.byref(h)))
        self.handle = h

    def tensors(self):
        n = ctypes.c_size_t()
        check(lib().th_st_count(self.handle, ctypes.byref(n)))
        out = {}
        for i in range(n.value):
            name, dt, nd = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_size_t()
            shape = (ctypes.c_size_t * 16)()
            check(lib().th_st_info(self.handle, i, ctypes.byref(name), ctypes.byref(dt), ctypes.byref(nd), shape, 16))
            out[name.value.decode()] = (ST_DTYPES[dt.value], tuple(shape[j] for j in range(nd.value)))
        return out

    def read_f32(self, name, n):
        out = np.empty(n, np.float32)
        check(lib().th_st_read_f32(self.handle, name.encode(), ptr(out), n))
        return out

    def upload(self, dev, name, dtype=F32):
        h = ctypes.c_void_p()
        check(lib().th_st_upload(dev.handle, self.handle, name.encode(), dtype, ctypes.byref(h)))
        return Buffer(dev, dtype, int(np.prod(self.tensors()[name][1], dtype=np.int64)), handle=h)

    def upload_q4(self, dev, name):
        h = ctypes.c_void_p()
        check(lib().th_st_upload_q4(dev.handle, self.handle, name.encode(), ctypes.byref(h)))
        rows, cols = self.tensors()[name][1]
        return QWeight(h, rows, cols, 4)

    def close(self):
        if self.handle:
            lib().th_st_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SamplingConfig(ctypes.Structure):
    """th_sampling_config = SamplingConfig (sampling.rs:6-20); stop_token < 0: None."""
    _fields_ = [("temperature", ctypes.c_double), ("top_k", ctypes.c_size_t), ("top_p", ctypes.c_double),
                ("repetition_penalty", ctypes.c_double), ("stop_token", ctypes.c_int64),
                ("max_tokens", ctypes.c_size_t)]

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0, stop_token=None,
                 max_tokens=256):
        super().__init__(temperature, top_k, top_p, repetition_penalty, -1 if stop_token is None else stop_token,
                         max_tokens)


class Sampler:
    """Sampler::with_seed + Sampler::sample (sampling.rs:67-160) through the C ABI."""

    def __init__(self, cfg, seed=42):
        self.cfg = cfg
        h = ctypes.c_void_p()
        check(lib().th_sampler_create(ctypes.byref(cfg), seed, ctypes.byref(h)))
        self.handle = h

    def sample(self, logits, past=()):
        lg = np.ascontiguousarray(logits, np.float32)
        pa = np.ascontiguousarray(past, np.int32)
        tok = ctypes.c_int32()
        check(lib().th_sampler_sample(self.handle, ptr(lg), lg.size, ptr(pa) if pa.size else None, pa.size,
                                      ctypes.byref(tok)))
        return tok.value

    def close(self):
        if self.handle:
            lib().th_sampler_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Graph:
    """A captured sequence of library calls, replayed with launch()."""

    def __init__(self, handle):
        self.handle = handle

    def launch(self):
        check(lib().th_graph_launch(self.handle))

    def free(self):
        if self.handle:
            lib().th_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipComputeDevice:
    """One device handle (one HIP stream), methods named as ComputeDevice's."""

    def __init__(self, ordinal=0):
        h = ctypes.c_void_p()
        check(lib().th_device_create(ordinal, ctypes.byref(h)))
        self.handle = h

    # -- buffer lifecycle (device.rs:44-80)
    def upload(self, data, dtype=F32):
        a = np.ascontiguousarray(data, dtype=_NP[dtype]).reshape(-1)
        b = Buffer(self, dtype, a.size)
        b.upload(a)
        return b

    def upload_u32(self, data):
        return self.upload(data, U32)

    def alloc(self, n, dtype=F32):
        return Buffer(self, dtype, n)

    def download(self, buf):
        return buf.to_numpy()

    def sync(self):
        check(lib().th_sync(self.handle))

    def zero_buffer(self, buf):
        check(lib().th_buffer_zero(buf.handle))

    def convert(self, src, dtype):
        out = self.alloc(src.n, dtype)
        check(lib().th_convert(self.handle, src.handle, out.handle))
        return out

    def memory_info(self):
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().th_memory_info(self.handle, ctypes.byref(f), ctypes.byref(t)))
        return f.value, t.value

    def timer_start(self):
        check(lib().th_timer_start(self.handle))

    def timer_stop(self):
        ms = ctypes.c_float()
        check(lib().th_timer_stop(self.handle, ctypes.byref(ms)))
        return ms.value

    def capture(self, fn):
        """Record the library calls fn() makes on this device's stream into a
        Graph (th_capture_begin / th_capture_end)."""
        check(lib().th_capture_begin(self.handle))
        h = ctypes.c_void_p()
        try:
            fn()
        except BaseException:
            # end the capture (the stream must leave capture mode) and drop its graph
            if lib().th_capture_end(self.handle, ctypes.byref(h)) == 0 and h:
                lib().th_graph_destroy(h)
            raise
        check(lib().th_capture_end(self.handle, ctypes.byref(h)))
        return Graph(h)

    # -- quantized weights
    def q4_upload_blocks(self, blocks, rows, cols, scale_dtype=F32):
        b = np.ascontiguousarray(blocks, Q4_BLOCK)
        h = ctypes.c_void_p()
        check(lib().th_q4_upload_blocks(self.handle, ptr(b), rows, cols, scale_dtype, ctypes.byref(h)))
        return QWeight(h, rows, cols, 4)

    def q4_upload_packed(self, nib, scales, rows, cols, scale_dtype=F16):
        n = np.ascontiguousarray(nib, np.uint8)
        s = np.ascontiguousarray(scales, np.uint16 if scale_dtype == F16 else np.float32)
        h = ctypes.c_void_p()
        check(lib().th_q4_upload_packed(self.handle, ptr(n), ptr(s), scale_dtype, rows, cols, ctypes.byref(h)))
        return QWeight(h, rows, cols, 4)

    def q8_upload_blocks(self, blocks, rows, cols):
        b = np.ascontiguousarray(blocks, Q8_BLOCK)
        h = ctypes.c_void_p()
        check(lib().th_q8_upload_blocks(self.handle, ptr(b), rows, cols, ctypes.byref(h)))
        return QWeight(h, rows, cols, 8)

    def q8_upload_rowwise(self, q, row_scale, rows, cols):
        qq = np.ascontiguousarray(q, np.int8)
        s = np.ascontiguousarray(row_scale, np.float32)
        h = ctypes.c_void_p()
        check(lib().th_q8_upload_rowwise(self.handle, ptr(qq), ptr(s), rows, cols, ctypes.byref(h)))
        return QWeight(h, rows, cols, 8)

    # -- quantized linear (matmul_b_transposed with a quantized B, device.rs:407)
    def gemm_q4(self, x, m, w, y=None):
        y = y or self.alloc(m * w.rows)
        check(lib().th_gemm_q4(self.handle, x.handle, m, w.handle, y.handle))
        return y

    def gemv_q8(self, x, m, w, y=None):
        y = y or self.alloc(m * w.rows)
        check(lib().th_gemv_q8(self.handle, x.handle, m, w.handle, y.handle))
        return y

    def bench_linear(self, x, m, weights, y, iters, use_graph=False):
        """Elapsed ms of `iters` quantized linears cycling through `weights`:
        launched one by one (use_graph False), replayed as a HIP graph (True)
        or as a sequence on the library's AQL queue ("aql")."""
        arr = (ctypes.c_void_p * len(weights))(*[w.handle.value for w in weights])
        ms = ctypes.c_float()
        mode = 2 if use_graph == "aql" else (1 if use_graph else 0)
        check(lib().th_bench_linear(self.handle, x.handle, m, arr, len(weights), y.handle, iters,
                                    mode, ctypes.byref(ms)))
        return ms.value

    # -- decode ops
    def rms_norm(self, data, weight, n_groups, dim, eps):
        out = self.alloc(n_groups * dim)
        check(lib().th_rms_norm(self.handle, data.handle, weight.handle, n_groups, dim, eps, out.handle))
        return out

    def rms_norm_residual(self, inp, residual, weight, n_groups, dim, eps):
        out, s = self.alloc(n_groups * dim), self.alloc(n_groups * dim)
        check(lib().th_rms_norm_residual(self.handle, inp.handle, residual.handle, weight.handle, n_groups, dim,
                                         eps, out.handle, s.handle))
        return out, s

    def rope_forward_cached(self, inp, cos_buf, sin_buf, seq_len, n_heads, head_dim, start_pos):
        out = self.alloc(seq_len * n_heads * head_dim)
        check(lib().th_rope_forward(self.handle, inp.handle, cos_buf.handle, sin_buf.handle, seq_len, n_heads,
                                    head_dim, start_pos, out.handle))
        return out

    def kv_attention(self, q, k_cache, v_cache, cache_start, q_len, n_heads, n_kv_heads, head_dim):
        out = self.alloc(q_len * n_heads * head_dim)
        check(lib().th_kv_attention(self.handle, q.handle, k_cache.handle, v_cache.handle, cache_start, q_len,
                                    n_heads, n_kv_heads, head_dim, out.handle))
        return out

    def swiglu_fused_buf(self, gate, up, numel):
        out = self.alloc(numel)
        check(lib().th_swiglu(self.handle, gate.handle, up.handle, numel, out.handle))
        return out

    def add_tensors_buf(self, a, b, numel):
        out = self.alloc(numel)
        check(lib().th_add(self.handle, a.handle, b.handle, numel, out.handle))
        return out

    def embedding(self, weight, ids, seq_len, dim):
        out = self.alloc(seq_len * dim)
        check(lib().th_embedding(self.handle, weight.handle, ids.handle, seq_len, dim, out.handle))
        return out

    def softmax(self, data, n_rows, row_len):
        out = self.alloc(n_rows * row_len)
        check(lib().th_softmax(self.handle, data.handle, n_rows, row_len, out.handle))
        return out

    def argmax(self, data, n_rows, n):
        out = self.alloc(n_rows, U32)
        check(lib().th_argmax(self.handle, data.handle, n_rows, n, out.handle))
        return out

    def mla_decode(self, q_nope, q_rope, cache, B, H, L, dn, dr, r, dv, w_uk, w_uv, sm_scale, out=None):
        """Absorbed MLA decode: q_nope/q_rope f32, cache bf16 [B][L][r+dr],
        w_uk/w_uv q8 rowwise; returns out f32 [B][H][dv]."""
        out = out or self.alloc(B * H * dv)
        check(lib().th_mla_decode(self.handle, q_nope.handle, q_rope.handle, cache.handle, B, H, L, dn, dr, r, dv,
                                  w_uk.handle, w_uv.handle, sm_scale, out.handle))
        return out

    # ---- dense operators (device.rs matmul / transpose_2d / reduce_sum / ...)
    def matmul(self, a, b, m, k, n, trans_a=False, trans_b=False, accumulate_into=None):
        c = accumulate_into if accumulate_into is not None else self.alloc(m * n)
        check(lib().th_matmul_ex(self.handle, a.handle, b.handle, m, k, n, int(trans_a), int(trans_b),
                                 int(accumulate_into is not None), c.handle))
        return c

    def matmul_b_transposed(self, a, b, m, k, n):
        return self.matmul(a, b, m, k, n, trans_b=True)

    def transpose_2d(self, buf, rows, cols):
        out = self.alloc(rows * cols)
        check(lib().th_transpose_2d(self.handle, buf.handle, rows, cols, out.handle))
        return out

    def reduce_sum(self, buf, shape, axis, accumulate_into=None):
        n_out = 1
        for i, d in enumerate(shape):
            if i != axis:
                n_out *= d
        out = accumulate_into if accumulate_into is not None else self.alloc(n_out)
        sh = (ctypes.c_size_t * len(shape))(*shape)
        check(lib().th_reduce_sum(self.handle, buf.handle, sh, len(shape), axis, int(accumulate_into is not None),
                                  out.handle))
        return out

    def bias_add(self, matrix, bias, numel, dim):
        out = self.alloc(numel)
        check(lib().th_bias_add(self.handle, matrix.handle, bias.handle, numel, dim, out.handle))
        return out

    def add_assign(self, dst, src):
        check(lib().th_add_assign(self.handle, dst.handle, src.handle))

    def elementwise(self, inputs, numel, f):
        """ComputeDevice::elementwise (device.rs:93): f(graph, vars) builds the
        output node from one variable per input buffer, as the reference's
        closure does under trace()."""
        g = ExprGraph()
        out_id = f(g, [g.var(i) for i in range(len(inputs))])
        nodes = g.array()
        out = self.alloc(numel)
        arr = (ctypes.c_void_p * max(len(inputs), 1))(*[b.handle for b in inputs])
        check(lib().th_elementwise_expr(self.handle, ptr(nodes), len(nodes), out_id, arr, len(inputs), numel,
                                        out.handle))
        return out

    def compile_kernel(self, source, entry="k0"):
        h = ctypes.c_void_p()
        check(lib().th_kernel_compile(self.handle, source.encode(), entry.encode(), ctypes.byref(h)))
        return h

    def run_kernel(self, kernel, inputs, numel):
        """A kernel from compile_kernel over numel elements (th_elementwise)."""
        out = self.alloc(numel)
        arr = (ctypes.c_void_p * max(len(inputs), 1))(*[b.handle for b in inputs])
        check(lib().th_elementwise(kernel, arr, len(inputs), numel, out.handle))
        return out

    def close(self):
        if self.handle:
            check(lib().th_device_destroy(self.handle))
            self.handle = None
