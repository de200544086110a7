"""The Rust binding (tang_amd/tang-compute-hip, source only: no Rust toolchain
in this image) against the C ABI it binds (include/tang_hip.h): every
function the header declares has an `extern "C"` declaration with the same
name, the same number of arguments and, argument by argument, the same kind
(pointer depth and constness, integer / float width); nothing is declared
that the header lacks.  Also: every required method of the reference's
ComputeDevice trait (crates/tang-compute/src/device.rs, the methods without a
default body) has an implementation in lib.rs, and the struct layouts the
binding repeats (th_q4_block, th_q8_block, th_llama_config,
th_sampling_config) list the header's fields in order."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tang_hip.h")
CRATE = os.path.join(ROOT, "tang_amd", "tang-compute-hip", "src")

C_BASE = {"int": "i32", "size_t": "usize", "float": "f32", "double": "f64", "uint64_t": "u64", "int64_t": "i64",
          "int32_t": "i32", "uint32_t": "u32", "uint8_t": "u8", "int8_t": "i8", "uint16_t": "u16", "char": "c_char", "void": "void",
          "th_dtype": "i32"}
RUST_BASE = {"c_int": "i32", "usize": "usize", "f32": "f32", "f64": "f64", "u64": "u64", "i64": "i64", "i32": "i32", "u32": "u32",
             "u8": "u8", "i8": "i8", "u16": "u16", "c_char": "c_char", "c_void": "void"}

# The required methods of `trait ComputeDevice` (device.rs:19-869): those
# declared without a default body.
REQUIRED = ["dialect", "upload", "upload_u32", "alloc", "download", "elementwise", "matmul", "softmax", "rms_norm",
            "embedding", "reduce_sum", "causal_attention", "kv_attention", "transpose_2d", "softmax_backward",
            "rms_norm_backward", "embedding_backward", "causal_attention_backward", "cross_entropy_forward_backward",
            "sync", "add_assign", "zero_buffer", "adamw_step"]


def _c_type(t):
    """C type -> (base, [const flags from the innermost pointer outwards])."""
    toks = t.replace("*", " * ").split()
    const_base = toks[0] == "const"
    if const_base:
        toks = toks[1:]
    base = C_BASE.get(toks[0], toks[0])
    quals = []  # per pointer level, innermost first: is the pointee const?
    pending = const_base
    for tok in toks[1:]:
        if tok == "*":
            quals.append(pending)
            pending = False
        elif tok == "const":
            pending = True
    return base, quals


def _rust_type(t):
    quals = []
    t = t.strip()
    while t.startswith("*"):
        m = re.match(r"\*(const|mut)\s+(.*)", t)
        quals.append(m.group(1) == "const")
        t = m.group(2).strip()
    return RUST_BASE.get(t, t), list(reversed(quals))


def header_functions():
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"^\s*((?:const\s+)?[A-Za-z_][\w\s\*]*?)\b(th_\w+)\s*\(([^;{]*?)\)\s*;", src,
                                      flags=re.M):
        params = [] if args.strip() in ("", "void") else [a.strip() for a in args.split(",")]
        kinds = [_c_type(re.match(r"(.*?)\w+$", p).group(1)) for p in params]
        out[name] = (_c_type(ret.strip()), kinds)
    return out


def rust_functions():
    src = open(os.path.join(CRATE, "ffi.rs")).read()
    block = src[src.index('extern "C" {'):]
    out = {}
    for name, args, ret in re.findall(r"pub fn (th_\w+)\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block):
        params = [a.strip() for a in args.split(",") if a.strip()]
        kinds = [_rust_type(p.split(":", 1)[1]) for p in params]
        out[name] = (_rust_type(ret) if ret else ("void", []), kinds)
    return out


def test_extern_block_matches_header():
    h, r = header_functions(), rust_functions()
    # every prototype line of the header is seen
    n_lines = len(re.findall(r"^(?:int|const char\*|uint64_t) th_\w+\(", open(HEADER).read(), flags=re.M))
    assert len(h) == n_lines > 75
    assert sorted(h) == sorted(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name in h:
        (hret, hargs), (rret, rargs) = h[name], r[name]
        assert len(hargs) == len(rargs), name
        assert hret == rret, (name, hret, rret)
        for i, (a, b) in enumerate(zip(hargs, rargs)):
            assert a == b, (name, i, a, b)


def _fields_c(struct_src):
    fields = []
    for decl in struct_src.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        m = re.match(r"([\w\s]+?)\s+([\w\s,\[\]]+)$", decl)
        names = [re.sub(r"\[.*\]", "", n).strip() for n in m.group(2).split(",")]
        fields += names
    return fields


def test_repeated_structs_match_header():
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    rs = open(os.path.join(CRATE, "ffi.rs")).read()
    for name in ("th_q4_block", "th_q8_block", "th_llama_config", "th_sampling_config", "th_expr_node"):
        m = re.search(r"typedef struct (?:\w+ )?\{([^}]*)\}\s*" + name + ";", src)
        c_fields = _fields_c(m.group(1))
        m2 = re.search(r"pub struct " + name + r" \{([^}]*)\}", rs)
        r_fields = re.findall(r"pub (\w+):", m2.group(1))
        assert c_fields == r_fields, (name, c_fields, r_fields)


def test_every_required_trait_method_is_implemented():
    src = open(os.path.join(CRATE, "lib.rs")).read()
    impl = src[src.index("impl ComputeDevice for HipComputeDevice"):src.index("// Quantized extension")]
    implemented = set(re.findall(r"\bfn (\w+)\s*\(", impl))
    missing = [m for m in REQUIRED if m not in implemented]
    assert not missing, missing


def test_every_entry_point_the_binding_calls_is_declared():
    src = open(os.path.join(CRATE, "lib.rs")).read()
    called = set(re.findall(r"ffi::(th_\w+)\s*\(", src))
    assert called <= set(header_functions()), sorted(called - set(header_functions()))


REF_DEVICE = "/root/reference/crates/tang-compute/src/device.rs"


def _split_top(s, sep=","):
    """Split at `sep` outside (), [], <>."""
    out, depth, cur = [], 0, ""
    for i, ch in enumerate(s):
        if ch in "([<":
            depth += 1
        elif ch in ")]>" and not (ch == ">" and s[i - 1] == "-"):
            depth -= 1
        if ch == sep and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [p.strip() for p in out if p.strip()]


def _signatures(src, buffer_names):
    """{method: (param types, return type)} of every `fn` in src, with the
    buffer type spelled B and whitespace removed."""
    sigs = {}
    for m in re.finditer(r"\bfn\s+(\w+)\s*\(", src):
        name, i, depth = m.group(1), m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(src[i], 0)
            i += 1
        params = src[m.end():i - 1]
        rest = src[i:]
        ret = re.match(r"\s*(?:->\s*([^{;]+?))?\s*(?:where[^{;]*)?[{;]", rest, flags=re.S)
        norm = lambda t: re.sub(r"\s+", "", re.sub(r"\b(%s)\b" % "|".join(buffer_names), "B", t))
        types = [norm(p.split(":", 1)[1]) for p in _split_top(params) if ":" in p]
        sigs[name] = (types, norm(ret.group(1) or "()"))
    return sigs


def _trait_body(src, start):
    i = src.index("{", src.index(start)) + 1
    depth = 1
    j = i
    while depth:
        depth += {"{": 1, "}": -1}.get(src[j], 0)
        j += 1
    return src[i:j - 1]


@pytest.mark.skipif(not os.path.exists(REF_DEVICE), reason="the reference checkout is not on this machine")
def test_implemented_trait_methods_have_the_reference_signatures():
    """Every method `impl ComputeDevice for HipComputeDevice` defines exists in
    the reference trait (crates/tang-compute/src/device.rs:19-869) with the
    same parameter types and return type (Self::Buffer = HipBuffer)."""
    ref = _signatures(_trait_body(open(REF_DEVICE).read(), "pub trait ComputeDevice"), [r"Self::Buffer"])
    src = open(os.path.join(CRATE, "lib.rs")).read()
    ours = _signatures(_trait_body(src, "impl ComputeDevice for HipComputeDevice"), ["HipBuffer"])
    assert len(ref) > 60 and len(ours) > 40
    bad = {n: (sig, ref.get(n)) for n, sig in ours.items() if ref.get(n) != sig}
    assert not bad, bad
    required = [n for n in ref if re.search(r"\bfn\s+%s\s*\([^{]*?\)\s*(->[^{;]*)?;" % n,
                                            _trait_body(open(REF_DEVICE).read(), "pub trait ComputeDevice"),
                                            flags=re.S)]
    assert sorted(required) == sorted(REQUIRED)


def test_extension_wrappers_cover_the_engines():
    """Safe wrappers exist for every configuration's entry points: the
    quantized linear, MLA decode, the MoE layer and the decode engine
    (greedy, prefill, safetensors load, and generate() with the sampler)."""
    src = open(os.path.join(CRATE, "lib.rs")).read()
    called = set(re.findall(r"ffi::(th_\w+)\s*\(", src))
    for fn in ("th_gemm_q4", "th_gemv_q8", "th_q8_upload_rowwise", "th_mla_decode", "th_moe_create",
               "th_moe_init_synthetic", "th_moe_forward", "th_moe_destroy", "th_llama_create", "th_llama_destroy",
               "th_llama_init_synthetic", "th_llama_load_safetensors", "th_llama_prefill", "th_llama_generate",
               "th_llama_generate_sampled", "th_sampler_create", "th_sampler_destroy", "th_elementwise_expr"):
        assert fn in called, fn
    for decl in ("pub trait LatentAttention", "pub struct HipMoe", "pub struct HipLlama",
                 "pub fn generate(&mut self, prompt: &[usize], config: &SamplingConfig, seed: u64) -> Vec<usize>"):
        assert decl in src, decl
    assert "Dialect::Cuda" not in src
