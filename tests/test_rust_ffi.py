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

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tang_hip.h")
CRATE = os.path.join(ROOT, "tang_amd", "tang-compute-hip", "src")

C_BASE = {"int": "i32", "size_t": "usize", "float": "f32", "double": "f64", "uint64_t": "u64", "int64_t": "i64",
          "int32_t": "i32", "uint8_t": "u8", "int8_t": "i8", "uint16_t": "u16", "char": "c_char", "void": "void",
          "th_dtype": "i32"}
RUST_BASE = {"c_int": "i32", "usize": "usize", "f32": "f32", "f64": "f64", "u64": "u64", "i64": "i64", "i32": "i32",
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
    for name in ("th_q4_block", "th_q8_block", "th_llama_config", "th_sampling_config"):
        m = re.search(r"typedef struct \{([^}]*)\}\s*" + name + ";", src)
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
