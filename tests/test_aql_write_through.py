"""The write-through contract of AQL sequences, checked on the built code.

A write-through sequence (tang_amd/csrc/aql.cpp) drops the release fence
between its kernels, which is safe only if every kernel in it stores what
later kernels read with write-through stores (`sc1`: relaxed agent-scope
atomic stores, which reach the coherence point before the kernel ends).
aql_record_launch refuses a kernel that WRITE_THROUGH_KERNELS does not list;
this test disassembles the library's gfx950 code objects and checks that
every global, buffer or flat store in every kernel a listed entry matches
carries `sc1`.  So a new kernel in the decode step, or a plain store added
to a listed kernel, fails here on the CPU before it can read stale data on
the GPU.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "tang_amd", "libtang_hip.so")
AQL_SRC = os.path.join(ROOT, "tang_amd", "csrc", "aql.cpp")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"


def write_through_table():
    src = open(AQL_SRC).read()
    body = src[src.index("WRITE_THROUGH_KERNELS[] = {"):]
    body = body[:body.index("};")]
    return re.findall(r'\{"(\w+)",\s*"(\w*)"\}', body)


def test_table_names_the_decode_step_kernels():
    table = write_through_table()
    kernels = {k for k, _ in table}
    assert {"q4_gemv_kernel", "attn_decode_kernel", "llama_argmax_embed_kernel", "aql_stamp_kernel"} <= kernels
    epis = {e for k, e in table if k == "q4_gemv_kernel"}
    assert {"EpiQKV", "EpiAddToSsq", "EpiSwiGLU", "EpiTileMax", "EpiStore"} <= epis


def disassembly(tmp_path):
    """{mangled kernel name: [store instruction lines]} over every gfx950 code
    object bundled in the library."""
    lib = str(tmp_path / "lib.so")
    shutil.copy(LIB, lib)
    subprocess.run([OBJDUMP, "--offloading", lib], check=True, capture_output=True, cwd=str(tmp_path))
    bundles = [str(p) for p in tmp_path.iterdir() if p.name.endswith("gfx950")]
    assert bundles, "no gfx950 code object in the library"
    stores = {}
    for b in bundles:
        out = subprocess.run([OBJDUMP, "-d", "--no-show-raw-insn", b], check=True, capture_output=True,
                             text=True).stdout
        cur = None
        for line in out.splitlines():
            m = re.match(r"^[0-9a-f]+ <(.*)>:$", line)
            if m:
                cur = m.group(1)
                stores.setdefault(cur, [])
                continue
            if cur and re.search(r"\b(global|buffer|flat)_store", line):
                stores[cur].append(line.split("//")[0].strip())
    return stores


@pytest.mark.skipif(not (os.path.exists(OBJDUMP) and os.path.exists(LIB)), reason="needs llvm-objdump and the built library")
def test_listed_kernels_store_write_through_only(tmp_path):
    table = write_through_table()
    stores = disassembly(tmp_path)
    matched = {k: [] for k in table}
    bad = []
    for name, lines in stores.items():
        entries = [(k, e) for k, e in table if k in name and e in name]
        if not entries:
            continue
        for ent in entries:
            matched[ent].append(name)
        bad += ["%s: %s" % (name[:120], ln) for ln in lines if not re.search(r"\bsc1\b", ln)]
    assert not [k for k, v in matched.items() if not v], "table entries that match no kernel: %s" % matched
    assert not bad, "plain stores in write-through kernels:\n" + "\n".join(bad[:20])
    # the check is not vacuous: the listed kernels do store, and a kernel
    # outside the table (the eager embedding) stores without sc1
    assert sum(len(stores[n]) for v in matched.values() for n in v) > 100
    emb = [n for n in stores if "llama_embed_kernel" in n and "argmax" not in n]
    assert emb and any(not re.search(r"\bsc1\b", ln) for n in emb for ln in stores[n])
