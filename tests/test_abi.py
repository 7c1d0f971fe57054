"""The C-ABI boundary without a GPU: every function include/*.h declares is exported by
libgpt2amd.so, the Python ctypes mirror has the C layout, and the host-only parts of the library
(backend tables, weight layout, file loaders' error paths) behave as the reference's do.
"""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
need_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no /root/reference)")


def header_text():
    txt = ""
    for f in sorted(os.listdir(INC)):
        if f.endswith(".h"):
            txt += open(os.path.join(INC, f)).read() + "\n"
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return re.sub(r"//[^\n]*", "", txt)


def declared_functions():
    txt = header_text()
    names = set()
    for m in re.finditer(r"^[ \t]*(?!static)(?:const\s+)?[A-Za-z_][\w \t\*]*?\b(gpt2_\w+)\s*\(", txt, re.M):
        names.add(m.group(1))
    inline = set(re.findall(r"static\s+inline\s+[\w\s\*]+?\b(gpt2_\w+)\s*\(", txt))
    return sorted(names - inline)


def declared_data():
    return sorted(set(re.findall(r"extern\s+const\s+GPT2Backend\s+(\w+)\s*;", header_text())))


def test_every_declared_symbol_is_exported(L):
    funcs = declared_functions()
    assert len(funcs) >= 50, funcs
    so = os.path.join(ROOT, "bare-metal-gpt2_amd", "libgpt2amd.so")
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [f for f in funcs + declared_data() if f not in exported]
    assert not missing, missing


def test_python_mirror_covers_header(pkg):
    missing = [f for f in declared_functions() if f not in pkg.SIGNATURES]
    assert not missing, missing
    assert sorted(pkg.DATA_SYMBOLS) == declared_data()


LAYOUT_C = r"""
#include <stdio.h>
#include <stddef.h>
#include "gpt2_kvcache.h"
#define S(T) printf(#T " %zu\n", sizeof(T));
#define O(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main(void) {
  S(GPT2Layer) S(GPT2Weights) O(GPT2Weights, layers) O(GPT2Weights, lnf_b)
  S(GPT2LayerGPU) S(GPT2QW) S(GPT2QLayerGPU) S(GPT2QWeightsGPU) O(GPT2QWeightsGPU, wte) O(GPT2QWeightsGPU, layers)
  S(GPT2WeightsGPU) O(GPT2WeightsGPU, layers) O(GPT2WeightsGPU, q)
  S(GPT2ScratchGPU) O(GPT2ScratchGPU, maxT) S(GPT2CapsGPU) O(GPT2CapsGPU, logits_all) O(GPT2CapsGPU, kv)
  S(GPT2KVCache) O(GPT2KVCache, len) S(GPT2Backend) O(GPT2Backend, gemv_q)
  return 0;
}
"""


def test_struct_layouts_match_c(pkg, tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(LAYOUT_C)
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", INC, str(src), "-o", str(exe)], check=True)
    vals = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                         check=True).stdout.splitlines())
    for key, v in vals.items():
        if "." in key:
            t, f = key.split(".")
            got = getattr(getattr(pkg, t), f).offset
        else:
            got = C.sizeof(getattr(pkg, key))
        assert got == int(v), (key, got, v)


def test_backend_tables(pkg, L):
    """Slot composition of the reference's backends (cuda/kernels.cuh:88-92, kernels_quant.cu:374-384,
    kvcache.cu:282-290): each stage fills more slots; lookup falls back to naive."""
    def slots(name):
        b = L.gpt2_backend_by_name(name.encode() if name else None).contents
        return b.name.decode(), {f: bool(getattr(b, f)) for f in ("matmul_q", "gemv", "gemv_q")}, b.matmul
    assert slots(None)[0] == "naive" and slots("bogus")[0] == "naive"
    assert slots("naive")[1] == {"matmul_q": False, "gemv": False, "gemv_q": False}
    assert slots("tiled")[1] == {"matmul_q": False, "gemv": False, "gemv_q": False}
    assert slots("flash")[1] == {"matmul_q": False, "gemv": False, "gemv_q": False}
    assert slots("gemv")[1] == {"matmul_q": False, "gemv": True, "gemv_q": False}
    assert slots("int8")[1] == {"matmul_q": True, "gemv": True, "gemv_q": True}
    assert slots("naive")[2] != slots("tiled")[2] == slots("int8")[2]
    for name in ("naive", "tiled", "flash", "int8", "gemv"):
        b = L.gpt2_backend_by_name(name.encode()).contents
        assert all(getattr(b, f) for f in ("embed", "layernorm", "matmul", "attention", "gelu", "add"))


def test_bind_weights_layout(pkg, L, synth):
    body = np.zeros(1, np.float32)
    w = pkg.GPT2Weights()
    assert L.gpt2_bind_weights(C.byref(w), body.ctypes.data) == pkg.TOTAL_PARAMS
    base = body.ctypes.data

    def off(p):
        return (C.cast(p, C.c_void_p).value - base) // 4
    got = [off(w.wte), off(w.wpe)]
    for Lyr in range(12):
        got += [off(getattr(w.layers[Lyr], n)) for n, _ in pkg.GPT2Layer._fields_]
    got += [off(w.lnf_g), off(w.lnf_b)]
    assert got == list(oracle.oracle_offsets())
    assert got == [synth.offsets()[n][0] for n, _, _ in synth.layout()]


def write_hdr(path, hdr, body=b""):
    with open(path, "wb") as f:
        f.write(np.asarray(hdr, np.int32).tobytes())
        f.write(body)


GOOD_HDR = [0x47505432, 1, 12, 12, 768, 50257, 1024, 3072, 2304, 0, 0, 0, 0, 0, 0, 0]


def crafted_weight_files(tmp_path):
    cases = {}
    p = tmp_path / "short_hdr.bin"
    p.write_bytes(b"\x32\x54\x50\x47")
    cases["short_header"] = (p, 2)
    for name, idx, val, code in (("magic", 0, 0x12345678, 3), ("version", 1, 2, 3), ("dims", 4, 512, 4),
                                 ("dtype", 9, 1, 5)):
        h = list(GOOD_HDR)
        h[idx] = val
        p = tmp_path / f"{name}.bin"
        write_hdr(p, h)
        cases[name] = (p, code)
    p = tmp_path / "short_body.bin"
    write_hdr(p, GOOD_HDR, np.zeros(1000, np.float32).tobytes())
    cases["short_body"] = (p, 7)
    cases["missing"] = (tmp_path / "nope.bin", 1)
    return cases


def test_load_weights_error_codes(L, pkg, tmp_path):
    """gpt2_load_weights keeps the reference loader's return codes (model/weights.c:16-39)."""
    for name, (path, code) in crafted_weight_files(tmp_path).items():
        w = pkg.GPT2Weights()
        assert L.gpt2_load_weights(str(path).encode(), C.byref(w)) == code, name
        assert not w.data


@need_ref
def test_load_weights_codes_equal_reference(L, pkg, tmp_path):
    for name, (path, code) in crafted_weight_files(tmp_path).items():
        rc_ref, _ = oracle.ref_offsets_from_file(str(path))
        assert rc_ref == code, name


def test_load_weights_full_file(L, pkg, synth, tmp_path):
    """A valid 'GPT2' v1 file loads bit-exact; one trailing byte is rejected with code 8."""
    body = synth.make_body(seed=11, plain=False)
    path = str(tmp_path / "w.bin")
    oracle.write_gpt2_file(path, body)
    w = pkg.GPT2Weights()
    assert L.gpt2_load_weights(path.encode(), C.byref(w)) == 0
    try:
        got = np.ctypeslib.as_array(w.data, shape=(pkg.TOTAL_PARAMS,))
        assert np.array_equal(got, body)
        fc = np.ctypeslib.as_array(w.layers[9].fc_w, shape=(3072 * 768,))
        assert np.array_equal(fc, synth.tensor(body, "h9.fc_w").reshape(-1))
    finally:
        L.gpt2_free_weights(C.byref(w))
    if oracle.ref_available():
        rc, offs = oracle.ref_offsets_from_file(path)
        assert rc == 0 and list(offs) == list(oracle.oracle_offsets())
    with open(path, "ab") as f:
        f.write(b"\0")
    w = pkg.GPT2Weights()
    assert L.gpt2_load_weights(path.encode(), C.byref(w)) == 8
    if oracle.ref_available():
        assert oracle.ref_offsets_from_file(path)[0] == 8
    os.remove(path)


QHDR = [0x38515047, 2, 12, 768, 50257, 3072, 2304, 49, 0, 0, 0, 0, 0, 0, 0, 0]


@pytest.mark.parametrize("case", ["missing", "short_header", "magic", "version", "dims", "short_flags",
                                  "short_q", "short_s", "trailing"])
def test_quant_file_errors(L, pkg, tmp_path, case):
    """'GPQ8' v2 loader rejects every malformed file before touching the GPU
    (cuda/kernels_quant.cu:89-120, tools/quantize.py:153-163)."""
    p = tmp_path / "q.bin"
    flags = np.zeros(49, np.int32)
    if case == "missing":
        p = tmp_path / "absent.bin"
    elif case == "short_header":
        p.write_bytes(np.asarray(QHDR[:5], np.int32).tobytes())
    elif case in ("magic", "version", "dims"):
        h = list(QHDR)
        h[{"magic": 0, "version": 1, "dims": 4}[case]] += 1
        write_hdr(p, h, flags.tobytes())
    elif case == "short_flags":
        write_hdr(p, QHDR, flags[:10].tobytes())
    elif case == "short_q":
        flags[3] = 1                       # layer 0 attn_proj: 768x768 codes + 768 scales
        write_hdr(p, QHDR, flags.tobytes() + b"\1" * 1000)
    elif case == "short_s":
        flags[3] = 1
        write_hdr(p, QHDR, flags.tobytes() + b"\1" * (768 * 768) + b"\0" * 100)
    elif case == "trailing":
        write_hdr(p, QHDR, flags.tobytes() + b"\0")
    q = pkg.GPT2QWeightsGPU()
    assert L.gpt2_quant_load_upload(str(p).encode(), None, C.byref(q)) == 1
    assert not q.qdata


def test_error_strings(L):
    assert L.gpt2_error_string(0) == b"no error"
    assert b"invalid argument" in L.gpt2_error_string(1000)


def test_c_caller_builds_and_links():
    """tests/c/boundary_caller.c compiles as C11 against include/ alone (gcc -Wall -Werror, done by
    __graft_entry__.build()), links libgpt2amd.so, and with no arguments prints its usage and exits 2
    before any device call."""
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = os.path.join(root, "tests", "c", "boundary_caller")
    assert os.path.exists(exe)
    deps = subprocess.run(["ldd", exe], capture_output=True, text=True).stdout
    assert "libgpt2amd.so" in deps and "not found" not in deps.split("libgpt2amd.so", 1)[1].splitlines()[0]
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr
