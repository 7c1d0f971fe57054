"""Writes the golden vectors under tests/golden/ from the reference's own code.

Run in the build container only (it needs /root/reference):
    python tests/golden/make_golden.py

ref_vectors.npz   inputs and outputs of the reference's cpu/forward_cpu.c helpers (matmul,
                  layernorm, gelu_new, attention) and of gpt2_forward_cpu on a seeded synthetic
                  model, computed by oracle/_ref/libref.so (the reference sources compiled by
                  oracle/Makefile).
quant_golden.npz  (w16 -> q, s) vectors from tools/quantize.py:quantize_rows, imported from the
                  reference tree: numpy's own rounding and dtype path, which no closed form pins.
gpq8_golden.json  what tools/quantize.py:main writes for a seeded synthetic model (a 'GPT2' v1 file
                  plus the manifest tools/export_gpt2.py would write beside it), for the default
                  scheme and for --fp16-keep head: the header and flags bytes, the file size, the
                  streamed-bytes and parameter counts and sha256(body) from its sidecar, and the
                  sha256 of the whole file.  Nothing else pins the 'GPQ8' v2 layout.

Only data is written (no reference source).  The forward's weights are not stored; the test
regenerates them with bare_metal_gpt2_amd.synth.make_body(seed=SEED_FWD, plain=False).
"""
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402
import oracle  # noqa: E402

REF_TOOLS = "/root/reference/tools/quantize.py"
SEED_FWD = 2024
FWD_IDS = np.array([464, 2068, 7586, 21831, 18045, 50256, 0, 13], np.int32)
LOGIT_COLS = np.r_[0:64, 50193:50257, 1000:50000:397]


def ref_vectors():
    rng = np.random.default_rng(99)
    out = {}
    for i, (M, N, K, bias) in enumerate([(5, 7, 33, True), (3, 11, 768, False), (4, 9, 3072, True)]):
        A = rng.standard_normal((M, K), dtype=np.float32)
        W = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
        b = rng.standard_normal(N, dtype=np.float32) * np.float32(0.01) if bias else None
        out[f"mm{i}_A"], out[f"mm{i}_W"] = A, W
        if b is not None:
            out[f"mm{i}_b"] = b
        out[f"mm{i}_C"] = oracle.ref_matmul(A, W, b)
    x = (rng.standard_normal((6, 768), dtype=np.float32) * np.float32(3) + np.float32(0.5))
    g = 1 + rng.standard_normal(768, dtype=np.float32) * np.float32(0.1)
    b = rng.standard_normal(768, dtype=np.float32) * np.float32(0.1)
    out.update(ln_x=x, ln_g=g, ln_b=b, ln_y=oracle.ref_layernorm(x, g, b))
    gx = np.concatenate([np.linspace(-8, 8, 257, dtype=np.float32),
                         rng.standard_normal(256, dtype=np.float32) * np.float32(3)])
    out.update(gelu_x=gx, gelu_y=oracle.ref_gelu(gx))
    qkv = rng.standard_normal((9, 2304), dtype=np.float32)
    out.update(attn_qkv=qkv, attn_y=oracle.ref_attention(qkv))

    pkg = __graft_entry__.load_package()
    import importlib
    synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    body = synth.make_body(seed=SEED_FWD, plain=False)
    # tensor offsets as the reference loader (model/weights.c) hands them out, from a real file
    path = "/tmp/golden_gpt2_fp32.bin"
    oracle.write_gpt2_file(path, body)
    rc, offs = oracle.ref_offsets_from_file(path)
    os.remove(path)
    assert rc == 0
    fwd = oracle.ref_forward(body, offs, FWD_IDS, logits_all=True)
    out.update(fwd_seed=np.array([SEED_FWD]), fwd_ids=FWD_IDS, fwd_final_ln=fwd["final_ln"],
               fwd_logit_cols=LOGIT_COLS, fwd_logits=fwd["logits"][:, LOGIT_COLS], ref_offsets=offs)
    del pkg
    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **out)


def quant_golden():
    spec = importlib.util.spec_from_file_location("ref_quantize", REF_TOOLS)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    rng = np.random.default_rng(7)
    cases = {}
    # random fp16-valued rows at several magnitudes
    w = rng.standard_normal((24, 96), dtype=np.float32) * np.float32(0.02)
    w[8:16] *= np.float32(50)
    w[16:] *= np.float32(1e-3)
    cases["rand"] = oracle.fp16_view(w)
    # exact ties (s = 1 and s = 2^-7), a dead row, single-entry rows, fp16 extremes
    t = np.zeros((8, 16), np.float32)
    t[0, :8] = [127, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 126.5]
    t[1, :6] = np.array([127, 2.5, 3.5, -2.5, -1.5, 0.5], np.float32) / np.float32(128)
    t[3, 5] = -0.001
    t[4, :] = oracle.fp16_view(np.linspace(-65504, 65504, 16).astype(np.float32))
    t[5, :] = oracle.fp16_view(np.full(16, 6e-8, np.float32))
    t[6, :] = oracle.fp16_view(rng.standard_normal(16, dtype=np.float32))
    t[7, :] = oracle.fp16_view(np.arange(16, dtype=np.float32) - 7.5)
    cases["special"] = oracle.fp16_view(t)
    out = {}
    for k, v in cases.items():
        q, s, _stats = mod.quantize_rows(v)
        out[f"{k}_w16"], out[f"{k}_q"], out[f"{k}_s"] = v, q, s
    np.savez_compressed(os.path.join(HERE, "quant_golden.npz"), **out)


SEED_GPQ8 = 4242
GPQ8_EXPORT_NAMES = ["wte", "wpe"] + [f"h{L}.{t}" for L in range(12) for t in (
    "ln_1.g", "ln_1.b", "attn.c_attn.w", "attn.c_attn.b", "attn.c_proj.w", "attn.c_proj.b",
    "ln_2.g", "ln_2.b", "mlp.c_fc.w", "mlp.c_fc.b", "mlp.c_proj.w", "mlp.c_proj.b")] + ["ln_f.g", "ln_f.b"]


def gpq8_golden():
    """Run the reference's tools/quantize.py main on a seeded synthetic 'GPT2' file (default scheme
    and --fp16-keep head) and keep the facts of each output file (the body is regenerated by the
    tests from SEED_GPQ8)."""
    import importlib
    import tempfile
    synth = importlib.import_module("bare_metal_gpt2_amd.synth") if "bare_metal_gpt2_amd" in sys.modules else None
    if synth is None:
        __graft_entry__.load_package()
        synth = importlib.import_module("bare_metal_gpt2_amd.synth")
    with tempfile.TemporaryDirectory() as tmp:
        _gpq8_golden(synth, tmp)


def _gpq8_golden(synth, tmp):
    import hashlib
    import json
    body = synth.make_body(seed=SEED_GPQ8, plain=False)
    src = os.path.join(tmp, "synth_fp32.bin")
    oracle.write_gpt2_file(src, body)
    # the manifest tools/export_gpt2.py writes beside the file (export_gpt2.py:92-107): byte offsets
    # of each tensor from the start of the file (64-byte header first)
    tensors, off = [], 64
    for (name, shape, _), ename in zip(synth.layout(), GPQ8_EXPORT_NAMES):
        n = int(np.prod(shape))
        tensors.append({"name": ename, "shape": list(shape), "offset": off, "bytes": 4 * n})
        off += 4 * n
    with open(src + ".json", "w") as f:
        json.dump({"tensors": tensors}, f)
    spec = importlib.util.spec_from_file_location("ref_quantize", REF_TOOLS)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out = {"seed": SEED_GPQ8, "plain": False, "variants": {}}
    for variant in ("none", "head"):
        dst = os.path.join(tmp, f"q_{variant}.bin")
        argv = sys.argv
        sys.argv = ["quantize.py", "--in", src, "--out", dst, "--fp16-keep", variant]
        try:
            mod.main()
        finally:
            sys.argv = argv
        side = json.load(open(dst + ".json"))
        raw = open(dst, "rb").read()
        n_t = int(np.frombuffer(raw[:64], np.int32)[7])
        flags = np.frombuffer(raw[64:64 + 4 * n_t], np.int32)
        out["variants"][variant] = {
            "keep": [int(f == 0) for f in flags],
            "prefix_hex": raw[:64 + 4 * n_t].hex(),
            "file_bytes": side["file_bytes"],
            "quantized_params": side["quantized_params"],
            "kept_fp16_params": side["kept_fp16_params"],
            "streamed_weight_bytes": side["streamed_weight_bytes"],
            "sha256_body": side["sha256"],
            "sha256_file": hashlib.sha256(raw).hexdigest(),
        }
        assert len(raw) == side["file_bytes"]
        os.remove(dst)
        os.remove(dst + ".json")
    os.remove(src)
    os.remove(src + ".json")
    with open(os.path.join(HERE, "gpq8_golden.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    if not oracle.ref_available():
        oracle.build()
    which = sys.argv[1:] or ["ref", "quant", "gpq8"]
    if "ref" in which:
        ref_vectors()
    if "quant" in which:
        quant_golden()
    if "gpq8" in which:
        gpq8_golden()
    print("wrote", os.listdir(HERE))
