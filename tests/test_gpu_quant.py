"""The INT8 scheme and the fp16 upload on the GPU, bit-exact against the CPU oracle.

k_quantize_rows (tools/quantize.py:58-73 on the device) must give the same int8 codes and fp32
scales as oracle.quantize_rows for every row; k_f32_to_f16 must give the same bits as the
oracle's IEEE round-to-nearest-even converter (itself pinned to F16C over all 2^32 inputs).
"""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def quantize_dev(pkg, L, w16):
    N, K = w16.shape
    dw = pkg.Dev.from_numpy(oracle.f32_to_f16(w16))
    dq, ds = pkg.Dev(N * K), pkg.Dev(N * 4)
    L.gpt2_quantize_rows(dq.ptr, ds.ptr, dw.ptr, N, K)
    L.gpt2_sync()
    pkg.check("quantize_rows")
    return dq.numpy(np.int8, (N, K)), ds.numpy(np.float32, (N,))


@pytest.mark.parametrize("N,K", [(2304, 768), (768, 768), (3072, 768), (768, 3072), (50257, 768)])
def test_device_quantizer_bit_exact(pkg, L, N, K):
    rng = np.random.default_rng(N ^ K)
    w16 = oracle.fp16_view(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    q, s = quantize_dev(pkg, L, w16)
    q_ref, s_ref, _ = oracle.quantize_rows(w16)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q, q_ref)


def test_device_quantizer_special_rows(pkg, L):
    K = 64
    rows = []
    rows.append(np.zeros(K, np.float32))                                  # dead row -> s = 1, q = 0
    r = np.zeros(K, np.float32); r[:6] = [127, 2.5, 3.5, -2.5, -3.5, 0.5]; rows.append(r)   # s = 1: ties
    r = np.zeros(K, np.float32); r[:4] = [127 / 128, 2.5 / 128, -1.5 / 128, 0.5 / 128]; rows.append(r)
    r = np.zeros(K, np.float32); r[3] = -0.001; rows.append(r)             # single negative entry
    rows.append(oracle.fp16_view(np.linspace(-65504, 65504, K).astype(np.float32)))  # fp16 extremes
    rows.append(oracle.fp16_view(np.full(K, 6e-8, np.float32)))            # subnormal fp16 values
    rng = np.random.default_rng(3)
    for _ in range(26):
        rows.append(oracle.fp16_view(rng.standard_normal(K, dtype=np.float32) * np.float32(10 ** rng.uniform(-4, 2))))
    w16 = oracle.fp16_view(np.stack(rows))
    q, s = quantize_dev(pkg, L, w16)
    q_ref, s_ref, dead = oracle.quantize_rows(w16)
    assert dead == 1 and s[0] == 1.0 and not q[0].any()
    assert list(q[1, :6]) == [127, 2, 4, -2, -4, 0]
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q, q_ref)


def test_quant_build_whole_model(pkg, L, synth):
    """gpt2_quant_build on the uploaded model == the oracle scheme on the fp16 view, all 48 trunk
    tensors; the head stays fp16 (q == NULL) by default."""
    body = synth.make_body(seed=77, plain=False)
    m = pkg.Model(body)
    try:
        m.quantize()
        assert m.q.wte.q is None
        shapes = {"qkv_w": (2304, 768), "attn_proj_w": (768, 768), "fc_w": (3072, 768), "proj_w": (768, 3072)}
        streamed = 0
        for Lyr in (0, 5, 11):
            for name, (N, K) in shapes.items():
                qw = getattr(m.q.layers[Lyr], name)
                q = np.empty((N, K), np.int8)
                s = np.empty(N, np.float32)
                L.gpt2_d2h(q.ctypes.data, qw.q, q.nbytes)
                L.gpt2_d2h(s.ctypes.data, qw.s, s.nbytes)
                q_ref, s_ref, _ = oracle.quantize_fp16_view(synth.tensor(body, f"h{Lyr}.{name}"))
                assert np.array_equal(q, q_ref), (Lyr, name)
                assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32)), (Lyr, name)
        for name, (N, K) in shapes.items():
            streamed += 12 * (N * K + 4 * N)
        streamed += 2 * 50257 * 768
        assert m.q.streamed_bytes == streamed == 162461184
    finally:
        m.free()


def test_f32_to_f16_kernel_bit_exact(pkg, L):
    rng = np.random.default_rng(5)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.99, 65520, -65520, 6.1035156e-05,
                        6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-10, 1.0009766,
                        1.00048828125, 1.000244140625, 2049.0, 2051.0], np.float32)
    bits = rng.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([special, bits.view(np.float32)])
    x = x[~np.isnan(x)]
    dx, dy = pkg.Dev.from_numpy(x), pkg.Dev(x.size * 2)
    L.gpt2_f32_to_f16(dy.ptr, dx.ptr, x.size)
    L.gpt2_sync()
    pkg.check("f32_to_f16")
    assert np.array_equal(dy.numpy(np.uint16, x.shape), oracle.f32_to_f16(x))


def test_upload_fp16_matches_oracle(pkg, L, synth):
    body = synth.make_body(seed=3, plain=False)
    m = pkg.Model(body)
    try:
        for name, ptr in (("wte", m.gpu.wte), ("h7.fc_w", m.gpu.layers[7].fc_w), ("lnf_b", m.gpu.lnf_b),
                          ("h0.ln1_g", m.gpu.layers[0].ln1_g), ("wpe", m.gpu.wpe)):
            ref = oracle.f32_to_f16(synth.tensor(body, name))
            got = np.empty(ref.shape, np.uint16)
            L.gpt2_d2h(got.ctypes.data, ptr, got.nbytes)
            assert np.array_equal(got, ref), name
    finally:
        m.free()


def test_quant_file_round_trip(pkg, L, synth, tmp_path):
    """'GPQ8' v2 written from device weights and loaded back gives identical codes and scales."""
    body = synth.make_body(seed=9)
    m = pkg.Model(body)
    path = str(tmp_path / "w.gpq8")
    try:
        m.quantize()
        assert L.gpt2_quant_write_file(path.encode(), C.byref(m.q), None) == 0
        q2 = pkg.GPT2QWeightsGPU()
        assert L.gpt2_quant_load_upload(path.encode(), None, C.byref(q2)) == 0
        assert q2.nq == m.q.nq and q2.ns == m.q.ns and q2.streamed_bytes == m.q.streamed_bytes
        a = np.empty(m.q.nq, np.int8)
        b = np.empty(m.q.nq, np.int8)
        L.gpt2_d2h(a.ctypes.data, m.q.qdata, a.nbytes)
        L.gpt2_d2h(b.ctypes.data, q2.qdata, b.nbytes)
        assert np.array_equal(a, b)
        L.gpt2_quant_free(C.byref(q2))
    finally:
        m.free()


@pytest.mark.parametrize("variant", ["none", "head"])
def test_gpq8_file_matches_reference_writer(pkg, L, synth, tmp_path, variant):
    """The library's 'GPQ8' v2 writer and loader against the file tools/quantize.py:main wrote for the
    same seeded model (tests/golden/gpq8_golden.json; default scheme and --fp16-keep head): the
    device-quantized weights written by gpt2_quant_write_file give the same header and flags bytes,
    the same file size, the same sha256 of the q/s body and of the whole file; gpt2_quant_load_upload
    reads it back with the sidecar's streamed-byte count and the same codes and scales."""
    import hashlib
    import json
    import os
    gold = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gpq8_golden.json")))
    want = gold["variants"][variant]
    body = synth.make_body(seed=gold["seed"], plain=gold["plain"])
    m = pkg.Model(body)
    path = str(tmp_path / f"w_{variant}.gpq8")
    keep = (C.c_int * len(want["keep"]))(*want["keep"])
    try:
        m.quantize(want["keep"])
        assert L.gpt2_quant_write_file(path.encode(), C.byref(m.q), keep) == 0
        raw = open(path, "rb").read()
        npre = len(want["prefix_hex"]) // 2
        assert raw[:npre].hex() == want["prefix_hex"]
        assert len(raw) == want["file_bytes"]
        assert hashlib.sha256(raw[npre:]).hexdigest() == want["sha256_body"]
        assert hashlib.sha256(raw).hexdigest() == want["sha256_file"]
        q2 = pkg.GPT2QWeightsGPU()
        assert L.gpt2_quant_load_upload(path.encode(), None, C.byref(q2)) == 0
        try:
            assert q2.streamed_bytes == want["streamed_weight_bytes"]
            assert q2.nq == m.q.nq and q2.ns == m.q.ns
            a, b = np.empty(m.q.nq, np.int8), np.empty(m.q.nq, np.int8)
            L.gpt2_d2h(a.ctypes.data, m.q.qdata, a.nbytes)
            L.gpt2_d2h(b.ctypes.data, q2.qdata, b.nbytes)
            assert np.array_equal(a, b)
            sa, sb = np.empty(m.q.ns, np.float32), np.empty(m.q.ns, np.float32)
            L.gpt2_d2h(sa.ctypes.data, m.q.sdata, sa.nbytes)
            L.gpt2_d2h(sb.ctypes.data, q2.sdata, sb.nbytes)
            assert np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
        finally:
            L.gpt2_quant_free(C.byref(q2))
    finally:
        m.free()
