"""Device assembly of the library's HIP sources for the compiled-code checks: hipcc -S with the
flags of bare-metal-gpt2_amd/csrc/Makefile, each source compiled once per test session.  CPU only
(hipcc cross-compiles gfx950 without a GPU)."""
import functools
import os
import re
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "bare-metal-gpt2_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-I" + os.path.join(ROOT, "include"),
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S"]
EXTRA = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],       # as in csrc/Makefile
         "attn_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


@functools.lru_cache(maxsize=None)
def _outdir():
    return tempfile.mkdtemp(prefix="g2asm_")


@functools.lru_cache(maxsize=None)
def device_asm(src):
    """The gfx950 assembly listing of csrc/<src> (skips the test when hipcc is absent)."""
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = os.path.join(_outdir(), src + ".s")
    r = subprocess.run([HIPCC, *FLAGS, *EXTRA.get(src, []), os.path.join(CSRC, src), "-o", out],
                       capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stderr[-2000:]
    with open(out) as f:
        return f.read()


def functions(asm):
    """{mangled kernel name: its listing lines} for every function of the listing."""
    return {m.group(1): m.group(2).splitlines()
            for m in re.finditer(r"^(_Z\S+):[^\n]*\n(.*?)^\s*s_endpgm", asm, re.S | re.M)}
