"""Compiled-code check of the persistent decode step's register plan (CPU only: hipcc -S, the flags
of csrc/Makefile).

The step holds each attention wave's q/k/v weight fragments (36 16-byte fragments, 144 registers) in
accumulation registers between layers and feeds them to v_mfma_f32_16x16x32_f16 as its A operand
straight from there.  Two ways a later change could quietly undo that, both of which would cost far
more than the MFMAs save: the compiler spilling to scratch memory (the kernel then reads and writes
private memory in every layer), or copying the fragments back to ordinary registers before each MFMA
(v_accvgpr_read in front of every use).  This test compiles decode.hip and checks, for both weight
formats: no scratch and no spills; 36 MFMAs whose A operand is an accumulation register (the q/k/v
GEMV); the fc block's MFMAs present as well; and the whole kernel within one wave's 512 registers,
so one work-group of four waves fits each CU as the step requires."""
import re

import pytest

from asm_util import device_asm, functions

KERNEL = re.compile(r"^_ZN2g216k_decode_persistILb([01])EEEvNS_6PDArgsE$")


def metadata(asm, name):
    """The kernel's .vgpr_count, .agpr_count, .vgpr_spill_count and .private_segment_fixed_size, read
    from its entry of the listing's kernel metadata (entries start with '  - ', fields on either side
    of .name)."""
    m = re.search(r"\.name:\s+" + re.escape(name) + r"\s*\n", asm)
    assert m, name
    start = asm.rfind("\n  - ", 0, m.start())
    end = asm.find("\n  - ", m.end())
    entry = asm[start:end if end > 0 else len(asm)]
    out = {}
    for key in ("vgpr_count", "agpr_count", "vgpr_spill_count", "private_segment_fixed_size"):
        k = re.search(r"\." + key + r":\s+(\d+)", entry)
        out[key] = int(k.group(1)) if k else None
    return out


@pytest.fixture(scope="module")
def decode_asm():
    return device_asm("decode.hip")


def test_both_weight_formats_compiled(decode_asm):
    names = [n for n in functions(decode_asm) if KERNEL.match(n)]
    assert sorted(KERNEL.match(n).group(1) for n in names) == ["0", "1"], names


@pytest.mark.parametrize("q8", ["0", "1"])
def test_no_scratch_and_fragments_in_accumulation_registers(decode_asm, q8):
    name = f"_ZN2g216k_decode_persistILb{q8}EEEvNS_6PDArgsE"
    lines = functions(decode_asm)[name]
    md = metadata(decode_asm, name)
    assert md["private_segment_fixed_size"] == 0, md
    assert md["vgpr_spill_count"] == 0, md
    assert md["agpr_count"] is not None and md["agpr_count"] >= 144, md   # the 36 q/k/v fragments
    assert md["vgpr_count"] <= 512, md                                    # VGPRs + AGPRs of one wave
    mfma = [ln.strip() for ln in lines if ln.strip().startswith("v_mfma_f32_16x16x32_f16")]
    a_from_acc = [ln for ln in mfma if re.match(r"v_mfma_f32_16x16x32_f16\s+\S+,\s+a\[", ln)]
    assert len(a_from_acc) >= 36, (len(a_from_acc), mfma[:4])
    assert len(mfma) >= 36 + 6, len(mfma)                                 # q/k/v blocks + the fc block
