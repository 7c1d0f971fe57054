"""Compiled-code check of the persistent kernels (work-groups that wait on each other): no loop may
narrow EXEC on its way back to its header (a lane-divergent latch) while a barrier lies inside it.

Why: such a loop lets some lanes of a wave cycle back to a barrier while the wave's other lanes wait
at the loop's exit for them.  The persistent prefill once compiled that way: with the ticket fetch and
the counter bumps under `threadIdx.x == 0`, lanes 1-63 of wave 0 (and waves 1-3) went from a task's
end straight back to the barrier before the next task word, re-reading the old one, while thread 0
waited -- the work-group re-ran its first task forever.  The kernels now branch only on wave-uniform
values around barriers; this test compiles them (hipcc -S, the flags of csrc/Makefile) and reads the
loop structure from the compiler's block comments.  CPU only: it needs hipcc, not a GPU."""
import re

import pytest

from asm_util import device_asm, functions


def blocks(lines):
    out, cur = [], None
    for i, line in enumerate(lines):
        m = re.match(r"^(\.LBB\d+_\d+|; %bb\.\d+):", line)
        if m:
            name = m.group(1) if m.group(1).startswith(".LBB") else f"bb@{i}"
            cur = {"name": name, "lines": []}
            out.append(cur)
        if cur is not None:
            cur["lines"].append(line)
    return out


def hazardous_loops(asm):
    """Loops (by header) with a lane-divergent latch and a barrier inside (nested loops included)."""
    bs = blocks(asm.splitlines())
    parent, inner = {}, {}
    for b in bs:
        head = "\n".join(b["lines"][:12])
        if re.search(r"This (?:Inner )?Loop Header: Depth=\d+", head):
            name = b["name"].lstrip(".").replace("LBB", "BB")
            parents = re.findall(r"Parent Loop (BB\d+_\d+) Depth=\d+", head)
            parent[name] = parents[-1] if parents else None
            inner[b["name"]] = name
        else:
            m = re.search(r"in Loop: Header=(BB\d+_\d+) Depth", head)
            inner[b["name"]] = m.group(1) if m else None

    def within(loop, target):
        while loop:
            if loop == target:
                return True
            loop = parent.get(loop)
        return False

    bad = []
    for loop in parent:
        label = "." + loop.replace("BB", "LBB")
        members = [k for k, b in enumerate(bs) if within(inner[b["name"]], loop)]
        barrier = any(x.strip().startswith("s_barrier") for k in members for x in bs[k]["lines"])
        divergent = False
        for k in members:
            body = "\n".join(bs[k]["lines"])
            jumps = re.search(r"^\s*s_c?branch\w* " + re.escape(label) + r"\s*$", body, re.M)
            falls = k + 1 < len(bs) and bs[k + 1]["name"] == label and not re.match(r"\s*s_branch ", bs[k]["lines"][-1])
            if (jumps or falls) and re.search(r"^\s*s_andn2_b64 exec, exec,", body, re.M):
                divergent = True
        if divergent and barrier:
            bad.append(loop)
    return bad


def test_scanner_flags_the_known_pattern():
    """The check itself: a loop whose latch narrows EXEC back to a header with a barrier is flagged,
    the same loop with a scalar latch is not."""
    def listing(latch):
        return "\n".join([
            ".LBB0_1:                                ; =>This Loop Header: Depth=1",
            "\ts_barrier",
            "\tds_read_b32 v2, v3",
            "; %bb.2:                                ;   in Loop: Header=BB0_1 Depth=1",
            latch,
            "\ts_cbranch_execnz .LBB0_1",
            "; %bb.3:",
            "\ts_endpgm",
        ])
    assert hazardous_loops(listing("\ts_andn2_b64 exec, exec, s[4:5]")) == ["BB0_1"]
    assert hazardous_loops(listing("\ts_and_b64 vcc, exec, s[4:5]")) == []


@pytest.mark.parametrize("src", ["prefill.hip", "decode.hip"])
def test_persistent_kernels_have_uniform_loops_around_barriers(src):
    asm = device_asm(src)
    assert "s_barrier" in asm and "Loop Header" in asm
    assert hazardous_loops(asm) == []


def test_persistent_prefill_counts_one_atomic_per_wave():
    """The persistent prefill's ticket fetch and counter bumps are made by all 64 lanes of wave 0 with
    the value 1 and read as multiples of 64 (a ticket is old / 64), so they are exact only if each
    wave's adds reach memory as ONE atomic of 64: interleaved single-lane adds of two work-groups
    could hand both the same ticket.  The compiler emits that single atomic (the active-lane count
    from s_bcnt1 added by one lane); this checks every atomic add of the kernel is in that form."""
    fns = {k: v for k, v in functions(device_asm("prefill.hip")).items() if "k_prefill_persist" in k}
    assert fns
    for name, lines in fns.items():
        sites = [i for i, x in enumerate(lines) if x.strip().startswith("global_atomic_add")]
        assert sites, name
        for i in sites:
            window = [x.strip() for x in lines[max(0, i - 5):i]]
            assert any(x.startswith("s_bcnt1_i32_b64") for x in window), f"{name}: per-lane atomic add at line {i}"
