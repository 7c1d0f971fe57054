"""Compiled-code check of the LDS-ring GEMMs: inside a k-loop, no wait for vector memory may sit in
front of a fragment read from LDS.

The k-loops fill their LDS ring with global_load_lds (loads that write LDS directly) and order those
writes themselves: an explicit `s_waitcnt vmcnt(n)` for the k-tiles about to be read, then a barrier.
The compiler adds a wait of its own ahead of any LDS read that it cannot prove disjoint from an LDS
load still in flight.  In the k-loop that wait covers the k-tiles just issued for later iterations,
so the loop stops overlapping loads with MFMAs: every iteration waits for its own prefetch.  The INT8
forms of k_gemm_dl compiled that way (two `s_waitcnt vmcnt(0)` per iteration, each right before a
`ds_read2st64_b64` or `ds_read_b128`), and so did the persistent prefill's INT8 tiles.  Moving the
kernel body into a device function whose pointer parameters are `__restrict__` gave the LDS reads
the alias scopes the compiler needs, and removing those waits made the INT8 trunk GEMMs ~10% faster
at P=512.  This test keeps it that way: it compiles the sources (hipcc -S, csrc/Makefile's flags) and
flags a vmcnt wait directly ahead of a 64- or 128-bit LDS read in a loop.  Waits ahead of 32-bit LDS
reads (the persistent kernel's task words, read after a barrier) are not k-loop fragment reads."""
import re

import pytest

from asm_util import device_asm, functions

FRAG_READ = re.compile(r"^ds_read(2st64)?_b(64|128)\b|^ds_read2(st64)?_b(32|64)\b")


def dma_alias_waits(lines):
    """Number of vmcnt waits directly ahead of a fragment-sized LDS read inside a loop."""
    n, in_loop = 0, False
    for i, line in enumerate(lines):
        if re.match(r"^(\.LBB\S+:|; %bb\.\d+:)", line):
            in_loop = "Loop" in line
        t = line.strip()
        if in_loop and t.startswith("s_waitcnt") and "vmcnt" in t and i + 1 < len(lines) \
                and FRAG_READ.match(lines[i + 1].strip()):
            n += 1
    return n


def test_scanner_flags_the_pattern():
    """The check itself: a vmcnt wait right before a 128-bit LDS read in a loop body is counted; the
    pipeline's own wait (before the barrier), a wait before a 32-bit read and a wait outside any loop
    are not."""
    head = ".LBB0_1:                                ; =>This Inner Loop Header: Depth=1"
    body = "; %bb.2:                                ;   in Loop: Header=BB0_1 Depth=1"
    own = [head, "\ts_waitcnt vmcnt(2)", "\t;;#ASMSTART", "\ts_waitcnt lgkmcnt(0)", "\ts_barrier", "\t;;#ASMEND",
           "\tglobal_load_lds_dwordx4 v[0:1], off"]
    assert dma_alias_waits(own + [body, "\tds_read_b128 v[4:7], v2"]) == 0
    assert dma_alias_waits(own + [body, "\ts_waitcnt vmcnt(0)", "\tds_read_b128 v[4:7], v2"]) == 1
    assert dma_alias_waits(own + [body, "\ts_waitcnt vmcnt(0)", "\tds_read2st64_b64 v[4:7], v2 offset1:8"]) == 1
    assert dma_alias_waits(own + [body, "\ts_waitcnt vmcnt(1)", "\tds_read_b32 v4, v2"]) == 0
    assert dma_alias_waits(["; %bb.0:", "\ts_waitcnt vmcnt(0)", "\tds_read_b128 v[4:7], v2"]) == 0


@pytest.mark.parametrize("src,kernel", [("gemm.hip", "k_gemm_dl"), ("prefill.hip", "k_prefill_persist")])
def test_lds_ring_loops_have_no_dma_alias_waits(src, kernel):
    fns = {k: v for k, v in functions(device_asm(src)).items()
           if kernel in k and any("global_load_lds" in x for x in v)}
    assert fns, f"no {kernel} kernel with global_load_lds in {src}"
    bad = {k: n for k, n in ((k, dma_alias_waits(v)) for k, v in fns.items()) if n}
    assert not bad, f"{len(bad)} of {len(fns)} kernels wait on their own prefetch: {sorted(bad)[:4]}"
