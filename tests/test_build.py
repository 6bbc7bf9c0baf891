"""Compiler resource checks of the gfx950 kernels (no GPU needed: hipcc cross-compiles).

A kernel that spills registers reads them back from scratch memory, and such a
reload waits for every memory operation issued before it (vmcnt counts in
issue order), stores included: in a kernel that streams dS out, one reload in
the loop costs a full memory drain.  Every kernel must build without spills or
scratch, and the hot ones within the LDS and occupancy their tiling assumes.
"""
import os
import shutil

import pytest

from swvr_amd import build

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not build.os.path.exists("/opt/rocm/bin/hipcc"),
                                reason="hipcc not installed")


@pytest.fixture(scope="module")
def usage():
    return build.resource_report()


def test_no_kernel_spills_or_uses_scratch(usage):
    assert usage, "no kernel resource remarks parsed"
    bad = {k: v for k, v in usage.items() if v.get("vgpr_spill", 0) or v.get("sgpr_spill", 0) or v.get("scratch", 0)}
    assert not bad, bad


@pytest.mark.parametrize("kernel", ["fwd_tile_kernel<bf16,64,0>", "bwd_scores_ring_kernel<bf16,64,0>",
                                    "bwd_gemm_kernel<bf16>", "bwd_scores_wide_kernel<bf16>",
                                    "fwd_stream_kernel<bf16,256>"])
def test_hot_kernels_run_two_waves_per_simd_within_lds(usage, kernel):
    """The headline tiles are 8 waves of 512 threads: two waves per SIMD, one workgroup per CU."""
    u = usage[kernel]
    assert u["occupancy"] >= 2 and u["vgprs"] + u.get("agprs", 0) <= 256, u
    assert u["lds"] <= 160 * 1024, u


def test_inline_assembly_declares_the_scalar_condition_code():
    """A scalar ALU op (s_add_u32 on M0 in the LDS-DMA batches, ...) writes SCC; inline assembly
    that does so must list "scc" as clobbered, or the compiler may keep a comparison's result in
    SCC across the block and branch or select on the overwritten value.  (That happened: the
    stage cursor of a one-slice-per-stage reduction read a stale SCC and reloaded the previous
    vocabulary tile.)"""
    import re
    csrc = os.path.join(os.path.dirname(build.__file__), "csrc")
    writes_scc = re.compile(r"\bs_(add|sub|addc|subb|and|or|xor|andn2|orn2|lshl|lshr|ashr|min|max|bfe|cmp|not|abs)")
    checked = 0
    for name in sorted(os.listdir(csrc)):
        if not name.endswith((".hip", ".hpp")):
            continue
        text = open(os.path.join(csrc, name)).read()
        for m in re.finditer(r"asm\s+volatile\s*\((.*?)\);", text, re.S):
            body = m.group(1)
            code = " ".join(re.findall(r'"((?:[^"\\]|\\.)*)"', body.split(":")[0]))
            if writes_scc.search(code):
                checked += 1
                assert '"scc"' in body, f"{name}: inline assembly writes SCC without declaring it: {code[:80]}"
    assert checked >= 2
