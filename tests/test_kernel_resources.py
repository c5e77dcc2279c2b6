"""CPU check of the hot MoE kernels' private (scratch) memory, from the
compiler's resource report for gfx950.

An index the compiler cannot resolve into the by-value MoeArgs kernel
argument makes it copy the whole struct to scratch in every thread (the
per-token kernels ran 4x slower that way); spills show up the same way.
The kernels listed here must use no scratch at all.
"""
import re
import subprocess
from pathlib import Path

import pytest

from logan_amd import build

CSRC = Path(build.CSRC)
HOT = {
    "moe.hip": [r"moe_gateup_kernelILi4ELi1E", r"moe_down_kernelILi4ELi16E", r"moe_route_tok_kernel",
                r"moe_group_kernel", r"moe_combine_kernel"],
    "moe_fused.hip": [r"moe_fused_b1_kernelILi4ELi1ELi16E"],
    "moe_mfma.hip": [r"moe_gateup_lds_kernel", r"moe_down_lds_kernel", r"moe_gateup_mfma_kernelILi4E",
                     r"moe_down_mfma_kernelILi4E", r"moe_mroute_kernel", r"moe_mgroup_kernel",
                     r"moe_mcombine_kernel"],
}


def _scratch_report(src: Path):
    cmd = [build.hipcc(), *build.HIPFLAGS, "-I", str(build.INCLUDE), "--cuda-device-only", "-c",
           str(src), "-o", "/dev/null", "-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out = {}
    name = None
    for line in r.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name:
            out[name] = int(m.group(1))
    return out


def test_hot_moe_kernels_use_no_scratch():
    try:
        build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    from concurrent.futures import ThreadPoolExecutor

    with ThreadPoolExecutor(len(HOT)) as ex:
        reps = dict(zip(sorted(HOT), ex.map(lambda s: _scratch_report(CSRC / s), sorted(HOT))))
    for src, pats in HOT.items():
        for pat in pats:
            hits = {k: v for k, v in reps[src].items() if re.search(pat, k)}
            assert hits, f"no kernel matches {pat} in {src}"
            bad = {k: v for k, v in hits.items() if v != 0}
            assert not bad, f"scratch in {src}: {bad}"
