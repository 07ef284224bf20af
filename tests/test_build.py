"""Every HIP kernel of the library compiles for gfx950 without register spills.

A kernel that spills runs out of scratch memory at a fraction of its speed
(an append fused into the decode attention once doubled its time that way),
and nothing in a parity test notices.  This compiles each translation unit
with the same flags as the library build plus the compiler's per-kernel
resource report, and fails on any kernel with spilled VGPRs or scratch use.
"""
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from aegaeon_amd.csrc import build

HIP_SOURCES = [s for s in build.SOURCES if s.endswith(".hip")]


def _report(src: str, out_dir: Path) -> str:
    cmd = [build._hipcc(), *build.COMMON_FLAGS, "-c", str(build.CSRC / src), "-o",
           str(out_dir / (Path(src).stem + ".o")), "-Rpass-analysis=kernel-resource-usage"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, f"{src} does not compile:\n{res.stderr[-4000:]}"
    return res.stderr


def _kernels(report: str):
    """(kernel name, {field: value}) per kernel of the resource report."""
    for block in report.split("Function Name: ")[1:]:
        name = block.split()[0]
        fields = {k: int(v) for k, v in re.findall(r"remark:\s+([A-Za-z ]+?)(?: \[[^\]]*\])?: (\d+)", block)}
        yield name, fields


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc is not installed")
def test_no_kernel_spills(tmp_path):
    with ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as ex:
        reports = dict(zip(HIP_SOURCES, ex.map(lambda s: _report(s, tmp_path), HIP_SOURCES)))
    seen, bad = 0, []
    for src, rep in reports.items():
        for name, f in _kernels(rep):
            seen += 1
            if f.get("VGPRs Spill", 0) or f.get("ScratchSize", 0):
                bad.append(f"{src}: {name}: {f.get('VGPRs Spill', 0)} VGPRs spilled, "
                           f"{f.get('ScratchSize', 0)} B/lane scratch")
    assert seen >= 20, f"only {seen} kernels found in the resource reports"
    assert not bad, "\n".join(bad)
