"""Every product kernel compiles for gfx950 without register spills (scratch
traffic). The resource report comes from hipcc's kernel-resource-usage remarks;
needs hipcc, no GPU."""

from __future__ import annotations

import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from jeeves_amd import build

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                                reason="needs hipcc")


def resource_report(source: Path, out: Path) -> list[tuple[str, int]]:
    cmd = [build.hipcc(), *build.HIPCC_FLAGS, f"-I{build.CSRC}", f"-I{build.ROOT / 'include'}", "-c", str(source),
           "-o", str(out), "-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    names = re.findall(r"remark: Function Name: (\S+)", r.stderr)
    scratch = [int(v) for v in re.findall(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", r.stderr)]
    assert len(names) == len(scratch)
    return list(zip(names, scratch))


def test_no_kernel_spills_registers(tmp_path):
    sources = sorted(build.CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=len(sources)) as pool:
        reports = list(pool.map(lambda s: resource_report(s, tmp_path / (s.stem + ".o")), sources))
    kernels = [k for rep in reports for k in rep]
    assert len(kernels) > 100  # every template instance the dispatchers can launch
    spilling = [(name, size) for name, size in kernels if size]
    assert not spilling, spilling
