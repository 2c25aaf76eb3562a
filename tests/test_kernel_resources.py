"""Compile-time checks of every product kernel for gfx950 (needs hipcc, no GPU):

* no kernel spills registers (scratch traffic), from hipcc's
  kernel-resource-usage remarks;
* no MFMA sits in an EXEC-masked region without a skip branch. gfx950 writes
  an MFMA's result even when EXEC is 0, so an MFMA that a divergent guard
  turns off but does not branch around still adds whatever its operand
  registers hold. (A decode kernel whose k bounds lived in vector registers
  had exactly this: the guarded third step of a two-step tail burst added
  address bits to the sums.)
"""

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

# Instructions that narrow EXEC to the lanes of a divergent branch, and the
# ones that restore it at the join.
EXEC_NARROW = re.compile(r"^\s*(s_and_saveexec_b64|s_andn2_saveexec_b64|s_or_saveexec_b64|s_andn1_saveexec_b64|"
                         r"s_(and|andn2|xor|mov|cselect)_b64\s+exec,)")
EXEC_RESTORE = re.compile(r"^\s*(s_or_b64\s+exec,\s*exec,|s_mov_b64\s+exec,\s*-1)")
FUNCTION_LABEL = re.compile(r"^([A-Za-z_][\w$]*):")


def compile_device(source: Path, out_dir: Path) -> tuple[str, str]:
    """(remarks, gfx950 assembly) of one source."""
    asm = out_dir / (source.stem + ".s")
    cmd = [build.hipcc(), *build.HIPCC_FLAGS, f"-I{build.CSRC}", f"-I{build.ROOT / 'include'}", "--cuda-device-only", "-S",
           str(source), "-o", str(asm), "-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return r.stderr, asm.read_text()


def unguarded_mfmas(asm: str) -> dict[str, list[int]]:
    """Functions with an MFMA after an EXEC-narrowing instruction and before
    both the matching restore and any s_cbranch_execz (a linear scan of the
    listing: per function, the lines of each such MFMA)."""
    bad: dict[str, list[int]] = {}
    fn, narrowed, guarded = None, False, False
    for no, line in enumerate(asm.splitlines(), 1):
        m = FUNCTION_LABEL.match(line)
        if m and not m.group(1).startswith(".L"):
            fn, narrowed, guarded = m.group(1), False, False
        elif EXEC_RESTORE.match(line):
            narrowed = guarded = False
        elif EXEC_NARROW.match(line):
            narrowed, guarded = True, False
        elif re.match(r"^\s*s_cbranch_execz", line):
            guarded = True
        elif narrowed and not guarded and re.match(r"^\s*v_mfma", line):
            bad.setdefault(fn, []).append(no)
    return bad


@pytest.fixture(scope="module")
def device_builds(tmp_path_factory) -> dict[str, tuple[str, str]]:
    out = tmp_path_factory.mktemp("asm")
    sources = sorted(build.CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=len(sources)) as pool:
        return dict(zip((s.name for s in sources), pool.map(lambda s: compile_device(s, out), sources)))


def test_no_kernel_spills_registers(device_builds):
    kernels = []
    for remarks, _ in device_builds.values():
        names = re.findall(r"remark: Function Name: (\S+)", remarks)
        scratch = [int(v) for v in re.findall(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", remarks)]
        assert len(names) == len(scratch)
        kernels += zip(names, scratch)
    assert len(kernels) > 100  # every template instance the dispatchers can launch
    spilling = [(name, size) for name, size in kernels if size]
    assert not spilling, spilling


def test_no_mfma_runs_under_a_masked_exec(device_builds):
    assert sum(len(re.findall(r"^\s*v_mfma", asm, re.M)) for _, asm in device_builds.values()) > 1000
    bad = {src: unguarded_mfmas(asm) for src, (_, asm) in device_builds.items()}
    bad = {src: fns for src, fns in bad.items() if fns}
    assert not bad, {src: sorted(fns)[:4] for src, fns in bad.items()}


def test_scan_finds_a_masked_mfma():
    """The scan on a hand-written listing: a guarded tail step's MFMA after
    s_and_saveexec with no skip branch is found; the same with s_cbranch_execz,
    or after the join, is not."""
    listing = """kern:
\ts_and_saveexec_b64 s[12:13], vcc
\tv_mfma_f32_16x16x128_f8f6f4 v[50:53], v[2:9], v[26:33], v[50:53]
\ts_or_b64 exec, exec, s[12:13]
ok:
\ts_and_saveexec_b64 s[12:13], vcc
\ts_cbranch_execz .LBB0_2
\tv_mfma_f32_16x16x128_f8f6f4 v[50:53], v[2:9], v[26:33], v[50:53]
\ts_or_b64 exec, exec, s[12:13]
\tv_mfma_f32_16x16x128_f8f6f4 v[50:53], v[2:9], v[26:33], v[50:53]
"""
    assert unguarded_mfmas(listing) == {"kern": [3]}
