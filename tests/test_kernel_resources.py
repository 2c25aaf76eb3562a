"""Compile-time checks of every product kernel for gfx950 (needs hipcc, no GPU):

* no kernel spills registers (scratch traffic), from hipcc's
  kernel-resource-usage remarks;
* no MFMA sits in an EXEC-masked region without a skip branch. gfx950 writes
  an MFMA's result even when EXEC is 0, so an MFMA that a divergent guard
  turns off but does not branch around still adds whatever its operand
  registers hold. (A decode kernel whose k bounds lived in vector registers
  had exactly this: the guarded third step of a two-step tail burst added
  address bits to the sums.)
* no kernel serializes its global loads: a load followed at once by a wait
  for every outstanding load, repeated, is what a load guarded one at a time
  next to its use compiles to (the quantizer's per-chunk loads were, one
  memory round trip per chunk);
* no kernel divides 64-bit integers by a run-time value: the expansion
  (~130 instructions, recognisable by its 2^32 and 2^-32 float constants)
  sat ahead of the first load of every workgroup in the decode and lockstep
  prefill kernels, whose K-split ranges were computed that way (1 us of a
  19 us decode GEMM, with the address arithmetic of its bursts); and every
  kernel issues its first global load within 450 instructions of its entry.
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


BRANCH = re.compile(r"^\s*(s_cbranch_\w+|s_branch)\s+(\S+)")
LABEL = re.compile(r"^(\.L\w+):")


def unguarded_mfmas(asm: str) -> dict[str, list[int]]:
    """Functions with an MFMA reached with EXEC narrowed by a divergent guard
    and neither restored nor checked by an s_cbranch_execz since: a scan of
    the listing that follows the branches (a branch taken in that state
    carries it to its label; an unconditional branch ends the fall-through),
    repeated until the labels' states settle. Per function, the lines of each
    such MFMA."""
    bad: dict[str, list[int]] = {}
    lines = asm.splitlines()
    starts = [i for i, line in enumerate(lines) if (m := FUNCTION_LABEL.match(line)) and not m.group(1).startswith(".L")]
    for s, e in zip(starts, starts[1:] + [len(lines)]):
        fn = FUNCTION_LABEL.match(lines[s]).group(1)
        entered: set[str] = set()  # labels some branch reaches with EXEC narrowed and unchecked
        while True:
            before = len(entered)
            found, state, falls = [], False, True
            for no in range(s + 1, e):
                line = lines[no]
                if m := LABEL.match(line):
                    state = (state and falls) or m.group(1) in entered
                    falls = True
                elif EXEC_RESTORE.match(line):
                    state = False
                elif EXEC_NARROW.match(line):
                    state = True
                elif re.match(r"^\s*s_cbranch_execz", line):
                    state = False
                elif m := BRANCH.match(line):
                    if state:
                        entered.add(m.group(2))
                    if m.group(1) == "s_branch":
                        state, falls = False, False
                elif re.match(r"^\s*(s_endpgm|s_setpc_b64)", line):
                    state, falls = False, False
                elif state and re.match(r"^\s*v_mfma", line):
                    found.append(no + 1)
            if len(entered) == before:
                break
        if found:
            bad[fn] = found
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
    # A narrowed block that branches away: the block laid out after it is
    # not reached in that state, the branch target is.
    listing = """kern:
\ts_and_saveexec_b64 s[4:5], s[16:17]
\ts_cbranch_scc1 .LBB0_9
\ts_branch .LBB0_8
.LBB0_7:
\tv_mfma_f32_16x16x128_f8f6f4 v[66:69], v[2:9], v[34:41], 0
.LBB0_8:
\ts_or_b64 exec, exec, s[4:5]
\ts_endpgm
.LBB0_9:
\tv_mfma_f32_16x16x128_f8f6f4 v[66:69], v[2:9], v[34:41], 0
\ts_branch .LBB0_7
"""
    assert unguarded_mfmas(listing) == {"kern": [6, 11]}


def serialized_loads(asm: str) -> dict[str, int]:
    """Per function, the global loads (not global -> LDS copies) whose next
    instruction waits for every outstanding vector-memory operation."""
    counts: dict[str, int] = {}
    fn = None
    lines = [line.strip() for line in asm.splitlines()]
    for no, line in enumerate(lines):
        if (m := FUNCTION_LABEL.match(line)) and not m.group(1).startswith(".L"):
            fn = m.group(1)
        elif line.startswith("global_load") and not line.startswith("global_load_lds"):
            nxt = next((u for u in lines[no + 1:no + 4] if u and not u.startswith(";")), "")
            if nxt.startswith("s_waitcnt") and "vmcnt(0)" in nxt:
                counts[fn] = counts.get(fn, 0) + 1
    return counts


def test_no_kernel_serializes_its_loads(device_builds):
    bad = {}
    for src, (_, asm) in device_builds.items():
        for fn, n in serialized_loads(asm).items():
            if n >= 3:
                bad[f"{src}:{fn[:80]}"] = n
    assert not bad, bad


def test_scan_finds_serialized_loads():
    listing = """kern:
\tglobal_load_dwordx4 v[2:5], v1, s[2:3]
\ts_waitcnt vmcnt(0)
\tv_pk_max_u16 v1, v1, v2
\tglobal_load_dwordx4 v[6:9], v1, s[2:3]
\tglobal_load_dwordx4 v[10:13], v1, s[2:3]
\ts_waitcnt vmcnt(1)
\tglobal_load_lds_dwordx4 v[2:3], off
\ts_waitcnt vmcnt(0)
"""
    assert serialized_loads(listing) == {"kern": 1}


def instructions_before_first_load(asm: str) -> dict[str, int]:
    """Per function, the instructions (labels, comments and directives not
    counted) ahead of its first global or buffer load; functions without one
    are left out."""
    counts: dict[str, int] = {}
    fn, n = None, 0
    for line in asm.splitlines():
        t = line.strip()
        if (m := FUNCTION_LABEL.match(t)) and not m.group(1).startswith(".L"):
            fn, n = m.group(1), 0
        elif fn is None or fn in counts or not t or t.startswith((";", ".")) or t.endswith(":"):
            continue
        elif t.startswith(("global_load", "buffer_load")):
            counts[fn] = n
        else:
            n += 1
    return counts


def test_every_kernel_loads_early(device_builds):
    late = {}
    for src, (_, asm) in device_builds.items():
        for fn, n in instructions_before_first_load(asm).items():
            if n > 450:
                late[f"{src}:{fn[:80]}"] = n
    assert not late, late


def test_scan_counts_instructions_before_the_first_load():
    listing = """kern:
\ts_load_dwordx4 s[4:7], s[0:1], 0x0
.LBB0_1:
\t; a comment
\ts_waitcnt lgkmcnt(0)
\tglobal_load_dwordx4 v[2:5], v1, s[2:3]
\tglobal_load_dwordx4 v[6:9], v1, s[2:3]
other:
\ts_endpgm
"""
    assert instructions_before_first_load(listing) == {"kern": 2}


DIV64_CONSTANTS = re.compile(r"0x4f800000|0x2f800000")


def divisions_64(asm: str) -> dict[str, int]:
    """Per function, the uses of 2^32 and 2^-32 as float constants: the
    float-reciprocal steps of a 64-bit integer division by a register."""
    counts: dict[str, int] = {}
    fn = None
    for line in asm.splitlines():
        if (m := FUNCTION_LABEL.match(line.strip())) and not m.group(1).startswith(".L"):
            fn = m.group(1)
        elif fn and DIV64_CONSTANTS.search(line):
            counts[fn] = counts.get(fn, 0) + 1
    return counts


def test_no_kernel_divides_64_bit_integers(device_builds):
    bad = {f"{src}:{fn[:80]}": n for src, (_, asm) in device_builds.items() for fn, n in divisions_64(asm).items()}
    assert not bad, bad


def test_scan_finds_a_64_bit_division():
    listing = """kern:
\tv_cvt_f32_u32_e32 v2, s5
\tv_madmk_f32 v2, v3, 0x4f800000, v2
\tv_rcp_f32_e32 v2, v2
\tv_mul_f32_e32 v3, 0x2f800000, v2
other:
\tv_rcp_iflag_f32_e32 v1, v1
\tv_mul_f32_e32 v1, 0x4f7ffffe, v1
"""
    assert divisions_64(listing) == {"kern": 2}
