"""The prefill kernels read their K fragments from LDS straight into AGPRs
with inline asm (`ds_read_b128 a[...]`) and wait for each one
(`s_waitcnt lgkmcnt(n)`) right before the MFMA that consumes it. The
compiler sees the asm outputs as ready when the asm block ends, so nothing it
schedules in between may touch those registers: no copy, move or spill of a
fragment before its wait. This test compiles both prefill sources with the
library's own flags and scans the gfx950 assembly: LDS operations complete
in issue order, so a fragment is ready once an `lgkmcnt` wait leaves fewer
LDS operations outstanding than were issued after it. Any instruction that
names a fragment AGPR before that point fails the test, as does any scratch
use or spill in these kernels. The scanner itself is checked on hand-written
sequences."""
import re
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO / "gemma.c_amd"))
from gemma_kv import build as kb  # noqa: E402

LDS_OP = re.compile(r"^\s*(ds_\w+|s_load\w*|s_buffer_load\w*)\b")
AGPR_LOAD = re.compile(r"^\s*ds_read\w*\s+(a\[(\d+):(\d+)\]|a(\d+))\s*,")
WAIT = re.compile(r"^\s*s_waitcnt\b(.*)$")
AGPR_REF = re.compile(r"\ba\[(\d+):(\d+)\]|\ba(\d+)\b")


def scan(lines):
    """Returns (line number, instruction) of every fragment register use
    before its LDS read is known complete."""
    queue = []    # outstanding LDS ops, oldest first: set of AGPRs each writes
    pending = {}  # AGPR -> the queue entry (a set) that writes it
    bad = []
    for no, raw in enumerate(lines, 1):
        line = raw.split(";")[0].rstrip()
        if not line.strip() or line.lstrip().startswith((".", "_")) or line.endswith(":"):
            if line.strip() == "s_endpgm":
                queue.clear()
                pending.clear()
            continue
        w = WAIT.match(line)
        if w:
            m = re.search(r"lgkmcnt\((\d+)\)", w.group(1))
            if m:
                keep = int(m.group(1))
                while len(queue) > keep:
                    done = queue.pop(0)
                    for reg in done:
                        pending.pop(reg, None)
            continue
        mnemonic = line.split()[0]
        load = AGPR_LOAD.match(line)
        operands = line[len(line) - len(line.lstrip()) + len(mnemonic):]
        for ref in AGPR_REF.finditer(operands if not load else operands.split(",", 1)[1]):
            lo = int(ref.group(1) if ref.group(1) is not None else ref.group(3))
            hi = int(ref.group(2) if ref.group(2) is not None else ref.group(3))
            if any(r in pending for r in range(lo, hi + 1)):
                bad.append((no, line.strip()))
                break
        if LDS_OP.match(line):
            writes = set()
            if load:
                lo = int(load.group(2) if load.group(2) is not None else load.group(4))
                hi = int(load.group(3) if load.group(3) is not None else load.group(4))
                writes = set(range(lo, hi + 1))
                for r in writes:
                    if r in pending:  # a second read into a register still in flight
                        bad.append((no, line.strip()))
            queue.append(writes)
            for r in writes:
                pending[r] = writes
        if mnemonic == "s_endpgm":
            queue.clear()
            pending.clear()
    return bad


def test_scanner_on_hand_written_sequences():
    ok = """
    ds_read_b128 a[64:67], v1
    ds_read_b128 a[68:71], v1 offset:16
    s_waitcnt lgkmcnt(1)
    v_mfma_f32_32x32x16_bf16 v[0:15], a[64:67], v[20:23], v[0:15]
    s_waitcnt lgkmcnt(0)
    v_mfma_f32_32x32x16_bf16 v[0:15], a[68:71], v[24:27], v[0:15]
    """.splitlines()
    assert scan(ok) == []
    early = """
    ds_read_b128 a[64:67], v1
    ds_read_b128 a[68:71], v1 offset:16
    s_waitcnt lgkmcnt(1)
    v_mfma_f32_32x32x16_bf16 v[0:15], a[68:71], v[24:27], v[0:15]
    """.splitlines()
    assert len(scan(early)) == 1          # the second read is not complete yet
    copy = """
    ds_read_b128 a[64:67], v1
    v_accvgpr_read_b32 v5, a65
    s_waitcnt lgkmcnt(0)
    """.splitlines()
    assert len(scan(copy)) == 1
    later_lds = """
    ds_read_b128 a[64:67], v1
    ds_write_b32 v2, v3
    s_waitcnt lgkmcnt(1)
    v_mfma_f32_32x32x16_bf16 v[0:15], a[64:67], v[20:23], v[0:15]
    """.splitlines()
    assert scan(later_lds) == []           # the later LDS write may still be in flight


@pytest.mark.parametrize("stem", ["prefill_attention", "prefill_norm_rope"])
def test_fragment_agprs_untouched_until_waited(stem, tmp_path):
    src = kb.CSRC_DIR / f"{stem}.hip"
    out = tmp_path / f"{stem}.s"
    cmd = [kb.HIPCC, *kb.HIP_FLAGS, *kb.EXTRA_FLAGS.get(stem, []), "--cuda-device-only", "-S",
           str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    text = out.read_text()
    lines = text.splitlines()
    assert any(AGPR_LOAD.match(l) for l in lines), "no fragment reads into AGPRs found"
    bad = scan(lines)
    assert bad == [], f"fragment AGPRs used before their LDS reads completed: {bad[:5]}"
    # No scratch: nothing of these kernels is spilled or kept in private memory.
    for m in re.finditer(r"\.private_segment_fixed_size:\s*(\d+)", text):
        assert int(m.group(1)) == 0
    for m in re.finditer(r"\.vgpr_spill_count:\s*(\d+)", text):
        assert int(m.group(1)) == 0
