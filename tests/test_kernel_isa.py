"""Static checks of the fused attention kernel's gfx950 code (CPU only: hipcc
cross-compiles it to assembly).

The K/V tiles are copied into LDS by ``buffer_load_dwordx4 ... lds`` and their
completion is awaited with an explicit ``s_waitcnt vmcnt(N)`` before the
barrier that publishes them, where N counts the buffer loads the wavefront
issues after the copies (vector-memory operations complete in issue order).  If
the compiler issued fewer loads there (moved one before the copies, or merged
two), the wait would let the barrier pass before the copies land.  This test
walks every kernel with direct copies: from each copy to the next explicit wait
(following the loop back-edge when the copy sits in the key loop) it counts the
vector-memory instructions and requires at least N of them.
"""

from __future__ import annotations

import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
CSRC = REPO / "disentangled-flash_amd" / "csrc"

VMEM = re.compile(r"^\s+(buffer|global|scratch)_(load|store|atomic)\w*\s")
COPY = re.compile(r"^\s+buffer_load_dwordx4\s.*\blds\b")
EXPLICIT_WAIT = re.compile(r"^\s+s_waitcnt vmcnt\((\d+)\)\s*$")


@pytest.fixture(scope="module")
def attention_asm(tmp_path_factory):
    sys.path.insert(0, str(CSRC))
    import build  # noqa: E402

    if shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "rel_attention.s"
    cmd = [build.hipcc(), *build.COMMON_FLAGS, "-I", str(CSRC), "--offload-device-only", "-S",
           str(CSRC / "rel_attention.hip"), "-o", str(out)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    assert result.returncode == 0, result.stderr[-2000:]
    return out.read_text()


def _kernels(asm: str):
    """(name, lines) of every rel_attention_kernel body."""
    names = re.findall(r"^(_ZN6dflash20rel_attention_kernel\w+):", asm, re.M)
    for name in names:
        start = asm.index(f"\n{name}:") + 1
        end = asm.index("s_endpgm", start)
        yield name, asm[start:end].splitlines()


def _explicit_waits(lines):
    """Indices of the vmcnt waits written as inline assembly (between ASMSTART/ASMEND)."""
    waits = {}
    inside = False
    for i, line in enumerate(lines):
        if ";;#ASMSTART" in line:
            inside = True
        elif ";;#ASMEND" in line:
            inside = False
        elif inside:
            m = EXPLICIT_WAIT.match(line)
            if m:
                waits[i] = int(m.group(1))
    return waits


def _loops(lines):
    """(header, back-edge) index pairs of the loops, from the compiler's loop comments."""
    loops = []
    for i, line in enumerate(lines):
        if "Loop Header" in line:
            label = line.split(":")[0].strip()
            back = max(j for j, other in enumerate(lines)
                       if re.search(rf"\bs_(c?)branch\w*\s+{re.escape(label)}\s*$", other))
            loops.append((i, back))
    return loops


def test_direct_copy_waits_cover_the_copies(attention_asm):
    checked = 0
    for name, lines in _kernels(attention_asm):
        copies = [i for i, line in enumerate(lines) if COPY.match(line)]
        if not copies:
            continue
        waits = _explicit_waits(lines)
        loops = _loops(lines)
        # Check after the last copy of each group (consecutive copies with no
        # other vector-memory instruction between them).
        groups = []
        for i in copies:
            if groups and not any(VMEM.match(lines[j]) and not COPY.match(lines[j])
                                  for j in range(groups[-1] + 1, i)):
                groups[-1] = i
            else:
                groups.append(i)
        for last in groups:
            path = list(range(last + 1, len(lines)))
            inner = [(h, e) for h, e in loops if h < last < e]
            if inner:
                h, e = min(inner, key=lambda he: he[1] - he[0])
                path = list(range(last + 1, e + 1)) + list(range(h, e + 1))
            count = 0
            for j in path:
                if j in waits:
                    assert count >= waits[j], (
                        f"{name}: {count} vector-memory instructions between the copies at line "
                        f"{last} and the wait vmcnt({waits[j]}) at line {j}")
                    checked += 1
                    break
                if VMEM.match(lines[j]) and not COPY.match(lines[j]):
                    count += 1
    assert checked > 0, "no kernel with direct copies was found"
