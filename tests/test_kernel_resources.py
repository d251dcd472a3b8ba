"""Static checks of the gfx950 code the library is built from (CPU only).

The streaming kernels wait for their buffer->LDS ring loads by counting
outstanding vector-memory operations (s_waitcnt vmcnt(N) with N fixed).  A
register spill adds scratch loads and stores to that count, and on gfx9 a
store can retire out of order with the loads, so such a kernel could read a
ring slot before its data arrived.  These tests compile the sources that
hold ring kernels to gfx950 assembly and require that every kernel using
buffer->LDS loads has no scratch (private segment) and fits its occupancy.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from gollek_amd import build

RING_SOURCES = ["gguf_gemm.hip", "gguf_gemm_tile.hip", "gguf_gemv_mfma.hip", "gguf_gemv_q6k_mfma.hip",
                "gguf_gemv_ring.hip", "gguf_moe_mfma.hip"]


def _assembly(src: str, tmp_path: Path) -> str:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / (src + ".s")
    flags = [f for f in build.compile_flags() if f != "-fPIC"]
    cmd = [hipcc, *flags, "-S", "--cuda-device-only", str(build.CSRC_DIR / src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def _kernels(asm: str):
    """(name, body, scratch bytes) per kernel of an assembly listing."""
    for m in re.finditer(r"^(_Z\w+):\s*;.*?$(.*?)^\.Lfunc_end\d+:", asm, re.M | re.S):
        name, body = m.group(1), m.group(2)
        tail = asm[m.end():m.end() + 4000]
        sm = re.search(r"; ScratchSize: (\d+)", tail)
        yield name, body, int(sm.group(1)) if sm else None


@pytest.mark.parametrize("src", RING_SOURCES)
def test_ring_kernels_do_not_spill(src, tmp_path):
    asm = _assembly(src, tmp_path)
    ring = [(n, s) for n, b, s in _kernels(asm) if re.search(r"buffer_load_dword\w*\s.*\blds\b", b)]
    assert ring, f"no buffer->LDS kernels found in {src}"
    bad = [n for n, s in ring if s != 0]
    assert not bad, f"kernels with scratch in {src}: {bad}"
