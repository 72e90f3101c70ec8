"""Checks of compiled code that the kernels' correctness depends on (CPU only: hipcc cross-compiles for gfx950).

The bf16 chunked-delta scan's loading waves keep their next chunk's register requests in flight across a barrier:
before it they wait with an explicit `s_waitcnt vmcnt(N)`, which is right only if exactly N loads were issued after
the wave's last direct-to-LDS load (gfx950 counts loads in one in-order counter). A different count would let a
stage be read before its direct loads land (N too large) or wait for the requests (N too small)."""
import importlib.util
import re
import shutil
import subprocess
from pathlib import Path

import pytest

NATIVE = Path(__file__).resolve().parents[1] / "metal-inference-engine_amd" / "native"
HIPCC = "/opt/rocm/bin/hipcc"
_spec = importlib.util.spec_from_file_location("rk_build", NATIVE / "build.py")
build = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(build)


@pytest.mark.skipif(shutil.which(HIPCC) is None, reason="hipcc not installed")
def test_loader_waits_count_its_register_requests(tmp_path):
    asm = tmp_path / "cols.s"
    cmd = [HIPCC, "-x", "hip", "-S", "--offload-device-only", str(NATIVE / "chunked_delta_cols.hip"), "-o", str(asm)]
    cmd += build.FLAGS + build.SOURCE_FLAGS.get("chunked_delta_cols.hip", [])
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln.strip() for ln in asm.read_text().splitlines()]
    checked = 0
    for i, ln in enumerate(lines):
        m = re.match(r"s_waitcnt vmcnt\((\d+)\) lgkmcnt\(0\)$", ln)
        if not m or i + 1 >= len(lines) or lines[i + 1] != "s_barrier":
            continue
        n, j = 0, i
        while j > 0:
            j -= 1
            if lines[j].startswith("global_load_lds") or lines[j] == "s_barrier":
                break
            if lines[j].startswith("global_load"):
                n += 1
        assert lines[j].startswith("global_load_lds"), f"no direct load before the wait at line {i}"
        assert n == int(m.group(1)), f"wait at line {i}: vmcnt({m.group(1)}) but {n} loads after the last direct load"
        checked += 1
    assert checked == 4, f"expected the 4 loader waits (2 waves x prologue / loop), found {checked}"
