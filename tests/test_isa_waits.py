"""Kernels that stage their activation rows in LDS by DMA wait for them by count: `s_waitcnt vmcnt(N)` after the
DMA loads and the weight and scale loads lets the N loads issued after the DMAs stay in flight, which is right only
if exactly N vector-memory loads follow the last DMA (loads complete in issue order). A compiler that merged, split
or moved those loads would make the kernel read LDS before its staging lands; this reads the built code object's
instructions (our own build) and checks the count."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HSACO = ROOT / "halo-flash_amd" / "_build" / "core.hsaco"
OBJDUMP = shutil.which("llvm-objdump", path="/opt/rocm/llvm/bin")


KERNELS = ["halo_gemv_q8a8s_l64_r1_b1", "halo_proj_q8q_l32_b1_t1", "halo_proj_q8q_l32_b4_t1", "halo_proj_q8q_l64_b4_t1",
           "halo_proj_q8q_l32_b8_t2", "halo_proj_q8q2_l32x64_b2", "halo_proj_q8q2_l32x64_b8", "halo_proj_q8q2_l64x64_b4"]


@pytest.fixture(scope="module")
def disasm():
    return subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", str(HSACO)], capture_output=True, text=True, check=True).stdout


@pytest.mark.skipif(not HSACO.exists() or OBJDUMP is None, reason="needs the built code object and llvm-objdump")
@pytest.mark.parametrize("kernel", KERNELS)
def test_staged_wait_count_matches_its_loads(disasm, kernel):
    """The one-token GEMV and the quantized-input projections stage their activation rows by DMA and wait for
    them by count while their weight loads stay in flight."""
    out = disasm
    m = re.search(r"<" + kernel + r">:\n(.*?)s_endpgm", out, re.S)
    assert m, "kernel not found in the code object"
    body = [ln.strip() for ln in m.group(1).splitlines()]
    last_dma = max(i for i, ln in enumerate(body) if ln.startswith("global_load_lds"))
    wait = next(i for i, ln in enumerate(body) if i > last_dma and ln.startswith("s_waitcnt") and "vmcnt(" in ln)
    n = int(re.search(r"vmcnt\((\d+)\)", body[wait]).group(1))
    loads = [ln for ln in body[last_dma + 1:wait] if re.match(r"(global|buffer)_load", ln)]
    assert len(loads) == n, f"{len(loads)} loads after the staging DMAs, wait allows {n} in flight"
    assert not any(ln.startswith("s_barrier") for ln in body[last_dma:wait]), "barrier before the staging wait"
