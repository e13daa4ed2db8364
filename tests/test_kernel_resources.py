"""Resource checks on the built gfx950 code objects of libt5hip.so (no GPU needed).

Every kernel must run without scratch (private segment) memory.  A kernel that spills its
registers to scratch still computes the right results, so the GPU parity tests cannot catch
it, but it is slow: the f16-weight GEMM producers once spilled 272-720 bytes per lane and ran
at two thirds of their speed.  The kernel metadata of the code objects gives each kernel's
.private_segment_fixed_size; the check reads it with the ROCm LLVM tools.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SO = ROOT / "witchcraft_amd" / "libt5hip.so"
LLVM = Path("/opt/rocm/llvm/bin")


def _kernels(tmp_path):
    objdump, readelf = LLVM / "llvm-objdump", LLVM / "llvm-readelf"
    if not SO.exists():
        pytest.skip("libt5hip.so is not built")
    if not objdump.exists() or not readelf.exists():
        pytest.skip("ROCm LLVM tools are not installed")
    lib = tmp_path / SO.name
    shutil.copy(SO, lib)
    subprocess.run([str(objdump), "--offloading", str(lib)], cwd=tmp_path, check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    out = {}
    for co in sorted(tmp_path.glob(SO.name + ".*gfx950")):
        notes = subprocess.run([str(readelf), "--notes", str(co)], check=True, capture_output=True,
                               text=True).stdout
        name = None
        for line in notes.splitlines():
            m = re.match(r"^    \.name:\s+(\S+)", line)
            if m:
                name = m.group(1)
            m = re.match(r"^    \.private_segment_fixed_size:\s+(\d+)", line)
            if m and name is not None:
                out[name] = int(m.group(1))
                name = None
    return out


def test_no_kernel_uses_scratch(tmp_path):
    k = _kernels(tmp_path)
    assert len(k) > 100, f"only {len(k)} kernels found in the code objects"
    for want in ("gemm_kernel", "gemv_kernel", "attn_relbias_kernel", "rmsnorm_kernel",
                 "matmul_t_stream_kernel", "pk_rans_enc"):
        assert any(want in n for n in k), want
    spilled = {n: s for n, s in k.items() if s}
    assert not spilled, f"kernels using scratch memory (bytes per lane): {spilled}"
