"""Resource checks of compiled kernels (CPU: hipcc cross-compiles for gfx950).

The MXFP4 prefill kernel keeps its next weight group in registers loaded by
inline assembly while the loads are in flight; a spill of those registers
would store them before they land, so the kernel must compile without VGPR
spills.  Its occupancy (three 256-thread workgroups per CU) also needs at
most 168 VGPRs and 32 KiB of LDS per workgroup.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "gaiban-lite_amd" / "csrc"


def kernel_metadata(src: Path, tmp_path: Path) -> dict[str, dict[str, int]]:
    from gaiban_lite_amd import build_ext

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / (src.stem + ".s")
    cmd = [hipcc, *build_ext.HIPCC_FLAGS, f"-I{ROOT / 'include'}", f"-I{CSRC}", "--cuda-device-only", "-S",
           str(src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    text = out.read_text()
    meta = {}
    for block in text.split("  - .agpr_count")[1:]:
        name = re.search(r"\.name:\s+(\S+)", block).group(1)
        fields = {k: int(v) for k, v in re.findall(r"\.(vgpr_count|vgpr_spill_count|sgpr_spill_count|"
                                                   r"group_segment_fixed_size):\s+(\d+)", block)}
        meta[name] = fields
    return meta


def test_mxfp4_prefill_kernel_has_no_spills_and_fits_three_workgroups(tmp_path):
    meta = kernel_metadata(CSRC / "experts_mx.hip", tmp_path)
    prefill = {k: v for k, v in meta.items() if "mx_prefill_kernel" in k}
    assert len(prefill) == 2
    for name, m in prefill.items():
        assert m["vgpr_spill_count"] == 0, name
        assert m["sgpr_spill_count"] == 0, name
        assert m["vgpr_count"] <= 168, (name, m["vgpr_count"])
        assert m["group_segment_fixed_size"] <= 32768, name
