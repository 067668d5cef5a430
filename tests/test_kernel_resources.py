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


def test_w8a8_prefill_kernel_fits_one_workgroup_per_cu(tmp_path):
    """The block-FP8 W8A8 prefill kernel (three LDS stages of tokens, weight
    strips and token scales): no spills, and its LDS within the 160 KiB of a
    gfx950 CU."""

    meta = kernel_metadata(CSRC / "linear.hip", tmp_path)
    prefill = {k: v for k, v in meta.items() if "w8a8_block_prefill_kernel" in k}
    assert len(prefill) == 2
    for name, m in prefill.items():
        assert m["vgpr_spill_count"] == 0, name
        assert m["sgpr_spill_count"] == 0, name
        assert m["group_segment_fixed_size"] <= 160 * 1024, name


def inflight_register_reads(asm: str, kernel: str) -> list[str]:
    """Instructions of `kernel` that read or overwrite a VGPR whose
    (non-LDS) inline-assembly load may still be in flight, in program order:
    vector memory operations complete in issue order and `s_waitcnt vmcnt(n)`
    leaves only the newest n outstanding.  The compiler's own loads (spill
    reloads included) count toward vmcnt but are not tracked as registers:
    the compiler waits for them itself on every path, whereas it knows nothing
    of the inline-assembly loads.  A read at the end of a loop body is seen
    with the loads the body left in flight, which is where a copy at the loop's
    back edge would sit."""

    start = asm.index(kernel + ":")
    body = asm[start:asm.index(".Lfunc_end", start)].split("\n")

    def regs(spec):
        spec = spec.strip()
        m = re.match(r"v\[(\d+):(\d+)\]", spec)
        if m:
            return set(range(int(m.group(1)), int(m.group(2)) + 1))
        m = re.match(r"v(\d+)$", spec)
        return {int(m.group(1))} if m else set()

    outstanding: list[set[int]] = []  # destination VGPRs of each vector memory op, in issue order
    bad = []
    inasm = False
    for line in body:
        raw = line.strip()
        if raw.startswith(";;#ASMSTART"):
            inasm = True
            continue
        if raw.startswith(";;#ASMEND"):
            inasm = False
            continue
        ins = line.split(";")[0].strip()
        if not ins or ins.startswith(".") or ins.endswith(":"):
            continue
        op = ins.split()[0]
        args = [a.strip() for a in ins[len(op):].split(",")]
        if op == "s_waitcnt" and "vmcnt" in ins:
            n = int(re.search(r"vmcnt\((\d+)\)", ins).group(1))
            outstanding = outstanding[len(outstanding) - n:] if n else []
            continue
        pending = set().union(*outstanding) if outstanding else set()
        touched = set().union(*(regs(a) for a in args)) if args else set()
        if op.startswith(("buffer_load", "global_load", "scratch_load")):
            if touched - regs(args[0]) & pending:
                bad.append(ins)
            outstanding.append(regs(args[0]) if inasm and not ins.endswith("lds") else set())
        elif op.startswith(("buffer_store", "global_store", "scratch_store", "buffer_atomic", "global_atomic")):
            if touched & pending:
                bad.append(ins)
            outstanding.append(set())
        elif op.startswith(("v_", "ds_")):
            if touched & pending:
                bad.append(ins)
    return bad


def test_mxfp4_prefill_reads_no_register_in_flight(tmp_path):
    """The MXFP4 prefill kernel's inline-asm weight loads land in registers
    that nothing may read (a copy, a spill) before its explicit wait."""

    from gaiban_lite_amd import build_ext

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / "mx.s"
    subprocess.run([hipcc, *build_ext.HIPCC_FLAGS, f"-I{ROOT / 'include'}", f"-I{CSRC}", "--cuda-device-only",
                    "-S", str(CSRC / "experts_mx.hip"), "-o", str(out)], check=True, capture_output=True)
    asm = out.read_text()
    names = re.findall(r"^(_Z\S*mx_prefill_kernel\S*):", asm, flags=re.M)
    assert len(names) == 2
    for name in names:
        assert inflight_register_reads(asm, name) == [], name


def loop_instructions(asm: str, kernel: str) -> list[str]:
    """The instructions of `kernel` inside loops: the blocks the compiler's
    listing marks as a loop header or as in a loop."""

    start = asm.index(kernel + ":")
    lines = asm[start:asm.index(".Lfunc_end", start)].split("\n")
    out, inloop = [], False
    for line in lines:
        s = line.strip()
        if s.startswith(".LBB") or s.startswith("; %bb."):
            inloop = "Loop" in s
            continue
        if inloop and s and not s.startswith((";", ".")):
            out.append(s)
    return out


def test_int4_prefill_kernel_register_weights(tmp_path):
    """The int4 (W4A16) prefill kernel keeps its next weight group in
    registers loaded by inline assembly as well, at three 256-thread
    workgroups per CU (at most 168 VGPRs, a third of the LDS): nothing reads
    those registers before the explicit wait (a spill of one would), and
    nothing inside the K loops touches scratch.  A few values that live
    across the loops (setup addresses) may be spilled outside them."""

    meta = kernel_metadata(CSRC / "experts.hip", tmp_path)
    prefill = {k: v for k, v in meta.items() if "expert_prefill_kernel" in k and "exact" not in k}
    assert len(prefill) == 2
    for name, m in prefill.items():
        assert m["vgpr_count"] <= 168, name
        assert m["sgpr_spill_count"] == 0, name
        assert m["group_segment_fixed_size"] <= 160 * 1024 // 3, name
    asm = _device_asm(CSRC / "experts.hip", tmp_path)
    for name in prefill:
        assert inflight_register_reads(asm, name) == [], name
        body = loop_instructions(asm, name)
        assert sum(1 for s in body if s.startswith("v_mfma")) >= 64, name
        assert [s for s in body if s.startswith("scratch_")] == [], name


def _device_asm(src: Path, tmp_path: Path) -> str:
    from gaiban_lite_amd import build_ext

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / (src.stem + ".s")
    subprocess.run([hipcc, *build_ext.HIPCC_FLAGS, f"-I{ROOT / 'include'}", f"-I{CSRC}", "--cuda-device-only",
                    "-S", str(src), "-o", str(out)], check=True, capture_output=True)
    return out.read_text()


def k_loop_bodies(asm: str, kernel: str) -> list[list[tuple[str, bool]]]:
    """The loops of `kernel` (loop header label to the last branch back to
    it) as (instruction, inside inline asm) pairs."""

    start = asm.index(kernel + ":")
    lines = asm[start:asm.index(".Lfunc_end", start)].split("\n")
    rows, inasm = [], False
    for line in lines:
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            inasm = True
        elif s.startswith(";;#ASMEND"):
            inasm = False
        rows.append((s, inasm))
    loops = []
    for i, (s, _) in enumerate(rows):
        if "Loop Header" not in s:
            continue
        label = s.split(":")[0]
        back = [k for k, (t, _) in enumerate(rows) if re.search(r"s_c?branch\w*\s+" + re.escape(label) + r"\b", t)]
        if back:
            loops.append(rows[i:max(back) + 1])
    return loops


def test_w8a8_gemm256_k_loop_is_one_block_with_only_its_own_copy_waits(tmp_path):
    """The 256-token block-FP8 kernel's K loop: no spills, LDS within a CU,
    no branch inside the loop body, and no vmcnt wait of the compiler's in
    it -- the copies' waits are inline asm, which the compiler does not
    count, so a wait of its own there (for a prologue load it still thinks
    outstanding) would also wait for the copies just issued and expose
    their whole latency every block; a branch lets the MFMAs of a block
    sink past that block's wait."""

    meta = kernel_metadata(CSRC / "linear.hip", tmp_path)
    gemm = {k: v for k, v in meta.items() if "w8a8_gemm256_kernel" in k}
    assert len(gemm) == 4  # 256 / 128 channels x tiled / row-major weights
    for name, m in gemm.items():
        assert m["vgpr_spill_count"] == 0, name
        assert m["group_segment_fixed_size"] <= 160 * 1024, name
    asm = _device_asm(CSRC / "linear.hip", tmp_path)
    for name in gemm:
        loops = k_loop_bodies(asm, name)
        dma_loops = [lp for lp in loops if any(a and "buffer_load" in s and " lds" in s for s, a in lp)]
        assert len(dma_loops) == 1, name
        body = dma_loops[0]
        assert sum(1 for s, _ in body if s.startswith("v_mfma")) > 0, name
        assert [s for s, a in body if not a and s.startswith("s_waitcnt") and "vmcnt" in s] == [], name
        branches = [s for s, _ in body if s.startswith(("s_cbranch", "s_branch"))]
        assert len(branches) == 1, (name, branches)  # the back edge only


def test_inflight_analysis_on_planted_code():
    """The in-flight check itself: a read of an inline-assembly load's
    destination before its wait is reported, the same read after
    `s_waitcnt vmcnt(0)` is not, and a compiler reload (waited for by the
    compiler) is not tracked; vmcnt(n) keeps only the newest n loads."""

    asm = "\n".join([
        "k:",
        "\t;;#ASMSTART",
        "\tbuffer_load_dwordx4 v[10:13], v2, s[4:7], s8 offen",
        "\t;;#ASMEND",
        "\tscratch_load_dword v5, off, off offset:8",
        "\tv_mov_b32_e32 v1, v5",
        "\tv_mov_b32_e32 v1, v11",
        "\ts_waitcnt vmcnt(1)",
        "\tv_mov_b32_e32 v1, v12",
        "\t;;#ASMSTART",
        "\tbuffer_load_dwordx4 v[20:23], v2, s[4:7], s8 offen",
        "\t;;#ASMEND",
        "\tglobal_load_dword v6, v[2:3], off",
        "\ts_waitcnt vmcnt(1)",
        "\tv_add_u32_e32 v1, v20, v1",
        "\ts_waitcnt vmcnt(0)",
        "\tv_add_u32_e32 v1, v21, v1",
        ".Lfunc_end0:",
    ])
    assert inflight_register_reads(asm, "k") == ["v_mov_b32_e32 v1, v11"]


def test_decode_kernels_keep_their_occupancy(tmp_path):
    """The persistent W4A16 decode kernels stream weights at a rate set by the
    resident workgroups: the deep-ring instances (RING 8) must fit three
    256-thread workgroups per CU (at most 168 VGPRs), the 4-deep ones four (at
    most 128), without scratch."""

    meta = kernel_metadata(CSRC / "experts.hip", tmp_path)
    dec = {k: v for k, v in meta.items() if "expert_decode_kernel" in k}
    assert len(dec) == 8
    for name, m in dec.items():
        ring = int(re.search(r"expert_decode_kernelILi\dELi(\d)E", name).group(1))
        assert m["vgpr_count"] <= {8: 168, 4: 128}[ring], (name, m["vgpr_count"])
        assert m["vgpr_spill_count"] == 0 and m["sgpr_spill_count"] == 0, name
