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


_LABEL = re.compile(r"^(\.LBB\d+_\d+):")
_BB = re.compile(r"^; %bb\.\d+:")


def mfmas_under_lane_mask(lines: list[str]) -> list[tuple[str, str]]:
    """MFMAs of one kernel's listing that can execute while EXEC holds only
    some lanes: a forward walk over the basic blocks (labels, fall-through and
    branch edges) that tracks the open `if` regions -- `s_and_saveexec_b64
    s[k]` (or `s_mov_b64 s[k], exec` then `s_mov_b64 exec, ...`) opens one
    keyed by the saved mask, `s_xor_b64 s[j], exec, s[k]` renames it (an
    if/else), `s_or_b64 exec, exec, s[k]` closes it.  Returns (block, MFMA)
    pairs reached with a region open."""

    blocks, cur = [], ["entry", []]
    for line in lines:
        s = line.strip()
        m = _LABEL.match(s)
        if m or _BB.match(s):
            blocks.append(cur)
            cur = [m.group(1) if m else s, []]
            continue
        if s and not s.startswith((";", ".")):
            cur[1].append(s)
    blocks.append(cur)
    index = {name: i for i, (name, _) in enumerate(blocks)}
    states, work, visits, bad = {0: ()}, [0], {}, set()
    while work:
        i = work.pop()
        open_, saved, succ, ends = list(states[i]), None, [], False
        for s in blocks[i][1]:
            t = s.replace(",", " ").split()
            op = t[0]
            if op == "s_and_saveexec_b64":
                open_.append(t[1])
            elif op == "s_xor_b64" and len(t) > 3 and t[2] == "exec" and open_ and open_[-1] == t[3]:
                open_[-1] = t[1]
            elif op == "s_mov_b64" and len(t) > 2 and t[2] == "exec":
                saved = t[1]
            elif op == "s_mov_b64" and t[1] == "exec":
                open_.append(saved or "?")
            elif op == "s_or_b64" and t[1] == "exec":
                key = t[3] if t[2] == "exec" else t[2]
                if key in open_:
                    while open_[-1] != key:
                        open_.pop()
                    open_.pop()
            elif op.startswith("v_mfma") and open_:
                bad.add((blocks[i][0], s))
            elif op.startswith("s_cbranch"):
                succ.append(t[1])
            elif op == "s_branch":
                succ.append(t[1])
                ends = True
            elif op == "s_endpgm":
                ends = True
        if not ends and i + 1 < len(blocks):
            succ.append(blocks[i + 1][0])
        for name in succ:
            j = index.get(name)
            if j is None:
                continue
            new = tuple(open_)
            if j in states and (states[j] == new or len(new) <= len(states[j])):
                continue
            states[j] = new
            visits[j] = visits.get(j, 0) + 1
            if visits[j] < 20:
                work.append(j)
    return sorted(bad)


def test_lane_mask_analysis_on_planted_code():
    """The EXEC-region walk itself: an MFMA inside `if` (saveexec ... or
    exec) is reported, one after the join is not, an if/else renamed by
    s_xor_b64 closes at its own join, and a region closed on a branch path
    laid out earlier (a loop latch) does not leak into later blocks."""

    inside = ["k:", "\tv_cmp_gt_i32_e32 vcc, s4, v0", "\ts_and_saveexec_b64 s[2:3], vcc",
              "\ts_cbranch_execz .LBB0_2", "; %bb.1:", "\tv_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]",
              ".LBB0_2:", "\ts_or_b64 exec, exec, s[2:3]", "\ts_endpgm"]
    assert [m for _, m in mfmas_under_lane_mask(inside)] == ["v_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]"]
    after = inside[:5] + ["\tv_mov_b32_e32 v1, 0"] + inside[6:8] + \
        ["\tv_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]", "\ts_endpgm"]
    assert mfmas_under_lane_mask(after) == []
    if_else = ["k:", "\ts_and_saveexec_b64 s[4:5], vcc", "\ts_xor_b64 s[6:7], exec, s[4:5]",
               "\ts_cbranch_execz .LBB0_2", "; %bb.1:", "\tv_mov_b32_e32 v1, 0", ".LBB0_2:",
               "\ts_andn2_saveexec_b64 s[6:7], s[6:7]", "\tv_mov_b32_e32 v1, 1",
               "\ts_or_b64 exec, exec, s[6:7]", "\tv_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]",
               "\ts_endpgm"]
    assert mfmas_under_lane_mask(if_else) == []
    latch = ["k:", "\ts_branch .LBB0_2", ".LBB0_1:", "\ts_or_b64 exec, exec, s[2:3]",
             "\tv_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]", "\ts_cbranch_scc1 .LBB0_3",
             ".LBB0_2:", "\ts_and_saveexec_b64 s[2:3], vcc", "\tv_mov_b32_e32 v1, 0", "\ts_branch .LBB0_1",
             ".LBB0_3:", "\tv_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]", "\ts_endpgm"]
    assert mfmas_under_lane_mask(latch) == []


# Kernels whose whole K loops run under an EXEC mask the compiler cannot
# prove uniform but that is uniform per wavefront at run time: the exact-
# scaling prefill kernel loops over a marked-block count read from LDS, the
# split gate GEMM over a per-wavefront K range.
_UNIFORM_MASKED_LOOPS = ("expert_prefill_exact_kernel", "gate_logits_split_kernel")


@pytest.mark.parametrize("src", ["experts.hip", "experts_mx.hip", "experts_fp8.hip", "experts_fp4.hip",
                                 "linear.hip", "gate.hip"])
def test_mfmas_never_run_under_a_lane_mask(src, tmp_path):
    """An MFMA is a cross-lane operation: its A and B operands and its result
    spread over all 64 lanes.  Executed under a partial EXEC mask (inside a
    per-lane `if`), lanes outside the mask contribute stale operand registers
    (a spill reload under that mask loads only the active lanes) and the
    products are wrong.  The compiler may sink the MFMAs of a peeled K loop's
    last groups into the epilogue's per-slot `rowid >= 0` branches, since
    their results feed only that epilogue; the W4A8-over-MXFP4 prefill kernel
    with register weights was built that way once and gave wrong rows for
    padded blocks.  No MFMA of these kernels may be reachable with an `if`
    region open."""

    asm = _device_asm(CSRC / src, tmp_path)
    names = re.findall(r"^(_Z\S+):", asm, re.M)
    checked = 0
    for name in names:
        start = asm.index(f"\n{name}:")
        body = asm[start: asm.index(".Lfunc_end", start)].splitlines()
        if not any(line.strip().startswith("v_mfma") for line in body):
            continue
        if any(k in name for k in _UNIFORM_MASKED_LOOPS):
            continue
        checked += 1
        assert mfmas_under_lane_mask(body) == [], name
    assert checked > 0
