"""Static check of the gfx950 assembly of every kernel: no VALU instruction
may write a register that an MFMA reads as srcA / srcB / srcC fewer than two
wait states before that MFMA.

The MFMA kernels issue their MFMAs as inline asm (to pin accumulators to
AGPRs or VGPRs and to order operand loads), and the compiler's hazard
recognizer does not see inside inline asm, so it inserts no wait states for
them.  The kernels provide the wait states themselves (``s_nop`` before an
MFMA whose operand a VALU instruction may just have written); this test
catches code where the compiler placed a copy or a spill reload of an
operand right in front of an MFMA (as happens when register pressure makes
it move values between the VGPR and AGPR files).  A second check covers the
other direction in the kernels whose MFMAs are inline asm: no instruction
may read a register (VGPR or AGPR) an MFMA wrote before the kernel's
explicit drain has passed, on any control-flow path, earlier than the wait
states the compiler itself inserts after a builtin MFMA of the same kind (a
probe compile measures that number).  CPU only: the assembly comes from
hipcc's device-only compile (no GPU needed)."""
import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from ops_amd import build as sfa_build

HIPCC = sfa_build.hipcc()
pytestmark = pytest.mark.skipif(shutil.which(HIPCC) is None and not os.path.exists(HIPCC),
                                reason="hipcc not available")

LOOKBACK = 5  # instructions examined before each MFMA


def _regs(spec):
    out = set()
    for m in re.finditer(r"([va])\[(\d+):(\d+)\]|([va])(\d+)\b", spec):
        if m.group(1):
            out |= {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
        else:
            out.add((m.group(4), int(m.group(5))))
    return out


def scan(asm: str):
    """[(kernel, mfma line, offending VALU line)] for every short RAW gap."""
    found = []
    for fm in re.finditer(r"^(_Z\S+):", asm, re.M):
        end = asm.find(".Lfunc_end", fm.end())
        body = [l.strip() for l in asm[fm.end():end].split("\n")
                if l.startswith("\t") and not l.startswith("\t;") and not l.startswith("\t.")]
        for i, ins in enumerate(body):
            if "v_mfma" not in ins:
                continue
            ops = ins.split(None, 1)[1].split(",")
            srcs = set().union(*[_regs(o) for o in ops[1:4]])
            waits = 0
            for j in range(i - 1, max(i - 1 - LOOKBACK, -1), -1):
                prev = body[j]
                if prev.startswith("s_nop"):
                    waits += int(prev.split()[1]) + 1
                    continue
                if prev.startswith("v_") and "mfma" not in prev and waits < 2:
                    dst = _regs(prev.split(None, 1)[1].split(",")[0])
                    if dst & srcs:
                        found.append((fm.group(1), ins, prev))
                waits += 1
    return found


# Kernels whose MFMAs are inline asm (the compiler inserts no wait states for
# them); kernels built on the MFMA builtins get theirs from the compiler.
INLINE_ASM_MFMA_KERNELS = ("dkv_keymajor_kernel", "fwd_mfma_kernel", "mla_bwd_dq_kernel", "mla_bwd_dkv_kernel")
DRAIN = 18  # wait states the inline-asm drains provide (at least) after an MFMA before VALU reads


def _kernel_bodies(asm: str, kernels):
    """(kernel name, instruction/label lines, label -> index) per kernel."""
    for fm in re.finditer(r"^(_Z\S+):", asm, re.M):
        if not any(k in fm.group(1) for k in kernels):
            continue
        end = asm.find(".Lfunc_end", fm.end())
        body = [l.strip() for l in asm[fm.end():end].split("\n")
                if (l.startswith("\t") and not l.startswith("\t;") and not l.startswith("\t.")) or l.startswith(".LBB")]
        labels = {l[:-1]: i for i, l in enumerate(body) if l.startswith(".LBB") and l.endswith(":")}
        yield fm.group(1), body, labels


def _reads(ins: str):
    """Registers an instruction reads (stores read every operand; MFMAs their
    srcA / srcB / srcC; other instructions every operand after the first)."""
    parts = ins.split(None, 1)
    if len(parts) < 2:
        return set()
    ops = parts[1].split(",")
    if ins.startswith(("ds_write", "global_store", "buffer_store", "flat_store")):
        return set().union(*[_regs(o) for o in ops])
    return set().union(*[_regs(o) for o in ops[1:]]) if len(ops) > 1 else set()


def scan_result_reads(asm: str, kernels=INLINE_ASM_MFMA_KERNELS, drain: int = DRAIN):
    """[(kernel, mfma, reader)] where an instruction reads a register (VGPR or
    AGPR) an MFMA wrote fewer than ``drain`` wait states later (1 per
    instruction, N + 1 per s_nop N).  Every control-flow path from the MFMA
    is followed: labels fall through, s_branch jumps to its target and
    s_cbranch_* continues on both sides (loop back-edges included); a path
    ends at s_endpgm, after ``drain`` wait states, or at an MFMA that rewrites the
    same registers (the hardware chains dependent accumulations).  An MFMA
    reading the result as srcA / srcB is a reader too."""
    found = []
    for name, body, labels in _kernel_bodies(asm, kernels):
        for i, ins in enumerate(body):
            if "v_mfma" not in ins:
                continue
            dst = _regs(ins.split(None, 1)[1].split(",")[0])
            if not dst:
                continue
            stack, seen, hits = [(i + 1, 0)], set(), set()
            while stack:
                pos, waits = stack.pop()
                while pos < len(body) and waits < drain:
                    if (pos, waits) in seen:
                        break
                    seen.add((pos, waits))
                    nxt = body[pos]
                    if nxt.startswith(".LBB"):
                        pos += 1
                        continue
                    if nxt.startswith("s_endpgm"):
                        break
                    if nxt.startswith("s_nop"):
                        waits += int(nxt.split()[1]) + 1
                        pos += 1
                        continue
                    if "v_mfma" in nxt:
                        mops = nxt.split(None, 1)[1].split(",")
                        if set().union(*[_regs(o) for o in mops[1:3]]) & dst:
                            hits.add(nxt)
                        if _regs(mops[0]) & dst:
                            break
                    elif nxt.startswith(("v_", "ds_", "global_", "buffer_", "flat_")) and _reads(nxt) & dst:
                        hits.add(nxt)
                    waits += 1
                    if nxt.startswith("s_branch"):
                        pos = labels.get(nxt.split()[1], len(body))
                        continue
                    if nxt.startswith("s_cbranch"):
                        tgt = labels.get(nxt.split()[-1])
                        if tgt is not None:
                            stack.append((tgt, waits))
                    pos += 1
            found += [(name, ins, h) for h in sorted(hits)]
    return found


def _device_asm(src: Path, out_dir: Path) -> str:
    out = out_dir / (src.stem + ".s")
    cmd = [HIPCC, *[f for f in sfa_build.HIPCC_FLAGS if f not in ("-shared", "-fPIC")], "--cuda-device-only",
           "-S", "-I", str(sfa_build.HERE.parent / "include"), str(src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out.read_text()


def test_scanner_flags_a_planted_hazard():
    # the scanner itself: a VALU write of an MFMA operand right before it is
    # reported, the same with two wait states of s_nop is not
    asm = ("_Zplanted:\n\tv_mov_b32_e32 v8, 0\n\tv_mfma_f32_32x32x16_bf16 v[0:15], v[8:11], a[0:3], v[0:15]\n"
           "\tv_mov_b32_e32 v9, 0\n\ts_nop 1\n\tv_mfma_f32_32x32x16_bf16 v[0:15], v[8:11], a[0:3], v[0:15]\n"
           "\tv_accvgpr_write_b32 a2, v1\n\tv_mfma_f32_32x32x16_bf16 v[0:15], v[8:11], a[0:3], v[0:15]\n"
           ".Lfunc_end0:\n")
    hits = scan(asm)
    assert [h[2] for h in hits] == ["v_mov_b32_e32 v8, 0", "v_accvgpr_write_b32 a2, v1"]


def test_no_valu_to_mfma_operand_hazards(tmp_path):
    sources = sfa_build.sources()
    assert sources
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        asms = list(ex.map(lambda s: _device_asm(Path(s), tmp_path), sources))
    n_mfma = sum(a.count("v_mfma") for a in asms)
    assert n_mfma > 500, "expected the MFMA kernels in the sources"
    hits = [h for a in asms for h in scan(a)]
    assert not hits, "VALU write of an MFMA operand without 2 wait states:\n" + "\n".join(
        f"{k[-60:]}: {v}  ->  {m}" for k, m, v in hits[:10])


def test_result_scanner_flags_a_planted_early_read():
    asm = ("_Zdkv_keymajor_kernel_planted:\n\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], a[0:3], v[0:15]\n"
           "\tv_add_f32_e32 v20, v3, v3\n"
           "\tv_mfma_f32_32x32x16_bf16 v[32:47], v[16:19], a[0:3], v[32:47]\n"
           "\ts_nop 7\n\ts_nop 7\n\ts_nop 3\n\tv_add_f32_e32 v20, v33, v33\n.Lfunc_end0:\n")
    hits = scan_result_reads(asm)
    assert [h[2] for h in hits] == ["v_add_f32_e32 v20, v3, v3"]


def test_result_scanner_follows_branches_and_agprs():
    # a read carried across the loop back-edge, an AGPR result read by
    # v_accvgpr_read on the taken side of a conditional branch, and the same
    # reads after a full drain (not reported)
    asm = ("_Zfwd_mfma_kernel_planted:\n"
           ".LBB0_1:\n\tv_add_f32_e32 v20, v1, v1\n"
           "\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[24:27], v[0:15]\n"
           "\ts_cbranch_scc1 .LBB0_1\n"
           "\tv_mfma_f32_32x32x16_bf16 a[0:15], v[16:19], v[24:27], a[0:15]\n"
           "\ts_cbranch_vccnz .LBB0_3\n"
           "\ts_nop 7\n\ts_nop 7\n\ts_nop 3\n"
           ".LBB0_3:\n\tv_accvgpr_read_b32 v30, a3\n"
           "\ts_nop 7\n\ts_nop 7\n\ts_nop 3\n\tv_add_f32_e32 v21, v2, v30\n\ts_endpgm\n.Lfunc_end0:\n")
    hits = scan_result_reads(asm)
    assert sorted(h[2] for h in hits) == ["v_accvgpr_read_b32 v30, a3", "v_add_f32_e32 v20, v1, v1"]


PROBE = """#include <hip/hip_runtime.h>
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
__global__ void probe(float* o, const bf16x8* a, const bf16x8* b) {
  f32x16 c = {};
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[threadIdx.x], b[threadIdx.x], c, 0, 0, 0);
  o[threadIdx.x] = c[0] * 3.0f;
}
"""


def required_read_wait_states(tmp_path: Path) -> int:
    """Wait states the compiler's own hazard recognizer puts between a
    builtin v_mfma_f32_32x32x16_bf16 and a VALU read of its result (the
    hardware requirement the inline-asm MFMAs must meet by hand)."""
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    asm = _device_asm(src, tmp_path)
    lines = [l.strip() for l in asm.split("\n") if l.startswith("\t")]
    i = next(j for j, l in enumerate(lines) if l.startswith("v_mfma_f32_32x32x16_bf16"))
    waits = 0
    for l in lines[i + 1:]:
        if l.startswith("s_nop"):
            waits += int(l.split()[1]) + 1
        elif l.startswith("v_"):
            return waits
        else:
            waits += 1
    raise AssertionError("no VALU read after the probe MFMA")


def test_no_early_reads_of_inline_asm_mfma_results(tmp_path):
    """No read of an inline-asm MFMA's result (including the compiler's own
    register copies around the tile loop, which come before the kernels'
    explicit drains) earlier than the hardware requirement."""
    need = required_read_wait_states(tmp_path)
    assert 8 <= need <= DRAIN, need
    srcs = [s for s in sfa_build.sources() if Path(s).stem in ("sfa_bwd_csr", "sfa_fwd_mfma", "sfa_bwd_mla")]
    assert len(srcs) == 3
    asms = [_device_asm(Path(s), tmp_path) for s in srcs]
    assert sum(a.count("v_mfma") for a in asms) > 300
    hits = [h for a in asms for h in scan_result_reads(a, drain=need)]
    assert not hits, "VGPR MFMA result read before the drain:\n" + "\n".join(
        f"{k[-60:]}: {m}  ->  {r}" for k, m, r in hits[:10])
