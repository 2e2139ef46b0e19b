"""The prefill kernels' inline MFMAs and what the compiler does around them (CPU).

The bf16 prefill issues its MFMAs as inline assembly, so the compiler does not
know their timing rules, and it inserts none of the wait states they need:

1. An MFMA's result arrives late.  The kernel waits that out itself before its
   own reads of S and O, but a copy the compiler adds on its own (an AGPR read
   to merge two control-flow paths, say) can read the registers too early.  An
   8-pass 32x32x16 MFMA needs 11 wait states; this test asks for 18.
2. An MFMA reads a source VGPR that a VALU instruction wrote at least 2 wait
   states after the write.  A copy the compiler makes of an operand right before
   the asm (from a register it parked in an AGPR, say) can be too close.

It compiles csrc/ca_flash.hip to gfx950 assembly, splits each
flash_bf16_p64_kernel into basic blocks, and propagates, per register, the fewest
wait states since an MFMA wrote it and since a VALU instruction wrote it (minimum
over predecessors, to a fixed point; `s_nop N` counts N + 1, any other
instruction 1).  Both rules are checked on every path.
"""

import os
import re
import shutil
import subprocess

import pytest

from conftest import PKG

NEED = 18      # an MFMA result read by another instruction
NEED_SRC = 2   # a VALU-written VGPR read by an MFMA
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
INF = 10 ** 9


def blocks_of(asm_lines):
    """Basic blocks: a label starts one, and so does the instruction after a branch
    (the fall-through blocks the compiler leaves unlabelled)."""
    blocks, order, cur = {"entry": []}, ["entry"], "entry"
    anon = 0
    for raw in asm_lines:
        line = raw.strip()
        if not line or line.startswith(";"):
            continue
        m = re.match(r"^(\.LBB\S+):", line)
        if m:
            cur = m.group(1)
            blocks[cur] = []
            order.append(cur)
            continue
        if line.startswith(".") or line.endswith(":"):
            continue
        ins = line.split(";")[0].strip()
        blocks[cur].append(ins)
        if ins.startswith(("s_cbranch", "s_branch")):
            anon += 1
            cur = f"fallthrough{anon}"
            blocks[cur] = []
            order.append(cur)
    succ = {b: [] for b in order}
    for i, b in enumerate(order):
        ins = [x for x in blocks[b] if x]
        for x in ins:
            m = re.match(r"s_(?:cbranch_\w+|branch)\s+(\.LBB\S+)", x)
            if m:
                succ[b].append(m.group(1))
        term = ins[-1] if ins else ""
        if not term.startswith(("s_branch", "s_endpgm")) and i + 1 < len(order):
            succ[b].append(order[i + 1])
    return blocks, order, succ


def regs_of(text):
    regs = []
    for m in re.finditer(r"\b([av])(\d+)\b|\b([av])\[(\d+):(\d+)\]", text):
        if m.group(1):
            regs.append((m.group(1), int(m.group(2))))
        else:
            regs += [(m.group(3), k) for k in range(int(m.group(4)), int(m.group(5)) + 1)]
    return regs


def operands(ins):
    """(destination text, source text) of an instruction; stores have no destination."""
    parts = ins.split(None, 1)
    if len(parts) < 2:
        return "", ""
    if parts[0].startswith(("ds_write", "buffer_store", "global_store")):
        return "", parts[1]
    if "," not in parts[1]:
        return parts[1], ""
    dst, srcs = parts[1].split(",", 1)
    return dst, srcs


def step(state, ins_list, report=None, where=""):
    """State: ("m", reg) -> wait states since an MFMA wrote reg, ("w", reg) -> since
    a VALU instruction wrote it."""
    st = dict(state)
    for ins in ins_list:
        if not ins:
            continue
        op = ins.split()[0]
        dst, srcs = operands(ins)
        if report is not None:
            for reg in regs_of(srcs):
                if op.startswith("v_mfma"):
                    if st.get(("w", reg), INF) < NEED_SRC:
                        report.append(f"{where}: {ins} (VALU wrote {reg[0]}{reg[1]} "
                                      f"{st[('w', reg)]} wait states before)")
                        break
                elif st.get(("m", reg), INF) < NEED:
                    report.append(f"{where}: {ins} ({st[('m', reg)]} wait states after the MFMA "
                                  f"that wrote {reg[0]}{reg[1]})")
                    break
        inc = int(ins.split()[1]) + 1 if op == "s_nop" else 1
        for key in st:
            st[key] = min(INF, st[key] + inc)
        if op.startswith("v_mfma"):
            for reg in regs_of(dst):
                st[("m", reg)] = 0
        elif op.startswith("v_"):
            for reg in regs_of(dst):
                st[("w", reg)] = 0
    return st


def hazards(asm_lines):
    blocks, order, succ = blocks_of(asm_lines)
    entry = {b: None for b in order}
    entry["entry"] = {}
    changed = True
    while changed:
        changed = False
        for b in order:
            if entry[b] is None:
                continue
            out = step(entry[b], blocks[b])
            for s in succ[b]:
                if s not in entry:
                    continue
                if entry[s] is None:
                    entry[s] = dict(out)
                    changed = True
                    continue
                merged = dict(entry[s])
                for reg, v in out.items():
                    if v < merged.get(reg, INF):
                        merged[reg] = v
                if merged != entry[s]:
                    entry[s] = merged
                    changed = True
    report = []
    for b in order:
        if entry[b] is not None:
            step(entry[b], blocks[b], report, b)
    return report


def test_checker_catches_an_early_read():
    """A read of an MFMA's result 3 wait states after it is reported; the same read
    after a 16-state guard plus two instructions is not."""
    bad = ["v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], 0", "s_nop 1",
           "v_accvgpr_read_b32 v8, a3", "s_endpgm"]
    good = ["v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], 0", "s_nop 7", "s_nop 7",
            "s_nop 1", "v_accvgpr_read_b32 v8, a3", "s_endpgm"]
    assert len(hazards(bad)) == 1 and hazards(good) == []
    # across a branch: the early path is found even though the linear order is long
    branchy = ["v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], 0", "s_cbranch_scc1 .LBB0_2",
               *["s_nop 7"] * 4, ".LBB0_2:", "v_accvgpr_read_b32 v8, a0", "s_endpgm"]
    assert len(hazards(branchy)) == 1
    # an MFMA source written by VALU one wait state before; two states later is fine
    src_bad = ["v_mov_b32 v2, 0", "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[0:3], 0", "s_endpgm"]
    src_good = ["v_mov_b32 v2, 0", "s_nop 1", "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[0:3], 0",
                "s_endpgm"]
    assert len(hazards(src_bad)) == 1 and hazards(src_good) == []


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_no_early_reads_of_inline_mfma_results(tmp_path):
    out = tmp_path / "flash.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(os.path.dirname(PKG), "include"),
           os.path.join(PKG, "csrc", "ca_flash.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    text = out.read_text().splitlines()
    found = 0
    for e, split in ((e, b) for e in (32, 64, 128) for b in (0, 1)):
        name = f"_ZN2ca21flash_bf16_p64_kernelILi{e}ELb{split}EEEvNS_11FlashParamsE:"
        start = next(i for i, x in enumerate(text) if x.startswith(name))
        end = next(i for i in range(start, len(text)) if text[i].startswith(".Lfunc_end"))
        body = text[start + 1:end]
        assert sum(1 for x in body if "v_mfma" in x) > 30
        report = hazards(body)
        assert report == [], f"E={e} split={split}:\n" + "\n".join(report[:10])
        found += 1
    assert found == 6
