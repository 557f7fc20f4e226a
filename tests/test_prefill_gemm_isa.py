"""The prefill GEMM issues its MFMAs and LDS reads as inline assembly (prefill_gemm.hip), so the compiler inserts none
of the MFMA hazard wait states; the kernel keeps them by construction. This checks that construction on the compiler's
own gfx950 assembly of prefill_gemm.hip, for every epilogue's kernel:

- a register an MFMA reads as an operand was last written by an LDS read, never by a VALU or vector memory
  instruction, on every path the control flow allows (a dataflow fixed point over the basic blocks, loop included);
- inside the K loop, no accumulator register is moved (v_accvgpr_*), so each tile stays in its own AGPRs;
- no register spills;
- on every path from an MFMA to an instruction that reads an accumulator, at least 32 wait states (four s_nop 7).
"""
import re
import subprocess
import tempfile
from pathlib import Path

import pytest

from nanochat_amd import native

SOURCE = native.CSRC / "prefill_gemm.hip"
VREG = re.compile(r"^([va])(?:\[(\d+):(\d+)\]|(\d+))$")


def regs(token):
    m = VREG.match(token.strip(","))
    if not m:
        return set()
    kind = m.group(1)
    if m.group(4) is not None:
        return {(kind, int(m.group(4)))}
    return {(kind, r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}


def parse(line):
    """(mnemonic, operand tokens) of an instruction line, or None for labels, directives and comments."""
    text = line.split(";")[0].strip()
    if not text or text.startswith(".") or text.endswith(":"):
        return None
    parts = text.split(None, 1)
    ops = [t.strip() for t in parts[1].split(",")] if len(parts) > 1 else []
    return parts[0], ops


@pytest.fixture(scope="module")
def kernels():
    with tempfile.TemporaryDirectory() as tmp:
        out = Path(tmp) / "pg.s"
        subprocess.run([native.hipcc(), *native.HIPCC_FLAGS, f"-I{native.CSRC}", "--cuda-device-only", "-S",
                        "-o", str(out), str(SOURCE)], check=True, capture_output=True)
        text = out.read_text()
    bodies = {}
    for m in re.finditer(r"^(_ZN2nc19prefill_gemm_kernelILi(-?\d+)ELi([012])EEEvNS_6PfGemmE\w*):[^\n]*\n(.*?)\n\.Lfunc_end", text,
                         re.S | re.M):
        bodies[(int(m.group(2)), int(m.group(3)))] = m.group(4).splitlines()
    return bodies, text


def blocks(lines):
    """The kernel's basic blocks in file order: (label, [(mnemonic, operands)], successor labels)."""
    out, label, body, n = [], "entry", [], 0

    def close(succ):
        nonlocal label, body, n
        out.append((label, body, succ))
        n += 1
        label, body = f"fall{n}", []

    for line in lines:
        s = line.split(";")[0].strip()
        if s.endswith(":") and s.startswith(".L"):
            if body or not label.startswith("fall"):
                close([s[:-1]])
            label = s[:-1]
            continue
        p = parse(line)
        if not p:
            continue
        body.append(p)
        mn, ops = p
        if mn == "s_branch":
            close([ops[0]])
        elif mn.startswith("s_cbranch"):
            close([ops[0], None])
        elif mn == "s_endpgm":
            close([])
    if body:
        out.append((label, body, []))
    # a fall-through successor is the next block in file order
    resolved = []
    for i, (lab, body, succ) in enumerate(out):
        nxt = out[i + 1][0] if i + 1 < len(out) else None
        resolved.append((lab, body, [nxt if t is None else t for t in succ if (t is not None or nxt)]))
    return resolved


def writer_kind(mn, ops):
    """What an instruction writes into its first operand's vector registers, or None."""
    if not ops or mn.startswith(("s_", "buffer_store", "global_store", "ds_write", "ds_store")):
        return None
    if mn.startswith("ds_read"):
        return "ds_read"
    if mn.startswith(("buffer_load", "global_load", "flat_load", "scratch_load")):
        return None if "lds" in ops else "vmem"
    if mn.startswith("v_mfma"):
        return "mfma"
    if mn.startswith(("v_", "ds_")):
        return "valu"
    return None


def mfma_operand_writers(lines):
    """For every MFMA (in any order of execution the control flow allows), the kinds of instruction that can have
    written its A and B operand registers last: a forward dataflow fixed point over the basic blocks."""
    bl = blocks(lines)
    index = {lab: i for i, (lab, _, _) in enumerate(bl)}
    state_in = {0: {}}
    work = [0]
    found = {}
    while work:
        i = work.pop()
        st = {r: set(k) for r, k in state_in[i].items()}
        for j, (mn, ops) in enumerate(bl[i][1]):
            if mn.startswith("v_mfma"):
                kinds = set()
                for r in regs(ops[1]) | regs(ops[2]):
                    kinds |= st.get(r, {"entry"})
                found.setdefault((i, j), set()).update(kinds)
            kind = writer_kind(mn, ops)
            if kind:
                for r in regs(ops[0]):
                    st[r] = {kind}
        for t in bl[i][2]:
            k = index[t]
            old = state_in.get(k)
            if old is None:
                state_in[k] = {r: set(v) for r, v in st.items()}
                work.append(k)
                continue
            changed = False
            for r in set(old) | set(st):
                merged = old.get(r, {"entry"}) | st.get(r, {"entry"})
                if merged != old.get(r, {"entry"}):
                    old[r] = merged
                    changed = True
            if changed:
                work.append(k)
    return found


def loop_lines(lines):
    """The lines of the basic blocks the compiler marks as inside a loop."""
    out, inside = [], False
    for line in lines:
        s = line.strip()
        if s.startswith(".LBB") or s.startswith("; %bb"):
            inside = "in Loop" in line or "Loop Header" in line
            continue
        if inside:
            out.append(line)
    return out


KERNELS = [(epi, mode) for epi in (0, 2, 3, 4) for mode in (0, 1, 2)]   # modes: whole tiles, split, thin


def test_every_epilogue_kernel_is_built(kernels):
    bodies, _ = kernels
    assert sorted(bodies) == KERNELS


def test_no_spills(kernels):
    bodies, text = kernels
    assert not any("scratch_" in l for b in bodies.values() for l in b)
    counts = re.findall(r"\.[sv]gpr_spill_count:\s+(\d+)", text)
    assert counts and all(int(c) == 0 for c in counts)


@pytest.mark.parametrize("epi", KERNELS)
def test_mfma_operands_come_from_lds_reads(kernels, epi):
    found = mfma_operand_writers(kernels[0][epi])
    assert len(found) >= 32, len(found)
    for where, kinds in found.items():
        assert kinds == {"ds_read"}, (epi, where, kinds)


@pytest.mark.parametrize("epi", KERNELS)
def test_accumulators_stay_in_place(kernels, epi):
    body = loop_lines(kernels[0][epi])
    assert any("v_mfma" in l for l in body)
    moves = [l.strip() for l in body if "v_accvgpr" in l]
    assert not moves, moves[:4]


def wait_states_before_agpr_reads(lines):
    """The fewest wait states between an MFMA and a later instruction (not an MFMA) that reads an AGPR, over every
    path the control flow allows: a forward fixed point of the minimum count since the last MFMA (s_nop N counts
    N + 1, any other instruction 1)."""
    bl = blocks(lines)
    index = {lab: i for i, (lab, _, _) in enumerate(bl)}
    INF = 1 << 30
    state_in = {0: INF}
    work = [0]
    fewest = INF
    while work:
        i = work.pop()
        ws = state_in[i]
        for mn, ops in bl[i][1]:
            if mn.startswith("v_mfma"):
                ws = 0
                continue
            srcs = ops[1:] if writer_kind(mn, ops) else ops
            if any(k == "a" for op in srcs for k, _ in regs(op)):
                fewest = min(fewest, ws)
            ws = min(INF, ws + (int(ops[0], 0) + 1 if mn == "s_nop" else 1))
        for t in bl[i][2]:
            k = index[t]
            if k not in state_in or ws < state_in[k]:
                state_in[k] = ws
                work.append(k)
    return fewest


@pytest.mark.parametrize("epi", KERNELS)
def test_accumulators_read_after_the_wait_states(kernels, epi):
    # 19 is the longest a 16-pass XDL result needs before a VALU reads it; the kernel waits 32
    assert wait_states_before_agpr_reads(kernels[0][epi]) >= 32


def test_checkers_see_the_hazards_they_look_for():
    """The checks against small hand-made listings: a VALU write reaching an MFMA operand around a loop's back edge,
    an accumulator move inside a loop, and an AGPR read too soon after an MFMA."""
    loop = """
        ds_read_b128 v[0:3], v20
        ds_read_b128 v[4:7], v20 offset:16
.LBB0_1:                                ; =>This Inner Loop Header: Depth=1
        v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]
        ds_read_b128 v[0:3], v20
        v_add_u32_e32 v4, 1, v4
        s_cbranch_scc1 .LBB0_1
; %bb.2:
        s_nop 7
        s_nop 7
        s_nop 7
        s_nop 7
        v_accvgpr_read_b32 v8, a0
        s_endpgm""".splitlines()
    found = mfma_operand_writers(loop)
    assert set().union(*found.values()) == {"ds_read", "valu"}
    assert wait_states_before_agpr_reads(loop) == 3 + 32   # the LDS read, the add and the branch, then the nops
    soon = [l for l in loop if l.strip() != "s_nop 7"]
    assert wait_states_before_agpr_reads(soon) == 3
    moving = loop[:4] + ["        v_accvgpr_mov_b32 a4, a0"] + loop[4:]
    assert any("v_accvgpr" in l for l in loop_lines(moving))
    clean = [l.replace("v_add_u32_e32 v4, 1, v4", "s_add_u32 s4, 1, s4") for l in loop]
    assert set().union(*mfma_operand_writers(clean).values()) == {"ds_read"}
