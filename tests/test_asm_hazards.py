"""Wait states around the inline-asm MFMAs of the bf16 dK/dV kernel (CPU).

bwd_dkdv_bf16_kernel (gonn_amd/csrc/attn_bwd.hip) issues its S and dP
products as inline asm (mfma_vacc), with VGPR accumulators and the K / V
fragments in AGPRs. The compiler's hazard recognizer does not look inside
inline asm, so the kernel supplies the wait states itself, in asm
statements that the registers pass through. This test compiles the file to
gfx950 assembly with the build's flags and scans every unmasked
instantiation, in program order:

- no instruction outside an asm statement reads or writes a VGPR that an
  inline MFMA wrote, until a statement with three s_nop 7 (24 wait states)
  has passed (the compiler once hoisted a register copy and the causal mask
  above an unconnected nop statement; the results were then wrong);
- no inline MFMA reads a pending result of another one as its A or B operand;
- after the first inline MFMA, nothing writes the AGPRs they read their B
  operand from (a write there would need wait states the compiler does not
  know of).
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _vregs(text):
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]", text):
        out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\bv(\d+)\b", text):
        out.add(int(m.group(1)))
    return out


def _aregs(text):
    m = re.search(r"\ba\[(\d+):(\d+)\]", text)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.search(r"\ba(\d+)\b", text)
    return {int(m.group(1))} if m else set()


def _scan(lines):
    """Violations of the rules above in one function's assembly lines."""
    bad, pending, asm, in_asm = [], set(), [], False
    srcb, first = set(), None
    for no, raw in enumerate(lines):
        ln = raw.strip()
        if ln.startswith(";;#ASMSTART"):
            in_asm, asm = True, []
            continue
        if ln.startswith(";;#ASMEND"):
            in_asm = False
            txt = " ".join(asm)
            if "v_mfma" in txt:
                ops = txt.split(None, 1)[1].split(",")
                if _vregs(ops[1]) & pending:
                    bad.append((no, txt))
                pending |= _vregs(ops[0])
                srcb |= _aregs(ops[2])
                first = no if first is None else first
            elif txt.count("s_nop 7") >= 3:
                pending.clear()
            continue
        if in_asm:
            asm.append(ln)
            continue
        if not ln or ln.startswith((";", ".")) or ln.endswith(":"):
            continue
        op = ln.split()[0]
        rest = ln.split(None, 1)[1] if " " in ln else ""
        if first is not None and op.startswith("v_accvgpr_") and not op.startswith("v_accvgpr_read"):
            if _aregs(rest.split(",")[0]) & srcb:
                bad.append((no, ln))
        if op.startswith("s_"):
            continue
        if _vregs(rest) & pending:
            bad.append((no, ln))
    return bad, first


@pytest.fixture(scope="module")
def bwd_asm(tmp_path_factory):
    from gonn_amd import build as gbuild
    hipcc = gbuild.HIPCC
    if not (os.path.exists(hipcc) or shutil.which(hipcc)):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "attn_bwd.s"
    src = os.path.join(gbuild.CSRC, "attn_bwd.hip")
    cmd = [hipcc, *[f for f in gbuild.CFLAGS if f != "-fPIC"],
           *gbuild.FILE_FLAGS.get("attn_bwd.hip", []), "--cuda-device-only", "-S", src, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text().split("\n")


def test_dkdv_inline_mfma_wait_states(bwd_asm):
    lines = bwd_asm
    starts = [i for i, ln in enumerate(lines)
              if re.match(r"^_ZN4gonn20bwd_dkdv_bf16_kernelILi\d+ELb[01]ELb0E\S*:", ln)]
    assert len(starts) == 4, "unmasked bwd_dkdv_bf16_kernel instantiations (D 64/128, causal or not)"
    for st in starts:
        end = next(i for i in range(st + 1, len(lines)) if lines[i].startswith(".Lfunc_end"))
        bad, first = _scan(lines[st:end])
        name = lines[st].split(":")[0]
        assert first is not None, f"{name}: no inline MFMA found"
        assert not bad, f"{name}: {len(bad)} accesses without wait states, first {bad[:3]}"


def test_scan_catches_a_hoisted_copy():
    """The checker itself: a VGPR copy of an inline MFMA result ahead of
    the wait-state statement is reported; after it, it is not."""
    mfma = [";;#ASMSTART", "v_mfma_f32_32x32x16_bf16 v[16:31], v[0:3], a[0:3], 0", ";;#ASMEND"]
    nops = [";;#ASMSTART", "s_nop 7", "s_nop 7", "s_nop 7", ";;#ASMEND"]
    copy = ["v_mov_b64_e32 v[40:41], v[16:17]"]
    bad, _ = _scan(mfma + copy + nops)
    assert len(bad) == 1
    bad, _ = _scan(mfma + nops + copy)
    assert not bad
    bad, _ = _scan(mfma + ["v_accvgpr_write_b32 a2, v5"] + nops)
    assert len(bad) == 1
