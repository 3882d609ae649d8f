"""CPU tier: wait states around the inline-assembly MFMAs and LDS DMA.

The dK/dV kernel (MfmaAgpr) issues 32x32x16 MFMAs from inline assembly, and
the prefill and decode kernels issue their global->LDS loads (buffer_load
... lds) from inline assembly. The compiler's hazard recognizer cannot see
inside the asm, so:

* it adds no wait states before its own reads of an asm MFMA's results --
  including register copies it inserts on its own. The kernels route every
  such result through a tied s_nop fence; no non-MFMA instruction may read
  or overwrite an MFMA destination register within 12 wait states of the
  MFMA, and no MFMA may take a pending result as its A or B operand;
* it adds none in front of an asm MFMA either: no VALU instruction may write
  an MFMA's A or B operand within 2 wait states before it (MfmaAgpr issues
  no padding, relying on this);
* in front of an LDS DMA, a VALU write of a descriptor SGPR (readfirstlane)
  needs 5 wait states and a write of M0 needs 1: dma_pin pads the first
  once per descriptor and each load the second.

This test compiles the sources for gfx950 (as the Makefile does) and checks
the assembly (instructions count 1 wait state, s_nop k counts k + 1).
"""

from __future__ import annotations

import concurrent.futures
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "tpu-native-pallas-flashattention_amd")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
NEED = 12

SOURCES = {
    "attn_bwd_dkv16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "attn_fwd.hip": [],
    "attn_bwd.hip": [],
    "attn_bwd_f32.hip": [],
    "attn_bwd_d256.hip": [],
    "decode_stream.hip": [],
}

# sources whose MFMAs are (partly) inline assembly: the result-read check
# (12 wait states, the 32x32x16 MFMA's) applies to these; every other MFMA is
# the compiler's own, padded by its hazard model for its shape
ASM_MFMA_SOURCES = ("attn_bwd_dkv16.hip",)

_REG = re.compile(r"([vas])\[(\d+):(\d+)\]|([vas])(\d+)$")


def _regs(tok: str) -> set:
    m = _REG.match(tok)
    if not m:
        return set()
    if m.group(1):
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    return {(m.group(4), int(m.group(5)))}


def scan(lines: list[str], need: int = NEED) -> list[str]:
    """Early reads/overwrites of MFMA results in one kernel's assembly."""
    found = []
    for i, line in enumerate(lines):
        s = line.strip()
        if not s.startswith("v_mfma"):
            continue
        dst = _regs(s.split()[1].rstrip(","))
        ws = 0
        for j in range(i + 1, min(i + 400, len(lines))):
            t = lines[j].strip()
            if not t or t.startswith((";", ".")) or t.endswith(":"):
                continue
            if t.startswith(("s_cbranch", "s_branch", "s_endpgm", "s_setpc")) or ws >= need:
                break
            if t.startswith("s_nop"):
                ws += int(t.split()[1]) + 1
                continue
            ws += 1
            ops = [o.rstrip(",") for o in t.split()[1:]]
            if t.startswith("v_mfma"):
                ab = set().union(*[_regs(o) for o in ops[1:3]]) if len(ops) >= 3 else set()
                if ab & dst:
                    found.append(f"{s} -> {t} (A/B read after {ws} wait states)")
                continue
            rd = set().union(*[_regs(o) for o in ops[1:]]) if len(ops) > 1 else set()
            wr = _regs(ops[0]) if ops else set()
            if (rd | wr) & dst:
                found.append(f"{s} -> {t} (after {ws} wait states)")
                break
    return found


def _ops(t: str) -> list[str]:
    return [o.rstrip(",") for o in t.split()[1:]]


def _is_valu(t: str) -> bool:
    return t.startswith("v_") and not t.startswith("v_mfma")


def scan_before(lines: list[str], asm_mfma: bool = True) -> list[str]:
    """Hazards in front of inline-assembly MFMAs (those accumulating in
    AGPRs, when asm_mfma: VALU write of A/B within 2 wait states) and LDS DMA
    loads (VALU write of a descriptor SGPR within 5, any write of M0 within
    1). Walks back from each such instruction over straight-line code; a
    label reached before enough wait states is a possible other predecessor
    and counts as a violation. The compiler pads its own MFMAs."""
    found = []
    body = [x.strip() for x in lines]
    # keep labels (".LBB0_3:"), drop comments and directives
    body = [x for x in body if x and not x.startswith(";") and (x.endswith(":") or not x.startswith("."))]
    for i, s in enumerate(body):
        if s.startswith("v_mfma") and asm_mfma and _ops(s)[0].startswith("a"):
            ops = _ops(s)
            need = {"valu": (set().union(*[_regs(o) for o in ops[1:3]]), 2)}
        elif s.startswith("buffer_load") and s.endswith("lds"):
            ops = _ops(s)
            need = {"valu": (_regs(ops[1]) if len(ops) > 1 else set(), 5), "m0": ({("m", 0)}, 1)}
        else:
            continue
        ws = 0
        for j in range(i - 1, max(i - 60, -1), -1):
            t = body[j]
            if max(n for _, n in need.values()) <= ws:
                break
            if t.endswith(":"):
                found.append(f"{s}: label {t} within {ws} wait states")
                break
            if t.startswith("s_nop"):
                ws += int(t.split()[1]) + 1
                continue
            dst = t.split()[1].rstrip(",") if len(t.split()) > 1 else ""
            if "m0" in need and ws < need["m0"][1] and dst == "m0":
                found.append(f"{s}: {t} writes M0 {ws} wait states before")
            regs, n = need["valu"]
            if ws < n and _is_valu(t) and _regs(dst) & regs:
                found.append(f"{s}: {t} writes an operand {ws} wait states before")
            ws += 1
    return found


def _kernels(asm: str) -> dict[str, list[str]]:
    out = {}
    for m in re.finditer(r"^(_Z\S+):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        body = asm[m.end():end]
        if "v_mfma" in body or " lds" in body:
            out[m.group(1)] = body.split("\n")
    return out


def _compile(src: str, extra: list[str], out_dir: str) -> str:
    out = os.path.join(out_dir, src + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{os.path.join(ROOT, 'include')}", *extra, "--offload-device-only", "-S",
           os.path.join(PKG, "csrc", src), "-o", out]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    with open(out) as f:
        return f.read()


@pytest.mark.skipif(not (os.path.exists(HIPCC) or shutil.which("hipcc")), reason="hipcc not available")
def test_inline_asm_mfma_results_are_fenced():
    with tempfile.TemporaryDirectory() as d, concurrent.futures.ThreadPoolExecutor(len(SOURCES)) as ex:
        asms = dict(zip(SOURCES, ex.map(lambda kv: _compile(kv[0], kv[1], d), SOURCES.items())))
    problems = []
    n_kernels = 0
    for src, asm in asms.items():
        for name, body in _kernels(asm).items():
            n_kernels += 1
            if src in ASM_MFMA_SOURCES:
                problems += [f"{src} {name[:60]}: {p}" for p in scan(body)]
            problems += [f"{src} {name[:60]}: {p}" for p in scan_before(body, src in ASM_MFMA_SOURCES)]
    assert n_kernels >= 20, f"expected the MFMA / LDS-DMA kernels of {list(SOURCES)}, found {n_kernels}"
    assert not problems, "\n".join(problems[:20])


def test_scan_before_flags_missing_padding():
    """The operand and DMA checks themselves: a planted VALU operand write,
    a readfirstlane right before a DMA and an M0 write right before a DMA are
    reported; the same sequences with enough padding are not."""
    mf = "v_mfma_f32_32x32x16_bf16 a[0:15], v[16:19], v[20:23], a[0:15]"
    assert len(scan_before(["v_mov_b32 v17, v1", mf])) == 1
    assert scan_before(["v_mov_b32 v17, v1", "s_nop 1", mf]) == []
    assert scan_before(["v_mov_b32 v30, v1", mf]) == []
    dma = "buffer_load_dwordx4 v1, s[36:39], 0 offen lds"
    assert len(scan_before(["v_readfirstlane_b32 s37, v3", "s_mov_b32 m0, s5", "s_nop 0", dma])) == 1
    assert scan_before(["v_readfirstlane_b32 s37, v3", "s_nop 4", "s_mov_b32 m0, s5", "s_nop 0", dma]) == []
    assert len(scan_before(["s_nop 7", "s_mov_b32 m0, s5", dma])) == 1
    assert len(scan_before([".LBB0_3:", dma])) == 1


def test_scan_flags_an_early_read():
    """The scan itself: a VALU read two instructions after an MFMA is
    reported; the same read behind a 16-state fence is not."""
    early = ["v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]",
             "v_mov_b32 v30, v31", "v_add_f32 v24, v3, v25"]
    fenced = early[:1] + ["s_nop 7", "s_nop 7"] + early[1:]
    copy = ["v_mfma_f32_32x32x16_bf16 a[0:15], v[16:19], v[20:23], a[0:15]", "v_accvgpr_mov_b32 a20, a15"]
    chained = ["v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]",
               "v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]"]
    operand = ["v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]",
               "v_mfma_f32_32x32x16_bf16 v[32:47], v[0:3], v[20:23], v[32:47]"]
    assert len(scan(early)) == 1
    assert scan(fenced) == []
    assert len(scan(copy)) == 1
    assert scan(chained) == []          # srcC chaining on the same registers is interlocked
    assert len(scan(operand)) == 1
