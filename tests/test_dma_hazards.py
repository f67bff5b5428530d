"""Static check of the global->LDS DMA loads in the built gfx950 code.

The kernels issue ``global_load_lds_dwordx4`` from inline assembly. An asm
statement's SGPR inputs are not covered by the compiler's hazard padding, and
on gfx950 a VMEM instruction that reads an SGPR last written by a VALU
instruction (``v_readfirstlane_b32``, ``v_readlane_b32``, a ``v_cmp`` or
carry-out) needs 5 wait states in between; one that reads M0 after an SALU
write of it needs 1. A read too early takes a stale base address: a wrong
address, a memory fault. This compiles the sources that hold DMA loads to
device assembly with the library's own flags and walks back from every DMA,
through fall-through and branch predecessors, to each operand's last writer.

It also pins the rule itself: for an ordinary buffer load after a
``v_readfirstlane_b32`` the compiler inserts ``s_nop 4`` (5 wait states).
"""

from __future__ import annotations

import re
import shutil
import subprocess
from collections import defaultdict
from concurrent.futures import ThreadPoolExecutor

import pytest

from tinyserver_amd import _build as B

DMA_SOURCES = ["paged_decode.hip", "varlen_prefill.hip", "varlen_prefill_w64.hip"]
VALU_SGPR_WS = 5  # VALU writes an SGPR -> VMEM reads it
SALU_M0_WS = 1  # SALU writes M0 -> LDS DMA reads it

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not B.Path("/opt/rocm/bin/hipcc").exists(),
                                reason="hipcc not available")


def _device_asm(src_path, tmp_path, extra=()):
    out = tmp_path / (B.Path(src_path).name + ".s")
    cmd = [B.hipcc(), *B.CFLAGS, *extra, "--cuda-device-only", "-S", str(src_path), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def _regs(tok: str) -> set[str]:
    tok = tok.strip()
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    m = re.fullmatch(r"(s\d+|m0)", tok)
    return {m.group(1)} if m else set()


_NO_DST = ("global_", "buffer_", "flat_", "scratch_", "ds_", "s_waitcnt", "s_nop", "s_branch", "s_cbranch", "s_barrier",
           "s_setprio", "s_sleep", "s_endpgm", "s_store", "s_dcache", "s_cmp", "s_bitcmp", "s_sendmsg")
_VALU_SDST2 = re.compile(r"_co_|div_scale|mad_u64_u32|mad_i64_i32")


def _writes(op: str, operands: list[str]) -> tuple[set[str], bool]:
    """SGPRs (and M0) an instruction writes, and whether it is a VALU op."""
    if op.startswith(_NO_DST) or not operands:
        return set(), False
    valu = op.startswith("v_")
    dst = _regs(operands[0])
    if valu and len(operands) > 1 and _VALU_SDST2.search(op):
        dst |= _regs(operands[1])
    return dst, valu


def _wait_states(op: str, operands: list[str]) -> int:
    return int(operands[0], 0) + 1 if op == "s_nop" else 1


def dma_hazards(asm: str) -> tuple[int, list[str]]:
    """Return (number of DMA sites, hazards found) for one assembly file."""
    body = [ln.split(";")[0].rstrip() for ln in asm.splitlines()]
    insts = {}  # line -> (op, operands)
    labels = {}
    func_start = set()
    for i, ln in enumerate(body):
        s = ln.strip()
        if not s:
            continue
        if re.match(r"^\S+:\s*$", ln):
            name = s[:-1]
            labels[name] = i
            if name.startswith("_Z"):
                func_start.add(i)
            continue
        if s.startswith("."):
            continue
        parts = s.split(None, 1)
        ops = [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []
        insts[i] = (parts[0], ops)
    branch_from = defaultdict(list)
    for i, (op, ops) in insts.items():
        if (op == "s_branch" or op.startswith("s_cbranch")) and ops:
            branch_from[ops[-1]].append(i)

    found: list[str] = []

    def walk(j: int, need: dict[str, int], ws: int, site: int, seen: set) -> None:
        while j >= 0 and need:
            if j in func_start:
                return
            if j in insts:
                op, ops = insts[j]
                dst, valu = _writes(op, ops)
                for r in list(need):
                    if r in dst:
                        req = SALU_M0_WS if (r == "m0" and not valu) else (VALU_SGPR_WS if valu else 0)
                        if ws < req:
                            found.append(f"line {site + 1}: {r} written by {op} at line {j + 1}, {ws} wait states before")
                        del need[r]
                ws += _wait_states(op, ops)
                if ws >= VALU_SGPR_WS:
                    return
            elif body[j].strip().endswith(":") and body[j].strip()[:-1] in labels:
                name = body[j].strip()[:-1]
                key = (j, ws)
                if key in seen:
                    return
                seen.add(key)
                for src in branch_from.get(name, []):
                    walk(src, dict(need), ws, site, seen)
                # fall-through from the previous instruction unless it is an unconditional branch / end
                k = j - 1
                while k >= 0 and k not in insts and k not in func_start:
                    k -= 1
                if k in insts and insts[k][0] in ("s_branch", "s_endpgm", "s_setpc_b64"):
                    return
            j -= 1

    n = 0
    for i, (op, ops) in insts.items():
        if not op.startswith("global_load_lds_"):
            continue
        n += 1
        need = {"m0": SALU_M0_WS}
        if len(ops) > 1 and ops[1] != "off":
            for r in _regs(ops[1]):
                need[r] = VALU_SGPR_WS
        walk(i - 1, need, 0, i, set())
    return n, found


@pytest.fixture(scope="module")
def asm_files(tmp_path_factory):
    tmp = tmp_path_factory.mktemp("asm")
    with ThreadPoolExecutor(max_workers=len(DMA_SOURCES)) as ex:
        texts = list(ex.map(lambda s: _device_asm(B.CSRC / s, tmp), DMA_SOURCES))
    return dict(zip(DMA_SOURCES, texts))


@pytest.mark.parametrize("src", DMA_SOURCES)
def test_no_dma_operand_hazards(asm_files, src):
    n, found = dma_hazards(asm_files[src])
    assert n > 0, f"no DMA sites found in {src}"
    assert not found, f"{len(found)} DMA operand hazards in {src}:\n" + "\n".join(found[:20])


def test_checker_flags_a_valu_written_base(tmp_path):
    """The rule and the checker: the compiler pads 5 wait states after a
    v_readfirstlane that feeds a buffer load's SGPR offset, and the checker
    flags a DMA whose base a v_readfirstlane wrote one wait state before."""
    src = tmp_path / "probe.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "__global__ void k(__amdgpu_buffer_rsrc_t r, const int* in, int* o) {\n"
        "  int s = __builtin_amdgcn_readfirstlane(in[threadIdx.x]);\n"
        "  o[threadIdx.x] = __builtin_amdgcn_raw_buffer_load_b32(r, threadIdx.x * 4, s, 0);\n"
        "}\n")
    asm = _device_asm(src, tmp_path)
    lines = [ln.strip() for ln in asm.splitlines()]
    i = next(k for k, ln in enumerate(lines) if ln.startswith("v_readfirstlane_b32"))
    j = next(k for k in range(i, len(lines)) if lines[k].startswith("buffer_load_dword"))
    pad = sum(int(ln.split()[1]) + 1 if ln.startswith("s_nop") else 1 for ln in lines[i + 1:j] if ln and not ln.startswith((".", ";")))
    assert pad >= VALU_SGPR_WS, lines[i:j + 1]

    bad = ("_Zk:\n\tv_readfirstlane_b32 s5, v3\n\tv_readfirstlane_b32 s4, v2\n"
           "\ts_mov_b32 m0, s6\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, s[4:5]\n\ts_endpgm\n")
    n, found = dma_hazards(bad)
    assert n == 1 and len(found) == 2, found
    good = bad.replace("s_nop 0", "s_nop 4")
    assert dma_hazards(good) == (1, [])
    # across a branch: the writer sits in a predecessor block
    branchy = ("_Zk:\n\tv_readfirstlane_b32 s4, v2\n\ts_cbranch_scc1 .LBB0_2\n\ts_nop 7\n.LBB0_2:\n"
               "\ts_mov_b32 m0, s6\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, s[4:5]\n\ts_endpgm\n")
    n, found = dma_hazards(branchy)
    assert n == 1 and len(found) == 1 and "s4" in found[0], found
