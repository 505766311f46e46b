"""Static check of the built gfx950 code: MFMA results read after a barrier.

The compiler counts a barrier, and the wait in front of it, as wait states
of the MFMA-to-VALU dependency, but a wavefront that reaches the barrier
last passes both at once; the fused kernel's buffered select, which read
its accumulators right after the tile barrier at exactly the compiler's
count, then saw stale values of the last accumulator registers now and
then (measured on the GPU: 8 more wait states removed it, 1 did not).
This test disassembles the device code of the library's own objects
(mlxvs_amd/_build, written by `python -m mlxvs_amd.build`) and, for every
MFMA, walks every path forward (branches followed) to the first VALU
instruction that reads its result.  On paths that cross an s_barrier it
counts the wait states that surely pass (each instruction one, s_nop N
N + 1; s_barrier and s_waitcnt none) and requires the MFMA's passes + 2
(the dependency) + 8 (the margin measured).  CPU only (LLVM's objdump).
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from mlxvs_amd import build as B

OBJECTS = ["knn_float.o", "knn_hamming.o"]
MARGIN = 8


def passes(op):
    # v_mfma_f32_32x32x16_f16 and the fp4/fp6 scaled MFMA run 8 passes here,
    # the fp32 32x32x2 one 16; anything else is taken as 16
    return 8 if ("32x32x16_f16" in op or "f8f6f4" in op) else 16


def need(op):
    return passes(op) + 2 + MARGIN


MIN_WAITS = need("v_mfma_f32_32x32x2_f32")  # 26
OBJDUMP = Path(B.HIPCC).resolve().parent.parent / "llvm" / "bin" / "llvm-objdump"
if not OBJDUMP.exists():
    OBJDUMP = Path("/opt/rocm/llvm/bin/llvm-objdump")


def _regs(spec):
    m = re.match(r"v\[(\d+):(\d+)\]$", spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", spec)
    return {int(m.group(1))} if m else set()


def parse(lines):
    """Instructions of an objdump listing: (function, op, text, branch target
    index or None), in address order."""
    base, insts, at = {}, [], {}
    func = None
    for line in lines:
        m = re.match(r"^([0-9a-f]+) <(\w+)>:", line)
        if m:
            func = m.group(2)
            base[func] = int(m.group(1), 16)
            continue
        m = re.match(r"^\s+(\S+)(.*?)\s*//\s*([0-9A-F]+):(.*)$", line)
        if not m or func is None:
            continue
        op, rest, addr, tail = m.group(1), m.group(2), int(m.group(3), 16), m.group(4)
        t = re.search(r"<(\w+)\+0x([0-9a-f]+)>", tail)
        tgt = (t.group(1), int(t.group(2), 16)) if t else None
        at[addr] = len(insts)
        insts.append([func, op, f"{op}{rest}", tgt])
    for ins in insts:
        if ins[3] is not None:
            f, off = ins[3]
            ins[3] = at.get(base.get(f, -1) + off)
    return insts


def barrier_reads(insts):
    """{function: (fewest wait states, the MFMA's need)} between an MFMA and
    a VALU read of its result over paths that cross an s_barrier, keeping
    per function the read with the least to spare."""

    def low(a, b):
        return b if a is None else (a if b is None else min(a, b))

    def walk(j, dst, waits, crossed, seen):
        # seen: the fewest wait states each (instruction, crossed) was reached
        # with; a later arrival with as many or more cannot find fewer
        best = None
        while j < len(insts) and waits < 2 * MIN_WAITS:
            if seen.get((j, crossed), 1 << 30) <= waits:
                return best
            seen[(j, crossed)] = waits
            func, op, text, tgt = insts[j]
            j += 1
            if op == "s_endpgm" or op.startswith("v_mfma"):
                return best
            if op == "s_barrier":
                crossed = True
            toks = re.findall(r"v\[\d+:\d+\]|v\d+", text)
            if op.startswith("v_") and toks:
                srcs = set().union(*(_regs(t) for t in toks[1:])) if len(toks) > 1 else set()
                if srcs & dst:
                    return low(best, waits) if crossed else best
                if _regs(toks[0]) & dst:
                    return best  # overwritten first
            if op == "s_nop":
                waits += int(text.split()[1], 0) + 1
            elif op not in ("s_barrier", "s_waitcnt"):
                waits += 1
            if op.startswith("s_cbranch") or op == "s_branch":
                if tgt is not None:
                    best = low(best, walk(tgt, dst, waits, crossed, seen))
                if op == "s_branch":
                    return best
        return best

    worst = {}
    for i, (func, op, text, _) in enumerate(insts):
        if op.startswith("v_mfma"):
            r = walk(i + 1, _regs(text.split()[1].rstrip(",")), 0, False, {})
            if r is not None:
                n = need(op)
                if func not in worst or r - n < worst[func][0] - worst[func][1]:
                    worst[func] = (r, n)
    return worst


@pytest.mark.parametrize("obj", OBJECTS)
def test_mfma_results_read_well_after_barriers(tmp_path, obj):
    src = B.BUILD / obj
    if not src.exists() or not OBJDUMP.exists():
        pytest.skip(f"no {src} (run python -m mlxvs_amd.build) or no {OBJDUMP}")
    local = tmp_path / obj
    shutil.copy(src, local)
    r = subprocess.run([str(OBJDUMP), "--offloading", str(local)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    dev = [p for p in tmp_path.iterdir() if "amdgcn" in p.name and "gfx950" in p.name]
    assert len(dev) == 1, [p.name for p in tmp_path.iterdir()]
    r = subprocess.run([str(OBJDUMP), "-d", "--no-show-raw-insn", str(dev[0])],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    insts = parse(r.stdout.split("\n"))
    assert sum(1 for i in insts if i[1].startswith("v_mfma")) > 0
    worst = barrier_reads(insts)
    if obj == "knn_float.o":
        # the fused kernels' buffered select reads its accumulators after the
        # tile barrier: finding none would mean the parser lost the code
        assert any("fused_kernel" in f for f in worst), sorted(worst)[:5]
    low = {f: w for f, w in worst.items() if w[0] < w[1]}
    assert not low, f"MFMA results read too soon after a barrier (wait states, needed): {low}"


def test_checker_flags_a_short_read():
    # the checker itself: reads after a barrier are reported with their wait
    # states and need, one without a barrier is not
    listing = """0000000000000000 <_ZShort>:
\tv_mfma_f32_32x32x2_f32 v[0:15], v20, v21, v[0:15]     // 000000000000: 0
\ts_waitcnt vmcnt(0)                                    // 000000000008: 0
\ts_barrier                                             // 00000000000C: 0
\tv_add_f32_e32 v30, v15, v15                           // 000000000010: 0
\ts_endpgm                                              // 000000000014: 0
0000000000000100 <_ZLong>:
\tv_mfma_f32_32x32x2_f32 v[0:15], v20, v21, v[0:15]     // 000000000100: 0
\ts_barrier                                             // 000000000108: 0
\ts_cbranch_scc1 3                                      // 00000000010C: 0 <_ZLong+0x1c>
\ts_nop 7                                               // 000000000110: 0
\ts_nop 7                                               // 000000000114: 0
\ts_nop 7                                               // 000000000118: 0
\ts_nop 7                                               // 00000000011C: 0
\ts_nop 7                                               // 000000000120: 0
\ts_nop 7                                               // 000000000124: 0
\tv_add_f32_e32 v30, v15, v15                           // 000000000128: 0
\ts_endpgm                                              // 00000000012C: 0
0000000000000200 <_ZNoBarrier>:
\tv_mfma_f32_32x32x2_f32 v[0:15], v20, v21, v[0:15]     // 000000000200: 0
\ts_nop 7                                               // 000000000208: 0
\tv_add_f32_e32 v30, v15, v15                           // 00000000020C: 0
\ts_endpgm                                              // 000000000210: 0
""".split("\n")
    worst = barrier_reads(parse(listing))
    # _ZShort: only the barrier and its wait lie between (they count none);
    # _ZLong: the branch skips three of the six nops: 1 + 24 = 25
    assert worst == {"_ZShort": (0, 26), "_ZLong": (25, 26)}
