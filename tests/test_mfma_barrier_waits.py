"""Static check of the built gfx950 code: MFMA results read after a barrier.

An MFMA does not interlock its result registers against VALU reads: the
program must leave a number of independent instructions (wait states)
between them, listed per MFMA kind and pass count in the ISA's table of
required independent instructions ("Dependency Resolution: Required
Independent Instructions" in the AMD Instinct CDNA3 and CDNA4 ISA reference
guides: an MFMA writing a VGPR followed by a VALU read of it).  The compiler
inserts them, and this test takes the counts from it: it compiles a probe
kernel per MFMA kind used here, an MFMA whose result is read at once, and
counts the wait states the compiler puts in between (for gfx950: 18 after
v_mfma_f32_32x32x2_f32, 12 after v_mfma_f32_32x32x16_f16 and after the FP4
v_mfma_scale_f32_32x32x64_f8f6f4).

The compiler also counts an s_barrier and the s_waitcnt in front of it as
one wait state each, but a wavefront that reaches the barrier last passes
both without a cycle to spare; the fused kernel's buffered select, which
read its accumulators right after the tile barrier at exactly the
compiler's count (16 instructions that surely pass, against 18), then saw
stale values of the last accumulator registers now and then (one more wait
state, 17, did not remove it; eight more did).  So on every path from an
MFMA across an s_barrier to the first VALU read of its result this test
counts the wait states that surely pass (each instruction one, s_nop N
N + 1, s_barrier and s_waitcnt none) and requires the ISA's count, with no
margin: the failure and both measured fixes agree with that count exactly.
Every library object that holds MFMAs is checked.  CPU only (hipcc and
LLVM's objdump on this build's own objects).
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from mlxvs_amd import build as B

MARGIN = 0
OBJDUMP = Path(B.HIPCC).resolve().parent.parent / "llvm" / "bin" / "llvm-objdump"
if not OBJDUMP.exists():
    OBJDUMP = Path("/opt/rocm/llvm/bin/llvm-objdump")

# one kernel per MFMA kind the library uses: the result read at once
PROBE = r"""
#include <hip/hip_runtime.h>
typedef float f16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef int i8v __attribute__((ext_vector_type(8)));
__global__ void p_f32(float* o, float a, float b) {
  f16v c = {};
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  o[threadIdx.x] = c[15] + 1.0f;
}
__global__ void p_f16(float* o, h8 a, h8 b) {
  f16v c = {};
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  o[threadIdx.x] = c[15] + 1.0f;
}
__global__ void p_fp4(float* o, i8v a, i8v b) {
  f16v c = {};
  c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 4, 4, 0, 0, 0, 0);
  o[threadIdx.x] = c[15] + 1.0f;
}
"""


def family(op):
    if "32x32x16_f16" in op:
        return "f16"
    if "f8f6f4" in op:
        return "fp4"
    if "32x32x2_f32" in op:
        return "f32"
    return None


def disassemble(obj: Path, tmp: Path):
    """The gfx950 device code of a host object, as objdump lines."""
    local = tmp / obj.name
    if obj.resolve() != local.resolve():
        shutil.copy(obj, local)
    r = subprocess.run([str(OBJDUMP), "--offloading", str(local)], capture_output=True, text=True,
                       cwd=tmp)
    assert r.returncode == 0, r.stderr[-2000:]
    dev = [p for p in tmp.iterdir() if p.name.startswith(local.name) and "amdgcn" in p.name
           and "gfx950" in p.name]
    if not dev:
        return []  # host code only
    assert len(dev) == 1, [p.name for p in tmp.iterdir()]
    r = subprocess.run([str(OBJDUMP), "-d", "--no-show-raw-insn", str(dev[0])],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stdout.split("\n")


@pytest.fixture(scope="module")
def required(tmp_path_factory):
    """{MFMA family: wait states the compiler puts before a VALU read of its
    result} from the probe kernels."""
    if not OBJDUMP.exists() or not Path(B.HIPCC).exists():
        pytest.skip("no hipcc / llvm-objdump")
    tmp = tmp_path_factory.mktemp("probe")
    src = tmp / "probe.hip"
    src.write_text(PROBE)
    obj = tmp / "probe.o"
    r = subprocess.run([B.HIPCC, "-O3", f"--offload-arch={B.ARCH}", "-x", "hip", "-c", str(src),
                        "-o", str(obj)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out = {}
    insts = parse(disassemble(obj, tmp))
    for i, (func, op, text, _) in enumerate(insts):
        fam = family(op)
        if fam is None:
            continue
        dst = _regs(text.split()[1].rstrip(","))
        waits = 0
        for _, op2, text2, _ in insts[i + 1:]:
            toks = re.findall(REG, text2)
            if op2.startswith("v_") and len(toks) > 1 and set().union(
                    *(_regs(t) for t in toks[1:])) & dst:
                break
            waits += int(text2.split()[1], 0) + 1 if op2 == "s_nop" else 1
        out[fam] = waits
    assert set(out) == {"f32", "f16", "fp4"}, out
    return out


REG = r"[va]\[\d+:\d+\]|[va]\d+"


def _regs(spec):
    """The vector (v) and accumulation (a) registers of an operand."""
    m = re.match(r"([va])\[(\d+):(\d+)\]$", spec)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", spec)
    return {f"{m.group(1)}{m.group(2)}"} if m else set()


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


def barrier_reads(insts, need):
    """{function: (fewest wait states, the MFMA's need)} between an MFMA and
    a VALU read of its result over paths that cross an s_barrier, keeping
    per function the read with the least to spare; need(op) is the count an
    MFMA's result needs."""
    cap = 2 * max(need("v_mfma_f32_32x32x2_f32"), 20)

    def low(a, b):
        return b if a is None else (a if b is None else min(a, b))

    def walk(j, dst, waits, crossed, seen):
        # seen: the fewest wait states each (instruction, crossed) was reached
        # with; a later arrival with as many or more cannot find fewer
        best = None
        while j < len(insts) and waits < cap:
            if seen.get((j, crossed), 1 << 30) <= waits:
                return best
            seen[(j, crossed)] = waits
            func, op, text, tgt = insts[j]
            j += 1
            if op == "s_endpgm" or op.startswith("v_mfma"):
                return best
            if op == "s_barrier":
                crossed = True
            toks = re.findall(REG, text)
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


def library_objects():
    return sorted(B.BUILD.glob("*.o")) if B.BUILD.exists() else []


def test_probe_counts(required):
    # the counts the ISA table gives for gfx950 (16-pass fp32 MFMA: 18;
    # 8-pass fp16 / FP4 MFMAs: 12), as the compiler applies them
    assert required == {"f32": 18, "f16": 12, "fp4": 12}


def test_mfma_results_read_well_after_barriers(tmp_path, required):
    objs = library_objects()
    if not objs:
        pytest.skip("no built objects (run python -m mlxvs_amd.build)")

    def need(op):
        fam = family(op)
        return (required[fam] if fam else max(required.values())) + MARGIN

    checked = []
    for obj in objs:
        d = tmp_path / obj.stem
        d.mkdir()
        insts = parse(disassemble(obj, d))
        if not any(i[1].startswith("v_mfma") for i in insts):
            continue
        checked.append(obj.name)
        worst = barrier_reads(insts, need)
        if obj.name == "knn_float.o":
            # the fused kernels' buffered select reads its accumulators after
            # the tile barrier: finding none would mean the parser lost the code
            assert any("fused_kernel" in f for f in worst), sorted(worst)[:5]
        low = {f: w for f, w in worst.items() if w[0] < w[1]}
        assert not low, f"{obj.name}: MFMA results read too soon after a barrier " \
                        f"(wait states, needed): {low}"
    # every object with MFMAs (the float and Hamming kernels) was checked
    assert {"knn_float.o", "knn_hamming.o"} <= set(checked), checked


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
    worst = barrier_reads(parse(listing), lambda op: 26)
    # _ZShort: only the barrier and its wait lie between (they count none);
    # _ZLong: the branch skips three of the six nops: 1 + 24 = 25
    assert worst == {"_ZShort": (0, 26), "_ZLong": (25, 26)}
