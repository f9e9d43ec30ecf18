"""Build ``libmlxq.so`` (the C-ABI HIP library) for gfx950 with hipcc.

Usage: ``python -m mlxcel_amd.build`` (also called by ``__graft_entry__.build()``).
Objects go to ``mlxcel_amd/_build/``; the library to ``mlxcel_amd/libmlxq.so``.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmlxq.so")
# bench.py's streaming-read reference kernel, kept out of the C-ABI library
BENCH_LIB = os.path.join(HERE, "libmlxq_bench.so")
BENCH_SOURCES = {"bench_read.hip": []}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-x", "hip",
    # no packed-FP32 VALU instructions (v_pk_fma_f32 and kin) in any kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]

# Per-file extras: the conversion kernels must round exactly like the
# reference's CPU code, so no FMA contraction there.
SOURCES = {
    "api.cpp": [],
    "qmv.hip": [],
    "qmv_rs.hip": [],
    "qmv_fr.hip": [],
    "qmv_b4.hip": [],
    "qmv_mid.hip": [],
    "qmv_mr.hip": [],
    "qmm_group.hip": [],
    "qmm.hip": [],
    "qmm_gen.hip": [],
    "moe.hip": [],
    "bias.hip": [],
    "copy.hip": [],
    "scratch.hip": [],
    "dequant.hip": ["-ffp-contract=off"],
}


def _compile(name: str, extra: list[str]) -> str:
    src = os.path.join(CSRC, name)
    obj = os.path.join(BUILD, name + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {name}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # The host pass does not know the packed-fp32 feature and says so; keep
    # anything else visible.
    noise = ("packed-fp32-ops", "not a recognized feature", "warning generated")
    for line in r.stderr.splitlines():
        if line.strip() and not any(n in line for n in noise):
            print(line, file=sys.stderr)
    return obj


def _verify_group_ring_waits() -> None:
    """qmm_group.hip waits for its LDS ring with a hand-counted
    `s_waitcnt vmcnt(2 n)`: 2 younger blocks of n vector-memory instructions
    each per wave (3 or 4 direct-to-LDS activation loads, one weight load per
    tile of the wave (3 or 2) and, without the LDS scale table, one scale load
    per tile: n = 6 with the table, 8 without).  If the compiler ever emitted a different number per block the
    wait would be wrong, so check each instantiation's AMD assembly (built
    here): 3 blocks before the first wait (and, with the scale table, its one
    staging load ahead of them), then exactly n loads after each of the 4
    waits of a ring turn."""
    src = os.path.join(CSRC, "qmm_group.hip")
    asm = os.path.join(BUILD, "qmm_group.device.s")
    cmd = [HIPCC, *COMMON, "--cuda-device-only", "-S", src, "-o", asm]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for qmm_group.hip:\n{r.stderr}")
    lines = open(asm).read().splitlines()
    prefix = "_ZN4mlxq22qmm_group_mxfp4_kernelILi"
    starts = [i for i, l in enumerate(lines) if l.startswith(prefix) and l.split(";")[0].rstrip().endswith(":")]
    seen = set()
    for start in starts:
        # _ZN4mlxq22qmm_group_mxfp4_kernelILi<SCL>ELi<tiles>EEEv...
        args = lines[start][len(prefix):].split("EEEv", 1)[0]
        scl, tiles = (int(v) for v in args.split("ELi"))
        xi = 4 if tiles == 2 else 3
        n = xi + tiles * (2 if scl == 0 else 1)
        end = next(i for i in range(start, len(lines)) if "s_endpgm" in lines[i])
        body = [l.strip() for l in lines[start:end]]
        wait = f"s_waitcnt vmcnt({2 * n})"
        marks = [i for i, l in enumerate(body) if l == wait and body[i + 1].startswith("s_barrier")]
        if len(marks) != 4:
            raise RuntimeError(f"qmm_group<{scl},{tiles}> ring check: expected 4 ring waits, found {len(marks)}")
        loads = lambda a, b: sum(1 for l in body[a:b] if l.startswith("buffer_load"))
        bounds = marks + [next(i for i in range(marks[-1], len(body)) if body[i].startswith("s_waitcnt vmcnt(0)"))]
        per = [loads(bounds[k] + 1, bounds[k + 1]) for k in range(4)]
        pro = loads(0, marks[0])
        want_pro = 3 * n + (0 if scl == 0 else 1)
        if per != [n] * 4 or pro != want_pro:
            raise RuntimeError(f"qmm_group<{scl},{tiles}> ring check: loads per ring step {per}, prologue {pro} "
                               f"(the kernel's vmcnt({2 * n}) assumes {n} per step and {want_pro} before the first wait)")
        seen.add((scl, tiles))
    if seen != {(0, 2), (4, 2), (16, 2), (4, 3), (16, 3)}:
        raise RuntimeError(f"qmm_group ring check: instantiations {sorted(seen)}")


_MFMA4 = "v_mfma_f32_4x4x4_16b_bf16"
_REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)\b)")


def _regs(operand_text: str) -> set:
    """The VGPRs / AGPRs an operand list names, as (file, index) pairs."""
    out = set()
    for kind, lo, hi, one in _REG.findall(operand_text):
        a, b = (int(lo), int(hi)) if lo else (int(one), int(one))
        out |= {(kind, k) for k in range(a, b + 1)}
    return out


def check_b4_mfma_chains(asm_text: str) -> int:
    """qmv_b4.hip writes its 4x4x4 MFMA accumulation chains as inline
    assembly, which the compiler's hazard recognizer does not see, so the
    wait states and register ties are the kernel's own.  Checks them in AMD
    assembly text: each MFMA's destination is disjoint from its A and B
    operands and its C operand is 0 or the destination itself; an `s_nop` of
    at least 1 (2 wait states) sits right before it; and after a chain's last
    MFMA, s_nop wait states add up to 16 before any other instruction names a
    destination register or the basic block ends.  Returns the number of
    MFMAs checked; raises RuntimeError at the first violation."""
    code = [l.split(";")[0].strip() for l in asm_text.splitlines()]
    code = [l for l in code if l and not l.startswith(".")]
    block_end = ("s_branch", "s_cbranch", "s_setpc", "s_endpgm")
    count = 0
    for i, ins in enumerate(code):
        if not ins.startswith(_MFMA4):
            continue
        count += 1
        ops = [o.strip() for o in ins[len(_MFMA4):].split(",")]
        d, a, b, c = (_regs(o) for o in ops[:4])
        where = f"qmv_b4 MFMA chain check, instruction {count} ({ins})"
        if d & (a | b):
            raise RuntimeError(f"{where}: destination overlaps A or B")
        if ops[3] != "0" and c != d:
            raise RuntimeError(f"{where}: C operand is neither 0 nor the destination")
        nop = re.fullmatch(r"s_nop (\d+)", code[i - 1])
        if not nop or int(nop.group(1)) < 1:
            raise RuntimeError(f"{where}: preceded by '{code[i - 1]}', not s_nop >= 1")
        waits = 0
        for nxt in code[i + 1:]:
            m = re.fullmatch(r"s_nop (\d+)", nxt)
            if m:
                waits += int(m.group(1)) + 1
                continue
            ends = nxt.endswith(":") or nxt.startswith(block_end)
            if not ends and not (_regs(nxt) & d):
                continue
            if nxt.startswith(_MFMA4):
                o2 = [o.strip() for o in nxt[len(_MFMA4):].split(",")]
                if _regs(o2[0]) == d and _regs(o2[3]) == d:
                    break  # the chain goes on
            if waits < 16:
                raise RuntimeError(f"{where}: result reached '{nxt}' after {waits} wait states (needs 16)")
            break
    if count == 0:
        raise RuntimeError("qmv_b4 MFMA chain check: no 4x4x4 MFMA found in the assembly")
    return count


B4_ASM = os.path.join(BUILD, "qmv_b4.device.s")


def _verify_b4_mfma_chains() -> None:
    """Builds qmv_b4.hip's AMD assembly and checks its MFMA chains."""
    src = os.path.join(CSRC, "qmv_b4.hip")
    cmd = [HIPCC, *COMMON, "--cuda-device-only", "-S", src, "-o", B4_ASM]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for qmv_b4.hip:\n{r.stderr}")
    check_b4_mfma_chains(open(B4_ASM).read())


def build(verbose: bool = True) -> str:
    """Compile every source and link libmlxq.so; always rebuilds."""
    if not os.path.exists(HIPCC) and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    os.makedirs(BUILD, exist_ok=True)
    srcs = {k: v for k, v in SOURCES.items() if os.path.exists(os.path.join(CSRC, k))}
    with ThreadPoolExecutor(max_workers=min(4, len(srcs))) as ex:
        objs = list(ex.map(lambda kv: _compile(*kv), srcs.items()))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    _verify_group_ring_waits()
    _verify_b4_mfma_chains()
    bobjs = [_compile(k, v) for k, v in BENCH_SOURCES.items()]
    tmp = BENCH_LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *bobjs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, BENCH_LIB)
    if verbose:
        print(f"built {LIB} and {BENCH_LIB}")
    return LIB


if __name__ == "__main__":
    build()
