"""CPU check of the gfx950 assembly of the library kernels (compiled here with hipcc -S).

The decode LDS/stream/ring kernels and the wide prefill kernels issue loads through inline asm (global_load_* into VGPRs, ds_read_b128)
so that the compiler's conservative waits do not serialise the weight stream.  The compiler does
not know those registers are written asynchronously, so the kernel re-binds them after each
explicit wait.  This test proves, for every instantiation, that no instruction reads or writes a
register of an in-flight untracked load before the explicit s_waitcnt that completes it (such an
access once turned an in-flight load into a wild address), and that no kernel spills to scratch.
"""
from __future__ import annotations

import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "w4a16-gemm_amd", "csrc")
HIPCC = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")


def _vregs(tok: str):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _parse(lines):
    """Instructions as (line, mnemonic, register args, in_asm, text) plus label -> index."""
    ins, labels, in_asm = [], {}, False
    for i, raw in enumerate(lines):
        t = raw.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        m = re.match(r"^(\.LBB\w+):", t)
        if m:
            labels[m.group(1)] = len(ins)
            continue
        if not t or t.startswith(";") or t.startswith(".") or t.endswith(":"):
            continue
        parts = t.split(None, 1)
        args = [a.strip().split()[0] for a in parts[1].split(",")] if len(parts) > 1 else []
        ins.append((i, parts[0], args, in_asm, t))
    return ins, labels


def _merge(a, b):
    """Join of two states: vmem queues aligned at their most recent op (element-wise union)."""
    qa, qb = a[0], b[0]
    n = max(len(qa), len(qb))
    qa = [frozenset()] * (n - len(qa)) + list(qa)
    qb = [frozenset()] * (n - len(qb)) + list(qb)
    return (tuple(x | y for x, y in zip(qa, qb)), a[1] | b[1])


def _step(state, ins, hazards=None):
    """Transfer function of one instruction; records hazards when a list is given."""
    queue, lgkm = list(state[0]), set(state[1])
    line, mnem, args, in_asm, t = ins
    if mnem == "s_waitcnt":
        m = re.search(r"vmcnt\((\d+)\)", t)
        if m:
            n = int(m.group(1))
            queue = queue[len(queue) - n:] if n < len(queue) else queue
        if "lgkmcnt(0)" in t and in_asm:
            lgkm = set()
        return (tuple(queue), frozenset(lgkm))
    pending = set(lgkm)
    for regs in queue:
        pending |= regs
    regs_here = set()
    for a in args:
        regs_here |= _vregs(a)
    # An LDS DMA (global_load_lds_*) writes LDS, not registers: its first operand is the address.
    lds_dma = mnem.startswith("global_load_lds")
    untracked = in_asm and ((mnem.startswith("global_load") and not lds_dma) or mnem.startswith("ds_read"))
    dst = _vregs(args[0]) if (untracked and args) else set()
    bad = sorted(((regs_here - dst) | (dst if untracked else set())) & pending)
    if bad and hazards is not None:
        hazards.append(f"line {line}: {t} touches pending v{bad}")
    if mnem.startswith("global_") or mnem.startswith("buffer_"):
        queue.append(frozenset(dst) if (untracked and mnem.startswith("global_load")) else frozenset())
        if len(queue) > 256:                               # fold the oldest entries together
            queue = [queue[0] | queue[1]] + queue[2:]
    if untracked and mnem.startswith("ds_read"):
        lgkm |= dst
    return (tuple(queue), frozenset(lgkm))


def check_kernel(lines):
    """Return a list of hazard descriptions for one kernel's assembly lines.

    Dataflow over the control-flow graph.  Every vector-memory instruction (global_*, buffer_*,
    including the LDS DMAs) is queued in issue order and `s_waitcnt vmcnt(n)` completes all but
    the n most recent.  Untracked loads are the loads inside inline-asm blocks; their destination
    registers stay pending until completed.  LDS reads inside asm blocks are pending until an asm
    `s_waitcnt lgkmcnt(0)`.  Any other instruction naming a pending register is a hazard."""
    ins, labels = _parse(lines)
    starts = sorted({0} | set(labels.values()) |
                    {k + 1 for k, x in enumerate(ins) if x[1].startswith("s_branch") or x[1].startswith("s_cbranch")
                     or x[1] == "s_endpgm"})
    starts = [b for b in starts if b < len(ins)]
    block_of = {b: j for j, b in enumerate(starts)}
    ends = starts[1:] + [len(ins)]
    succ = []
    for b, e in zip(starts, ends):
        last = ins[e - 1]
        tgt = [labels[a] for a in last[2] if a in labels] if last[1].startswith("s_") and "branch" in last[1] else []
        nxt = [e] if e < len(ins) and not last[1].startswith("s_branch") and last[1] != "s_endpgm" else []
        succ.append([block_of[x] for x in tgt + nxt if x in block_of])
    empty = ((), frozenset())
    inp = {0: empty}
    work = [0]
    while work:
        j = work.pop()
        st = inp[j]
        for x in ins[starts[j]:ends[j]]:
            st = _step(st, x)
        for k in succ[j]:
            new = st if k not in inp else _merge(inp[k], st)
            if k not in inp or new != inp[k]:
                inp[k] = new
                work.append(k)
    hazards = []
    for j, b in enumerate(starts):
        if j not in inp:
            continue
        st = inp[j]
        for x in ins[b:ends[j]]:
            st = _step(st, x, hazards)
    return hazards


@pytest.fixture(scope="module")
def isa(tmp_path_factory):
    """Device assembly of every HIP source of the library, compiled with its build flags."""
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    import sys
    sys.path.insert(0, os.path.join(ROOT, "w4a16-gemm_amd"))
    import build
    d = tmp_path_factory.mktemp("isa")
    text = []
    for src, _ in build.SOURCES:
        if not src.endswith(".hip"):
            continue
        out = d / (src + ".s")
        flags = [f for f in build.compile_flags(src) if f != "-fPIC"]
        subprocess.run([HIPCC, *flags, "-S", "--cuda-device-only", os.path.join(CSRC, src), "-o", str(out)],
                       check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
        text.append(out.read_text())
    return "\n".join(text)


def _kernels(text):
    ks = {}
    for m in re.finditer(r"^(_ZN5w4a16\w+):", text, re.M):
        end = text.find("s_endpgm", m.end())
        ks[m.group(1)] = text[m.end():end].splitlines()
    return ks


def test_untracked_load_registers_untouched_until_waited(isa):
    ks = _kernels(isa)
    lds = [k for k in ks if any(n in k for n in ("decode_stream_kernel", "decode_ring_kernel",
                                                  "prefill_wide_kernel", "prefill_wide_pipe_kernel",
                                                  "prefill_stream_kernel",
                                                  "prefill_group_kernel"))]
    assert len(lds) >= 16 + 20 + 3 + 2 + 2, list(ks)
    problems = {k: check_kernel(ks[k]) for k in lds}
    bad = {k: v[:5] for k, v in problems.items() if v}
    assert not bad, bad


def test_checker_flags_a_hoisted_use():
    """The checker itself catches the failure pattern (use of an in-flight asm-load register)."""
    lines = [";;#ASMSTART", "global_load_dwordx4 v[2:5], v[8:9], off", ";;#ASMEND",
             "v_permlane32_swap_b32_e32 v2, v4", ";;#ASMSTART", "s_waitcnt vmcnt(0)", ";;#ASMEND"]
    assert check_kernel(lines)
    ok = [";;#ASMSTART", "global_load_dwordx4 v[2:5], v[8:9], off", ";;#ASMEND",
          ";;#ASMSTART", "s_waitcnt vmcnt(0)", ";;#ASMEND", "v_permlane32_swap_b32_e32 v2, v4"]
    assert not check_kernel(ok)


def test_checker_treats_lds_dma_operands_as_inputs():
    """An asm LDS DMA's VGPR operand is its address (reusable at once); an asm register load's
    first operand is a destination (pending until its wait)."""
    dma = [";;#ASMSTART", "s_mov_b32 m0, s4", "global_load_lds_dword v7, s[2:3]", ";;#ASMEND", "v_xor_b32_e32 v8, 4, v7"]
    assert not check_kernel(dma)
    reg = [";;#ASMSTART", "global_load_dword v7, v[2:3], off", ";;#ASMEND", "v_xor_b32_e32 v8, 4, v7"]
    assert check_kernel(reg)


def test_no_bit_cast_of_vector_element():
    """clang (ROCm 7.2) lowers __builtin_bit_cast(T, v.y) as a load from &v, i.e. it reads v.x;
    the device sources must copy a vector element to a scalar before bit-casting it."""
    bad = []
    for name in os.listdir(CSRC):
        if name.endswith((".hip", ".h")):
            for i, line in enumerate(open(os.path.join(CSRC, name)), 1):
                if re.search(r"__builtin_bit_cast\([^,]+,\s*[\w\[\]]+(\.[xyzw]|\[\d+\])\s*\)", line):
                    bad.append(f"{name}:{i}: {line.strip()}")
    assert not bad, bad


def test_no_kernel_spills(isa):
    sizes = re.findall(r"; ScratchSize: (\d+)", isa)
    assert sizes and all(int(s) == 0 for s in sizes), sizes


def _loop_bodies(lines):
    """Instruction texts of each innermost loop (from a 'Loop Header' label to its back-branch)."""
    items, heads = [], []
    for raw in lines:
        t = raw.strip()
        if "Loop Header" in t:
            heads.append((len(items), t.split(":")[0]))
        if not t or t.startswith(";") or (t.startswith(".") and "Loop Header" not in t):
            continue
        items.append(t)
    loops = []
    for start, label in heads:
        end = next((i for i in range(start + 1, len(items)) if "cbranch" in items[i] and label in items[i]), None)
        if end is not None:
            loops.append(items[start:end + 1])
    return loops


def test_wide_prefill_accumulators_stay_in_place(isa):
    """The wide prefill main loop keeps its MFMA accumulators in place: no accumulator register
    copies or AGPR<->VGPR transfers (the default scheduler's allocation rotated them through
    copies, serialising the MFMA pipe)."""
    ks = {k: v for k, v in _kernels(isa).items() if "prefill_wide_kernel" in k or "prefill_wide_pipe_kernel" in k}
    # ten configs (one of them the pipelined kernel), six of them also with the second
    # accumulator set of the long-K segments (Lb1E; checked for spills and load hazards by the
    # tests above, their loop holds the segment-close branch)
    assert len(ks) == 16 and sum("Lb1E" in k for k in ks) == 6, list(ks)
    for name, lines in ks.items():
        if "Lb1E" in name:
            continue
        bm, bn, wm, wn, _, depth = (int(v) for v in
                                    re.search(r"ILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELb0ELi(\d+)EE", name).groups())
        tm, tn = bm // wm // 32, bn // wn // 32
        loops = [l for l in _loop_bodies(lines) if any("v_mfma" in t for t in l)]
        assert len(loops) == 1, (name, len(loops))
        ops = [t.split()[0] for t in loops[0]]
        # `depth` chunks per loop iteration; one chunk of a (32 tm) x (32 tn) wave tile = 8 tm tn
        # 16x16x32 MFMAs' work (a 32x32x16 counts twice)
        work = ops.count("v_mfma_f32_16x16x32_f16") + 2 * ops.count("v_mfma_f32_32x32x16_f16")
        assert work == 8 * tm * tn * depth, (name, work)
        moves = [o for o in ops if o.startswith("v_accvgpr")]
        assert not moves, (name, len(moves))
