"""Static check of the wide GEMM's gfx950 code (hipcc -S here, no GPU). Its inline-asm buffer loads
are asynchronous and the compiler does not know when their destination registers are written: every
read or write of such a register must come after an s_waitcnt vmcnt that has retired the load
(vector-memory operations retire in issue order, so vmcnt(N) retires all but the last N). The last
K groups issue loads for groups past the end of the tile that nothing in the K loop waits for; if
the epilogue reused one of their registers before a wait, a late load would overwrite it (an
address register turned to 0 faults the store that uses it).

The check is a data-flow pass over the basic blocks of each kernel: the state is the ordered list of
outstanding vector-memory operations with the registers of those that are inline-asm loads; at a
join the lists are aligned at their most recent entries and merged."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "comfy-quant-bench_amd", "csrc", "mq_gemm_wide.hip")
GEN = os.path.join(ROOT, "comfy-quant-bench_amd", "_build", "gen")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")

KERNEL = re.compile(r"^(_ZN2mq12_GLOBAL__N_116gemm_wide_kernel\w+):")


def vregs(tok):
    m = re.match(r"^v\[(\d+):(\d+)\]$", tok)
    if m:
        return frozenset(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"^v(\d+)$", tok)
    return frozenset({int(m.group(1))}) if m else frozenset()


def parse(body):
    """[(kind, op or label, args, is an inline-asm load into registers)]"""
    ins, in_asm = [], False
    for line in body:
        if ";;#ASMSTART" in line:
            in_asm = True
            continue
        if ";;#ASMEND" in line:
            in_asm = False
            continue
        t = line.split(";")[0].strip()
        m = re.match(r"^(\.LBB\w+):", t)
        if m:
            ins.append(("label", m.group(1), [], False))
            continue
        if not t or t.startswith("."):
            continue
        parts = t.split(None, 1)
        args = [a.strip() for a in parts[1].split(",")] if len(parts) > 1 else []
        asm_load = in_asm and parts[0].startswith("buffer_load") and not t.endswith(" lds")
        ins.append(("op", parts[0], args, asm_load))
    return ins


def blocks(ins):
    """Basic blocks (lists of instruction indices) and their successor blocks."""
    starts = {0}
    for i, (kind, op, _, _) in enumerate(ins):
        if kind == "label":
            starts.add(i)
        elif op.startswith(("s_branch", "s_cbranch")) or op == "s_endpgm":
            starts.add(i + 1)
    starts = sorted(s for s in starts if s < len(ins))
    bl = [list(range(s, e)) for s, e in zip(starts, starts[1:] + [len(ins)])]
    label_block = {ins[b[0]][1]: k for k, b in enumerate(bl) if ins[b[0]][0] == "label"}
    succ = []
    for k, b in enumerate(bl):
        kind, op, args, _ = ins[b[-1]]
        s = []
        if kind == "op" and op.startswith(("s_branch", "s_cbranch")):
            s.append(label_block[args[0]])
            if op.startswith("s_cbranch") and k + 1 < len(bl):
                s.append(k + 1)
        elif not (kind == "op" and op == "s_endpgm") and k + 1 < len(bl):
            s.append(k + 1)
        succ.append(s)
    return bl, succ


def merge(a, b):
    n = max(len(a), len(b))
    a = (frozenset(),) * (n - len(a)) + tuple(a)
    b = (frozenset(),) * (n - len(b)) + tuple(b)
    return tuple(x | y for x, y in zip(a, b))[-64:]


def hazards(body):
    ins = parse(body)
    bl, succ = blocks(ins)
    entry, work, found = {0: ()}, [0], set()
    while work:
        k = work.pop()
        state = list(entry[k])
        for i in bl[k]:
            kind, op, args, asm_load = ins[i]
            if kind != "op":
                continue
            if op == "s_waitcnt":
                m = re.search(r"vmcnt\((\d+)\)", " ".join(args))
                if m and len(state) > int(m.group(1)):
                    state = state[len(state) - int(m.group(1)):]
                continue
            touched = frozenset().union(*(vregs(a) for a in args)) if args else frozenset()
            pending = frozenset().union(*state) if state else frozenset()
            if touched & pending:
                found.add((i, op, tuple(sorted(touched & pending))))
            if op.startswith(("buffer_", "global_", "scratch_", "flat_")):
                state = (state + [vregs(args[0]) if asm_load else frozenset()])[-64:]
        for s in succ[k]:
            new = merge(entry[s], state) if s in entry else tuple(state)
            if entry.get(s) != new:
                entry[s] = new
                work.append(s)
    return sorted(found)


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("asm") / "wide.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "-w", "-I", GEN, "--cuda-device-only", "-S", SRC, "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text().split("\n")


def test_async_load_registers_untouched_until_waited(asm):
    seen = 0
    for i, line in enumerate(asm):
        m = KERNEL.match(line)
        if not m:
            continue
        end = next(j for j in range(i, len(asm)) if asm[j].startswith(".Lfunc_end"))
        found = hazards(asm[i:end])
        seen += 1
        assert not found, f"{m.group(1)}: registers of pending inline-asm loads touched: {found[:4]}"
    assert seen >= 12
