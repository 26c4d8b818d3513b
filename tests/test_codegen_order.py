"""The cross-workgroup hand-overs of the built library, checked in its gfx950 machine code.

Three kernels add other workgroups' results inside one launch:
* GemvSplitBf16Kernel (the K splits of a column group) and DecodeAttentionKernel (the chunks
  of a head) store their partial results with agent-scope relaxed atomic stores
  (`global_store ... sc1`, written through to the level every XCD reads), bump an arrival
  counter with an agent-scope atomic add, and the workgroup that completes the count reads
  the partials with agent-scope relaxed atomic loads (`global_load ... sc1`);
* GreedyKernel does the same with an acquire-release add (`buffer_wbl2 sc1` before it,
  `buffer_inv sc1` after it).

What makes the hand-over correct is the order of those instructions in the code the compiler
emitted, so this test reads it from `libaccel_hip.so` itself (the device code objects are
unbundled with clang-offload-bundler and disassembled with llvm-objdump), builds each kernel's
control-flow graph, and checks on every path:
1. from a partial store to the counter's add there is an `s_waitcnt vmcnt(0)` (all of the
   thread's stores acknowledged) and, where other threads store, an `s_barrier` (all of the
   workgroup's); with the acquire-release add, a `buffer_wbl2 sc1`;
2. the add returns its value (`sc0`); from it to the barrier that releases the readers there is
   an `s_waitcnt vmcnt(0)` (and, with the acquire-release add, a `buffer_inv sc1`), and no
   agent-scope store;
3. from the kernel's entry to any partial load there is that barrier.
A compiler that hoisted a load above the arrival or sank a store below it fails here.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "accelep_amd" / "libaccel_hip.so"
LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

# (kernel name fragment, other threads store partials (a barrier is needed before the add),
#  acquire-release add)
KERNELS = [
    ("GemvSplitBf16KernelILb1EE", True, False),
    ("GemvSplitBf16KernelILb0EE", True, False),
    ("21DecodeAttentionKernel", True, False),
    ("12GreedyKernel", False, True),
]


def _tool(name):
    path = LLVM / name
    return str(path) if path.exists() else shutil.which(name)


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    """{kernel symbol: [(address, instruction text, branch target address or None)]}."""
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    tools = {n: _tool(n) for n in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")}
    missing = [n for n, p in tools.items() if p is None]
    if missing:
        pytest.skip(f"ROCm LLVM tools missing: {missing}")
    tmp = tmp_path_factory.mktemp("codegen")
    fat = tmp / "fat.bin"
    subprocess.run([tools["llvm-objcopy"], f"--dump-section=.hip_fatbin={fat}", str(LIB), str(tmp / "copy.so")],
                   check=True, capture_output=True)
    data = fat.read_bytes()
    # One offload bundle per translation unit, back to back in the section.
    starts = [m.start() for m in re.finditer(rb"__CLANG_OFFLOAD_BUNDLE__", data)] + [len(data)]
    funcs = {}
    for i, (a, b) in enumerate(zip(starts, starts[1:])):
        bundle = tmp / f"bundle{i}.bin"
        bundle.write_bytes(data[a:b])
        obj = tmp / f"device{i}.o"
        r = subprocess.run([tools["clang-offload-bundler"], "--unbundle", "--type=o", f"--input={bundle}",
                            f"--targets={TARGET}", f"--output={obj}"], capture_output=True, text=True)
        if r.returncode != 0 or not obj.exists() or obj.stat().st_size == 0:
            continue
        dis = subprocess.run([tools["llvm-objdump"], "-d", "--mcpu=gfx950", str(obj)], capture_output=True, text=True,
                             check=True).stdout
        funcs.update(_parse(dis))
    assert funcs, "no gfx950 code object found in the library"
    return funcs


def _parse(dis):
    out = {}
    name = None
    base = 0
    for line in dis.splitlines():
        head = re.match(r"^([0-9a-f]+) <(.+)>:$", line)
        if head:
            base, name = int(head.group(1), 16), head.group(2)
            out[name] = []
            continue
        if name is None:
            continue
        ins = re.match(r"^\s+(\S.*?)\s*//\s*([0-9A-Fa-f]+):", line)
        if not ins:
            continue
        text, addr = ins.group(1).strip(), int(ins.group(2), 16)
        target = None
        if text.startswith(("s_cbranch", "s_branch")):
            t = re.search(r"<([^<>]+?)(?:\+0x([0-9a-f]+))?>\s*$", line)
            assert t and t.group(1) == name, f"branch out of {name}: {line}"
            target = base + int(t.group(2) or "0", 16)
        out[name].append((addr, text, target))
    return out


def _find(funcs, fragment):
    names = [n for n in funcs if fragment in n]
    assert len(names) == 1, f"{fragment}: {names}"
    return names[0], funcs[names[0]]


def _is(text, op, *operands):
    words = text.replace(",", " ").split()
    return words[0].startswith(op) and all(o in words for o in operands)


@pytest.mark.parametrize("fragment,barrier_before_add,acq_rel", KERNELS, ids=[k[0] for k in KERNELS])
def test_partials_are_handed_over_in_order(kernels, fragment, barrier_before_add, acq_rel):
    name, ins = _find(kernels, fragment)
    assert handover_errors(ins, barrier_before_add, acq_rel) == [], name


def test_checker_reports_planted_mistakes(kernels):
    """Each mistake, planted in a copy of the listing, is reported: the checker is not vacuous."""
    _, gemv = _find(kernels, KERNELS[0][0])
    _, greedy = _find(kernels, KERNELS[3][0])
    texts = [t for _, t, _ in gemv]
    ia = next(i for i, t in enumerate(texts) if _is(t, "global_atomic_add", "sc0"))
    bar = next(i for i, t in enumerate(texts) if _is(t, "s_barrier") and i > ia)
    last_store = max(i for i, t in enumerate(texts[:ia]) if _is(t, "global_store", "sc1"))
    first_load = min(i for i, t in enumerate(texts) if _is(t, "global_load", "sc1"))

    def replaced(ins, pick, text="s_nop 0"):
        return [(a, text if pick(i, t) else t, tg) for i, (a, t, tg) in enumerate(ins)]

    # the barrier that releases the readers taken out
    errs = handover_errors(replaced(gemv, lambda i, t: i == bar), True, False)
    assert any("barrier" in e for e in errs), errs
    # the wait for the partial stores taken out
    errs = handover_errors(replaced(gemv, lambda i, t: last_store < i < ia and "vmcnt(0)" in t), True, False)
    assert any("without a wait" in e for e in errs), errs
    # the wait for the add's value taken out
    errs = handover_errors(replaced(gemv, lambda i, t: ia < i < bar and "vmcnt(0)" in t), True, False)
    assert any("follow the add without a wait" in e for e in errs), errs
    # a partial load hoisted above the arrival
    hoisted = gemv[:ia] + [(gemv[ia][0] - 2, gemv[first_load][1], None)] + gemv[ia:]
    errs = handover_errors(hoisted, True, False)
    assert any("without the barrier" in e for e in errs), errs
    # a partial store sunk below the arrival
    sunk = gemv[:ia + 1] + [(gemv[ia][0] + 2, gemv[last_store][1], None)] + gemv[ia + 1:]
    errs = handover_errors(sunk, True, False)
    assert any("store can follow the arrival" in e for e in errs), errs
    # the acquire of the greedy pick's add taken out
    errs = handover_errors(replaced(greedy, lambda i, t: _is(t, "buffer_inv", "sc1")), False, True)
    assert any("without an acquire" in e for e in errs), errs


def handover_errors(ins, barrier_before_add, acq_rel):
    """The ways the listing `ins` breaks the hand-over order (empty when it holds)."""
    texts = [t for _, t, _ in ins]
    adds = [i for i, t in enumerate(texts) if _is(t, "global_atomic_add", "sc0")]
    if len(adds) != 1:
        return [f"expected one returning atomic add, found {len(adds)}"]
    ia = adds[0]
    succ = _successors(ins)
    errors = []

    def where(i):
        return f"+{ins[i][0] - ins[0][0]:#x}"

    def reaches(starts, goals, blocked):
        """Some path from a successor of `starts` reaches `goals` through no `blocked` node."""
        return any(_reaches(succ, n, goals, blocked) for st in starts for n in succ[st])

    waits = {i for i, t in enumerate(texts) if _is(t, "s_waitcnt") and "vmcnt(0)" in t}
    barriers = {i for i, t in enumerate(texts) if _is(t, "s_barrier")}

    # 1. partial stores -> wait (-> barrier / release) -> add
    stores = [i for i, t in enumerate(texts) if _is(t, "global_store", "sc1") and i < ia]
    if not stores:
        errors.append("no agent-scope partial store before the arrival")
    elif reaches(stores, {ia}, waits):
        errors.append("a path from a partial store reaches the add without a wait")
    if stores and barrier_before_add and reaches(stores, {ia}, barriers):
        errors.append("a path from a partial store reaches the add without a barrier")
    if stores and acq_rel:
        wbl2 = {i for i, t in enumerate(texts) if _is(t, "buffer_wbl2", "sc1")}
        if reaches(stores, {ia}, wbl2):
            errors.append("a path from a partial store reaches the add without a release")

    # 2. add -> wait (-> acquire) -> the barrier that releases the readers
    after = [i for i in sorted(barriers) if i > ia]
    if not after:
        return errors + ["no barrier after the arrival"]
    bar = after[0]
    if reaches([ia], {bar}, waits):
        errors.append(f"the barrier at {where(bar)} can follow the add without a wait")
    late = {i for i, t in enumerate(texts) if _is(t, "global_store", "sc1")}
    if reaches([ia], late, {bar}):
        errors.append(f"an agent-scope store can follow the arrival before the barrier at {where(bar)}")
    if acq_rel:
        inv = {i for i, t in enumerate(texts) if _is(t, "buffer_inv", "sc1")}
        if reaches([ia], {bar}, inv):
            errors.append(f"the barrier at {where(bar)} can follow the add without an acquire")

    # 3. entry -> that barrier -> every partial load
    loads = {i for i, t in enumerate(texts) if _is(t, "global_load", "sc1")}
    if not loads:
        errors.append("no agent-scope partial load")
    elif _reaches(succ, 0, loads, {bar}):
        errors.append(f"a partial load is reachable without the barrier at {where(bar)}")
    return errors


def _successors(ins):
    """Control-flow successors of each instruction (by index)."""
    index = {addr: i for i, (addr, _, _) in enumerate(ins)}
    succ = []
    for i, (addr, text, target) in enumerate(ins):
        nxt = [i + 1] if i + 1 < len(ins) else []
        op = text.split()[0]
        if op == "s_endpgm" or op.startswith("s_setpc") or op == "s_trap":
            succ.append([])
        elif target is not None:
            assert target in index, f"branch into the middle of an instruction at {addr:#x}"
            succ.append([index[target]] if op == "s_branch" else nxt + [index[target]])
        else:
            succ.append(nxt)
    return succ


def _reaches(succ, start, goals, blocked):
    seen, todo = set(), [start]
    while todo:
        n = todo.pop()
        if n in seen or n in blocked:
            continue
        if n in goals:
            return True
        seen.add(n)
        todo.extend(succ[n])
    return False
