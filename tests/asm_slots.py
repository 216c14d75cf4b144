"""Static check of the persistent verify kernel's inline-asm weight ring.

k_mk2's compute waves stream weights through a ring of AGPR slots: an inline
`global_load ... ; SLOTLOAD` writes a slot, and a later inline
`s_waitcnt vmcnt(N) ; SLOTWAIT <slot registers>` must guarantee that load has
landed before anything reads the slot.  The compiler cannot see either
(inline asm), so two invariants hold only by construction and a compiler or
source change can silently break them:

1. no instruction other than the slot's own SLOTWAIT touches a slot register
   while its load may still be in flight (the compiler may move or copy
   registers around inline asm it does not understand);
2. at each SLOTWAIT, vmcnt(N) really covers the named slot's load: on this
   architecture the vector-memory counter retires in order, so a load is
   complete after `vmcnt(N)` only if at least N vector-memory instructions
   were issued after it on EVERY path to the wait.

The checker parses the AMD assembly of the kernel (built here from source),
splits it into basic blocks, and runs a forward dataflow analysis over the
compute-wave path (from the `; CPATH_BEGIN` marker, up to the IO-wave path):
the state maps each in-flight slot register to the minimum number of
vector-memory instructions issued after its load over all paths (the join is
the minimum, so the analysis is conservative).
"""
import re

VMEM_PREFIX = ("global_", "buffer_", "flat_", "scratch_")
BRANCH = ("s_branch", "s_cbranch")
CAP = 1 << 10
_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_VMCNT = re.compile(r"vmcnt\((\d+)\)")


def regs(text):
    """The v/a registers an instruction names."""
    out = set()
    for m in _REG.finditer(text):
        if m.group(2) is not None:
            out |= {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
        else:
            out.add((m.group(4), int(m.group(5))))
    return out


def parse(lines):
    """(kind, text) items: 'label', 'op', and the inline-asm kinds 'load'
    (SLOTLOAD), 'wait' (SLOTWAIT), 'asm' (any other inline asm)."""
    items, in_asm, buf = [], False, []
    for line in lines:
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm, buf = True, []
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            t = " ".join(buf)
            items.append(("load" if "SLOTLOAD" in t else "wait" if "SLOTWAIT" in t else "asm", t))
            continue
        if in_asm:
            buf.append(s)
            continue
        if not s or s.startswith(";"):
            continue
        if re.match(r"^[.\w$]+:", s) and not s.startswith(".") or re.match(r"^\.LBB\w*:", s):
            items.append(("label", s.split(":")[0]))
            continue
        if s.startswith("."):
            continue
        items.append(("op", s))
    return items


def blocks_of(items):
    blocks, cur = [], []
    for k, t in items:
        if k == "label":
            if cur:
                blocks.append(cur)
            cur = [(k, t)]
            continue
        cur.append((k, t))
        if k == "op" and (t.startswith(BRANCH) or t.startswith(("s_endpgm", "s_setpc"))):
            blocks.append(cur)
            cur = []
    if cur:
        blocks.append(cur)
    labels = {b[0][1]: i for i, b in enumerate(blocks) if b[0][0] == "label"}
    succ = {}
    for i, b in enumerate(blocks):
        k, t = b[-1]
        s = []
        if k == "op" and t.startswith("s_branch"):
            s = [labels[t.split()[1]]]
        elif k == "op" and t.startswith(("s_endpgm", "s_setpc")):
            s = []
        else:
            if k == "op" and t.startswith("s_cbranch"):
                s.append(labels[t.split()[1]])
            if i + 1 < len(blocks):
                s.append(i + 1)
        succ[i] = s
    return blocks, succ


def _step(item, state, report, where):
    """Apply one item to state {reg: min VMEM ops issued after its load};
    report(msg) is called for violations."""
    k, t = item
    vm = _VMCNT.search(t)
    if k == "load":
        for r in state:
            state[r] = min(CAP, state[r] + 1)
        dest = t.split()[1].rstrip(",")
        for r in regs(dest):
            state[r] = 0
        return
    if k == "wait":
        n = int(vm.group(1))
        for r in [r for r, c in state.items() if c >= n]:
            del state[r]
        named = regs(t.split("SLOTWAIT", 1)[1])
        left = named & set(state)
        if left:
            report(f"{where}: SLOTWAIT vmcnt({n}) does not cover its slot "
                   f"{sorted(left)[:4]} (too few vector-memory ops issued after the load)")
            for r in left:
                del state[r]
        return
    # an ordinary instruction or other inline asm
    if vm and "s_waitcnt" in t:
        n = int(vm.group(1))
        for r in [r for r, c in state.items() if c >= n]:
            del state[r]
    touched = regs(t) & set(state)
    if touched:
        report(f"{where}: '{t[:90]}' touches in-flight slot register(s) {sorted(touched)[:4]}")
    if k == "op" and t.startswith(VMEM_PREFIX):
        for r in state:
            state[r] = min(CAP, state[r] + 1)


def check(asm_text, begin="CPATH_BEGIN", end="IOPATH_BEGIN"):
    """Returns (violations, stats) for the paths from every block holding
    the `begin` marker (one per instantiation of the kernel; blocks holding
    `end` are not entered); stats are summed over them."""
    blocks, succ = blocks_of(parse(asm_text.split("\n")))
    starts = [i for i, b in enumerate(blocks) if any(begin in t for _, t in b)]
    if not starts:
        raise ValueError(f"no '{begin}' marker")
    bad, total = [], {"paths": len(starts), "blocks": 0, "slot_loads": 0, "slot_waits": 0,
                      "iterations": 0}
    for st in starts:
        b, s = _check_from(blocks, succ, st, end)
        bad += b
        for k in ("blocks", "slot_loads", "slot_waits"):
            total[k] += s[k]
        total["iterations"] = max(total["iterations"], s["iterations"])
    return sorted(set(bad)), total


def _check_from(blocks, succ, start, end):
    stop = {i for i, b in enumerate(blocks) if any(end in t for _, t in b)}
    starts = [start]
    reach, todo = set(), [starts[0]]
    while todo:
        x = todo.pop()
        if x in reach or x in stop:
            continue
        reach.add(x)
        todo += succ[x]
    for i in reach:
        k, t = blocks[i][-1]
        if k == "op" and t.startswith("s_setpc"):
            raise ValueError("calls on the compute path are not analysed")
    IN = {i: None for i in reach}
    IN[starts[0]] = {}

    def run(i, report):
        st = dict(IN[i])
        for j, it in enumerate(blocks[i]):
            _step(it, st, report, f"block {i} item {j}")
        return st

    changed, iters = True, 0
    while changed:
        changed, iters = False, iters + 1
        if iters > 500:
            raise RuntimeError("dataflow did not converge")
        for i in sorted(reach):
            if IN[i] is None:
                continue
            out = run(i, lambda m: None)
            for j in succ[i]:
                if j not in reach:
                    continue
                if IN[j] is None:
                    IN[j] = dict(out)
                    changed = True
                    continue
                for r, c in out.items():
                    if r not in IN[j] or c < IN[j][r]:
                        IN[j][r] = c if r not in IN[j] else min(c, IN[j][r])
                        changed = True
    bad = []
    for i in sorted(reach):
        if IN[i] is not None:
            run(i, bad.append)
    n_load = sum(1 for i in reach for k, _ in blocks[i] if k == "load")
    n_wait = sum(1 for i in reach for k, _ in blocks[i] if k == "wait")
    return sorted(set(bad)), {"blocks": len(reach), "slot_loads": n_load, "slot_waits": n_wait,
                              "iterations": iters}
