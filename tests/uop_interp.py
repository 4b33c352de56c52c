"""A CPU interpreter of linear kernel listings (test infrastructure).

It executes ``uop/linearize.py``'s listings work-item by work-item over numpy arrays, with
numpy scalar arithmetic of each dtype (integers wrap, floats round as numpy rounds them), so the
linearizer's index arithmetic, loops, gates and accumulators are checked on the CPU
independently of the HIP renderer.  The work-items of a workgroup share its DEFINE_LOCAL arrays
and run in turns between BARRIERs (each runs until its next barrier, then the next one runs).
bf16 and FP8 are not interpreted.
"""

from __future__ import annotations

import warnings

import numpy as np

NP = {"bool": np.bool_, "int8": np.int8, "uint8": np.uint8, "int16": np.int16, "uint16": np.uint16,
      "int32": np.int32, "uint32": np.uint32, "int64": np.int64, "uint64": np.uint64, "float16": np.float16,
      "float32": np.float32, "float64": np.float64}


def _alu(op: str, dt: str, v: list):
    t = NP[dt]
    if op == "WHERE":
        return v[1] if v[0] else v[2]
    if op == "CMPLT":
        return np.bool_(v[0] < v[1])
    if op == "CMPNE":
        return np.bool_(v[0] != v[1])
    if op == "CMPEQ":
        return np.bool_(v[0] == v[1])
    if op == "ADD":
        return t(v[0] + v[1])
    if op == "SUB":
        return t(v[0] - v[1])
    if op == "MUL":
        return t(v[0] * v[1])
    if op == "MAX":
        return t(max(v[0], v[1]))
    if op == "IDIV":
        q = abs(int(v[0])) // abs(int(v[1]))
        return t(q if (v[0] < 0) == (v[1] < 0) else -q)
    if op == "MOD":
        return t(int(v[0]) - int(v[1]) * int(_alu("IDIV", dt, v)))
    if op == "FDIV":
        return t(v[0] / v[1])
    if op == "NEG":
        return t(-v[0])
    if op == "AND":
        return t(v[0] & v[1])
    if op == "OR":
        return t(v[0] | v[1])
    if op == "XOR":
        return t(v[0] ^ v[1])
    if op == "SHL":
        return t(v[0] << v[1])
    if op == "SHR":
        return t(v[0] >> v[1])
    if op == "MULACC":
        return t(v[0] * v[1] + v[2])
    if op == "SQRT":
        return t(np.sqrt(v[0]))
    if op == "RECIPROCAL":
        return t(t(1) / v[0])
    if op == "EXP2":
        return t(np.exp2(v[0]))
    if op == "LOG2":
        return t(np.log2(v[0]))
    if op == "SIN":
        return t(np.sin(v[0]))
    if op == "TRUNC":
        return t(np.trunc(v[0]))
    raise NotImplementedError(op)


def run(listing, buffers: dict[int, np.ndarray], var_vals: dict[str, int] | None = None) -> None:
    """Execute ``listing`` for every work-item; ``buffers`` maps PARAM slots to flat arrays that
    stores write in place."""
    uops = listing.uops
    var_vals = var_vals or {}
    # matching block ends
    ends, stack = {}, []
    for i, u in enumerate(uops):
        if u.op.name in ("RANGE", "IF"):
            stack.append(i)
        elif u.op.name in ("END", "ENDIF"):
            ends[stack.pop()] = i
    groups, local = listing.global_size[0], listing.local_size[0]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        for g in range(groups):
            shared: dict[int, np.ndarray] = {}
            items = [_item(uops, ends, buffers, var_vals, g, lid, shared) for lid in range(local)]
            while items:  # one turn: every live work-item runs to its next barrier
                alive = []
                for it in items:
                    try:
                        next(it)
                        alive.append(it)
                    except StopIteration:
                        pass
                if alive and len(alive) != len(items):
                    raise AssertionError("work-items of one workgroup reached different barriers")
                items = alive


def _item(uops, ends, buffers, var_vals, gidx, lidx, shared):
    val: dict[int, object] = {}
    ptr: dict[int, tuple] = {}
    regs: dict[int, np.ndarray] = {}
    loops: list[tuple[int, int, int]] = []  # (range position, counter, bound)
    pc = 0

    def get(s):
        return NP[s.dtype.name](s.arg) if s.op.name == "CONST" else val[id(s)]

    while pc < len(uops):
        u = uops[pc]
        op, dt = u.op.name, (u.dtype.name if u.dtype is not None else None)
        if op == "PARAM":
            pass
        elif op == "DEFINE_VAR":
            val[id(u)] = np.int32(var_vals[u.arg[0]])
        elif op == "CONST":
            val[id(u)] = NP[dt](u.arg)
        elif op == "SPECIAL":
            val[id(u)] = np.int32(gidx if u.arg.startswith("g") else lidx)
        elif op == "DEFINE_REG":
            regs[id(u)] = np.zeros(u.arg[0], NP[dt])
        elif op == "DEFINE_LOCAL":
            regs[id(u)] = shared.setdefault(id(u), np.zeros(u.arg[0], NP[dt]))
        elif op == "BARRIER":
            yield
        elif op == "INDEX":
            base = u.src[0]
            arr = regs[id(base)] if base.op.name in ("DEFINE_REG", "DEFINE_LOCAL") else buffers[base.arg.slot]
            gate = bool(get(u.src[2])) if len(u.src) > 2 else True
            ptr[id(u)] = (arr, int(get(u.src[1])), gate)
        elif op == "LOAD":
            arr, i, gate = ptr[id(u.src[0])]
            if gate:
                if not 0 <= i < len(arr):  # a device would read outside the buffer
                    raise IndexError(f"load of element {i} of a {len(arr)}-element buffer")
                val[id(u)] = arr[i]
            else:
                val[id(u)] = get(u.src[1]) if len(u.src) > 1 else NP[dt](0)
        elif op == "STORE":
            arr, i, gate = ptr[id(u.src[0])]
            if gate:
                if not 0 <= i < len(arr):
                    raise IndexError(f"store to element {i} of a {len(arr)}-element buffer")
                arr[i] = get(u.src[1])
        elif op == "RANGE":
            bound = int(get(u.src[0]))
            if bound <= 0:
                pc = ends[pc] + 1
                continue
            loops.append((pc, 0, bound))
            val[id(u)] = np.int32(0)
        elif op == "END":
            start, count, bound = loops[-1]
            if count + 1 < bound:
                loops[-1] = (start, count + 1, bound)
                val[id(uops[start])] = np.int32(count + 1)
                pc = start + 1
                continue
            loops.pop()
        elif op == "IF":
            if not get(u.src[0]):
                pc = ends[pc] + 1
                continue
        elif op == "ENDIF":
            pass
        elif op == "CAST":
            val[id(u)] = NP[dt](get(u.src[0]))
        elif op == "BITCAST":
            val[id(u)] = np.array(get(u.src[0])).view(NP[dt])[()]
        else:
            val[id(u)] = _alu(op, dt, [get(s) for s in u.src])
        pc += 1
