"""Scheduled kernel -> linear kernel listing (the codegen step between a SINK and the renderer).

A scheduled kernel (``ops.py``) is a SINK over ``END(STORE(INDEX(param, i), value), *ranges)``
items: every item stores one value per point of its ranges, and REDUCE nodes inside the values
fold their own ranges.  The listing assigns one work-item to each point of the stored ranges
and turns every REDUCE into a loop over its ranges with a register accumulator:

* work-item ``g = gidx0 * L + lidx0`` (``L`` work-items per workgroup), guarded by ``g < total``;
  the stored ranges are the digits of ``g`` in their own bounds, the last range fastest;
* ``REDUCE(x, *r, arg=op)``: ``DEFINE_REG`` accumulator set to op's identity, ``RANGE`` loops over
  ``r`` (``END`` closes each), the accumulator updated with ``x`` inside; the parts of ``x`` that
  do not depend on ``r`` are computed once, before the loops;
* an ``INDEX`` read as a value becomes a ``LOAD`` (a gated index loads 0 where its gate is false);
  an ``INDEX`` a STORE writes through stays an address.

When every REDUCE of the stored values folds at least ``GROUP_MIN`` points over constant bounds
and none is nested in another, one workgroup computes each stored point instead: work-item
``lidx0`` folds points ``lidx0, lidx0 + L, ...`` of each reduction into its register accumulator
(the last chunk's surplus work-items read a valid point and fold the identity), the
accumulators meet in a ``DEFINE_LOCAL`` array by a halving tree with a ``BARRIER`` after every
level, and work-item 0 stores.

The listing uses tinygrad's codegen ops (SPECIAL, DEFINE_REG, RANGE/END, IF/ENDIF, LOAD, STORE),
so ``MI355XRenderer.render`` renders it as it would render a listing made by tinygrad.  The
reference hands this step to tinygrad (its renderer receives tinygrad's listing,
alexandreteles/tinygrad-dx12 src/tinygrad_dx12/renderer/cstyle.py:665-678); this is the
restatement a standalone backend needs.  It does no tiling or vectorisation: a matrix product
reaches the MFMA GEMMs through ``codegen/uop_matmul.py`` instead.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

from tinygrad_mi355x.uop.ops import ALU, AxisType, DType, KernelInfo, Ops, UOp, dtypes

LOCAL = 256  # work-items per workgroup
GROUP_MIN = 256  # reduction length from which a workgroup folds each stored point


@dataclass(frozen=True)
class LinearKernel:
    """A kernel listing and its launch: ``params`` in slot order, ``variables`` in name order."""

    name: str
    uops: tuple[UOp, ...]
    params: tuple[UOp, ...]
    variables: tuple[UOp, ...]
    global_size: tuple[int, int, int]
    local_size: tuple[int, int, int]


def _identity(op: Ops, dt: DType) -> UOp:
    if op is Ops.ADD:
        return UOp.const(dt, 0)
    if op is Ops.MUL:
        return UOp.const(dt, 1)
    return UOp.const(dt, dtypes.min(dt))  # MAX


def _items(sink: UOp) -> list[tuple[UOp, tuple[UOp, ...]]]:
    """The (STORE, stored ranges) items of a kernel; every item shares one range list."""
    if sink.op is not Ops.SINK or not sink.src:
        raise ValueError("a kernel is a SINK of stores")
    items = []
    for x in sink.src:
        store, ranges = (x.src[0], tuple(x.src[1:])) if x.op is Ops.END else (x, ())
        if store.op is not Ops.STORE or store.src[0].op is not Ops.INDEX:
            raise ValueError(f"kernel item {x.op.name} is not a (closed) STORE through an INDEX")
        items.append((store, ranges))
    if any(set(r) != set(items[0][1]) for _, r in items):
        raise ValueError("the stores of one kernel must share their ranges")
    order = items[0][1]
    for r in order:
        if r.op is not Ops.RANGE or r.src[0].op is not Ops.CONST:
            raise ValueError("stored ranges need constant bounds")
        if r.arg[-1] is AxisType.REDUCE:
            raise ValueError("a REDUCE range cannot be stored over")
    return [(s, order) for s, _ in items]


def _grouped(items) -> bool:
    """Whether the stored values' reductions are long, flat and of constant length."""
    reduces = [u for store, _ in items for u in store.src[1].toposort() if u.op is Ops.REDUCE]
    if not reduces:
        return False
    for r in reduces:
        if any(u.op is Ops.REDUCE for u in r.src[0].toposort()):
            return False
        if any(x.op is not Ops.RANGE or x.src[0].op is not Ops.CONST for x in r.src[1:]):
            return False
        if math.prod(x.src[0].arg for x in r.src[1:]) < GROUP_MIN:
            return False
    return True


class _Emitter:
    def __init__(self) -> None:
        self.out: list[UOp] = []
        self.scopes: list[dict[UOp, UOp]] = [{}]
        self.regs = self.loops = self.loads = 0
        self.free_cache: dict[UOp, frozenset] = {}
        self.group: tuple[UOp, int] | None = None  # (lidx0, work-items) when a workgroup folds each point

    def put(self, u: UOp) -> UOp:
        self.out.append(u)
        return u

    def find(self, node: UOp) -> UOp | None:
        for scope in reversed(self.scopes):
            if node in scope:
                return scope[node]
        return None

    def bind(self, node: UOp, value: UOp) -> UOp:
        self.scopes[-1][node] = value
        return value

    def free(self, node: UOp) -> frozenset:
        """The RANGEs ``node`` depends on that no REDUCE inside it folds."""
        got = self.free_cache.get(node)
        if got is not None:
            return got
        for n in node.toposort():
            if n in self.free_cache:
                continue
            if n.op is Ops.RANGE:
                f = frozenset({n}) | self.free_cache[n.src[0]]
            elif n.op is Ops.REDUCE:
                f = (self.free_cache[n.src[0]] - frozenset(n.src[1:])).union(
                    *(self.free_cache[r.src[0]] for r in n.src[1:]))
            else:
                f = frozenset().union(*(self.free_cache[s] for s in n.src))
            self.free_cache[n] = f
        return self.free_cache[node]

    def in_scope(self, ranges: frozenset) -> bool:
        return all(self.find(r) is not None for r in ranges)

    def address(self, node: UOp) -> UOp:
        """An INDEX as an address into its (already listed) buffer.  Addresses are bound under
        their own key: one INDEX can be both read (a LOAD) and written through."""
        key = ("address", node)
        found = self.find(key)
        if found is not None:
            return found
        buf = self.find(node.src[0])
        if buf is None:
            raise ValueError(f"INDEX of an unlisted {node.src[0].op.name}")
        src = (buf, *(self.value(s) for s in node.src[1:]))
        return self.bind(key, self.put(UOp(Ops.INDEX, node.dtype, src)))

    def _pending(self, root: UOp) -> list[UOp]:
        """The unlisted nodes ``root`` needs, each after its sources (iterative: expression
        chains may be thousands deep); a REDUCE is listed with its body by ``reduce``."""
        order: list[UOp] = []
        seen: set[int] = set()
        stack: list[tuple[UOp, bool]] = [(root, False)]
        while stack:
            n, done = stack.pop()
            if done:
                order.append(n)
                continue
            if id(n) in seen or self.find(n) is not None:
                continue
            seen.add(id(n))
            stack.append((n, True))
            if n.op is not Ops.REDUCE:
                stack.extend((x, False) for x in reversed(n.src))
        return order

    def value(self, node: UOp) -> UOp:
        found = self.find(node)
        if found is not None:
            return found
        for n in self._pending(node):
            if self.find(n) is None:
                self._emit(n)
        return self.find(node)

    def _emit(self, node: UOp) -> None:
        """List one node whose sources are listed."""
        op = node.op
        if op is Ops.CONST:  # constants belong to the outermost scope
            self.scopes[0][node] = node
            self.put(node)
        elif op is Ops.RANGE:
            raise ValueError("a RANGE is used outside its loop")
        elif op is Ops.INDEX:
            self.bind(node, self.put(UOp(Ops.LOAD, node.dtype, (self.address(node),))))
        elif op is Ops.LOAD:  # explicit load of an INDEX (with an optional alternative value)
            src = (self.address(node.src[0]), *(self.find(s) for s in node.src[1:]))
            self.bind(node, self.put(UOp(Ops.LOAD, node.dtype, src)))
        elif op is Ops.REDUCE:
            self.grouped_reduce(node) if self.group is not None else self.reduce(node)
        elif op in ALU or op in (Ops.CAST, Ops.BITCAST):
            self.bind(node, self.put(UOp(op, node.dtype, tuple(self.find(s) for s in node.src), node.arg)))
        elif op in (Ops.PARAM, Ops.DEFINE_VAR):
            raise ValueError(f"{op.name} of slot/name {node.arg} is not a kernel parameter")
        else:
            raise ValueError(f"{op.name} cannot be a value in a scheduled kernel")

    def hoist_invariants(self, x: UOp) -> None:
        """List the parts of a REDUCE body that no loop of it changes, before its loops."""
        for n in x.toposort():
            if n.op not in (Ops.RANGE, Ops.PARAM, Ops.DEFINE_VAR) and self.in_scope(self.free(n)):
                self.value(n)

    def reduce(self, node: UOp) -> UOp:
        x, ranges = node.src[0], node.src[1:]
        if not ranges or any(r.op is not Ops.RANGE for r in ranges):
            raise ValueError("REDUCE folds RANGEs")
        acc = self.put(UOp(Ops.DEFINE_REG, node.dtype, (), (1, self.regs)))
        self.regs += 1
        slot = self.put(UOp(Ops.INDEX, node.dtype, (acc, UOp.const(dtypes.index, 0))))
        self.put(UOp(Ops.STORE, None, (slot, self.put(_identity(node.arg, node.dtype)))))
        # loop-invariant parts of the body first, in dependency order (the body stores nothing,
        # so its loads may move) -- but only ahead of loops that surely run: with a variable or
        # zero bound the loop may run no iteration, and a load hoisted out of it would read an
        # address the original kernel never touches (e.g. b[n - 1] at n = 0)
        if all(r.src[0].op is Ops.CONST and r.src[0].arg > 0 for r in ranges):
            self.hoist_invariants(x)
        loops = []
        for r in ranges:
            bound = self.value(r.src[0])
            loop = self.put(UOp(Ops.RANGE, dtypes.index, (bound,), (r.arg[0], self.loops)))
            self.loops += 1
            loops.append(loop)
            self.scopes.append({})
            self.bind(r, loop)
        body = self.value(x)
        cur = self.put(self.reg_load(slot))
        self.put(UOp(Ops.STORE, None, (slot, self.put(UOp(node.arg, node.dtype, (cur, body))))))
        for loop in reversed(loops):
            self.scopes.pop()
            self.put(UOp(Ops.END, None, (loop,)))
        return self.bind(node, self.put(self.reg_load(slot)))

    def const(self, dt, value) -> UOp:
        return self.value(UOp.const(dt, value))

    def alu(self, op: Ops, dt, *src: UOp) -> UOp:
        return self.put(UOp(op, dt, src))

    def grouped_reduce(self, node: UOp) -> UOp:
        """REDUCE folded by the workgroup (see the module docstring)."""
        lidx, local = self.group
        idx = dtypes.index
        x, ranges = node.src[0], node.src[1:]
        bounds = [r.src[0].arg for r in ranges]
        total = math.prod(bounds)
        ident = _identity(node.arg, node.dtype)
        acc = self.put(UOp(Ops.DEFINE_REG, node.dtype, (), (1, self.regs)))
        self.regs += 1
        slot = self.put(UOp(Ops.INDEX, node.dtype, (acc, UOp.const(idx, 0))))
        self.put(UOp(Ops.STORE, None, (slot, self.value(ident))))
        if total > 0:  # loop-invariant parts first (the loop surely runs)
            self.hoist_invariants(x)
        loop = self.put(UOp(Ops.RANGE, idx, (self.const(idx, -(-total // local)),), ("group", self.loops)))
        self.loops += 1
        self.scopes.append({})
        p = self.alu(Ops.ADD, idx, self.alu(Ops.MUL, idx, loop, self.const(idx, local)), lidx)
        gate = None
        if total % local:
            gate = self.alu(Ops.CMPLT, dtypes.bool, p, self.const(idx, total))
            p = self.put(UOp(Ops.WHERE, idx, (gate, p, self.const(idx, total - 1))))  # in-bounds point
        stride = 1
        for r, n in reversed(list(zip(ranges, bounds))):
            v = p if stride == 1 else self.alu(Ops.IDIV, idx, p, self.const(idx, stride))
            if stride * n < total:
                v = self.alu(Ops.MOD, idx, v, self.const(idx, n))
            self.bind(r, v)
            stride *= n
        body = self.value(x)
        if gate is not None:
            body = self.put(UOp(Ops.WHERE, node.dtype, (gate, body, self.value(ident))))
        self.put(UOp(Ops.STORE, None, (slot, self.put(UOp(node.arg, node.dtype, (self.put(self.reg_load(slot)), body))))))
        self.scopes.pop()
        self.put(UOp(Ops.END, None, (loop,)))
        # halving tree over the workgroup's accumulators in LDS
        lds = self.put(UOp(Ops.DEFINE_LOCAL, node.dtype, (), (local, self.regs)))
        self.regs += 1
        mine = self.put(UOp(Ops.INDEX, node.dtype, (lds, lidx)))
        self.put(UOp(Ops.STORE, None, (mine, self.put(self.reg_load(slot)))))
        self.barrier()
        half = local // 2
        while half >= 1:
            self.put(UOp(Ops.IF, None, (self.alu(Ops.CMPLT, dtypes.bool, lidx, self.const(idx, half)),)))
            other = self.put(UOp(Ops.INDEX, node.dtype, (lds, self.alu(Ops.ADD, idx, lidx, self.const(idx, half)))))
            a, b = self.put(self.reg_load(mine)), self.put(self.reg_load(other))
            self.put(UOp(Ops.STORE, None, (mine, self.put(UOp(node.arg, node.dtype, (a, b))))))
            self.put(UOp(Ops.ENDIF, None, ()))
            self.barrier()
            half //= 2
        first = self.put(UOp(Ops.INDEX, node.dtype, (lds, UOp.const(idx, 0))))
        return self.bind(node, self.put(self.reg_load(first)))

    def barrier(self) -> None:
        self.loads += 1
        self.put(UOp(Ops.BARRIER, None, (), self.loads))

    def reg_load(self, slot: UOp) -> UOp:
        """A read of the accumulator; each is its own UOp (the value changes between reads)."""
        self.loads += 1
        return UOp(Ops.LOAD, slot.dtype, (slot,), self.loads)


def linearize(sink: UOp, local: int = LOCAL) -> LinearKernel:
    """The linear listing and launch of scheduled kernel ``sink``."""
    items = _items(sink)
    nodes = sink.toposort()
    params = sorted((u for u in nodes if u.op is Ops.PARAM), key=lambda u: u.arg.slot)
    slots = [p.arg.slot for p in params]
    if len(set(slots)) != len(slots):
        raise ValueError("two PARAMs share a slot")
    variables = sorted((u for u in nodes if u.op is Ops.DEFINE_VAR), key=lambda u: u.arg[0])
    order = items[0][1]
    bounds = [r.src[0].arg for r in order]
    total = math.prod(bounds)
    if total >= 2**31:
        raise ValueError("a kernel stores fewer than 2^31 points")
    if any(p.max_numel() >= 2**31 for p in params):
        raise ValueError("kernel buffers hold fewer than 2^31 elements (32-bit indexing)")
    e = _Emitter()
    for u in (*params, *variables):
        e.bind(u, e.put(u))
    if _grouped(items):
        return _linearize_grouped(sink, items, e, params, variables, order, bounds, total, local)
    local = max(64, min(local, -(-total // 64) * 64))
    groups = -(-total // local)
    gidx = e.put(UOp(Ops.SPECIAL, dtypes.index, (UOp.const(dtypes.index, groups),), "gidx0"))
    lidx = e.put(UOp(Ops.SPECIAL, dtypes.index, (UOp.const(dtypes.index, local),), "lidx0"))
    g = e.put(UOp(Ops.ADD, dtypes.index, (e.put(UOp(Ops.MUL, dtypes.index, (gidx, e.value(UOp.const(dtypes.index, local))))), lidx)))
    guarded = total % local != 0
    if guarded:
        e.put(UOp(Ops.IF, None, (e.put(UOp(Ops.CMPLT, dtypes.bool, (g, e.value(UOp.const(dtypes.index, total))))),)))
    stride = 1
    for r, n in reversed(list(zip(order, bounds))):
        v = g
        if stride > 1:
            v = e.put(UOp(Ops.IDIV, dtypes.index, (v, e.value(UOp.const(dtypes.index, stride)))))
        if stride * n < total:
            v = e.put(UOp(Ops.MOD, dtypes.index, (v, e.value(UOp.const(dtypes.index, n)))))
        e.bind(r, v)
        stride *= n
    for store, _ in items:
        target, value = store.src
        address = e.address(target)
        e.put(UOp(Ops.STORE, None, (address, e.value(value))))
    if guarded:
        e.put(UOp(Ops.ENDIF, None, ()))
    name = sink.arg.name if isinstance(sink.arg, KernelInfo) else "kernel"
    return LinearKernel(name, tuple(e.out), tuple(params), tuple(variables), (groups, 1, 1), (local, 1, 1))


def _linearize_grouped(sink, items, e: _Emitter, params, variables, order, bounds, total, local) -> LinearKernel:
    """One workgroup per stored point: the stored ranges are the digits of gidx0."""
    idx = dtypes.index
    gidx = e.put(UOp(Ops.SPECIAL, idx, (UOp.const(idx, total),), "gidx0"))
    lidx = e.put(UOp(Ops.SPECIAL, idx, (UOp.const(idx, local),), "lidx0"))
    e.group = (lidx, local)
    stride = 1
    for r, n in reversed(list(zip(order, bounds))):
        v = gidx if stride == 1 else e.alu(Ops.IDIV, idx, gidx, e.const(idx, stride))
        if stride * n < total:
            v = e.alu(Ops.MOD, idx, v, e.const(idx, n))
        e.bind(r, v)
        stride *= n
    # every work-item takes part in the reductions; work-item 0 stores
    stores = [(e.address(store.src[0]), e.value(store.src[1])) for store, _ in items]
    e.put(UOp(Ops.IF, None, (e.alu(Ops.CMPEQ, dtypes.bool, lidx, e.const(idx, 0)),)))
    for address, value in stores:
        e.put(UOp(Ops.STORE, None, (address, value)))
    e.put(UOp(Ops.ENDIF, None, ()))
    name = sink.arg.name if isinstance(sink.arg, KernelInfo) else "kernel"
    return LinearKernel(name, tuple(e.out), tuple(params), tuple(variables), (total, 1, 1), (local, 1, 1))
