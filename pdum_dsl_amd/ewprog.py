"""Lowering of pointwise chains to the elementwise register programs that
libpdhip's interpreter runs (pdh_ew_program, include/pdhip.h).

A chain is a DAG of tl.pointwise / consts / iotas / broadcasts over LEAVES:
params (or any node the caller materializes) read with LOAD, and, in a
contraction epilogue, the accumulator read with ACC. Every node is evaluated
at the coordinates of one output lattice (``dims``); a leaf whose dims are a
subset of the lattice is read with stride 0 along the missing dims, which is
exactly the reference's broadcast (tl.repeat_like / tl.repeat add stride-0
dims, dialect.py:175-205).

Registers are allocated over a topological order with last-use freeing; a
chain that needs more than PDH_EW_MAX_REGS live values, more operands than
PDH_EW_MAX_OPERANDS or more instructions than PDH_EW_MAX_INSNS refuses.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

from . import _lib as L

# tl.pointwise markers -> opcodes (the reference's numpy markers, dsl/markers.py)
_UNARY = {"neg": "NEG", "exp": "EXP", "log": "LOG", "sqrt": "SQRT", "tanh": "TANH", "sin": "SIN", "cos": "COS",
          "abs": "ABS", "floor": "FLOOR"}
_BINARY = {"add": "ADD", "sub": "SUB", "mul": "MUL", "div": "DIV", "maximum": "MAX", "minimum": "MIN",
           "eq": "EQ", "ne": "NE", "lt": "LT", "le": "LE", "gt": "GT", "ge": "GE"}
_VIEW = ("tl.repeat_like", "tl.repeat", "tl.stage")
_GELU_C = 0.7978845608028654  # sqrt(2/pi), the composite zoo.gelu marker's constant (zoo_common.py:19-20)


class Unlowerable(Exception):
    """The chain has a node the elementwise program cannot express."""


@dataclass
class Lowered:
    insns: list  # (op, dst, a, b, c, imm)
    out_reg: int
    operands: tuple  # the node each LOAD slot reads (a leaf, or a view chain over one), slot order
    dims: tuple  # output lattice dims (ir.Dim), outermost first
    bases: tuple = ()  # the leaf under each slot (views peeled)
    # per slot: leaf dim name -> (coefficients by lattice dim name, constant):
    # the leaf coordinate as an affine form of the slot's coordinates
    views: tuple = ()

    def operand_view(self, i: int, leaf_strides: dict) -> tuple:
        """(element strides over ``dims``, element offset) at which slot ``i``
        reads its leaf, given the leaf's strides by dim name: lattice index
        j_d along dim d is coordinate d.start + j_d, the leaf coordinate along
        b is sum_d coef_bd (d.start + j_d) + const_b, and its storage index
        that minus b's start."""
        forms = self.views[i]
        start = {d.name: d.start for d in self.bases[i].type.dims}
        strides = [sum(cf.get(d.name, 0) * int(leaf_strides[b]) for b, (cf, _c) in forms.items()) for d in self.dims]
        first = {d.name: d.start for d in self.dims}
        off = sum((c + sum(v * first[dn] for dn, v in cf.items()) - start[b]) * int(leaf_strides[b])
                  for b, (cf, c) in forms.items())
        return strides, off

    def offset_reads(self) -> int:
        """Slots whose reads do not start at their leaf's first element in
        lattice order (a shifted or strided view)."""
        return sum(1 for forms in self.views if any(c or list(cf.values()) != [1] for cf, c in forms.values()))

    def program(self, out_strides, operand_strides) -> L.EwProgram:
        """The C struct, given the output's and each operand's element
        strides over ``dims`` (0 where an operand lacks a dim)."""
        p = L.EwProgram()
        p.n_insns = len(self.insns)
        p.n_operands = len(self.operands)
        p.ndim = len(self.dims)
        p.out_reg = self.out_reg
        for d, dim in enumerate(self.dims):
            p.shape[d] = dim.size
            p.start[d] = dim.start
            p.out_stride[d] = int(out_strides[d])
        for i, st in enumerate(operand_strides):
            for d in range(len(self.dims)):
                p.in_stride[i][d] = int(st[d])
        for j, (op, dst, a, b, c, imm) in enumerate(self.insns):
            ins = p.insns[j]
            ins.op, ins.dst, ins.a, ins.b, ins.c, ins.imm = L.EW[op], dst, a, b, c, float(imm)
        return p


def _const_value(n):
    if n.op in ("core.const", "tl.const"):
        return float(n.attr("value"))
    return None


def lower(root, dims, leaves: dict, acc=None, acc_scale: float | None = None, allow_views: bool = False) -> Lowered:
    """Lower the chain ending at ``root``. ``leaves`` maps id(node) -> node
    for nodes read with LOAD (slot order = first use). A chain of layout views
    over a leaf (tl.rename, tl.stage; with ``allow_views`` also tl.shift,
    tl.slice, tl.select, tl.window, tl.decimate and tl.diagonal: affine views whose
    offset and strides the caller applies through ``Lowered.operand_view``)
    is one LOAD slot: views move no data. ``acc`` is
    the node read with ACC (a contraction's fold), if any; ``acc_scale``
    multiplies it (a mean's finalize)."""
    names = tuple(d.name for d in dims)
    order: list = []
    seen: set = set()
    walkable = ("tl.rename", "tl.stage") + (
        ("tl.shift", "tl.slice", "tl.select", "tl.window", "tl.decimate", "tl.diagonal") if allow_views else ())

    def base_of(x):
        while x.op in walkable and id(x) not in leaves:
            x = x.args[0]
        return x if id(x) in leaves else None

    def is_leaf(x):  # a stage over a leaf is skipped as a view instead (the leaf is the slot)
        return id(x) in leaves or (x.op in walkable and x.op != "tl.stage" and base_of(x) is not None)

    def view_of(x):
        """Each dim of the frame being walked, as an affine form (coefficients
        over the slot's dims, constant), from the slot down to its leaf."""
        cur = {n: ({n: 1}, 0) for n in x.type.names}
        while id(x) not in leaves:
            if x.op == "tl.shift":  # in = out - delta
                deltas = dict(x.attr("deltas"))
                cur = {nm: (cf, c - int(deltas.get(nm, 0))) for nm, (cf, c) in cur.items()}
            elif x.op == "tl.rename":
                inv = {new: old for old, new in x.attr("mapping")}
                cur = {inv.get(nm, nm): v for nm, v in cur.items()}
            elif x.op == "tl.window":  # in[x] = out[x] + dilation out[k]
                nm, dil = x.attr("name"), int(x.attr("dilation", 1))
                (cx, c0), (ck, c1) = cur.pop(nm), cur.pop(x.attr("k_name"))
                cf = dict(cx)
                for k, v in ck.items():
                    cf[k] = cf.get(k, 0) + dil * v
                cur[nm] = (cf, c0 + dil * c1)
            elif x.op == "tl.decimate":  # in[x] = factor out[x] + phase
                nm, f = x.attr("name"), int(x.attr("factor"))
                cx, c0 = cur[nm]
                cur[nm] = ({k: f * v for k, v in cx.items()}, f * c0 + int(x.attr("phase", 0)) % f)
            elif x.op == "tl.select":  # the fixed dims read one coordinate
                for nm, i in x.attr("coords"):
                    cur[nm] = ({}, int(i))
            elif x.op == "tl.diagonal":  # every part reads the diagonal's coordinate
                parts = x.attr("parts")
                e = cur.pop(x.attr("name"))
                for pn in ((parts,) if isinstance(parts, str) else tuple(parts)):
                    cur[pn] = e
            x = x.args[0]  # tl.slice / tl.stage: the same coordinates
        return cur

    def visit(n):  # post-order over the chain, stopping at leaves
        stack = [(n, False)]
        while stack:
            x, done = stack.pop()
            if done:
                order.append(x)
                continue
            if id(x) in seen:
                continue
            seen.add(id(x))
            stack.append((x, True))
            if is_leaf(x) or (acc is not None and x is acc):
                continue
            if x.op in _VIEW or x.op == "tl.round_to":
                stack.append((x.args[0], False))
            elif x.op == "tl.pointwise":
                for a in reversed(x.args):
                    stack.append((a, False))

    visit(root)

    def skip_view(x):
        while x.op in _VIEW and id(x) not in leaves and x is not acc:
            x = x.args[0]
        return x

    uses: dict[int, int] = {}
    for x in order:
        if x.op in ("tl.pointwise", "tl.round_to") and not is_leaf(x) and x is not acc:
            for a in x.args:
                a = skip_view(a)
                uses[id(a)] = uses.get(id(a), 0) + 1
    root_v = skip_view(root)
    uses[id(root_v)] = uses.get(id(root_v), 0) + 1

    insns: list = []
    reg: dict[int, int] = {}
    free = list(range(L.EW_MAX_REGS - 1, -1, -1))
    slots: list = []

    def alloc():
        if not free:
            raise Unlowerable(f"the chain needs more than {L.EW_MAX_REGS} live registers")
        return free.pop()

    def release(x):
        uses[id(x)] -= 1
        if uses[id(x)] == 0 and x is not root_v:
            free.append(reg[id(x)])

    for x in order:
        if x.op in _VIEW and id(x) not in leaves and x is not acc:
            continue
        if id(x) in reg:
            continue
        if acc is not None and x is acc:
            r = alloc()
            insns.append(("ACC", r, 0, 0, 0, 0.0))
            if acc_scale is not None:
                k = alloc()
                insns.append(("CONST", k, 0, 0, 0, float(acc_scale)))
                insns.append(("MUL", r, r, k, 0, 0.0))
                free.append(k)
        elif is_leaf(x):
            if len(slots) >= L.EW_MAX_OPERANDS:
                raise Unlowerable(f"the chain reads more than {L.EW_MAX_OPERANDS} operands")
            for nm in x.type.names:
                if nm not in names:
                    raise Unlowerable(f"operand dim {nm!r} is not an output dim")
            slots.append(x)
            r = alloc()
            insns.append(("LOAD", r, len(slots) - 1, 0, 0, 0.0))
        elif _const_value(x) is not None:
            r = alloc()
            insns.append(("CONST", r, 0, 0, 0, _const_value(x)))
        elif x.op == "tl.round_to":  # encode-then-decode; fp32 values already are f32
            src = skip_view(x.args[0])
            xr = reg[id(src)]
            release(src)
            r = alloc()
            enc = x.attr("encoding")
            insns.append(("MAX", r, xr, xr, 0, 0.0) if enc == "f32" else (("RBF16" if enc == "bf16" else "RF16"), r, xr,
                                                                          0, 0, 0.0))
        elif x.op == "tl.iota":
            nm = x.attr("name")
            if nm not in names:
                raise Unlowerable(f"iota over {nm!r}, which is not an output dim")
            r = alloc()
            insns.append(("IOTA", r, names.index(nm), 0, 0, 0.0))
        elif x.op == "tl.pointwise" and x.attr("f") == "zoo.gelu":
            # the composite marker, expanded in its own association order:
            # 0.5 * x * (1 + tanh(c * (x + 0.044715 * x * x * x)))
            src = skip_view(x.args[0])
            xr = reg[id(src)]
            r, c = alloc(), alloc()  # x stays live until the last instruction reads it
            insns += [("CONST", c, 0, 0, 0, 0.044715), ("MUL", r, c, xr, 0, 0.0), ("MUL", r, r, xr, 0, 0.0),
                      ("MUL", r, r, xr, 0, 0.0), ("ADD", r, xr, r, 0, 0.0), ("CONST", c, 0, 0, 0, _GELU_C),
                      ("MUL", r, c, r, 0, 0.0), ("TANH", r, r, 0, 0, 0.0), ("CONST", c, 0, 0, 0, 1.0),
                      ("ADD", r, c, r, 0, 0.0), ("CONST", c, 0, 0, 0, 0.5), ("MUL", c, c, xr, 0, 0.0),
                      ("MUL", r, c, r, 0, 0.0)]
            free.append(c)
            release(src)
        elif x.op == "tl.pointwise" and x.attr("f") == "zoo.gelu.d0":
            # the marker's partial: 0.5 ((1 + t) + x (1 - t^2) c (1 + 3 * 0.044715 x^2)), t = tanh(u)
            src = skip_view(x.args[0])
            xr = reg[id(src)]
            r, c, s_, w = alloc(), alloc(), alloc(), alloc()
            insns += [("CONST", c, 0, 0, 0, 0.044715), ("MUL", r, c, xr, 0, 0.0), ("MUL", r, r, xr, 0, 0.0),
                      ("MUL", r, r, xr, 0, 0.0), ("ADD", r, xr, r, 0, 0.0), ("CONST", c, 0, 0, 0, _GELU_C),
                      ("MUL", r, c, r, 0, 0.0), ("TANH", r, r, 0, 0, 0.0),  # r = t
                      ("MUL", s_, xr, xr, 0, 0.0), ("CONST", c, 0, 0, 0, 0.134145), ("MUL", s_, c, s_, 0, 0.0),
                      ("CONST", c, 0, 0, 0, 1.0), ("ADD", s_, s_, c, 0, 0.0), ("CONST", w, 0, 0, 0, _GELU_C),
                      ("MUL", s_, w, s_, 0, 0.0),  # s = c (1 + 3 a x^2)
                      ("MUL", w, r, r, 0, 0.0), ("SUB", w, c, w, 0, 0.0), ("MUL", s_, s_, w, 0, 0.0),
                      ("MUL", s_, s_, xr, 0, 0.0),  # s = x (1 - t^2) c (1 + 3 a x^2)
                      ("ADD", r, r, c, 0, 0.0), ("ADD", r, r, s_, 0, 0.0), ("CONST", c, 0, 0, 0, 0.5),
                      ("MUL", r, c, r, 0, 0.0)]
            free.extend((c, s_, w))
            release(src)
        elif x.op == "tl.pointwise":
            f = x.attr("f")
            srcs = [skip_view(a) for a in x.args]
            regs = [reg[id(a)] for a in srcs]
            for a in srcs:
                release(a)
            if f == "stop_gradient":  # identity in value: max(x, x) is a move
                r = alloc()
                insns.append(("MAX", r, regs[0], regs[0], 0, 0.0))
            elif f in _UNARY:
                r = alloc()
                insns.append((_UNARY[f], r, regs[0], 0, 0, 0.0))
            elif f in _BINARY:
                r = alloc()
                insns.append((_BINARY[f], r, regs[0], regs[1], 0, 0.0))
            elif f == "where":
                r = alloc()
                insns.append(("WHERE", r, regs[0], regs[1], regs[2], 0.0))
            else:
                raise Unlowerable(f"marker {f!r} has no opcode")
        else:
            raise Unlowerable(f"{x.op} is not elementwise-program vocabulary")
        reg[id(x)] = r
    if len(insns) > L.EW_MAX_INSNS:
        raise Unlowerable(f"{len(insns)} instructions (max {L.EW_MAX_INSNS})")
    return Lowered(insns, reg[id(root_v)], tuple(slots), tuple(dims), tuple(base_of(x) for x in slots),
                   tuple(view_of(x) for x in slots))


def with_slots(prog, first: int, total: int):
    """The program reading its operands from slots first.. of a table of
    ``total`` (its LOADs and strides moved up by ``first``)."""
    new = L.EwProgram()
    new.n_insns, new.ndim, new.out_reg, new.n_operands = prog.n_insns, prog.ndim, prog.out_reg, total
    for d in range(prog.ndim):
        new.shape[d], new.start[d], new.out_stride[d] = prog.shape[d], prog.start[d], prog.out_stride[d]
    for i in range(prog.n_operands):
        for d in range(prog.ndim):
            new.in_stride[first + i][d] = prog.in_stride[i][d]
    for j in range(prog.n_insns):
        src, dst = prog.insns[j], new.insns[j]
        dst.op, dst.dst, dst.a, dst.b, dst.c, dst.imm = src.op, src.dst, src.a, src.b, src.c, src.imm
        if src.op == L.EW["LOAD"]:
            dst.a = src.a + first
    return new


def splitk_sum(prog, S: int, plane_strides=None):
    """The epilogue program ``prog`` (which reads the contraction's sum with
    ACC) rewritten to read that sum as the total of S partial planes: slots
    0..S-1 hold the planes (strides ``plane_strides`` over prog's lattice,
    default the output's), prog's own operands move up by S, and the sum,
    added in plane order, replaces ACC. None when the operand table or the
    registers cannot hold it."""
    if S < 2 or prog.n_operands + S > L.EW_MAX_OPERANDS or prog.n_insns + 2 * S > L.EW_MAX_INSNS:
        return None
    used = {int(prog.out_reg)} | {int(prog.insns[j].dst) for j in range(prog.n_insns)}
    free = [r for r in range(L.EW_MAX_REGS) if r not in used]
    if len(free) < 2:
        return None
    ra, rb = free[0], free[1]
    new = L.EwProgram()
    new.ndim, new.out_reg, new.n_operands = prog.ndim, prog.out_reg, prog.n_operands + S
    for d in range(prog.ndim):
        new.shape[d], new.start[d], new.out_stride[d] = prog.shape[d], prog.start[d], prog.out_stride[d]
        for i in range(S):
            new.in_stride[i][d] = prog.out_stride[d] if plane_strides is None else int(plane_strides[d])
        for i in range(prog.n_operands):
            new.in_stride[S + i][d] = prog.in_stride[i][d]
    seq = [(L.EW["LOAD"], ra, 0, 0, 0, 0.0)]
    for i in range(1, S):
        seq += [(L.EW["LOAD"], rb, i, 0, 0, 0.0), (L.EW["ADD"], ra, ra, rb, 0, 0.0)]
    for j in range(prog.n_insns):
        src = prog.insns[j]
        op, dst, a, b, c, imm = src.op, src.dst, src.a, src.b, src.c, src.imm
        if op == L.EW["ACC"]:
            op, a, b = L.EW["MAX"], ra, ra  # max(x, x) = x, NaN included
        elif op == L.EW["LOAD"]:
            a = a + S
        seq.append((op, dst, a, b, c, imm))
    new.n_insns = len(seq)
    for j, (op, dst, a, b, c, imm) in enumerate(seq):
        ins = new.insns[j]
        ins.op, ins.dst, ins.a, ins.b, ins.c, ins.imm = op, dst, a, b, c, imm
    return new


def merge_dims(prog, groups):
    """Merge groups of consecutive lattice dims of a program into one dim each
    (e.g. (unit, t, nh, hk) -> (unit, t, nh*hk)). A group merges when every
    view's strides over it compose densely (outer = inner * size) or are all
    zero; an IOTA over a dim in a group of several refuses (Unlowerable)."""
    n_old = prog.ndim
    sizes = [int(prog.shape[d]) for d in range(n_old)]
    for j in range(prog.n_insns):
        ins = prog.insns[j]
        if ins.op == L.EW["IOTA"]:
            g = next(gi for gi, grp in enumerate(groups) if ins.a in grp)
            if len(groups[g]) > 1:
                raise Unlowerable("an iota over a flattened dim has no merged form")
    if any(int(prog.start[d]) != 0 for grp in groups if len(grp) > 1 for d in grp):
        raise Unlowerable("a flattened dim must start at 0")

    def merge(strides):
        out = []
        for grp in groups:
            st = [int(strides[d]) for d in grp]
            if all(s == 0 for s in st):
                out.append(0)
                continue
            for a, b in zip(grp[:-1], grp[1:]):
                if int(strides[a]) != int(strides[b]) * sizes[b]:
                    raise Unlowerable("a view's strides do not compose across a flattened dim")
            out.append(st[-1])
        return out

    out_st = merge(prog.out_stride)
    in_st = [merge(prog.in_stride[i]) for i in range(prog.n_operands)]
    iota_dim = {d: gi for gi, grp in enumerate(groups) for d in grp}
    new = L.EwProgram()
    new.n_insns, new.n_operands, new.ndim, new.out_reg = prog.n_insns, prog.n_operands, len(groups), prog.out_reg
    for gi, grp in enumerate(groups):
        new.shape[gi] = math.prod(sizes[d] for d in grp)
        new.start[gi] = int(prog.start[grp[0]]) if len(grp) == 1 else 0
        new.out_stride[gi] = out_st[gi]
        for i in range(prog.n_operands):
            new.in_stride[i][gi] = in_st[i][gi]
    for j in range(prog.n_insns):
        src, dst = prog.insns[j], new.insns[j]
        dst.op, dst.dst, dst.a, dst.b, dst.c, dst.imm = src.op, src.dst, src.a, src.b, src.c, src.imm
        if src.op == L.EW["IOTA"]:
            dst.a = iota_dim[src.a]
    return new


def strides_over(arr_strides, arr_names, dims) -> list:
    """Element strides of an array (dims ``arr_names``) over the lattice
    ``dims``: the array's stride where it has the dim, 0 (broadcast) where not."""
    out = []
    for d in dims:
        out.append(arr_strides[arr_names.index(d.name)] if d.name in arr_names else 0)
    return out


__all__ = ["Lowered", "Unlowerable", "lower", "merge_dims", "strides_over", "with_slots"]
