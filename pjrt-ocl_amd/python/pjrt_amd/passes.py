"""Fusion passes over a lowered tensor program, and liveness arena packing.

These rewrite the VMProgram instruction list the StableHLO lowering produced, in
place and index-stable (a removed instruction becomes OP_NOP, so region
sub-list ranges stay valid), as the reference's post-lowering passes do
(python/pjrt_ocl/lowering.py:3027-3106).  Each pass matches one idiom on the
tensor instructions and leaves anything that does not match exactly untouched:
an unfused program is correct, only slower.

  compose_affines      x*s1+t1 then *s2+t2 -> one affine (lowering.py:1378-1431)
  fuse_matmul_views    transpose / reshape gathers folded into matmul operand
                       reads (lowering.py:2381-2452)
  fuse_views           gathers folded into elementwise operand views
                       (lowering.py:1481-1545)
  dce                  dead instructions -> NOP (lowering.py:1434-1466)
  fuse_norm            softmax and layernorm-core idioms -> one row op
                       (lowering.py:1561-1724); the reference's seg <= 1024 gate
                       (lowering.py:1553) is lifted: the row kernels here stream
                       rows of any length
  fuse_norm_epilogue   extension: a layernorm's gamma / beta, a GELU after it
                       and a final f32 -> bf16 / f16 convert join the one row op
                       (OP_LAYERNORM_AFFINE)
  fuse_gelu            the tanh-GELU idiom -> OP_GELU (lowering.py:1737-1876)
  fuse_mma_epilogue    the elementwise chain after a matmul -> its store
                       epilogue (lowering.py:2486-2601); extended with per-column
                       bias (source 2), constant operands (source 3, e.g. relu),
                       any binary micro-op and a final convert to bf16 / f16
  fuse_region          remaining same-size f32 map chains -> OP_MAP_REGION
                       (lowering.py:2071-2378)
  fuse_attention       DOT(Q K^T) [* scale] [causal mask] -> softmax -> DOT(P V)
                       -> OP_FLASH_ATTN (lowering.py:2664-2810); extended with
                       the causal mask and bf16 converts around P and the output
  finalize_matmul_views  DOT views / epilogue mirrored into aux
                       (lowering.py:2455-2466)
  reuse_arena          arena offsets by liveness in scheduler phase time
                       (lowering.py:2813-2973)

Order: the reference folds region chains before matmul epilogues; here the
epilogue pass runs first, because this build's epilogue takes per-column biases
and constant operands, so a matmul's bias / activation tail becomes part of its
store instead of a region of its own.
"""
from __future__ import annotations

import math
import os

import numpy as np

from . import vmprogram as V

_REGION_OPS = (V.OP_WHILE, V.OP_IF, V.OP_FOR)


def _off(name: str) -> bool:
    return os.environ.get(name, "1") == "0"


def _bits(x: float) -> int:
    return V.f32_bits(x)


def _f(bits: int) -> float:
    return V.bits_f32(bits)


# ---- analysis helpers ------------------------------------------------------------------------

def reads_of(ins: V.Instr, prog: V.VMProgram) -> set:
    """Buffers an instruction reads (region ops: their cond buffer only; the
    sub-list instructions are analysed where they stand)."""
    from .scheduler import _instr_reads
    if ins.op == V.OP_NOP:
        return set()
    if ins.op in (V.OP_WHILE, V.OP_IF):
        return {ins.dst}
    if ins.op == V.OP_FOR:
        return set()
    return _instr_reads(ins, prog)


def writes_of(ins: V.Instr) -> set:
    if ins.op in (V.OP_NOP, V.OP_FOR, V.OP_WHILE, V.OP_IF):
        return set()
    if ins.op == V.OP_ARGMAX_SEG:
        return {ins.dst, ins.b}
    return {ins.dst}


def scopes(prog: V.VMProgram) -> list:
    """Scope id of every instruction: 0 for the root list, one id per region
    sub-list (cond, body, then, else)."""
    sc = [0] * len(prog.instrs)
    nxt = 1
    for i, ins in enumerate(prog.instrs):
        ranges = []
        if ins.op in (V.OP_WHILE, V.OP_IF):
            ranges = [(ins.a, ins.a + ins.b), (ins.n, ins.n + ins.imm)]
        elif ins.op == V.OP_FOR:
            ranges = [(ins.n, ins.n + ins.imm)]
        for lo, hi in ranges:
            for j in range(lo, hi):
                sc[j] = nxt
            nxt += 1
    return sc


class _Index:
    """Writers and readers of every buffer over the live instructions."""

    def __init__(self, prog: V.VMProgram):
        self.prog = prog
        self.writers: dict = {}
        self.readers: dict = {}
        for i, ins in enumerate(prog.instrs):
            if ins.op == V.OP_NOP:
                continue
            for b in writes_of(ins):
                self.writers.setdefault(b, []).append(i)
            for b in reads_of(ins, prog):
                self.readers.setdefault(b, []).append(i)

    def unique_writer(self, buf: int):
        w = self.writers.get(buf, ())
        return w[0] if len(w) == 1 else None

    def producer(self, buf: int, op: int = None):
        w = self.unique_writer(buf)
        if w is None:
            return None
        ins = self.prog.instrs[w]
        return ins if op is None or ins.op == op else None

    def live_readers(self, buf: int) -> list:
        return [j for j in self.readers.get(buf, ()) if self.prog.instrs[j].op != V.OP_NOP
                and buf in reads_of(self.prog.instrs[j], self.prog)]


def _elems(prog, buf) -> int:
    b = prog.buffers[buf]
    return b.size_bytes // V.DT_SIZE[b.dtype]


def _dt(prog, buf) -> int:
    return prog.buffers[buf].dtype


def _const_values(prog) -> dict:
    """f32 constant buffers whose elements are all equal -> that value."""
    out = {}
    for bid, data in prog.consts:
        if prog.buffers[bid].dtype == V.DT_F32 and len(data) >= 4:
            arr = np.frombuffer(bytes(data), "<f4")
            if np.all(arr == arr[0]) or (np.isnan(arr).all()):
                out[bid] = float(arr[0])
    return out


def _view_desc(prog, view1: int):
    """(dims, strides, offset) of a view aux offset + 1."""
    off = view1 - 1
    aux = prog.aux
    rank = aux[off]
    dims = [aux[off + 1 + k] for k in range(rank)]
    st = [_i32(aux[off + 1 + rank + k]) for k in range(rank)]
    return dims, st, _i32(aux[off + 1 + 2 * rank])


def _i32(u: int) -> int:
    u &= 0xFFFFFFFF
    return u - (1 << 32) if u >= 1 << 31 else u


def _is_row_broadcast(prog, view1: int, seg: int) -> bool:
    """The view reads element i of its output from source element i % seg (a
    [seg] vector repeated over rows)."""
    dims, st, off = _view_desc(prog, view1)
    if off != 0:
        return False
    inner = 1
    for d in range(len(dims) - 1, -1, -1):
        if dims[d] == 1:
            continue
        if inner < seg:
            if st[d] != inner:
                return False
            inner *= dims[d]
        elif st[d] != 0:
            return False
    return inner == seg


def _is_splat(prog, view1: int) -> bool:
    dims, st, off = _view_desc(prog, view1)
    return off == 0 and all(s == 0 or d == 1 for d, s in zip(dims, st))


def _is_identity_view(prog, view1: int, n: int) -> bool:
    dims, st, off = _view_desc(prog, view1)
    if off != 0 or int(np.prod(dims)) != n:
        return False
    acc = 1
    for d in range(len(dims) - 1, -1, -1):
        if dims[d] != 1 and st[d] != acc:
            return False
        acc *= dims[d]
    return True


# ---- compose_affines (lowering.py:1378-1431) -------------------------------------------------

def compose_affines(prog: V.VMProgram) -> None:
    if _off("PJRT_OCL_COMPOSE_AFFINE"):
        return
    outs = set(prog.outputs)
    sc = scopes(prog)
    changed = True
    while changed:
        changed = False
        ix = _Index(prog)
        for i, ins in enumerate(prog.instrs):
            if ins.op != V.OP_AFFINE_F32:
                continue
            w = ix.unique_writer(ins.a)
            if w is None or sc[w] != sc[i]:
                continue
            inner = prog.instrs[w]
            if inner.op != V.OP_AFFINE_F32 or ins.a in outs or len(ix.live_readers(ins.a)) != 1:
                continue
            s1, t1, s2, t2 = (np.float32(_f(x)) for x in (inner.imm, inner.imm2, ins.imm, ins.imm2))
            prog.instrs[i] = V.Instr(V.OP_AFFINE_F32, dst=ins.dst, a=inner.a, b=inner.a, n=ins.n,
                                     imm=_bits(float(s1 * s2)), imm2=_bits(float(t1 * s2 + t2)))
            prog.instrs[w] = V.Instr(V.OP_NOP)
            changed = True
            break


# ---- dce (lowering.py:1434-1466) ------------------------------------------------------------

def dce(prog: V.VMProgram) -> None:
    live_buf = set(prog.outputs) | set(prog.inputs)
    live = [False] * len(prog.instrs)
    for i, ins in enumerate(prog.instrs):
        if ins.op in _REGION_OPS:
            live[i] = True
            if ins.op != V.OP_FOR:
                live_buf.add(ins.dst)
    changed = True
    while changed:
        changed = False
        for i, ins in enumerate(prog.instrs):
            if ins.op == V.OP_NOP:
                continue
            if not live[i] and writes_of(ins) & live_buf:
                live[i] = True
                changed = True
            if live[i]:
                for b in reads_of(ins, prog):
                    if b not in live_buf:
                        live_buf.add(b)
                        changed = True
    for i, ins in enumerate(prog.instrs):
        if ins.op != V.OP_NOP and not live[i]:
            prog.instrs[i] = V.Instr(V.OP_NOP)


# ---- view folding (lowering.py:1481-1545, 2381-2452) -----------------------------------------

VIEWABLE_EW = frozenset({
    V.OP_ADD_F32, V.OP_SUB_F32, V.OP_MUL_F32, V.OP_DIV_F32, V.OP_MAX_F32, V.OP_MIN_F32, V.OP_POW_F32,
    V.OP_ATAN2_F32, V.OP_REMAINDER_F32, V.OP_NEG_F32, V.OP_EXP_F32, V.OP_LOG_F32, V.OP_SQRT_F32,
    V.OP_RSQRT_F32, V.OP_TANH_F32, V.OP_ABS_F32, V.OP_FLOOR_F32, V.OP_CEIL_F32, V.OP_SIGN_F32,
    V.OP_LOG1P_F32, V.OP_EXPM1_F32, V.OP_CBRT_F32, V.OP_SIN_F32, V.OP_COS_F32, V.OP_TAN_F32,
    V.OP_ROUND_NEAREST_EVEN_F32, V.OP_ROUND_NEAREST_AFZ_F32, V.OP_COPY_F32, V.OP_GELU})
_BINARY_VIEW = frozenset({V.OP_ADD_F32, V.OP_SUB_F32, V.OP_MUL_F32, V.OP_DIV_F32, V.OP_MAX_F32,
                          V.OP_MIN_F32, V.OP_POW_F32, V.OP_ATAN2_F32, V.OP_REMAINDER_F32})


def _gather_foldable(prog, ix, sc, gi, g) -> bool:
    """A gather whose output is a pure view of its source: written once, its
    source not rewritten later in the gather's scope, not a program output."""
    if g.op != V.OP_GATHER_STRIDED or g.dst in set(prog.outputs):
        return False
    if len(ix.writers.get(g.dst, ())) != 1:
        return False
    return not any(w > gi for w in ix.writers.get(g.a, ()))


def fuse_matmul_views(prog: V.VMProgram) -> None:
    if _off("PJRT_OCL_MM_VIEWFOLD"):
        return
    sc = scopes(prog)
    changed = True
    while changed:
        changed = False
        ix = _Index(prog)
        for gi, g in enumerate(prog.instrs):
            if not _gather_foldable(prog, ix, sc, gi, g):
                continue
            readers = ix.live_readers(g.dst)
            if not readers:
                continue

            def ok(r):
                if r.op != V.OP_DOT:
                    return False
                if (r.a == g.dst and r.aview) or (r.b == g.dst and r.bview):
                    return False
                return (r.a == g.dst and not r.aview) or (r.b == g.dst and not r.bview)
            if not all(ok(prog.instrs[j]) for j in readers):
                continue
            for j in readers:
                r = prog.instrs[j]
                if r.a == g.dst and not r.aview:
                    r.a, r.aview = g.a, g.aux + 1
                if r.b == g.dst and not r.bview:
                    r.b, r.bview = g.a, g.aux + 1
            prog.instrs[gi] = V.Instr(V.OP_NOP)
            changed = True
            break


def fuse_views(prog: V.VMProgram) -> None:
    if _off("PJRT_OCL_VIEWFOLD"):
        return
    sc = scopes(prog)
    changed = True
    while changed:
        changed = False
        ix = _Index(prog)
        for gi, g in enumerate(prog.instrs):
            if not _gather_foldable(prog, ix, sc, gi, g) or _dt(prog, g.dst) != V.DT_F32:
                continue
            readers = ix.live_readers(g.dst)
            if not readers:
                continue

            def ok(r):
                if r.op not in VIEWABLE_EW or _dt(prog, r.dst) != V.DT_F32:
                    return False
                if r.a == g.dst and r.imm:
                    return False
                if r.op in _BINARY_VIEW and r.b == g.dst and r.imm2:
                    return False
                return r.a == g.dst or (r.op in _BINARY_VIEW and r.b == g.dst)
            if not all(ok(prog.instrs[j]) for j in readers):
                continue
            for j in readers:
                r = prog.instrs[j]
                if r.a == g.dst:
                    r.a, r.imm = g.a, g.aux + 1
                if r.op in _BINARY_VIEW and r.b == g.dst:
                    r.b, r.imm2 = g.a, g.aux + 1
            prog.instrs[gi] = V.Instr(V.OP_NOP)
            changed = True
            break


# ---- fuse_norm (lowering.py:1561-1724) ------------------------------------------------------

def fuse_norm(prog: V.VMProgram) -> None:
    """softmax: max -> x - max -> exp -> sum -> exp / sum  => OP_SOFTMAX.
    layernorm core: mean = sum / seg; xc = x - mean; var = sum(xc * xc) / seg;
    r = rsqrt(var + eps) (or (var + eps) ** -0.5); xc * r  => one row op (the
    two-pass variance of the program, OP_LAYERNORM_AFFINE without gamma/beta)."""
    if _off("PJRT_OCL_FUSE_NORM"):
        return
    outs = set(prog.outputs)
    sc = scopes(prog)
    consts = _const_values(prog)
    changed = True
    while changed:
        changed = False
        ix = _Index(prog)
        instrs = prog.instrs

        def src(buf, view):
            """The buffer a (possibly viewed) operand reads, if the view is a row
            broadcast of a [rows] vector (or no view)."""
            return buf

        def readers_op(buf, op):
            return [(j, instrs[j]) for j in ix.live_readers(buf) if instrs[j].op == op]

        def row_bcast(ins, which, vec_buf, rows, seg):
            """operand `which` (a/b) of ins reads vec_buf[rows] broadcast along seg."""
            buf, view = (ins.a, ins.imm) if which == "a" else (ins.b, ins.imm2)
            if buf != vec_buf or not view:
                return False
            dims, st, off = _view_desc(prog, view)
            if off != 0 or int(np.prod(dims)) != rows * seg:
                return False
            # element (r, c) reads vec[r]: the inner seg elements have stride 0,
            # the outer axes index vec row-major
            inner, outer, ok = 1, 1, True
            for d in range(len(dims) - 1, -1, -1):
                if dims[d] == 1:
                    continue
                if inner < seg:
                    ok &= st[d] == 0
                    inner *= dims[d]
                else:
                    ok &= st[d] == outer
                    outer *= dims[d]
            return ok and inner == seg and outer == rows

        def div_by_const(buf, rows, seg):
            """readers of buf of the form buf / seg (scalar constant)."""
            out = []
            for j, d in readers_op(buf, V.OP_DIV_F32):
                if d.a == buf and not d.imm and d.n == rows and consts.get(d.b) == float(seg) and \
                        (not d.imm2 or _is_splat(prog, d.imm2)) and sc[j] == sc[ix.unique_writer(buf)]:
                    out.append((j, d))
            return out

        for ri, R in enumerate(instrs):
            if R.op != V.OP_REDUCE_SEG or _dt(prog, R.dst) != V.DT_F32:
                continue
            kind, seg = R.imm >> 28, R.imm & 0x0FFFFFFF
            X, rows = R.a, R.n
            total = rows * seg
            if seg == 0 or _dt(prog, X) != V.DT_F32:
                continue
            if kind == V.RED_MAX:                           # softmax
                for si, SUB in readers_op(X, V.OP_SUB_F32):
                    if SUB.a != X or SUB.imm or SUB.n != total or not row_bcast(SUB, "b", R.dst, rows, seg):
                        continue
                    for ei, EXP in readers_op(SUB.dst, V.OP_EXP_F32):
                        if EXP.imm or len(ix.live_readers(SUB.dst)) != 1:
                            continue
                        sums = [(j, r) for j, r in readers_op(EXP.dst, V.OP_REDUCE_SEG)
                                if r.imm == ((V.RED_SUM << 28) | seg) and r.n == rows]
                        divs = [(j, d) for j, d in readers_op(EXP.dst, V.OP_DIV_F32)
                                if d.a == EXP.dst and not d.imm and d.n == total]
                        for (r2i, R2), (di, DIV) in ((s, d) for s in sums for d in divs):
                            if not row_bcast(DIV, "b", R2.dst, rows, seg):
                                continue
                            if len({sc[x] for x in (ri, si, ei, r2i, di)}) != 1 or (DIV.dst in outs and X == DIV.dst):
                                continue
                            instrs[di] = V.Instr(V.OP_SOFTMAX, dst=DIV.dst, a=X, b=X, n=rows, imm=seg)
                            changed = True
                            break
                        if changed:
                            break
                    if changed:
                        break
            elif kind == V.RED_SUM:                         # layernorm core
                for mi, MU in div_by_const(R.dst, rows, seg):
                    subs = [(j, s) for j, s in readers_op(X, V.OP_SUB_F32)
                            if s.a == X and not s.imm and s.n == total and row_bcast(s, "b", MU.dst, rows, seg)]
                    for si, SUB in subs:
                        xc = SUB.dst
                        sq = [(j, m) for j, m in readers_op(xc, V.OP_MUL_F32)
                              if m.a == xc and m.b == xc and not m.imm and not m.imm2 and m.n == total]
                        for qi, SQ in sq:
                            r2 = [(j, r) for j, r in readers_op(SQ.dst, V.OP_REDUCE_SEG)
                                  if r.imm == ((V.RED_SUM << 28) | seg) and r.n == rows]
                            for r2i, R2 in r2:
                                for vi, VAR in div_by_const(R2.dst, rows, seg):
                                    hit = _norm_tail(prog, ix, instrs, VAR, xc, rows, seg, total, consts, row_bcast)
                                    if hit is None:
                                        continue
                                    oi, OUT, eps = hit
                                    if len({sc[x] for x in (ri, mi, si, qi, r2i, vi, oi)}) != 1:
                                        continue
                                    if OUT.dst in outs and X == OUT.dst:
                                        continue
                                    desc = prog.aux.__len__()
                                    prog.aux.extend([V.LN_TWO_PASS, 0])
                                    instrs[oi] = V.Instr(V.OP_LAYERNORM_AFFINE, dst=OUT.dst, a=X, b=X, n=rows,
                                                         imm=seg, imm2=_bits(eps), aux=desc)
                                    changed = True
                                    break
                                if changed:
                                    break
                            if changed:
                                break
                        if changed:
                            break
                    if changed:
                        break
            if changed:
                break


def _norm_tail(prog, ix, instrs, VAR, xc, rows, seg, total, consts, row_bcast):
    """var -> + eps -> rsqrt (or ** -0.5) -> xc * r.  Returns (index, OUT, eps)."""
    for ai in ix.live_readers(VAR.dst):
        AFF = instrs[ai]
        if AFF.op != V.OP_AFFINE_F32 or AFF.a != VAR.dst or _f(AFF.imm) != 1.0:
            continue
        eps = _f(AFF.imm2)
        for pi in ix.live_readers(AFF.dst):
            P = instrs[pi]
            ok = (P.op == V.OP_RSQRT_F32 and P.a == AFF.dst and not P.imm) or \
                 (P.op == V.OP_POW_F32 and P.a == AFF.dst and not P.imm and consts.get(P.b) == -0.5)
            if not ok:
                continue
            for oi in ix.live_readers(P.dst):
                OUT = instrs[oi]
                if OUT.op != V.OP_MUL_F32 or OUT.n != total:
                    continue
                if OUT.a == xc and not OUT.imm and row_bcast(OUT, "b", P.dst, rows, seg):
                    return oi, OUT, eps
                if OUT.b == xc and not OUT.imm2 and row_bcast(OUT, "a", P.dst, rows, seg):
                    return oi, OUT, eps
    return None


def fuse_norm_epilogue(prog: V.VMProgram) -> None:
    """Extension: a layernorm row op followed by y * gamma + beta (per-column f32
    vectors), then GELU, then a convert to bf16 / f16 -> one row op with the
    LAYERNORM_SEG flags (one read, one write)."""
    if _off("PJRT_OCL_FUSE_NORM"):
        return
    outs = set(prog.outputs)
    sc = scopes(prog)
    changed = True
    while changed:
        changed = False
        ix = _Index(prog)
        instrs = prog.instrs
        for li, LN in enumerate(instrs):
            if LN.op != V.OP_LAYERNORM_AFFINE:
                continue
            flags, beta = prog.aux[LN.aux], prog.aux[LN.aux + 1]
            rows, seg = LN.n, LN.imm
            total = rows * seg
            cur = LN.dst
            if cur in outs or _dt(prog, cur) != V.DT_F32:
                continue
            rs = ix.live_readers(cur)
            if len(rs) != 1 or sc[rs[0]] != sc[li]:
                continue
            j = rs[0]
            C = instrs[j]
            new = None
            if not flags & (V.LN_AFFINE | V.LN_GELU) and C.op == V.OP_MUL_F32 and C.n == total:
                vec = None
                if C.a == cur and not C.imm and _row_vector(prog, C.imm2, seg, total):
                    vec = C.b
                elif C.b == cur and not C.imm2 and _row_vector(prog, C.imm, seg, total):
                    vec = C.a
                if vec is not None and _dt(prog, vec) == V.DT_F32 and _elems(prog, vec) == seg:
                    # + beta must follow
                    rs2 = ix.live_readers(C.dst)
                    if len(rs2) == 1 and C.dst not in outs and sc[rs2[0]] == sc[li]:
                        k = rs2[0]
                        A = instrs[k]
                        bvec = None
                        if A.op == V.OP_ADD_F32 and A.n == total:
                            if A.a == C.dst and not A.imm and _row_vector(prog, A.imm2, seg, total):
                                bvec = A.b
                            elif A.b == C.dst and not A.imm2 and _row_vector(prog, A.imm, seg, total):
                                bvec = A.a
                        if bvec is not None and _dt(prog, bvec) == V.DT_F32 and _elems(prog, bvec) == seg \
                                and _written_before(ix, bvec, li) and _written_before(ix, vec, li):
                            new = (flags | V.LN_AFFINE, vec, bvec, A.dst, [j, k])
            elif not flags & V.LN_GELU and C.op == V.OP_GELU and C.a == cur and not C.imm and C.n == total:
                new = (flags | V.LN_GELU, LN.b, beta, C.dst, [j])
            elif C.op == V.OP_CONVERT and C.a == cur and C.n == total and \
                    _dt(prog, C.dst) in (V.DT_BF16, V.DT_F16, V.DT_F32):
                new = (flags, LN.b, beta, C.dst, [j])
            if new is None:
                continue
            nflags, gamma, nbeta, dst, consumed = new
            off = len(prog.aux)
            prog.aux.extend([nflags, nbeta if nflags & V.LN_AFFINE else 0])
            last = consumed[-1]
            instrs[last] = V.Instr(V.OP_LAYERNORM_AFFINE, dst=dst, a=LN.a,
                                   b=gamma if nflags & V.LN_AFFINE else LN.a, n=rows, imm=seg,
                                   imm2=LN.imm2, aux=off,
                                   reads_hint=(nbeta,) if nflags & V.LN_AFFINE else ())
            for x in [li] + consumed[:-1]:
                instrs[x] = V.Instr(V.OP_NOP)
            changed = True
            break


def _row_vector(prog, view1: int, seg: int, total: int) -> bool:
    """An elementwise operand that reads a [seg] vector once per row: a
    row-broadcast view, or the plain vector when there is one row."""
    if view1:
        return _is_row_broadcast(prog, view1, seg)
    return total == seg


def _written_before(ix, buf, idx) -> bool:
    return all(w < idx for w in ix.writers.get(buf, ()))


# ---- fuse_gelu (lowering.py:1737-1876) ------------------------------------------------------

_GELU_CUBE = float(np.float32(0.044715))
_GELU_SQRT = float(np.float32(0.7978845608))


def _close(v, ref, rtol=1e-6) -> bool:
    return v is not None and abs(v - ref) <= rtol * abs(ref) + 1e-12


def fuse_gelu(prog: V.VMProgram) -> None:
    """x * (s_t * (tanh(0.7978845608 * (x + 0.044715 * x^3)) + 1)), with the x
    factor x itself or s_x * x and s_x * s_t == 0.5 => OP_GELU."""
    if _off("PJRT_OCL_FUSE_GELU"):
        return
    outs = set(prog.outputs)
    changed = True
    while changed:
        changed = False
        ix = _Index(prog)
        instrs = prog.instrs

        def prod(buf, op):
            return ix.producer(buf, op)

        def affine(buf, s, t):
            a = prod(buf, V.OP_AFFINE_F32)
            if a is None or not _close(_f(a.imm), s) or not _close(_f(a.imm2), t):
                return None
            return a

        def backbone(tin, total):
            A = affine(tin, _GELU_SQRT, 0.0)
            if A is None or A.n != total:
                return None
            ADD = prod(A.a, V.OP_ADD_F32)
            if ADD is None or ADD.n != total or ADD.imm or ADD.imm2:
                return None
            for X, cb in ((ADD.a, ADD.b), (ADD.b, ADD.a)):
                C = affine(cb, _GELU_CUBE, 0.0)
                if C is None or C.n != total:
                    continue
                M3 = prod(C.a, V.OP_MUL_F32)
                if M3 is None or M3.n != total or M3.imm or M3.imm2:
                    continue
                x2 = M3.b if M3.a == X else (M3.a if M3.b == X else None)
                if x2 is None:
                    continue
                M2 = prod(x2, V.OP_MUL_F32)
                if M2 is None or M2.n != total or M2.imm or M2.imm2 or M2.a != X or M2.b != X:
                    continue
                return X
            return None

        for oi, OUT in enumerate(instrs):
            if OUT.op != V.OP_MUL_F32 or OUT.imm or OUT.imm2:
                continue
            total = OUT.n
            for tf, xf in ((OUT.a, OUT.b), (OUT.b, OUT.a)):
                TF = prod(tf, V.OP_AFFINE_F32)
                if TF is None or TF.n != total:
                    continue
                s_t = _f(TF.imm)
                if not _close(_f(TF.imm2), s_t):
                    continue
                TANH = prod(TF.a, V.OP_TANH_F32)
                if TANH is None or TANH.n != total or TANH.imm:
                    continue
                X = backbone(TANH.a, total)
                if X is None:
                    continue
                if xf == X:
                    s_x = 1.0
                else:
                    XF = prod(xf, V.OP_AFFINE_F32)
                    if XF is None or XF.a != X or XF.n != total or not _close(_f(XF.imm2), 0.0):
                        continue
                    s_x = _f(XF.imm)
                if not _close(s_x * s_t, 0.5) or (OUT.dst in outs and X == OUT.dst):
                    continue
                instrs[oi] = V.Instr(V.OP_GELU, dst=OUT.dst, a=X, b=X, n=total)
                changed = True
                break
            if changed:
                break


# ---- fuse_mma_epilogue (lowering.py:2486-2601) ----------------------------------------------

_EPI_BIN = {V.OP_ADD_F32: V.SUB_ADD, V.OP_MUL_F32: V.SUB_MUL, V.OP_SUB_F32: V.SUB_SUB,
            V.OP_DIV_F32: V.SUB_DIV, V.OP_MAX_F32: V.SUB_MAX, V.OP_MIN_F32: V.SUB_MIN}
_COMMUTES = {V.OP_ADD_F32, V.OP_MUL_F32, V.OP_MAX_F32, V.OP_MIN_F32}


def fuse_mma_epilogue(prog: V.VMProgram) -> None:
    if _off("PJRT_OCL_FUSE_MMA_EPI"):
        return
    outs = set(prog.outputs)
    sc = scopes(prog)
    consts = _const_values(prog)
    ix = _Index(prog)
    instrs = prog.instrs
    for di, DOT in enumerate(instrs):
        if DOT.op != V.OP_DOT or DOT.epi:
            continue
        M, N, G = DOT.n, DOT.imm >> 16, max(1, DOT.imm2)
        total = M * N * G
        if N == 1 and G == 1:
            continue                    # the RED_SEG dot mode has no epilogue
        if _dt(prog, DOT.dst) != V.DT_F32:
            continue
        micros, consumed, res = [], [], 0
        cur = DOT.dst
        last = DOT.dst
        while True:
            rs = [j for j in ix.live_readers(cur) if j != di]
            if len(rs) != 1 or cur in outs or len(ix.writers.get(cur, ())) != 1:
                break
            ci = rs[0]
            c = instrs[ci]
            if sc[ci] != sc[di] or len(ix.writers.get(c.dst, ())) != 1:
                break
            if c.op == V.OP_CONVERT and c.a == cur and c.n == total and \
                    _dt(prog, c.dst) in (V.DT_BF16, V.DT_F16):
                consumed.append(ci)
                last = c.dst
                break                   # the store converts; nothing follows it
            if c.n != total or _dt(prog, c.dst) != V.DT_F32:
                break
            if c.op == V.OP_GELU and c.a == cur and not c.imm:
                micros.append((V.SUB_GELU, 0, 0, 0))
            elif c.op == V.OP_AFFINE_F32 and c.a == cur:
                micros.append((V.SUB_AFFINE, 0, c.imm, c.imm2))
            elif c.op in _EPI_BIN:
                if c.a == cur and not c.imm:
                    other, oview = c.b, c.imm2
                elif c.b == cur and not c.imm2 and c.op in _COMMUTES:
                    other, oview = c.a, c.imm
                else:
                    break
                kind = _EPI_BIN[c.op]
                if other == cur:
                    break
                if oview and _is_splat(prog, oview) and other in consts:
                    micros.append((kind, 3, _bits(consts[other]), 0))            # constant operand
                elif res == 0 and oview and _is_row_broadcast(prog, oview, N) and \
                        _dt(prog, other) == V.DT_F32 and _elems(prog, other) == N and _written_before(ix, other, di):
                    micros.append((kind, 2, 0, 0))                              # per-column vector
                    res = other
                elif res == 0 and not oview and _dt(prog, other) == V.DT_F32 and _elems(prog, other) == total \
                        and _written_before(ix, other, di) and other != c.dst:
                    micros.append((kind, 1, 0, 0))                              # residual per element
                    res = other
                else:
                    break
            else:
                break
            consumed.append(ci)
            last = c.dst
            cur = c.dst
        if not consumed:
            continue
        desc = [len(micros)]
        for kind, src, s, t in micros:
            desc += [kind, src, s & 0xFFFFFFFF, t & 0xFFFFFFFF]
        off = len(prog.aux)
        prog.aux.extend(desc)
        for ci in consumed:
            instrs[ci] = V.Instr(V.OP_NOP)
        DOT.dst = last
        if micros:
            DOT.epi, DOT.epi_res = off + 1, res
            if res:
                DOT.reads_hint = tuple(DOT.reads_hint) + (res,)
        ix = _Index(prog)


# ---- fuse_region (lowering.py:2071-2378) ----------------------------------------------------

_REGION_KIND = {V.OP_ADD_F32: (V.SUB_ADD, 2), V.OP_SUB_F32: (V.SUB_SUB, 2), V.OP_MUL_F32: (V.SUB_MUL, 2),
                V.OP_DIV_F32: (V.SUB_DIV, 2), V.OP_MAX_F32: (V.SUB_MAX, 2), V.OP_MIN_F32: (V.SUB_MIN, 2),
                V.OP_POW_F32: (V.SUB_POW, 2), V.OP_NEG_F32: (V.SUB_NEG, 1), V.OP_EXP_F32: (V.SUB_EXP, 1),
                V.OP_LOG_F32: (V.SUB_LOG, 1), V.OP_SQRT_F32: (V.SUB_SQRT, 1), V.OP_RSQRT_F32: (V.SUB_RSQRT, 1),
                V.OP_TANH_F32: (V.SUB_TANH, 1), V.OP_ABS_F32: (V.SUB_ABS, 1), V.OP_AFFINE_F32: (V.SUB_AFFINE, 1),
                V.OP_GELU: (V.SUB_GELU, 1), V.OP_FLOOR_F32: (V.SUB_FLOOR, 1), V.OP_CEIL_F32: (V.SUB_CEIL, 1),
                V.OP_SIGN_F32: (V.SUB_SIGN, 1), V.OP_LOG1P_F32: (V.SUB_LOG1P, 1),
                V.OP_EXPM1_F32: (V.SUB_EXPM1, 1), V.OP_SIN_F32: (V.SUB_SIN, 1), V.OP_COS_F32: (V.SUB_COS, 1)}
_REGION_SLOTS = 8
_REGION_MAXIN = 8


def fuse_region(prog: V.VMProgram) -> None:
    """Connected chains of same-size f32 map ops whose intermediates are read
    only inside the chain -> one OP_MAP_REGION at the chain's last op (one load
    per input, one store).  Gates: operands read directly (no views), every
    member written once, at most 8 inputs and 8 register slots."""
    if _off("PJRT_OCL_FUSE_REGION"):
        return
    outs = set(prog.outputs)
    sc = scopes(prog)
    changed = True
    while changed:
        changed = False
        ix = _Index(prog)
        instrs = prog.instrs

        def eligible(i):
            ins = instrs[i]
            k = _REGION_KIND.get(ins.op)
            if k is None or _dt(prog, ins.dst) != V.DT_F32:
                return False
            if ins.op != V.OP_AFFINE_F32 and (ins.imm or (k[1] == 2 and ins.imm2)):
                return False
            ops = (ins.a, ins.b) if k[1] == 2 else (ins.a,)
            if any(_dt(prog, b) != V.DT_F32 or _elems(prog, b) < ins.n for b in ops):
                return False
            return len(ix.writers.get(ins.dst, ())) == 1

        def operands(ins):
            return (ins.a, ins.b) if _REGION_KIND[ins.op][1] == 2 else (ins.a,)

        for root, R in enumerate(instrs):
            if not eligible(root):
                continue
            # the root's value must leave the chain: read outside or an output
            members = {root}
            frontier = [root]
            while frontier:
                m = frontier.pop()
                for b in operands(instrs[m]):
                    w = ix.unique_writer(b)
                    if w is None or w in members or not eligible(w) or sc[w] != sc[root]:
                        continue
                    if instrs[w].n != R.n or b in outs:
                        continue
                    if any(r not in members and r != m for r in ix.live_readers(b)):
                        # b is also read outside: it can only join if every reader is a member
                        rd = set(ix.live_readers(b))
                        if not rd <= members | {m}:
                            continue
                    members.add(w)
                    frontier.append(w)
            if len(members) < 2:
                continue
            # no member's dst may be read outside the region except the root's
            if any(set(ix.live_readers(instrs[m].dst)) - members for m in members if m != root):
                continue
            order = sorted(members)
            produced = {instrs[m].dst for m in order}
            inputs = []
            for m in order:
                for b in operands(instrs[m]):
                    if b not in produced and b not in inputs:
                        inputs.append(b)
            if not 1 <= len(inputs) <= _REGION_MAXIN:
                continue
            # inputs must hold the same values at every member's position
            lo = order[0]
            if any(any(lo <= w <= root for w in ix.writers.get(b, ())) for b in inputs):
                continue
            slot = _region_slots(order, instrs, inputs, R.dst, operands)
            if slot is None:
                continue
            micro = []
            for m in order:
                ins = instrs[m]
                kind, ar = _REGION_KIND[ins.op]
                ops = operands(ins)
                a_s = slot[ops[0]]
                b_s = slot[ops[1]] if ar == 2 else a_s
                s, t = (ins.imm, ins.imm2) if ins.op == V.OP_AFFINE_F32 else (0, 0)
                micro += [kind, slot[("d", m)], a_s, b_s, s, t]
            desc = [len(inputs), slot[("d", root)], len(order)] + [slot[b] for b in inputs] + micro + inputs
            off = len(prog.aux)
            prog.aux.extend(desc)
            for m in order:
                if m != root:
                    instrs[m] = V.Instr(V.OP_NOP)
            instrs[root] = V.Instr(V.OP_MAP_REGION, dst=R.dst, a=inputs[0], b=inputs[-1], n=R.n, aux=off,
                                   region_inputs=tuple(inputs))
            changed = True
            break


def _region_slots(order, instrs, inputs, out_buf, operands):
    """Linear-scan register slots (lowering.py:1953-1999): inputs live from the
    start, each member's value from its definition to its last use."""
    last = {}
    for i, m in enumerate(order):
        for b in operands(instrs[m]):
            last[b] = i
    slot, active, free, nxt = {}, {}, [], 0

    def alloc():
        nonlocal nxt
        if free:
            return free.pop()
        nxt += 1
        return nxt - 1
    for b in inputs:
        slot[b] = alloc()
        active[b] = slot[b]
    for i, m in enumerate(order):
        for v in [v for v in active if last.get(v, -1) < i]:
            free.append(active.pop(v))
        s = alloc()
        d = instrs[m].dst
        slot[("d", m)] = s
        slot[d] = s
        active[d] = s
        if nxt > _REGION_SLOTS:
            return None
    return slot


# ---- fuse_attention (lowering.py:2664-2810) --------------------------------------------------

def fuse_attention(prog: V.VMProgram) -> None:
    """DOT1(Q, K^T) [* scale] [masked by a causal select] -> softmax [-> convert]
    -> DOT2(P, V) [-> convert] => OP_FLASH_ATTN.  Q, K, V keep the matmuls' folded
    views.  The mask is recognised by evaluating its predicate, which depends on
    iotas and constants only, and comparing it with the causal rule
    key <= query + (C - T)."""
    if _off("PJRT_OCL_FLASH"):
        return
    outs = set(prog.outputs)
    sc = scopes(prog)
    consts = _const_values(prog)
    changed = True
    while changed:
        changed = False
        ix = _Index(prog)
        instrs = prog.instrs
        for si, SM in enumerate(instrs):
            if SM.op != V.OP_SOFTMAX:
                continue
            C, rows = SM.imm, SM.n
            consumed = []
            scale = 1.0
            causal = 0
            cur = SM.a
            dot1 = None
            for _ in range(6):
                if cur in outs or len(ix.live_readers(cur)) != 1:
                    break
                w = ix.unique_writer(cur)
                if w is None or sc[w] != sc[si]:
                    break
                P = instrs[w]
                if P.op == V.OP_DOT:
                    dot1 = w
                    break
                if P.op == V.OP_AFFINE_F32 and not P.imm2 and P.n == rows * C:
                    scale *= _f(P.imm)
                elif P.op in (V.OP_MUL_F32, V.OP_DIV_F32) and not P.imm and P.imm2 and P.n == rows * C and \
                        _is_splat(prog, P.imm2) and P.b in consts and consts[P.b] not in (0.0,):
                    scale = scale * consts[P.b] if P.op == V.OP_MUL_F32 else scale / consts[P.b]
                elif P.op == V.OP_SELECT_F32 and not causal:
                    neg = _eval_const(prog, ix, _peel_broadcast(prog, ix, P.b))
                    if neg is None or neg.size != 1 or not (float(neg[0]) == -math.inf or float(neg[0]) <= -1e30):
                        break
                    mask = _eval_const(prog, ix, _peel_broadcast(prog, ix, P.imm))
                    if mask is None or not _is_causal(mask, C):
                        break
                    causal = 1
                    consumed.append(w)
                    cur = P.a
                    continue
                elif P.op == V.OP_GATHER_STRIDED and _is_identity_view(prog, P.aux + 1, P.n):
                    pass
                else:
                    break
                consumed.append(w)
                cur = P.a
            if dot1 is None:
                continue
            D1 = instrs[dot1]
            G1, M1, N1, hd = max(1, D1.imm2), D1.n, D1.imm >> 16, D1.imm & 0xFFFF
            if N1 != C or G1 * M1 != rows or hd > 256 or len(ix.live_readers(D1.dst)) != 1:
                continue
            if D1.epi:
                e = D1.epi - 1
                if prog.aux[e] != 1 or prog.aux[e + 1] != V.SUB_AFFINE or prog.aux[e + 2] != 0 or \
                        _f(prog.aux[e + 4]) != 0.0:
                    continue
                scale *= _f(prog.aux[e + 3])
            fwd = ix.live_readers(SM.dst)
            if SM.dst in outs or len(fwd) != 1:
                continue
            p_buf, d2i = SM.dst, fwd[0]
            mid = []
            if instrs[d2i].op == V.OP_CONVERT:
                cv = instrs[d2i]
                nxt = ix.live_readers(cv.dst)
                if cv.dst in outs or len(nxt) != 1:
                    continue
                mid.append(d2i)
                p_buf, d2i = cv.dst, nxt[0]
            D2 = instrs[d2i]
            if D2.op != V.OP_DOT or D2.a != p_buf or D2.aview or D2.epi:
                continue
            G2, M2, N2, K2 = max(1, D2.imm2), D2.n, D2.imm >> 16, D2.imm & 0xFFFF
            if G2 != G1 or M2 != M1 or K2 != C or N2 != hd:
                continue
            out, tail = D2.dst, []
            rs = ix.live_readers(out)
            if len(rs) == 1 and out not in outs and instrs[rs[0]].op == V.OP_CONVERT and \
                    instrs[rs[0]].a == out and sc[rs[0]] == sc[si]:
                tail = [rs[0]]
                out = instrs[rs[0]].dst
            adt = _dt(prog, D1.a)
            if _dt(prog, D1.b) != adt or _dt(prog, D2.b) != adt or scale <= 0 and causal:
                continue
            if len({sc[x] for x in [dot1, si, d2i] + consumed + mid + tail}) != 1:
                continue
            qv, kv, vv = (_canonical_view(prog, v, n) for v, n in
                          ((D1.aview, G1 * M1 * hd), (D1.bview, G1 * hd * C), (D2.bview, G1 * C * hd)))
            kt = [3, G1, hd, C, C * hd, 1, hd, 0]
            if kv and _merged(*_view_desc(prog, kv)) == _merged(kt[1:4], kt[4:7], 0):
                kv = len(prog.aux) + 1            # the plain transpose of a [G, C, hd] K
                prog.aux.extend(kt)
            last = tail[-1] if tail else d2i
            free = sorted(consumed + [dot1, si] + mid + ([d2i] if tail else []))
            qa, kb, vb = D1.a, D1.b, D2.b
            placed = []
            if (adt in (V.DT_BF16, V.DT_F16) and hd % 8 == 0 and 8 <= hd <= 256 or
                    adt == V.DT_F32 and hd % 4 == 0 and 4 <= hd <= 128) and scale > 0 and \
                    (qv or vv or not (kv and prog.aux[kv - 1:kv + 7] == kt)):
                # the matrix-core kernel reads Q and V as plain [G, rows, hd]
                # and K as the transpose of a plain [G, C, hd]: strided operands
                # (the heads of a fused QKV projection) are gathered into that
                # layout first, in slots the fused chain frees
                plan = _attn_gathers(prog, qa, kb, vb, qv, kv, vv, G1, M1, C, hd, adt, kt)
                placed = _place_gathers(ix, sc, si, free, last, plan)
                if placed is not None:
                    for slot, ins in placed:
                        free.remove(slot)
                    qa, kb, vb, qv, kv, vv = plan[-1]
                else:
                    placed = []
            desc = len(prog.aux)
            prog.aux.extend([G1, M1, C, hd, _bits(scale), causal, qv, kv, vv])
            for j in free:
                instrs[j] = V.Instr(V.OP_NOP)
            for slot, ins in placed:
                instrs[slot] = ins
            instrs[last] = V.Instr(V.OP_FLASH_ATTN, dst=out, a=qa, b=kb, n=G1, imm=M1, imm2=vb,
                                   aux=desc, reads_hint=(vb,))
            changed = True
            break


def _attn_gathers(prog, qa, kb, vb, qv, kv, vv, G, M, C, hd, adt, kt):
    """Gathers that put attention operands in the matrix-core layout: a list of
    (source buffer, gather instruction) and, last, the new (q, k, v buffers,
    q, k, v views); None when K's view is not one over [G, hd, C]."""
    plan = []
    if not (kv and prog.aux[kv - 1:kv + 7] == kt):
        # B reads K^T [G, hd, C]: gather K [G, C, hd] with the last two axes swapped
        if kv:
            dims, st, off = _view_desc(prog, kv)
            if list(dims) == [hd, C] and G == 1:
                dims, st = [1, hd, C], [0] + list(st)
            if list(dims) != [G, hd, C]:
                return None
        else:
            st, off = [hd * C, C, 1], 0
        k = _new_buffer(prog, G * C * hd, adt)
        d = len(prog.aux)
        prog.aux.extend([3, G, C, hd, st[0], st[2], st[1], off])
        plan.append((kb, V.Instr(V.OP_GATHER_STRIDED, dst=k, a=kb, n=G * C * hd, aux=d)))
        kb = k
        kv = len(prog.aux) + 1
        prog.aux.extend(kt)
    if qv:
        q = _new_buffer(prog, G * M * hd, adt)
        plan.append((qa, V.Instr(V.OP_GATHER_STRIDED, dst=q, a=qa, n=G * M * hd, aux=qv - 1)))
        qa, qv = q, 0
    if vv:
        v = _new_buffer(prog, G * C * hd, adt)
        plan.append((vb, V.Instr(V.OP_GATHER_STRIDED, dst=v, a=vb, n=G * C * hd, aux=vv - 1)))
        vb, vv = v, 0
    plan.append((qa, kb, vb, qv, kv, vv))
    return plan


def _place_gathers(ix, sc, si, free, last, plan):
    """(slot, instruction) for each gather of ``plan``: a freed slot after the
    last write of its source in the chain's scope, before ``last``; None if
    some gather finds none."""
    if plan is None:
        return None
    taken, out = set(), []
    for src, ins in plan[:-1]:
        after = max([w for w in ix.writers.get(src, ()) if sc[w] == sc[si] and w < last], default=-1)
        slot = next((j for j in free if j > after and j not in taken and j < last), None)
        if slot is None:
            return None
        taken.add(slot)
        out.append((slot, ins))
    return out


# ---- fuse_decode_attention (extension: no reference counterpart) ------------------------------

def fuse_decode_attention(prog: V.VMProgram) -> None:
    """The decode step of a decoder with a KV cache, in either of the two forms
    a JAX program writes per layer:

        masked:  K' = dynamic_update_slice(K, k, pos)   V' likewise with v
                 s = dot(q, K'^T) [* scale];  s = select(key <= pos, s, -inf)
                 o = dot(softmax(s) [-> convert], V') [-> convert]
        append:  KK = concatenate([K, k], 1)   VV likewise     (no mask;
                 o = dot(softmax(dot(q, KK^T) [* scale]), VV)  tools/bench_decode.py:47-52)

    => OP_DECODE_ATTN (krow when the keys are rows [H, C, hd]): one pass over the
    two caches instead of five barrier-separated ops, the append form without
    copying the caches into the concatenation.  The reference runs both chains
    op by op (python/pjrt_ocl/lowering.py:2664-2690 fuses only the constant-mask
    prefill form).  The mask is proven by evaluating its predicate for every
    position in [-2, C + 2]; the updates' position must be the same buffer, and
    the fused op runs before the updates (it reads cache columns before pos,
    which they do not write).  The append form reads the caches with pos = C."""
    if _off("PJRT_OCL_DECODE_ATTN"):
        return
    outs = set(prog.outputs)
    sc = scopes(prog)
    consts = _const_values(prog)
    changed = True
    while changed:
        changed = False
        ix = _Index(prog)
        instrs = prog.instrs
        for si, SM in enumerate(instrs):
            if SM.op != V.OP_SOFTMAX:
                continue
            m = _match_decode(prog, ix, sc, consts, outs, si)
            if m is None:
                continue
            (q, kbuf, vbuf, kc, vc, posb, H, C, hd, krow, scale, out, chain, last, qgather, dk, dv, masked) = m
            desc = len(prog.aux)
            prog.aux.extend([hd | int(krow) << 16 | int(masked) << 17, kbuf, vbuf, posb, _bits(scale)])
            fused = V.Instr(V.OP_DECODE_ATTN, dst=out, a=q, b=kc, n=H, imm=C, imm2=vc, aux=desc,
                            reads_hint=(vc, kbuf, vbuf, posb))
            # the op reads cache columns before pos only, which the updates do
            # not touch: it can run before them, so that they share a phase with
            # what follows instead of delaying the attention by one.  Only when
            # nothing else reads the caches in between.
            seq = ([qgather] if qgather is not None else []) + [fused]
            slots = sorted(set(chain) | {last})
            others = [j for b in (kc, vc) for j in ix.live_readers(b)
                      if masked and min(dk, dv) < j <= last and j not in chain and j not in (dk, dv)]
            if masked and not others:
                seq += [instrs[dk], instrs[dv]] if dk < dv else [instrs[dv], instrs[dk]]
                slots = sorted(set(slots) | {dk, dv})
            for j in slots:
                instrs[j] = V.Instr(V.OP_NOP)
            for j, ins in zip(slots, seq):
                instrs[j] = ins
            changed = True
            break


def _match_decode(prog, ix, sc, consts, outs, si):
    """The pieces of one decode attention around softmax ``si``, or None: the
    masked form (caches updated at pos, keys <= pos) or the append form (keys
    and values concatenated with the step's own, no mask)."""
    instrs = prog.instrs
    SM = instrs[si]
    nkeys, rows = SM.imm, SM.n
    consumed, scale, sel, dot1 = [], 1.0, None, None
    cur = SM.a
    for _ in range(6):
        if cur in outs or len(ix.live_readers(cur)) != 1:
            return None
        w = ix.unique_writer(cur)
        if w is None or sc[w] != sc[si]:
            return None
        P = instrs[w]
        if P.op == V.OP_DOT:
            dot1 = w
            break
        if P.op == V.OP_AFFINE_F32 and not P.imm2 and P.n == rows * nkeys:
            scale *= _f(P.imm)
        elif P.op in (V.OP_MUL_F32, V.OP_DIV_F32) and not P.imm and P.imm2 and P.n == rows * nkeys and \
                _is_splat(prog, P.imm2) and P.b in consts and consts[P.b] not in (0.0,):
            scale = scale * consts[P.b] if P.op == V.OP_MUL_F32 else scale / consts[P.b]
        elif P.op == V.OP_SELECT_F32 and sel is None and P.n == rows * nkeys:
            neg = _eval_const(prog, ix, _peel_broadcast(prog, ix, P.b))
            if neg is None or neg.size != 1 or not (float(neg[0]) == -math.inf or float(neg[0]) <= -1e30):
                return None
            sel = w
        elif P.op == V.OP_GATHER_STRIDED and _is_identity_view(prog, P.aux + 1, P.n):
            pass
        else:
            return None
        consumed.append(w)
        cur = P.a
    if dot1 is None:
        return None
    D1 = instrs[dot1]
    M1, N1, hd, G1, av1, bv1, epi1, _ = _dot_fields_pass(D1)
    if M1 != 1 or N1 != nkeys or G1 != rows or len(ix.live_readers(D1.dst)) != 1 or D1.dst in outs:
        return None
    if epi1:
        e = epi1 - 1
        if prog.aux[e] != 1 or prog.aux[e + 1] != V.SUB_AFFINE or prog.aux[e + 2] != 0 or \
                _f(prog.aux[e + 4]) != 0.0:
            return None
        scale *= _f(prog.aux[e + 3])
    H = G1
    # forward: softmax [-> convert] -> DOT2 [-> convert]
    fwd = ix.live_readers(SM.dst)
    if SM.dst in outs or len(fwd) != 1:
        return None
    p_buf, d2i, mid = SM.dst, fwd[0], []
    if instrs[d2i].op == V.OP_CONVERT:
        cv = instrs[d2i]
        nxt = ix.live_readers(cv.dst)
        if cv.dst in outs or len(nxt) != 1:
            return None
        mid.append(d2i)
        p_buf, d2i = cv.dst, nxt[0]
    D2 = instrs[d2i]
    if D2.op != V.OP_DOT or D2.a != p_buf:
        return None
    M2, N2, K2, G2, av2, bv2, epi2, _ = _dot_fields_pass(D2)
    if av2 or epi2 or G2 != H or M2 != 1 or K2 != nkeys or N2 != hd:
        return None
    out, tail = D2.dst, []
    rs = ix.live_readers(out)
    if len(rs) == 1 and out not in outs and instrs[rs[0]].op == V.OP_CONVERT and \
            instrs[rs[0]].a == out and sc[rs[0]] == sc[si]:
        tail = [rs[0]]
        out = instrs[rs[0]].dst
    adt = _dt(prog, D1.a)
    if adt not in (V.DT_F32, V.DT_F16, V.DT_BF16) or _dt(prog, D1.b) != adt or _dt(prog, D2.b) != adt \
            or _dt(prog, out) != adt or _elems(prog, out) != H * hd:
        return None
    if len({sc[x] for x in [dot1, si, d2i] + consumed + mid + tail}) != 1:
        return None
    last = tail[-1] if tail else d2i
    # the keys as dot1 reads them: rows [H, nkeys, hd] (read through the
    # transpose) or K^T [H, hd, nkeys]
    kview = _canonical_view(prog, bv1, H * hd * nkeys)
    if _elems(prog, D1.b) != H * nkeys * hd or _elems(prog, D2.b) != H * nkeys * hd or \
            _canonical_view(prog, bv2, H * nkeys * hd):
        return None
    if kview == 0:
        krow = False
    elif _merged(*_view_desc(prog, kview)) == _merged([H, hd, nkeys], [nkeys * hd, 1, hd], 0):
        krow = True
    else:
        return None
    if sel is not None:
        m = _masked_decode_parts(prog, ix, sc, instrs[sel].imm, D1, D2, dot1, d2i, last, H, nkeys, hd,
                                 krow, adt)
    else:
        m = _append_decode_parts(prog, ix, sc, D1, D2, dot1, last, H, nkeys, hd, krow, adt)
    if m is None:
        return None
    kc, vc, kbuf, vbuf, posb, C, masked, dk, dv = m
    if hd % 8 or hd > 256 or C % 8 or C < 8 or C > 0xFFFF:
        return None
    # nothing rewrites what the fused op reads between its sources and ``last``
    # (no region op in between either: its sub-list could)
    lo = min(x for x in (dk, dv, dot1) if x is not None)
    if any(instrs[j].op in _REGION_OPS for j in range(lo, last) if sc[j] == sc[si]):
        return None
    srcs = [(kc, dk), (vc, dv), (kbuf, dk), (vbuf, dv), (D1.a, dot1)]
    if masked:
        srcs += [(posb, dk), (posb, dv)]
    for buf, since in srcs:
        if any((since if since is not None else dot1) < w <= last for w in ix.writers.get(buf, ())):
            return None
    # q: the dot's A rows [H, 1, hd], contiguous
    qv = _canonical_view(prog, av1, H * hd)
    q, qgather = D1.a, None
    if qv or _elems(prog, D1.a) != H * hd:
        dims, st, off = _view_desc(prog, qv) if qv else ([H * hd], [1], 0)
        if _merged(dims, st, off) != (((H * hd, 1),), off) and _merged(dims, st, off) != ((), off):
            return None
        q = _new_buffer(prog, H * hd, adt)
        vdesc = len(prog.aux)
        prog.aux.extend([1, H * hd, 1, off])
        qgather = V.Instr(V.OP_GATHER_STRIDED, dst=q, a=D1.a, n=H * hd, aux=vdesc)
    if posb is None:
        posb = _new_buffer(prog, 1, V.DT_I32)
        prog.consts.append((posb, np.array([C], "<i4").tobytes()))
    chain = consumed + [dot1, si, d2i] + mid + tail
    return (q, kbuf, vbuf, kc, vc, posb, H, C, hd, krow, scale, out, chain, last, qgather, dk, dv, masked)


def _masked_decode_parts(prog, ix, sc, pred, D1, D2, dot1, d2i, last, H, C, hd, krow, adt):
    """The masked form: the caches dot1 / dot2 read were just updated at pos
    (dynamic_update_slice, the same position buffer for both) and the mask is
    key <= pos.  (kc, vc, k, v, pos, C, masked, update_k, update_v) or None."""
    kc, vc = D1.b, D2.b
    dk = _last_writer(ix, kc, dot1, sc)
    dv = _last_writer(ix, vc, d2i, sc)
    if dk is None or dv is None:
        return None
    uk = _dus_fields(prog, prog.instrs[dk])
    uv = _dus_fields(prog, prog.instrs[dv])
    if uk is None or uv is None:
        return None
    kdims, kids, kbuf = uk
    vdims, vids, vbuf = uv
    if tuple(kdims) != ((H, 1, hd) if krow else (H, hd, 1)) or tuple(vdims) != (H, 1, hd):
        return None
    posb = kids[1] if krow else kids[2]
    if vids[1] != posb or prog.buffers[posb].dtype != V.DT_I32 or _elems(prog, posb) != 1:
        return None
    if _elems(prog, kbuf) != H * hd or _elems(prog, vbuf) != H * hd or _dt(prog, kbuf) != adt or \
            _dt(prog, vbuf) != adt:
        return None
    if not _mask_is_key_le_pos(prog, ix, pred, posb, C):
        return None
    return kc, vc, kbuf, vbuf, posb, C, True, dk, dv


def _append_decode_parts(prog, ix, sc, D1, D2, dot1, last, H, nkeys, hd, krow, adt):
    """The append form (tools/bench_decode.py:47-52): the keys are
    concatenate([K cache, k], axis 1) and the values likewise, both as rows
    [H, C + 1, hd], every key visible.  The op then reads the caches in place
    with pos = C.  (kc, vc, k, v, None, C, masked, None, None) or None."""
    if not krow:
        return None
    C = nkeys - 1
    got = []
    for buf in (D1.b, D2.b):
        ws = ix.writers.get(buf, ())
        if len(ws) != 2 or len([j for j in ix.live_readers(buf) if j not in ws]) != 1:
            return None
        parts = {}
        for w in ws:
            S_ = prog.instrs[w]
            if S_.op != V.OP_SCATTER or not S_.disjoint or sc[w] != sc[dot1] or w > dot1:
                return None
            a = S_.aux
            rank = prog.aux[a]
            if rank != 3:
                return None
            dims = tuple(prog.aux[a + 1:a + 4])
            st = tuple(prog.aux[a + 4:a + 7])
            off = prog.aux[a + 7]
            if st != (nkeys * hd, hd, 1):
                return None
            parts[(dims, off)] = S_.a
        cache, new = parts.get(((H, C, hd), 0)), parts.get(((H, 1, hd), C * hd))
        if cache is None or new is None or prog.instrs[ws[0]].disjoint != prog.instrs[ws[1]].disjoint:
            return None
        if _elems(prog, cache) != H * C * hd or _elems(prog, new) != H * hd or _dt(prog, cache) != adt or \
                _dt(prog, new) != adt:
            return None
        got.append((cache, new))
    (kc, kbuf), (vc, vbuf) = got
    return kc, vc, kbuf, vbuf, None, C, False, None, None


def _dot_fields_pass(ins):
    """(M, N, K, G, aview, bview, epi, epi_res) of an in-memory OP_DOT."""
    return (ins.n, ins.imm >> 16, ins.imm & 0xFFFF, max(1, ins.imm2), ins.aview, ins.bview, ins.epi,
            ins.epi_res)


def _last_writer(ix, buf, before, sc):
    """The last instruction before ``before`` in the same scope that writes
    ``buf``, if it is a dynamic_update_slice; None otherwise."""
    ws = [w for w in ix.writers.get(buf, ()) if w < before and sc[w] == sc[before]]
    if not ws:
        return None
    w = max(ws)
    if ix.prog.instrs[w].op != V.OP_DYNAMIC_UPDATE_SLICE or ix.prog.instrs[w].dst != buf:
        return None
    return w


def _dus_fields(prog, ins):
    """(update dims, start buffers, update buffer) of a dynamic_update_slice
    (aux: rank, update dims, strides, clamps, zeros, start buffers, is64)."""
    a = ins.aux
    rank = prog.aux[a]
    if rank != 3 or prog.aux[a + 1 + 5 * rank]:
        return None
    dims = prog.aux[a + 1:a + 1 + rank]
    ids = prog.aux[a + 1 + 4 * rank:a + 1 + 5 * rank]
    return dims, ids, ins.a


def _mask_is_key_le_pos(prog, ix, pred, posb, C) -> bool:
    """The select predicate is key <= pos on every row, for every pos in
    [-2, C + 2] and 3 C (all keys for pos >= C - 1, none for pos < 0)."""
    pred = _peel_broadcast(prog, ix, pred)
    keys = np.arange(C)
    for v in list(range(-2, C + 3)) + [3 * C]:
        m = _eval_const(prog, ix, pred, env={posb: np.array([v], np.int64)})
        if m is None or m.size % C:
            return False
        if not np.array_equal(m.reshape(-1, C) != 0, np.broadcast_to(keys <= v, (m.size // C, C))):
            return False
    return True


def _new_buffer(prog, n, dt) -> int:
    """A fresh buffer of n elements at the arena's end (reuse_arena packs it)."""
    size = n * V.DT_SIZE[dt]
    off = -(-prog.arena_bytes // V.ARENA_ALIGN) * V.ARENA_ALIGN
    prog.buffers.append(V.Buffer(off, size, dt))
    prog.arena_bytes = off + max(-(-size // V.ARENA_ALIGN) * V.ARENA_ALIGN, V.ARENA_ALIGN)
    if hasattr(prog, "_overlap_groups"):
        try:
            del prog._overlap_groups
        except AttributeError:
            pass
    return len(prog.buffers) - 1


def _merged(dims, st, off=None):
    """A view with size-1 axes dropped and contiguous axes merged (the same
    index map, fewest axes), for comparing descriptors."""
    if off is None:
        dims, st, off = dims
    out = []
    for d, s_ in zip(dims, st):
        if d == 1:
            continue
        if out and out[-1][1] == s_ * d:
            out[-1] = (out[-1][0] * d, s_)
        else:
            out.append((d, s_))
    return tuple(out), off


def _canonical_view(prog, view1, n):
    """0 for an identity view (a contiguous read), else the view."""
    if view1 and _is_identity_view(prog, view1, n):
        return 0
    return view1


def _is_causal(mask: np.ndarray, C: int) -> bool:
    """mask (one [T, C] block, repeated over batch-heads by the broadcast that
    fed the select) is the causal rule key <= query + (C - T)."""
    if mask.size % C:
        return False
    m = mask.reshape(-1, C) != 0
    T = m.shape[0]
    want = np.arange(C)[None, :] <= np.arange(T)[:, None] + (C - T)
    return bool(np.array_equal(m, want))


def _peel_broadcast(prog, ix, buf):
    """The source of a chain of broadcasting gathers (each output element i reads
    source element i % |source|): an attention mask or fill value is computed
    once at [T, C] (or as a scalar) and broadcast over batch and heads."""
    for _ in range(8):
        g = ix.producer(buf, V.OP_GATHER_STRIDED)
        if g is None:
            return buf
        n_src = _elems(prog, g.a)
        if n_src == 0 or not _is_row_broadcast(prog, g.aux + 1, n_src):
            return buf
        buf = g.a
    return buf


def _eval_const(prog, ix, buf, depth=0, env=None):
    """Value of a buffer computed only from iotas, fills and constants (the
    predicate of an attention mask), evaluated on the host; None otherwise.
    ``env`` gives values for runtime buffers (a decode position)."""
    if depth > 12:
        return None
    if env and buf in env:
        return np.asarray(env[buf]).reshape(-1)
    for b, data in prog.consts:
        if b == buf:
            return np.frombuffer(bytes(data), V.DT_NUMPY[_dt(prog, b)]).copy()
    w = ix.unique_writer(buf)
    if w is None:
        return None
    ins = prog.instrs[w]
    n = _elems(prog, ins.dst)
    if ins.op == V.OP_IOTA_DIM:
        rank = prog.aux[ins.aux]
        dims = prog.aux[ins.aux + 1:ins.aux + 1 + rank]
        dim = prog.aux[ins.aux + 1 + rank]
        return np.indices(dims)[dim].reshape(-1).astype(np.int64)
    if ins.op == V.OP_FILL_F32:
        dt = _dt(prog, ins.dst)
        v = _f(ins.imm) if dt in (V.DT_F32, V.DT_F16, V.DT_BF16, V.DT_F64) else _i32(ins.imm)
        return np.full(n, v)
    if ins.op == V.OP_GATHER_STRIDED:
        src = _eval_const(prog, ix, ins.a, depth + 1, env)
        if src is None:
            return None
        dims, st, off = _view_desc(prog, ins.aux + 1)
        idx = np.full(int(np.prod(dims)), off, np.int64)
        rem = np.arange(idx.size, dtype=np.int64)
        for d in range(len(dims) - 1, -1, -1):
            idx += (rem % dims[d]) * st[d]
            rem //= dims[d]
        return src[idx]
    if n > (1 << 24):
        return None
    if ins.op in (V.OP_CMP_F32, V.OP_ADD_F32, V.OP_SUB_F32, V.OP_AND, V.OP_OR):
        if ins.op in (V.OP_ADD_F32, V.OP_SUB_F32) and (ins.imm or ins.imm2):
            return None
        a = _eval_const(prog, ix, ins.a, depth + 1, env)
        b = _eval_const(prog, ix, ins.b, depth + 1, env)
        if a is None or b is None:
            return None
        if ins.op == V.OP_CMP_F32:
            fn = (np.equal, np.not_equal, np.less, np.less_equal, np.greater, np.greater_equal)[ins.imm]
            return fn(a, b).astype(np.uint8)
        return {V.OP_ADD_F32: np.add, V.OP_SUB_F32: np.subtract, V.OP_AND: np.logical_and,
                V.OP_OR: np.logical_or}[ins.op](a, b)
    if ins.op in (V.OP_CONVERT, V.OP_COPY_F32):
        return _eval_const(prog, ix, ins.a, depth + 1, env)
    return None


# ---- finalize_matmul_views (lowering.py:2455-2466) --------------------------------------------

def finalize_matmul_views(prog: V.VMProgram) -> None:
    for ins in prog.instrs:
        if ins.op == V.OP_DOT and (ins.aview or ins.bview or ins.epi):
            ins.aux = len(prog.aux)
            prog.aux.extend([ins.aview, ins.bview, ins.epi, ins.epi_res])


# ---- alias_slices (extension) -------------------------------------------------------------------

def alias_slices(prog: V.VMProgram) -> None:
    """A gather that copies one contiguous, 16-byte aligned run of its source
    (a row slice such as q, k, v out of a decode step's fused projection)
    becomes a buffer of its own on the source's bytes, and the copy goes: its
    readers read the source in place.  The source must be written by exactly one
    instruction (or be a constant) and not be a program input or output (those
    are bound to caller memory, not the arena); the slice must be written only
    by the gather and not be an output.  The scheduler orders accesses to
    overlapping buffers as accesses to one (scheduler.overlap_groups), and
    reuse_arena moves them together.  The reference keeps such slices as
    strided views that each consumer re-reads (lowering.py:1481-1545)."""
    if _off("PJRT_OCL_ALIAS_SLICES"):
        return
    ports = set(prog.inputs) | set(prog.outputs)
    const_bufs = {b for b, _ in prog.consts}
    ix = _Index(prog)
    changed = False
    for gi, g in enumerate(prog.instrs):
        if g.op != V.OP_GATHER_STRIDED or g.dst in ports or g.a in ports or g.a == g.dst:
            continue
        if ix.writers.get(g.dst, []) != [gi]:
            continue
        if g.a not in const_bufs and len(ix.writers.get(g.a, ())) != 1:
            continue
        if g.a in const_bufs and ix.writers.get(g.a):
            continue
        dims, st, off = _view_desc(prog, g.aux + 1)
        n = int(np.prod(dims)) if dims else 1
        runs, _ = _merged(dims, st, off)
        if n != g.n or not (runs == () or runs == ((n, 1),)):
            continue
        src, dst = prog.buffers[g.a], prog.buffers[g.dst]
        esz = V.DT_SIZE[src.dtype]
        if dst.dtype != src.dtype or off < 0 or (off + n) * esz > src.size_bytes or (off * esz) % 16:
            continue
        dst.arena_byte_offset = src.arena_byte_offset + off * esz
        prog.instrs[gi] = V.Instr(V.OP_NOP)
        changed = True
    if changed and hasattr(prog, "_overlap_groups"):
        try:
            del prog._overlap_groups
        except AttributeError:
            pass


# ---- reuse_arena (lowering.py:2813-2973) ------------------------------------------------------

def reuse_arena(prog: V.VMProgram, cfg=None) -> None:
    """Pack buffer offsets by liveness measured in scheduler phases: two buffers
    share bytes only if a grid barrier separates the last use of one from the
    first write of the other.  Inputs, outputs and constants live the whole
    program; everything a loop or branch touches lives for the region's whole
    phase; buffers that alias (a slice kept as a buffer of its own) move with
    their parent.  The phases run instructions as soon as their dependencies
    allow, not in program order, so the lifetimes must also be disjoint in
    program order: the program stays correct when run one instruction after
    another (the tensor-level semantics the oracle executes)."""
    from . import scheduler as S
    if _off("PJRT_OCL_ARENA_REUSE"):
        return
    bufs = prog.buffers
    nb = len(bufs)
    if not nb:
        return
    cfg = cfg or S.DeviceConfig.from_env()
    sched = S._Scheduler(prog, cfg)
    levels = sched.levels(list(range(prog.main_len)))
    # a level the scheduler may join to the one before it (completion flags in
    # place of the barrier between them) shares that level's phase time
    joined = sched.joined_levels(levels)
    phase = {}
    region_roots = []
    ph = -1
    for k, (kind, payload) in enumerate(levels):
        if k not in joined:
            ph += 1
        if kind == "compute":
            for i in payload:
                phase[i] = ph
        else:
            phase[payload] = ph
            region_roots.append((payload, ph))
    order = {i: i for i in range(prog.main_len)}       # program-order position
    for r, ph in region_roots:
        stack = [r]
        while stack:
            ins = prog.instrs[stack.pop()]
            ranges = []
            if ins.op in (V.OP_WHILE, V.OP_IF):
                ranges = [(ins.a, ins.a + ins.b), (ins.n, ins.n + ins.imm)]
            elif ins.op == V.OP_FOR:
                ranges = [(ins.n, ins.n + ins.imm)]
            for lo_, hi_ in ranges:
                for j in range(lo_, hi_):
                    phase[j] = ph
                    order[j] = r
                    stack.append(j)
    # layernorms staged inside a GEMV run in the GEMV's phase
    for dot_i, ln_i in sched.ln_pro.items():
        if dot_i in phase:
            phase[ln_i] = phase[dot_i]
    n_ph = ph + 1
    lo = [n_ph + 1] * nb
    hi = [-1] * nb
    lo2 = [prog.main_len + 1] * nb
    hi2 = [-1] * nb

    def touch(b, t, t2):
        if 0 <= b < nb:
            lo[b] = min(lo[b], t)
            hi[b] = max(hi[b], t)
            lo2[b] = min(lo2[b], t2)
            hi2[b] = max(hi2[b], t2)
    for i, ins in enumerate(prog.instrs):
        if ins.op == V.OP_NOP or i not in phase:
            continue
        for b in reads_of(ins, prog) | writes_of(ins):
            touch(b, phase[i], order[i])
    end, end2 = n_ph, prog.main_len
    for b in set(prog.inputs):
        lo[b] = lo2[b] = 0
        hi[b] = max(hi[b], 0)
        hi2[b] = max(hi2[b], 0)
    for b in set(prog.outputs):
        lo[b] = min(lo[b], 0)
        lo2[b] = min(lo2[b], 0)
        hi[b], hi2[b] = end, end2
    for b, _ in prog.consts:
        lo[b], hi[b] = 0, end
        lo2[b], hi2[b] = 0, end2
    # alias groups (arena-overlapping buffers of the bump layout) move as one;
    # the scheduler keeps ordering by them, not by the packed overlaps
    group = list(S.overlap_groups(prog))
    prog.alias_groups = group
    members = {}
    for b in range(nb):
        members.setdefault(group[b], []).append(b)
    units = []
    for root, mem in members.items():
        base = min(bufs[m].arena_byte_offset for m in mem)
        top = max(bufs[m].arena_byte_offset + bufs[m].size_bytes for m in mem)
        l = min(lo[m] for m in mem)
        h = max(hi[m] for m in mem)
        units.append((root, mem, base, top - base, l, h, min(lo2[m] for m in mem), max(hi2[m] for m in mem)))

    def aligned(x):
        return -(-x // V.ARENA_ALIGN) * V.ARENA_ALIGN
    live_units = [u for u in units if u[5] >= 0]
    live_units.sort(key=lambda u: (-aligned(u[3]), -(u[5] - u[4]), u[0]))
    placed = []
    arena_end = 0
    new_off = {}
    for root, mem, base, size, l, h, l2, h2 in live_units:
        size_a = max(aligned(size), V.ARENA_ALIGN)
        conflicts = sorted((o, e) for (pl, ph_, pl2, ph2, o, e) in placed
                           if not (h < pl or ph_ < l) or not (h2 < pl2 or ph2 < l2))
        off = 0
        for c0, c1 in conflicts:
            if off + size_a <= c0:
                break
            off = max(off, c1)
        placed.append((l, h, l2, h2, off, off + size_a))
        arena_end = max(arena_end, off + size_a)
        for m in mem:
            new_off[m] = off + bufs[m].arena_byte_offset - base
    # buffers no instruction touches (intermediates a fusion replaced) keep no
    # arena bytes at all
    for root, mem, base, size, l, h, _, _ in units:
        if h < 0:
            for m in mem:
                new_off[m] = 0
                bufs[m].size_bytes = 0
    for b in range(nb):
        bufs[b].arena_byte_offset = new_off[b]
        arena_end = max(arena_end, new_off[b] + bufs[b].size_bytes)
    prog.arena_bytes = max(arena_end, V.ARENA_ALIGN)
    if hasattr(prog, "_overlap_groups"):
        try:
            del prog._overlap_groups
        except AttributeError:
            pass


# ---- driver ------------------------------------------------------------------------------------

def run_all(prog: V.VMProgram) -> None:
    """The pass pipeline (lowering.py:3027-3106, with the order noted above)."""
    compose_affines(prog)
    fuse_matmul_views(prog)
    fuse_views(prog)
    dce(prog)
    fuse_norm(prog)
    fuse_gelu(prog)
    dce(prog)
    fuse_norm_epilogue(prog)
    dce(prog)
    fuse_mma_epilogue(prog)
    dce(prog)
    fuse_decode_attention(prog)
    dce(prog)
    fuse_attention(prog)
    dce(prog)
    fuse_region(prog)
    dce(prog)
    finalize_matmul_views(prog)
    alias_slices(prog)
