"""StableHLO -> VMProgram lowering (the front end of the compile path).

Mirrors the reference's lowering (python/pjrt_ocl/lowering.py:2976-3119 and the
op handlers of python/pjrt_ocl/ops/*.py): walk the public ``@main`` of a
StableHLO module, emit tensor instructions per op through the graph builder
(``graph.Graph``), lower ``while``/``if`` regions after the root list, then run
the fusion passes (``passes.py``) and the liveness-based arena packing, and
schedule the result for the device.

Semantics kept from the reference, each noted where it is implemented:
  * a multiply / add / subtract by a broadcast f32 scalar constant becomes one
    OP_AFFINE (``_affine_st``, lowering.py:503-548);
  * broadcast / transpose / slice / reverse are strided gathers that the view
    passes fold into their consumers (ops/shape.py:57-190);
  * ``dot_general`` is canonicalised to C[G,M,N] = A[G,M,K] B[G,K,N] with the
    operand permutations as gathers (ops/dot.py:94-161);
  * counted ``while`` loops (lax.fori_loop / scan) are detected and unrolled or
    become OP_FOR; other loops are OP_WHILE with a cond sub-list
    (lowering.py:718-996, 1017-1186);
  * a while body result produced by one elementwise op, or a
    dynamic_update_slice of its own carry, is written into the carry in place
    (lowering.py:1067-1140).

Extensions of this build: bf16/f16 results of dot_general are honoured (the
reference always produces f32, ops/dot.py:158); the variadic (value, index)
reduce that ``jnp.argmax`` emits lowers to OP_ARGMAX_SEG (the reference rejects
it, ops/reduce.py:165-168).
"""
from __future__ import annotations

import math
import os

import numpy as np

from . import graph as G
from . import mlir as M
from . import vmprogram as V


class LoweringError(NotImplementedError):
    """A valid program beyond this lowering's op / type coverage (the lowering
    service exits 2 for it, lower_service.py:11-18)."""


DT_OF_ELEM = {"f32": V.DT_F32, "f64": V.DT_F64, "f16": V.DT_F16, "bf16": V.DT_BF16, "i1": V.DT_BOOL,
              "i32": V.DT_I32, "si32": V.DT_I32, "ui32": V.DT_U32, "i64": V.DT_I64, "si64": V.DT_I64}
FLOAT_DTS = (V.DT_F32, V.DT_F64, V.DT_F16, V.DT_BF16)

BINARY = {"add": V.OP_ADD_F32, "subtract": V.OP_SUB_F32, "multiply": V.OP_MUL_F32, "divide": V.OP_DIV_F32,
          "maximum": V.OP_MAX_F32, "minimum": V.OP_MIN_F32, "power": V.OP_POW_F32, "atan2": V.OP_ATAN2_F32,
          "remainder": V.OP_REMAINDER_F32, "and": V.OP_AND, "or": V.OP_OR, "xor": V.OP_XOR,
          "shift_left": V.OP_SHL, "shift_right_logical": V.OP_SHR_L, "shift_right_arithmetic": V.OP_SHR_A}
UNARY = {"negate": "neg", "exponential": "exp", "log": "log", "sqrt": "sqrt", "rsqrt": "rsqrt", "tanh": "tanh",
         "abs": "abs", "floor": "floor", "ceil": "ceil", "sign": "sign", "log_plus_one": "log1p",
         "exponential_minus_one": "expm1", "cbrt": "cbrt", "sine": "sin", "cosine": "cos", "tan": "tan",
         "round_nearest_even": "rint", "round_nearest_afz": "round", "not": "not"}
CMP = {"EQ": "EQ", "NE": "NE", "LT": "LT", "LE": "LE", "GT": "GT", "GE": "GE"}
# reduce body op -> reduce kind (V.RED_*) and the kind's identity
RED_KIND = {"stablehlo.add": V.RED_SUM, "stablehlo.maximum": V.RED_MAX, "stablehlo.minimum": V.RED_MIN,
            "stablehlo.multiply": V.RED_PROD, "stablehlo.and": V.RED_AND, "stablehlo.or": V.RED_OR,
            "stablehlo.xor": V.RED_XOR}
IDENTITY_OPS = {"stablehlo.optimization_barrier", "sdy.sharding_constraint", "stablehlo.custom_call@Sharding",
                "mhlo.sharding"}


def _env_int(name: str, default: int) -> int:
    try:
        return int(os.environ.get(name, str(default)))
    except ValueError:
        return default


def _dtype(ty) -> int:
    if not isinstance(ty, M.TensorType):
        raise LoweringError(f"unsupported type {ty} (ranked static tensors only)")
    dt = DT_OF_ELEM.get(ty.elem)
    if dt is None:
        raise LoweringError(f"unsupported element type {ty.elem}")
    return dt


def _rm_strides(shape):
    st, acc = [0] * len(shape), 1
    for d in range(len(shape) - 1, -1, -1):
        st[d] = acc
        acc *= shape[d]
    return st


class Lowerer:
    """Per-module lowering state (the reference's ``_Ctx``, lowering.py:352-407)."""

    def __init__(self, module: M.Module):
        self.mod = module
        self.g = G.Graph()
        self.env: dict = {}          # Value -> graph Tensor
        self.cval: dict = {}         # Value -> numpy value of a constant
        self.sbcast: dict = {}       # Value -> float: broadcast of an f32 scalar constant
        self.depth = 0
        self.inplace: set = set()    # dynamic_update_slice ops that write their loop carry

    # ---- values ---------------------------------------------------------------------------
    def t(self, v: M.Value) -> G.Tensor:
        try:
            return self.env[v]
        except KeyError:
            raise LoweringError(f"no buffer for value %{v.name}") from None

    def bind(self, v: M.Value, t: G.Tensor) -> None:
        want = tuple(v.type.shape) if isinstance(v.type, M.TensorType) else None
        if want is not None and tuple(t.shape) != want:
            if G._prod(want) != t.n:
                raise LoweringError(f"internal: %{v.name} expects {want}, got {t.shape}")
            t = self.g.reshape(t, want)
        self.env[v] = t

    # ---- driver -----------------------------------------------------------------------------
    def lower(self) -> V.VMProgram:
        main = self.mod.main
        for a in main.args:
            self.env[a] = self.g.input(a.type.shape, _dtype(a.type))
        results = self.block(main.body.ops)
        used = {t.buf for t in self.g.inputs} | {b for b, _ in self.g.consts}
        for v in results:
            t = self.g.materialize(self.t(v))
            if t.buf in used:
                # an output must be a buffer of its own that some instruction
                # writes (ports bind outputs; constants never are program I/O)
                t = self._copy(t)
            used.add(t.buf)
            self.g.output(t)
        return self.g.build()

    def block(self, ops, stop=("func.return",)):
        """Lower a straight-line op list; returns the terminator's operand values."""
        for op in ops:
            if op.name in stop or op.name == "stablehlo.return":
                return list(op.operands)
            self.op(op)
        return []

    def op(self, op: M.Op) -> None:
        name = op.name
        short = name.split(".", 1)[1] if name.startswith("stablehlo.") else None
        if short in BINARY:
            return self.binary(op, short)
        if short in UNARY:
            return self.unary(op, UNARY[short])
        fn = getattr(self, "op_" + (short or name.replace(".", "_")), None)
        if fn is None:
            if name in IDENTITY_OPS or name.startswith("sdy."):
                for r, o in zip(op.results, op.operands):
                    self.bind(r, self.t(o))
                return
            raise LoweringError(f"unsupported op {name}")
        fn(op)

    def _copy(self, t: G.Tensor) -> G.Tensor:
        dst = self.g._new(t.shape, t.dtype)
        self.g.copy_into(dst, t)
        return dst

    # ---- elementwise (ops/elementwise.py:98-168, 349-431) -------------------------------------
    def binary(self, op, short):
        a, b = (self.t(x) for x in op.operands)
        dt = _dtype(op.results[0].type)
        opcode = BINARY[short]
        if dt == V.DT_F32 and short in ("add", "subtract", "multiply"):
            ls, rs = self.sbcast.get(op.operands[0]), self.sbcast.get(op.operands[1])
            if (rs is None) != (ls is None):
                # x (op) scalar constant -> one affine pass (lowering.py:503-548)
                other, c, other_is_lhs = (a, rs, True) if rs is not None else (b, ls, False)
                if short == "multiply":
                    s, t = c, 0.0
                elif short == "add":
                    s, t = 1.0, c
                else:
                    s, t = (1.0, -c) if other_is_lhs else (-1.0, c)
                self.bind(op.results[0], self.g.affine(other, s, t))
                return
        if a.shape != b.shape:
            raise LoweringError(f"{op.name}: operand shapes differ ({a.shape} vs {b.shape})")
        self.bind(op.results[0], self.g._binop(opcode, a, b))

    def unary(self, op, name):
        x = self.t(op.operands[0])
        if name == "not" and x.dtype in FLOAT_DTS:
            raise LoweringError("not of a float tensor")
        self.bind(op.results[0], self.g.unary(name, x))

    def op_logistic(self, op):
        """logistic(x) = 1 / (1 + exp(-x)) (ops/elementwise.py)."""
        x = self.t(op.operands[0])
        e = self.g.unary("exp", self.g.unary("neg", x))
        d = self.g.affine(e, 1.0, 1.0)
        one = self.g.broadcast(self.g.scalar(1.0), x.shape, ())
        self.bind(op.results[0], self.g.div(one, d))

    def op_is_finite(self, op):
        self.bind(op.results[0], self.g.is_finite(self.t(op.operands[0])))

    def op_clamp(self, op):
        lo, x, hi = (self.t(v) for v in op.operands)
        lo = lo if lo.shape == x.shape else self.g.broadcast(lo, x.shape, ())
        hi = hi if hi.shape == x.shape else self.g.broadcast(hi, x.shape, ())
        self.bind(op.results[0], self.g.minimum(self.g.maximum(x, lo), hi))

    def op_compare(self, op):
        a, b = (self.t(x) for x in op.operands)
        direction = M.attr_enum(op.attr("comparison_direction"))
        ctype = op.attr("compare_type")
        if ctype is not None and M.attr_enum(ctype) == "UNSIGNED" and a.dtype == V.DT_I32:
            a, b = self.g.bitcast(a, "u32"), self.g.bitcast(b, "u32")
        if ctype is not None and M.attr_enum(ctype) == "TOTALORDER":
            raise LoweringError("compare with TOTALORDER")
        self.bind(op.results[0], self.g.compare(a, b, CMP[direction]))

    def op_select(self, op):
        p, a, b = (self.t(x) for x in op.operands)
        if p.shape != a.shape:
            p = self.g.broadcast(p, a.shape, ())
        self.bind(op.results[0], self.g.select(p, a, b))

    def op_convert(self, op):
        x = self.t(op.operands[0])
        dt = _dtype(op.results[0].type)
        if dt == x.dtype:
            self.bind(op.results[0], x)
            return
        self.bind(op.results[0], self.g.convert(x, dt))

    def op_bitcast_convert(self, op):
        x = self.t(op.operands[0])
        dt = _dtype(op.results[0].type)
        if V.DT_SIZE[dt] != V.DT_SIZE[x.dtype]:
            raise LoweringError("bitcast_convert between widths")
        self.bind(op.results[0], self.g.bitcast(x, dt) if dt != x.dtype else x)

    # ---- constants and creation (ops/making.py:70-155; lowering.py:551-585) ------------------
    def op_constant(self, op):
        a = op.attr("value")
        ty = op.results[0].type
        dt = _dtype(ty)
        if not isinstance(a, M.DenseAttr):
            raise LoweringError("constant without a dense value")
        arr = a.array().reshape(ty.shape)
        self.cval[op.results[0]] = arr
        self.bind(op.results[0], self.g.const(arr, dt))

    def op_iota(self, op):
        ty = op.results[0].type
        dim = M.attr_int(op.attr("iota_dimension"))
        dt = _dtype(ty)
        if dt in (V.DT_I32, V.DT_U32, V.DT_I64):
            self.bind(op.results[0], self.g.iota(ty.shape, dim, dt))
            return
        i = self.g.iota(ty.shape, dim, "i32")
        self.bind(op.results[0], self.g.convert(i, dt))

    # ---- shape (ops/shape.py:57-190) ----------------------------------------------------------
    def op_broadcast_in_dim(self, op):
        src = op.operands[0]
        x = self.t(src)
        shape = op.results[0].type.shape
        dims = M.attr_ints(op.attr("broadcast_dimensions"))
        c = self.cval.get(src)
        if c is not None and c.size == 1 and x.dtype == V.DT_F32:
            self.sbcast[op.results[0]] = float(c.reshape(-1)[0])
        if c is not None and c.size == 1:
            # a read-only view with zero strides: a splat of any size costs nothing
            self.cval[op.results[0]] = np.broadcast_to(c.reshape(()), shape)
        if G._prod(shape) == x.n and list(dims) == sorted(dims):
            # adds or drops only size-1 axes: a reshape, no data movement
            self.bind(op.results[0], self.g.reshape(x, shape))
            return
        self.bind(op.results[0], self.g.broadcast(x, shape, dims))

    def op_reshape(self, op):
        x = self.t(op.operands[0])
        shape = op.results[0].type.shape
        c = self.cval.get(op.operands[0])
        if c is not None:
            splat = c.ndim and not any(c.strides)
            self.cval[op.results[0]] = np.broadcast_to(c[(0,) * c.ndim], shape) if splat else c.reshape(shape)
            if c.size == 1 and x.dtype == V.DT_F32 and op.operands[0] in self.sbcast:
                self.sbcast[op.results[0]] = self.sbcast[op.operands[0]]
        self.bind(op.results[0], self.g.reshape(x, shape))

    def op_transpose(self, op):
        x = self.t(op.operands[0])
        perm = M.attr_ints(op.attr("permutation"))
        if perm == list(range(len(perm))):
            self.bind(op.results[0], x)
            return
        self.bind(op.results[0], self.g.transpose(x, perm))

    def op_slice(self, op):
        x = self.t(op.operands[0])
        starts = M.attr_ints(op.attr("start_indices"))
        limits = M.attr_ints(op.attr("limit_indices"))
        strides = M.attr_ints(op.attr("strides")) if op.attr("strides") is not None else None
        self.bind(op.results[0], self.g.slice(x, starts, limits, strides))

    def op_reverse(self, op):
        x = self.g.materialize(self.t(op.operands[0]))
        dims = set(M.attr_ints(op.attr("dimensions")))
        st = _rm_strides(x.shape)
        strides = [-st[d] if d in dims else st[d] for d in range(len(st))]
        off = sum((x.shape[d] - 1) * st[d] for d in dims)
        self.bind(op.results[0], self.g.gather(x, x.shape, strides, off))

    def op_concatenate(self, op):
        parts = [self.t(v) for v in op.operands]
        axis = M.attr_int(op.attr("dimension"))
        self.bind(op.results[0], self.g.concatenate(parts, axis))

    def op_pad(self, op):
        x = self.g.materialize(self.t(op.operands[0]))
        pv = self.cval.get(op.operands[1])
        lo = M.attr_ints(op.attr("edge_padding_low"))
        hi = M.attr_ints(op.attr("edge_padding_high"))
        interior = M.attr_ints(op.attr("interior_padding"))
        if pv is None or any(interior) or min(lo + hi) < 0:
            raise LoweringError("pad with a runtime pad value, interior or negative padding")
        shape = op.results[0].type.shape
        out = self.g.fill(shape, float(pv.reshape(-1)[0]) if x.dtype in FLOAT_DTS else int(pv.reshape(-1)[0]),
                          x.dtype)
        ost = _rm_strides(shape)
        self.g.scatter_into(out, x, ost, sum(lo[d] * ost[d] for d in range(len(shape))))
        self.bind(op.results[0], out)

    # ---- dynamic slices and gathers (ops/dynslice.py:85-127; gather_index.py:130-146) --------
    def op_dynamic_slice(self, op):
        x = self.t(op.operands[0])
        starts = [self.g.materialize(self.t(v)) for v in op.operands[1:]]
        sizes = M.attr_ints(op.attr("slice_sizes"))
        self.bind(op.results[0], self.g.dynamic_slice(x, starts, sizes))

    def op_dynamic_update_slice(self, op):
        x = self.g.materialize(self.t(op.operands[0]))
        upd = self.t(op.operands[1])
        starts = [self.g.materialize(self.t(v)) for v in op.operands[2:]]
        if op in self.inplace:
            # the update of a loop carry whose old value nothing else reads
            # (Lowerer.inplace_updates): written into the carry itself
            self.g.dynamic_update_slice(x, upd, starts)
            self.bind(op.results[0], x)
            return
        # out-of-place: an identity gather copies the operand, then the update is
        # scattered into the copy (in place when a loop carry allows it)
        out = self.g.gather(x, x.shape, _rm_strides(x.shape), 0)
        self.g.dynamic_update_slice(out, upd, starts)
        self.bind(op.results[0], out)

    def op_gather(self, op):
        """The embedding-lookup form: rows of a rank-2 table by an index tensor."""
        table, idx = (self.t(v) for v in op.operands)
        dn = op.attr("dimension_numbers")
        f = dn.fields if isinstance(dn, M.StructAttr) else {}
        sizes = M.attr_ints(op.attr("slice_sizes"))
        ivd = f.get("index_vector_dim", len(idx.shape))
        if (len(table.shape) == 2 and f.get("collapsed_slice_dims") == [0] and f.get("start_index_map") == [0]
                and sizes == [1, table.shape[1]] and f.get("offset_dims") == [len(op.results[0].type.shape) - 1]):
            if ivd < len(idx.shape):
                if idx.shape[ivd] != 1:
                    raise LoweringError("gather with a multi-component index vector")
                idx = self.g.reshape(idx, idx.shape[:ivd] + idx.shape[ivd + 1:])
            self.bind(op.results[0], self.g.take_rows(table, idx))
            return
        raise LoweringError("gather other than a row lookup of a rank-2 table")

    # ---- contractions (ops/dot.py:94-161) ------------------------------------------------------
    def op_dot_general(self, op):
        a, b = (self.t(v) for v in op.operands)
        dn = op.attr("dot_dimension_numbers")
        f = dn.fields if isinstance(dn, M.StructAttr) else {}
        lb, rb = f.get("lhs_batching_dimensions", []), f.get("rhs_batching_dimensions", [])
        lc, rc = f.get("lhs_contracting_dimensions", []), f.get("rhs_contracting_dimensions", [])
        self.bind(op.results[0], self.dot(a, b, lb, rb, lc, rc, _dtype(op.results[0].type)))

    def op_dot(self, op):
        a, b = (self.t(v) for v in op.operands)
        rc = [0] if len(b.shape) >= 1 else []
        self.bind(op.results[0], self.dot(a, b, [], [], [len(a.shape) - 1], rc, _dtype(op.results[0].type)))

    def dot(self, a, b, lb, rb, lc, rc, out_dt):
        la, ra = len(a.shape), len(b.shape)
        lf = [d for d in range(la) if d not in lb and d not in lc]
        rf = [d for d in range(ra) if d not in rb and d not in rc]
        Gn = G._prod([a.shape[d] for d in lb])
        Mn = G._prod([a.shape[d] for d in lf])
        Kn = G._prod([a.shape[d] for d in lc])
        Nn = G._prod([b.shape[d] for d in rf])
        if Kn != G._prod([b.shape[d] for d in rc]) or Gn != G._prod([b.shape[d] for d in rb]):
            raise LoweringError("dot_general: dimension sizes disagree")
        if out_dt not in (V.DT_F32, V.DT_BF16, V.DT_F16):
            raise LoweringError("dot_general result must be f32, bf16 or f16")
        if a.dtype != b.dtype or a.dtype not in (V.DT_F32, V.DT_BF16, V.DT_F16):
            raise LoweringError("dot_general operands must share a float dtype (f32, bf16, f16)")
        if Nn > 0xFFFF or Kn > 0xFFFF:
            raise LoweringError("dot_general N / K beyond the 16-bit DOT encoding")
        pa, pb = lb + lf + lc, rb + rc + rf
        if pa != list(range(la)):
            a = self.g.transpose(a, pa)
        if pb != list(range(ra)):
            b = self.g.transpose(b, pb)
        if Gn == 1:
            a2 = self.g.reshape(a, (Mn, Kn))
            b2 = self.g.reshape(b, (Kn, Nn))
        else:
            a2 = self.g.reshape(a, (Gn, Mn, Kn))
            b2 = self.g.reshape(b, (Gn, Kn, Nn))
        return self.g.dot(a2, b2, out_dtype=out_dt)

    # ---- reductions (ops/reduce.py:162-247) --------------------------------------------------
    def op_reduce(self, op):
        n_in = len(op.operands) // 2
        dims = sorted(M.attr_ints(op.attr("dimensions")))
        if n_in == 2:
            return self.argmax_reduce(op, dims)
        if n_in != 1:
            raise LoweringError(f"reduce over {n_in} inputs")
        x = self.g.materialize(self.t(op.operands[0]))
        init = self.cval.get(op.operands[1])
        body = op.regions[0][0]
        kinds = [o for o in body.ops if o.name != "stablehlo.return"]
        if len(kinds) != 1 or kinds[0].name not in RED_KIND:
            raise LoweringError("reduce body other than one add/max/min/mul/and/or/xor")
        kind = RED_KIND[kinds[0].name]
        out = self.reduce(x, dims, kind)
        # a non-identity init joins the result once (op(reduce, init))
        if init is None or not _is_identity(kind, float(init.reshape(-1)[0]) if init.size else 0.0):
            iv = self.g.broadcast(self.t(op.operands[1]), out.shape, ()) if out.shape else self.t(op.operands[1])
            comb = {V.RED_SUM: "add", V.RED_MAX: "maximum", V.RED_MIN: "minimum", V.RED_PROD: "mul",
                    V.RED_AND: "bit_and", V.RED_OR: "bit_or", V.RED_XOR: "bit_xor"}[kind]
            out = getattr(self.g, comb)(out, iv)
        self.bind(op.results[0], out)

    def reduce(self, x, dims, kind):
        rank = len(x.shape)
        if not dims:
            return x
        if len(dims) == rank:
            return self.g.reduce_all(x, kind)
        keep = [d for d in range(rank) if d not in dims]
        if dims == list(range(rank - len(dims), rank)):          # a suffix
            outer = tuple(x.shape[d] for d in keep)
            r = self.g.reduce_last(self.g.reshape(x, outer + (G._prod([x.shape[d] for d in dims]),)), kind)
            return self.g.reshape(r, outer)
        if len(dims) == 1:
            return self.g.reduce_axis(x, dims[0], kind)
        # general: move the reduced axes last
        xt = self.g.transpose(x, keep + dims)
        outer = tuple(x.shape[d] for d in keep)
        r = self.g.reduce_last(self.g.reshape(xt, outer + (G._prod([x.shape[d] for d in dims]),)), kind)
        return self.g.reshape(r, outer)

    def argmax_reduce(self, op, dims):
        """The variadic (value, index) reduce of jnp.argmax / argmin over the last
        axis, its index operand an iota along that axis (extension: the reference
        rejects it, ops/reduce.py:165-168)."""
        x = self.g.materialize(self.t(op.operands[0]))
        rank = len(x.shape)
        idx_op = op.operands[1]
        if dims != [rank - 1]:
            raise LoweringError("argmax/argmin over an axis other than the last")
        body = op.regions[0][0]
        cmps = [M.attr_enum(o.attr("comparison_direction")) for o in body.ops if o.name == "stablehlo.compare"]
        pa, pi, qa, qi = body.args[0], body.args[1], body.args[2], body.args[3]
        value_cmp = [o for o in body.ops if o.name == "stablehlo.compare" and set(o.operands) == {pa, qa}
                     and M.attr_enum(o.attr("comparison_direction")) in ("GT", "LT")]
        if not value_cmp or not cmps:
            raise LoweringError("variadic reduce other than argmax / argmin")
        vc = value_cmp[0]
        d = M.attr_enum(vc.attr("comparison_direction"))
        is_max = (d == "GT") == (vc.operands[0] is pa)
        if x.dtype not in FLOAT_DTS:
            raise LoweringError("argmax over integers")
        idx_dt = _dtype(idx_op.type)
        src = x if is_max else self.g.unary("neg", x)
        val, idx = self.g.argmax_last(src, V.DT_NAMES[idx_dt])
        if not is_max:
            val = self.g.unary("neg", val)
        self.bind(op.results[0], val)
        self.bind(op.results[1], idx)

    # ---- calls and control flow (lowering.py:629-660, 936-1330) --------------------------------
    def op_func_call(self, op):
        callee = op.attr("callee")
        name = callee.name if isinstance(callee, M.SymbolRef) else str(callee)
        f = self.mod.funcs.get(name)
        if f is None:
            raise LoweringError(f"call to unknown function @{name}")
        if self.depth > 32:
            raise LoweringError("call nesting too deep")
        for arg, val in zip(f.body.args, op.operands):
            self.env[arg] = self.t(val)
            if val in self.cval:
                self.cval[arg] = self.cval[val]
            if val in self.sbcast:
                self.sbcast[arg] = self.sbcast[val]
        self.depth += 1
        rets = self.block(f.body.ops)
        self.depth -= 1
        for r, v in zip(op.results, rets):
            self.bind(r, self.t(v))
            if v in self.cval:
                self.cval[r] = self.cval[v]
            if v in self.sbcast:
                self.sbcast[r] = self.sbcast[v]

    def op_while(self, op):
        cond, body = op.regions[0][0], op.regions[1][0]
        fixed = detect_fixed_trip(op, self.cval)
        mode = os.environ.get("PJRT_OCL_WHILE", "auto").strip().lower()
        if fixed is not None and mode != "while":
            trip, k, init, step = fixed
            n_ops = _count_ops(body.ops, self.mod)
            small = trip <= _env_int("PJRT_OCL_UNROLL_TRIPS", 64) or trip * n_ops <= _env_int("PJRT_OCL_UNROLL_OPS",
                                                                                               2048)
            body_bytes = _result_bytes(body.ops)
            if mode == "unroll" or (mode == "auto" and small and trip * body_bytes
                                    <= (_env_int("PJRT_OCL_UNROLL_ARENA_MB", 256) << 20)):
                return self.unroll(op, trip, k, init, step)
        else:
            fixed = None
        g = self.g
        carries = []
        for v in op.operands:
            src = g.materialize(self.t(v))
            c = g._new(src.shape, src.dtype)
            g.copy_into(c, src)                  # init copy: the carries are mutable
            carries.append(c)
        cond_list, cond_buf = [], None
        if fixed is None:
            g.begin()
            for a, c in zip(cond.args, carries):
                self.env[a] = c
            (res,) = self.block(cond.ops)
            cond_buf = g.materialize(self.t(res))
            cond_list = g.end()
        g.begin()
        for a, c in zip(body.args, carries):
            self.env[a] = c
        self.inplace |= inplace_updates(body)
        rets = [g.materialize(self.t(v)) for v in self.block(body.ops)]
        self.commit_carries(carries, rets)
        body_list = g.end()
        if fixed is None:
            g.while_loop(cond_buf, cond_list, body_list)
        else:
            g.for_loop(fixed[0], body_list)
        for r, c in zip(op.results, carries):
            self.bind(r, c)

    def commit_carries(self, carries, rets):
        """Write a body's results into its carries (lowering.py:1055-1180): in
        place when the result's only producer is an elementwise op or a
        dynamic_update_slice of that very carry, no other body instruction reads
        the carry after that producer and no other result is the carry itself;
        otherwise by a copy, through a temporary when another result reads the
        carry (a swap or a passthrough must not see it overwritten)."""
        g = self.g
        body = g._stack[-1]
        writers, readers = {}, {}
        for i, ins in enumerate(body):
            writers.setdefault(ins.dst, []).append(i)
            for b in _reads(ins, g):
                if b == ins.dst and ins.op in (V.OP_DYNAMIC_UPDATE_SLICE, V.OP_SCATTER):
                    continue        # a partial write keeps the rest of its own dst
                readers.setdefault(b, []).append(i)
        nested = any(ins.op in V.REGION_OPS for ins in body)
        carry_bufs = {c.buf for c in carries}
        ret_bufs = [x.buf for x in rets]
        done = [False] * len(carries)
        for k, (c, r) in enumerate(zip(carries, rets)):
            if nested or r.buf == c.buf:
                done[k] = r.buf == c.buf
                continue
            w = writers.get(r.buf, [])
            if r.buf in carry_bufs or readers.get(r.buf) or ret_bufs.count(r.buf) != 1 or c.buf in ret_bufs:
                continue
            if len(w) == 1 and body[w[0]].op in INPLACE_SAFE:
                # an elementwise producer may read the carry itself (same index)
                if r.n == c.n and all(i < w[0] for i in readers.get(c.buf, []) if i != w[0]) \
                        and c.buf not in writers:
                    body[w[0]].dst = c.buf
                    done[k] = True
            elif len(w) == 2:
                cp, dus = body[w[0]], body[w[1]]
                if (cp.op == V.OP_GATHER_STRIDED and dus.op == V.OP_DYNAMIC_UPDATE_SLICE and cp.a == c.buf
                        and _identity_gather(g.aux, cp.aux, c.n) and readers.get(c.buf) == [w[0]]
                        and c.buf not in writers):
                    cp.op = V.OP_NOP
                    cp.dst = cp.a = 0
                    dus.dst = c.buf
                    done[k] = True
        # copies: first into the carries that no pending result reads, then into
        # the others; a result that is itself such a carry goes through a
        # temporary taken before any copy (a swap)
        pending = {r.buf for k, r in enumerate(rets) if not done[k]}
        late = {k for k, c in enumerate(carries) if not done[k] and c.buf in pending}
        late_bufs = {carries[k].buf for k in late}
        temps = {k: self._copy(rets[k]) for k in late if rets[k].buf in late_bufs}
        for k, (c, r) in enumerate(zip(carries, rets)):
            if not done[k] and k not in late:
                g.copy_into(c, r)
        for k in sorted(late):
            g.copy_into(carries[k], temps.get(k, rets[k]))

    def unroll(self, op, trip, k, init, step):
        """Inline a counted loop's body ``trip`` times (lowering.py:893-934): the
        counter becomes a constant per iteration."""
        body = op.regions[1][0]
        cur = [self.t(v) for v in op.operands]
        cdt = cur[k].dtype
        for it in range(trip):
            for j, a in enumerate(body.args):
                self.env[a] = cur[j]
            cv = np.array(init + it * step, V.DT_NUMPY[cdt])
            self.env[body.args[k]] = self.g.const(cv, cdt)
            self.cval[body.args[k]] = cv
            rets = self.block(body.ops)
            cur = [self.t(v) for v in rets]
        for r, t in zip(op.results, cur):
            self.bind(r, t)

    def op_if(self, op):
        g = self.g
        pred = g.materialize(self.t(op.operands[0]))
        outs = [g._new(r.type.shape, _dtype(r.type)) for r in op.results]
        lists = []
        for region in op.regions:
            g.begin()
            rets = [g.materialize(self.t(v)) for v in self.block(region[0].ops)]
            for o, r in zip(outs, rets):
                g.copy_into(o, r)
            lists.append(g.end())
        g.if_(pred, lists[0], lists[1])
        for r, o in zip(op.results, outs):
            self.bind(r, o)

    def op_case(self, op):
        """case(index) as a chain of ifs on index == k (the last branch is the
        default, as for an out-of-range index)."""
        g = self.g
        index = g.materialize(self.t(op.operands[0]))
        outs = [g._new(r.type.shape, _dtype(r.type)) for r in op.results]
        n = len(op.regions)

        def branch(k):
            g.begin()
            rets = [g.materialize(self.t(v)) for v in self.block(op.regions[k][0].ops)]
            for o, r in zip(outs, rets):
                g.copy_into(o, r)
            return g.end()

        def chain(k):
            if k == n - 1:
                return branch(k)
            g.begin()
            flag = g.compare(index, g.scalar(k, V.DT_NAMES[index.dtype]), "EQ")
            g.if_(flag, branch(k), chain(k + 1))
            return g.end()

        for ins in chain(0):
            g.emit(ins)
        for r, o in zip(op.results, outs):
            self.bind(r, o)


def inplace_updates(body: M.Block) -> set:
    """The dynamic_update_slice ops of a loop body that can write their loop
    carry in place (lowering.py:1055-1180 commits DUS carries in place the same
    way): the op updates block argument k, its result is what the body returns
    at position k, and nothing else in the body (nested regions included) uses
    argument k, so the carry's old value is dead once the update has run.  Other
    readers of the result then read the carry."""
    uses: dict = {}

    def walk(ops):
        for o in ops:
            for v in o.operands:
                uses[v] = uses.get(v, 0) + 1
            for region in o.regions:
                for blk in region:
                    walk(blk.ops)
    walk(body.ops)
    if not body.ops or body.ops[-1].name != "stablehlo.return":
        return set()
    producer = {r: o for o in body.ops for r in o.results}
    rets = body.ops[-1].operands
    out = set()
    for k, (arg, v) in enumerate(zip(body.args, rets)):
        o = producer.get(v)
        if o is None or o.name != "stablehlo.dynamic_update_slice" or o.operands[0] is not arg:
            continue
        if uses.get(arg, 0) == 1 and sum(r is v for r in rets) == 1:
            out.add(o)
    return out


INPLACE_SAFE = frozenset({
    V.OP_ADD_F32, V.OP_MUL_F32, V.OP_SUB_F32, V.OP_DIV_F32, V.OP_MAX_F32, V.OP_MIN_F32, V.OP_POW_F32,
    V.OP_ATAN2_F32, V.OP_REMAINDER_F32, V.OP_NEG_F32, V.OP_EXP_F32, V.OP_LOG_F32, V.OP_SQRT_F32,
    V.OP_RSQRT_F32, V.OP_TANH_F32, V.OP_ABS_F32, V.OP_FLOOR_F32, V.OP_CEIL_F32, V.OP_SIGN_F32,
    V.OP_LOG1P_F32, V.OP_EXPM1_F32, V.OP_CBRT_F32, V.OP_SIN_F32, V.OP_COS_F32, V.OP_TAN_F32,
    V.OP_ROUND_NEAREST_EVEN_F32, V.OP_ROUND_NEAREST_AFZ_F32, V.OP_COPY_F32, V.OP_CONVERT, V.OP_BITCAST,
    V.OP_CMP_F32, V.OP_SELECT_F32, V.OP_AND, V.OP_OR, V.OP_XOR, V.OP_NOT, V.OP_IS_FINITE, V.OP_AFFINE_F32,
    V.OP_SHL, V.OP_SHR_L, V.OP_SHR_A, V.OP_GELU})


def _reads(ins: V.Instr, g: G.Graph) -> set:
    from .scheduler import _instr_reads

    class _P:
        pass
    p = _P()
    p.aux = g.aux
    p.buffers = None
    try:
        return _instr_reads(ins, p)
    except (AttributeError, TypeError, IndexError):
        return {ins.a, ins.b} | set(ins.reads_hint)


def _identity_gather(aux, off: int, n: int) -> bool:
    rank = aux[off]
    dims = [aux[off + 1 + i] for i in range(rank)]
    st = [aux[off + 1 + rank + i] for i in range(rank)]
    src_off = aux[off + 1 + 2 * rank]
    if src_off != 0 or G._prod(dims) != n:
        return False
    want = _rm_strides(dims)
    return all(dims[i] == 1 or (st[i] & 0xFFFFFFFF) == want[i] for i in range(rank))


def _is_identity(kind: int, v: float) -> bool:
    if kind == V.RED_SUM or kind == V.RED_OR or kind == V.RED_XOR:
        return v == 0
    if kind == V.RED_PROD:
        return v == 1
    if kind == V.RED_MAX:
        return v == -math.inf or v <= -3.4028234663852886e38
    if kind == V.RED_MIN:
        return v == math.inf or v >= 3.4028234663852886e38
    if kind == V.RED_AND:
        return v != 0
    return False


def _count_ops(ops, mod, depth=0) -> int:
    if depth > 4:
        return 0
    n = 0
    for o in ops:
        if o.name in ("stablehlo.return", "func.return", "stablehlo.constant"):
            continue
        if o.name == "func.call":
            f = mod.funcs.get(o.attr("callee").name)
            n += _count_ops(f.body.ops, mod, depth + 1) if f else 1
            continue
        n += 1
        for region in o.regions:
            for blk in region:
                n += _count_ops(blk.ops, mod, depth + 1)
    return n


def _result_bytes(ops) -> int:
    total = 0
    for o in ops:
        if o.name in ("stablehlo.return", "func.return", "stablehlo.constant"):
            continue
        for r in o.results:
            if isinstance(r.type, M.TensorType) and r.type.elem in DT_OF_ELEM:
                total += r.type.n * V.DT_SIZE[DT_OF_ELEM[r.type.elem]]
    return total


def detect_fixed_trip(op: M.Op, cval: dict):
    """The counted-loop pattern of lax.fori_loop / scan (lowering.py:718-784):
    a scalar integer carry k with a constant init, a cond that is exactly
    ``compare LT (arg_k, constant)`` (not UNSIGNED), and a body returning
    ``add(arg_k, constant step)`` with step > 0.  Returns (trips, k, init, step)
    or None."""
    cond, body = op.regions[0][0], op.regions[1][0]
    consts = {}
    cmp = ret = None
    for o in cond.ops:
        if o.name == "stablehlo.constant":
            consts[o.results[0]] = o.attr("value").array().reshape(-1)
        elif o.name == "stablehlo.compare":
            if cmp is not None:
                return None
            cmp = o
        elif o.name == "stablehlo.return":
            ret = o
        else:
            return None
    if cmp is None or ret is None or ret.operands[0] is not cmp.results[0]:
        return None
    if M.attr_enum(cmp.attr("comparison_direction")) != "LT":
        return None
    ct = cmp.attr("compare_type")
    if ct is not None and M.attr_enum(ct) == "UNSIGNED":
        return None
    if cmp.operands[0] not in cond.args:
        return None
    k = cond.args.index(cmp.operands[0])

    def scalar(v, table):
        a = table.get(v)
        if a is None or a.size != 1 or not np.issubdtype(a.dtype, np.integer):
            return None
        return int(a.reshape(-1)[0])

    limit = scalar(cmp.operands[1], {**cval, **consts})
    init = scalar(op.operands[k], cval)
    if limit is None or init is None:
        return None
    bconsts = {o.results[0]: o.attr("value").array().reshape(-1) for o in body.ops if o.name == "stablehlo.constant"}
    bret = next((o for o in body.ops if o.name == "stablehlo.return"), None)
    if bret is None:
        return None
    upd = next((o for o in body.ops if bret.operands[k] in o.results), None)
    if upd is None or upd.name != "stablehlo.add":
        return None
    arg = body.args[k]
    table = {**cval, **bconsts}
    if upd.operands[0] is arg:
        step = scalar(upd.operands[1], table)
    elif upd.operands[1] is arg:
        step = scalar(upd.operands[0], table)
    else:
        return None
    if step is None or step <= 0:
        return None
    trip = max(0, (limit - init + step - 1) // step)
    if trip >= 1 << 31:
        return None
    return trip, k, init, step


# ---- entry points -------------------------------------------------------------------------------

def lower_module(module: M.Module, fuse: bool = True) -> V.VMProgram:
    """A parsed module's public @main -> a VMProgram (tensor sections), fused and
    with its arena packed by liveness; ``io_aliases`` holds the donations the
    program can take (``donation_aliases``)."""
    from . import passes
    prog = Lowerer(module).lower()
    if fuse:
        passes.run_all(prog)
    else:
        passes.dce(prog)
        passes.finalize_matmul_views(prog)
    passes.reuse_arena(prog)
    if prog.arena_bytes >= 1 << 31:
        raise LoweringError(f"arena of {prog.arena_bytes} bytes exceeds the 31-bit offset space "
                            f"(bit 31 of a handle marks an I/O port)")
    prog.io_aliases = donation_aliases(prog, module.main)
    return prog


def donation_aliases(prog: V.VMProgram, main: M.Func, cfg=None) -> list:
    """[(input, output)] pairs a donated argument may share memory with: the
    argument carries ``tf.aliasing_output`` (what jax.jit(donate_argnums=...)
    emits), the two have the same byte size, neither is also an output / input,
    and every instruction reading the input runs in an earlier phase (a grid
    barrier earlier) than every instruction writing the output, so on shared
    memory no write can overtake a read.  Loops and branches count as one phase
    each, as in passes.reuse_arena."""
    from . import passes
    from . import scheduler as S
    pairs = []
    for i in range(len(prog.inputs)):
        a = main.arg_attr(i, "tf.aliasing_output")
        if a is None:
            continue
        try:
            o = M.attr_int(a)
        except M.MlirSyntaxError:
            continue
        if 0 <= o < len(prog.outputs):
            pairs.append((i, o))
    if not pairs:
        return []
    cfg = cfg or S.DeviceConfig.from_env()
    sched = S._Scheduler(prog, cfg)
    phase = {}
    for ph, (kind, payload) in enumerate(sched.levels(list(range(prog.main_len)))):
        roots = payload if kind == "compute" else [payload]
        for r in roots:
            stack = [r]
            while stack:
                k = stack.pop()
                phase[k] = ph
                ins = prog.instrs[k]
                if ins.op in (V.OP_WHILE, V.OP_IF):
                    stack += list(range(ins.a, ins.a + ins.b)) + list(range(ins.n, ins.n + ins.imm))
                elif ins.op == V.OP_FOR:
                    stack += list(range(ins.n, ins.n + ins.imm))
    for dot_i, ln_i in sched.ln_pro.items():         # a layernorm staged in its GEMV runs there
        if dot_i in phase:
            phase[ln_i] = phase[dot_i]
    grp = S.overlap_groups(prog)
    out = []
    for i, o in pairs:
        bi, bo = prog.inputs[i], prog.outputs[o]
        if prog.buffers[bi].size_bytes != prog.buffers[bo].size_bytes or bi in prog.outputs or bo in prog.inputs:
            continue
        reads = [phase[k] for k, ins in enumerate(prog.instrs)
                 if ins.op != V.OP_NOP and k in phase and grp[bi] in {grp[b] for b in passes.reads_of(ins, prog)}]
        writes = [phase[k] for k, ins in enumerate(prog.instrs)
                  if ins.op != V.OP_NOP and k in phase and grp[bo] in {grp[b] for b in passes.writes_of(ins)}]
        if writes and (not reads or max(reads) < min(writes)):
            out.append((i, o))
    return out


def lower_text(text: str, fuse: bool = True) -> V.VMProgram:
    try:
        mod = M.parse_module(text)
    except M.MlirSyntaxError as e:
        raise LoweringError(f"cannot read the program: {e}") from None
    return lower_module(mod, fuse=fuse)


def artifact_to_text(artifact: bytes) -> str:
    """PJRT_Client_Compile program bytes -> MLIR text.  Text passes through; a
    VHLO portable artifact (MLIR bytecode, magic 'ML\\xefR') is deserialized and
    printed in the generic form with jaxlib's own bindings (lowering.py:3145-3157),
    which must then be importable."""
    data = bytes(artifact)
    if data[:4] == b"ML\xefR":
        try:
            from jaxlib.mlir import ir
            from jaxlib.mlir.dialects import stablehlo
        except ImportError:
            raise LoweringError("a VHLO portable artifact needs jaxlib's MLIR bindings to deserialize; "
                                "pass the program as MLIR text instead") from None
        ctx = ir.Context()
        try:
            from jaxlib.mlir._mlir_libs import _sdy
            _sdy.register_dialect(ctx, load=True)
        except Exception:  # noqa: BLE001 -- older jaxlib without Shardy
            pass
        module = stablehlo.deserialize_portable_artifact(ctx, data)
        return module.operation.get_asm(print_generic_op_form=True)
    try:
        return data.decode("utf-8")
    except UnicodeDecodeError:
        raise LoweringError("program bytes are neither MLIR text nor a VHLO artifact") from None


def lower_artifact(artifact: bytes) -> V.VMProgram:
    return lower_text(artifact_to_text(artifact))


def lower_and_schedule(artifact: bytes, cfg=None, with_aliases: bool = False):
    """Program bytes -> VMProgram v3 bytes with the schedule for the device the
    environment describes (PJRT_OCL_NLANES / _EW_TS / _MMA_T, scheduler.py:135-153);
    with ``with_aliases`` the pair (bytes, [(input, output)] donation aliases)."""
    from . import scheduler as S
    prog = lower_artifact(artifact)
    cfg = cfg or S.DeviceConfig.from_env()
    blob = V.serialize(prog, S.schedule_program(prog, cfg))
    return (blob, list(getattr(prog, "io_aliases", []))) if with_aliases else blob
