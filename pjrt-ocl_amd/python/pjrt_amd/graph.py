"""Tensor-graph builder: emits VMProgram tensor instructions.

This is the instruction-selection layer of the lowering: every StableHLO op the
front-end understands becomes one or more calls here, and hand-written programs
(tests, benchmarks) use it directly.  The instructions it emits follow the
reference lowering's encodings op for op (python/pjrt_ocl/ops/*.py handlers,
lowering.py:286-331), so the resulting bytes are a reference-format program.

    g = Graph()
    x = g.input((8, 4), "f32")
    y = g.add(x, g.const(np.ones((8, 4), np.float32)))
    g.output(y)
    prog = g.build()              # VMProgram (tensor sections, arena laid out)
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

from . import vmprogram as V


def _prod(shape) -> int:
    return int(math.prod(shape)) if len(shape) else 1


def _row_major_strides(shape):
    st, acc = [0] * len(shape), 1
    for d in range(len(shape) - 1, -1, -1):
        st[d] = acc
        acc *= shape[d]
    return st


def _dt(d) -> int:
    if isinstance(d, str):
        return V.DT_BY_NAME[d]
    return int(d)


@dataclasses.dataclass(frozen=True)
class Tensor:
    buf: int
    shape: tuple
    dtype: int
    # optional strided view over ``buf`` (aux word offset + 1); set only on
    # values produced by ``view`` and consumed by ops that accept views
    view: int = 0

    @property
    def n(self) -> int:
        return _prod(self.shape)


class GraphError(ValueError):
    pass


class Graph:
    def __init__(self):
        self.buffers: list = []         # [(n_elems, dtype)]
        self.instrs: list = []          # root instruction list being built
        self.regions: list = []         # finished sub-lists appended at build
        self.aux: list = []
        self.consts: list = []          # [(buf, bytes)]
        self.inputs: list = []
        self.outputs: list = []
        self._stack: list = []          # instruction lists under construction
        self._disjoint = 0
        self.aliases: dict = {}         # buffer -> (parent buffer, byte offset)

    # ---- buffers / io -----------------------------------------------------
    def _new(self, shape, dtype) -> Tensor:
        shape = tuple(int(s) for s in shape)
        self.buffers.append((_prod(shape), _dt(dtype)))
        return Tensor(len(self.buffers) - 1, shape, _dt(dtype))

    def input(self, shape, dtype="f32") -> Tensor:
        t = self._new(shape, dtype)
        self.inputs.append(t)
        return t

    def const(self, value, dtype=None) -> Tensor:
        arr = np.asarray(value)
        if dtype is None:
            dtype = {np.float32: V.DT_F32, np.int32: V.DT_I32,
                     np.uint32: V.DT_U32, np.bool_: V.DT_BOOL,
                     np.int64: V.DT_I64, np.float64: V.DT_F64,
                     np.float16: V.DT_F16}.get(arr.dtype.type, V.DT_F32)
        dt = _dt(dtype)
        if dt == V.DT_BF16 and arr.dtype != np.uint16:
            raw = V.f32_to_bf16(arr.astype(np.float32))
        elif dt == V.DT_BOOL:
            raw = arr.astype(np.uint8)
        else:
            raw = arr.astype(V.DT_NUMPY[dt])
        t = self._new(arr.shape, dt)
        self.consts.append((t.buf, np.ascontiguousarray(raw).tobytes()))
        return t

    def scalar(self, v, dtype="f32") -> Tensor:
        dt = _dt(dtype)
        if dt == V.DT_BF16:
            return self.const(np.asarray(v, np.float32), dt)
        return self.const(np.asarray(v, V.DT_NUMPY[dt] if dt != V.DT_BOOL else np.uint8), dt)

    def output(self, *ts: Tensor) -> None:
        for t in ts:
            self.outputs.append(t)

    def add_aux(self, words) -> int:
        off = len(self.aux)
        self.aux.extend(int(w) & 0xFFFFFFFF for w in words)
        return off

    def emit(self, ins: V.Instr) -> None:
        (self._stack[-1] if self._stack else self.instrs).append(ins)

    # ---- views (strided reads folded into consumers) ------------------------
    def view(self, src: Tensor, out_shape, in_strides, src_off=0) -> Tensor:
        """A strided view ``out[i] = src[src_off + sum_d coord_d(i) * stride_d]``
        that elementwise and matmul consumers read in place."""
        rank = len(out_shape)
        off = self.add_aux([rank] + list(out_shape) + list(in_strides) + [src_off])
        return Tensor(src.buf, tuple(out_shape), src.dtype, view=off + 1)

    def broadcast_view(self, src: Tensor, out_shape, dims) -> Tensor:
        """broadcast_in_dim as a view: src axis k maps to out axis dims[k]."""
        st = _row_major_strides(src.shape)
        in_strides = [0] * len(out_shape)
        for k, d in enumerate(dims):
            if src.shape[k] != 1:
                in_strides[d] = st[k]
        return self.view(src, out_shape, in_strides)

    def transpose_view(self, src: Tensor, perm) -> Tensor:
        st = _row_major_strides(src.shape)
        return self.view(src, [src.shape[p] for p in perm], [st[p] for p in perm])

    def alias(self, src: Tensor, elem_off: int, shape) -> Tensor:
        """A contiguous slice of ``src`` as a buffer of its own that shares src's
        memory (no copy): elements [elem_off, elem_off + prod(shape)).  The
        scheduler orders accesses to overlapping buffers like accesses to one."""
        src = self.materialize(src)
        shape = tuple(int(x) for x in shape)
        if elem_off < 0 or elem_off + _prod(shape) > src.n:
            raise GraphError("alias outside its source")
        byte_off = elem_off * V.DT_SIZE[src.dtype]
        if byte_off % 16:
            raise GraphError("alias offset must keep 16-byte alignment")
        parent, base = self.aliases.get(src.buf, (src.buf, 0))
        t = self._new(shape, src.dtype)
        self.aliases[t.buf] = (parent, base + byte_off)
        return t

    def materialize(self, t: Tensor) -> Tensor:
        if not t.view:
            return t
        dst = self._new(t.shape, t.dtype)
        self.emit(V.Instr(V.OP_GATHER_STRIDED, dst=dst.buf, a=t.buf, n=t.n,
                          aux=t.view - 1))
        return dst

    # ---- shape ops ------------------------------------------------------------
    def reshape(self, t: Tensor, shape) -> Tensor:
        t = self.materialize(t)
        if _prod(shape) != t.n:
            raise GraphError("reshape changes element count")
        return Tensor(t.buf, tuple(shape), t.dtype)

    def gather(self, src: Tensor, out_shape, in_strides, src_off=0) -> Tensor:
        return self.materialize(self.view(self.materialize(src), out_shape,
                                          in_strides, src_off))

    def broadcast(self, src: Tensor, out_shape, dims) -> Tensor:
        return self.materialize(self.broadcast_view(self.materialize(src),
                                                    out_shape, dims))

    def transpose(self, src: Tensor, perm) -> Tensor:
        return self.materialize(self.transpose_view(self.materialize(src), perm))

    def slice(self, src: Tensor, starts, limits, strides=None) -> Tensor:
        src = self.materialize(src)
        strides = strides or [1] * len(starts)
        st = _row_major_strides(src.shape)
        out_shape = [max(0, -(-(l - s) // k)) for s, l, k in zip(starts, limits, strides)]
        return self.gather(src, out_shape, [st[d] * strides[d] for d in range(len(st))],
                           sum(starts[d] * st[d] for d in range(len(st))))

    def scatter_into(self, dst: Tensor, src: Tensor, out_strides, out_off,
                     disjoint: int = 0) -> None:
        src = self.materialize(src)
        rank = len(src.shape)
        off = self.add_aux([rank] + list(src.shape) + list(out_strides) + [out_off])
        self.emit(V.Instr(V.OP_SCATTER, dst=dst.buf, a=src.buf, n=src.n, aux=off,
                          disjoint=disjoint))

    def concatenate(self, parts, axis: int) -> Tensor:
        shape = list(parts[0].shape)
        shape[axis] = sum(p.shape[axis] for p in parts)
        out = self._new(shape, parts[0].dtype)
        ost = _row_major_strides(shape)
        self._disjoint += 1
        pos = 0
        for p in parts:
            self.scatter_into(out, p, ost, pos * ost[axis], self._disjoint)
            pos += p.shape[axis]
        return out

    # ---- elementwise ------------------------------------------------------------
    def _binop(self, op, a: Tensor, b: Tensor, out_dtype=None) -> Tensor:
        if a.shape != b.shape:
            raise GraphError(f"shape mismatch {a.shape} vs {b.shape}")
        dt = a.dtype if out_dtype is None else _dt(out_dtype)
        viewable = a.dtype == V.DT_F32 and op in (
            V.OP_ADD_F32, V.OP_MUL_F32, V.OP_SUB_F32, V.OP_DIV_F32,
            V.OP_MAX_F32, V.OP_MIN_F32, V.OP_POW_F32)
        if not viewable:
            a, b = self.materialize(a), self.materialize(b)
        dst = self._new(a.shape, dt)
        self.emit(V.Instr(op, dst=dst.buf, a=a.buf, b=b.buf, n=a.n, imm=a.view,
                          imm2=b.view))
        return dst

    def _unop(self, op, a: Tensor, out_dtype=None) -> Tensor:
        viewable = a.dtype == V.DT_F32 and op in (
            V.OP_COPY_F32, V.OP_NEG_F32, V.OP_EXP_F32, V.OP_LOG_F32,
            V.OP_SQRT_F32, V.OP_RSQRT_F32, V.OP_TANH_F32, V.OP_ABS_F32,
            V.OP_GELU)
        if not viewable:
            a = self.materialize(a)
        dst = self._new(a.shape, a.dtype if out_dtype is None else out_dtype)
        self.emit(V.Instr(op, dst=dst.buf, a=a.buf, n=a.n, imm=a.view))
        return dst

    def add(self, a, b): return self._binop(V.OP_ADD_F32, a, b)
    def mul(self, a, b): return self._binop(V.OP_MUL_F32, a, b)
    def sub(self, a, b): return self._binop(V.OP_SUB_F32, a, b)
    def div(self, a, b): return self._binop(V.OP_DIV_F32, a, b)
    def maximum(self, a, b): return self._binop(V.OP_MAX_F32, a, b)
    def minimum(self, a, b): return self._binop(V.OP_MIN_F32, a, b)
    def pow(self, a, b): return self._binop(V.OP_POW_F32, a, b)
    def atan2(self, a, b): return self._binop(V.OP_ATAN2_F32, a, b)
    def remainder(self, a, b): return self._binop(V.OP_REMAINDER_F32, a, b)
    def bit_and(self, a, b): return self._binop(V.OP_AND, a, b)
    def bit_or(self, a, b): return self._binop(V.OP_OR, a, b)
    def bit_xor(self, a, b): return self._binop(V.OP_XOR, a, b)
    def shl(self, a, b): return self._binop(V.OP_SHL, a, b)
    def shr_l(self, a, b): return self._binop(V.OP_SHR_L, a, b)
    def shr_a(self, a, b): return self._binop(V.OP_SHR_A, a, b)

    def unary(self, name: str, a: Tensor) -> Tensor:
        op = {"copy": V.OP_COPY_F32, "neg": V.OP_NEG_F32, "exp": V.OP_EXP_F32,
              "log": V.OP_LOG_F32, "sqrt": V.OP_SQRT_F32,
              "rsqrt": V.OP_RSQRT_F32, "tanh": V.OP_TANH_F32,
              "abs": V.OP_ABS_F32, "floor": V.OP_FLOOR_F32,
              "ceil": V.OP_CEIL_F32, "sign": V.OP_SIGN_F32,
              "log1p": V.OP_LOG1P_F32, "expm1": V.OP_EXPM1_F32,
              "cbrt": V.OP_CBRT_F32, "sin": V.OP_SIN_F32, "cos": V.OP_COS_F32,
              "tan": V.OP_TAN_F32, "rint": V.OP_ROUND_NEAREST_EVEN_F32,
              "round": V.OP_ROUND_NEAREST_AFZ_F32, "not": V.OP_NOT,
              "gelu": V.OP_GELU}[name]
        return self._unop(op, a)

    def gelu(self, a): return self._unop(V.OP_GELU, a)

    def affine(self, a: Tensor, s: float, t: float) -> Tensor:
        a = self.materialize(a)
        dst = self._new(a.shape, a.dtype)
        self.emit(V.Instr(V.OP_AFFINE_F32, dst=dst.buf, a=a.buf, n=a.n,
                          imm=V.f32_bits(s), imm2=V.f32_bits(t)))
        return dst

    def fill(self, shape, value, dtype="f32") -> Tensor:
        dt = _dt(dtype)
        dst = self._new(shape, dt)
        if dt in (V.DT_F32, V.DT_F16, V.DT_BF16, V.DT_F64):
            bits = V.f32_bits(value)
        else:
            bits = int(value) & 0xFFFFFFFF
        self.emit(V.Instr(V.OP_FILL_F32, dst=dst.buf, n=dst.n, imm=bits))
        return dst

    def iota_flat(self, n: int, dtype="f32") -> Tensor:
        dst = self._new((n,), dtype)
        self.emit(V.Instr(V.OP_IOTA_F32, dst=dst.buf, n=n))
        return dst

    def iota(self, shape, dim: int, dtype="i32") -> Tensor:
        dst = self._new(shape, dtype)
        off = self.add_aux([len(shape)] + list(shape) + [dim])
        self.emit(V.Instr(V.OP_IOTA_DIM, dst=dst.buf, n=dst.n, aux=off))
        return dst

    def compare(self, a: Tensor, b: Tensor, pred: str) -> Tensor:
        a, b = self.materialize(a), self.materialize(b)
        p = {"EQ": 0, "NE": 1, "LT": 2, "LE": 3, "GT": 4, "GE": 5}[pred]
        dst = self._new(a.shape, V.DT_BOOL)
        self.emit(V.Instr(V.OP_CMP_F32, dst=dst.buf, a=a.buf, b=b.buf, n=a.n, imm=p))
        return dst

    def select(self, pred: Tensor, on_true: Tensor, on_false: Tensor) -> Tensor:
        pred, on_true, on_false = map(self.materialize, (pred, on_true, on_false))
        dst = self._new(on_true.shape, on_true.dtype)
        self.emit(V.Instr(V.OP_SELECT_F32, dst=dst.buf, a=on_true.buf,
                          b=on_false.buf, n=dst.n, imm=pred.buf))
        return dst

    def convert(self, a: Tensor, dtype) -> Tensor:
        a = self.materialize(a)
        dst = self._new(a.shape, dtype)
        self.emit(V.Instr(V.OP_CONVERT, dst=dst.buf, a=a.buf, n=a.n))
        return dst

    def bitcast(self, a: Tensor, dtype) -> Tensor:
        a = self.materialize(a)
        if V.DT_SIZE[a.dtype] != V.DT_SIZE[_dt(dtype)]:
            raise GraphError("bitcast between different widths")
        dst = self._new(a.shape, dtype)
        self.emit(V.Instr(V.OP_BITCAST, dst=dst.buf, a=a.buf, n=a.n))
        return dst

    def is_finite(self, a: Tensor) -> Tensor:
        a = self.materialize(a)
        dst = self._new(a.shape, V.DT_BOOL)
        self.emit(V.Instr(V.OP_IS_FINITE, dst=dst.buf, a=a.buf, n=a.n))
        return dst

    def lts(self, a: Tensor, b: Tensor) -> Tensor:
        dst = self._new((), V.DT_F32)
        self.emit(V.Instr(V.OP_LTS_F32, dst=dst.buf, a=a.buf, b=b.buf, n=1))
        return dst

    # ---- reductions ------------------------------------------------------------
    def reduce_all(self, a: Tensor, kind: int, ew_ts: int = 4096) -> Tensor:
        from .scheduler import red_chunk
        a = self.materialize(a)
        chunk = red_chunk(a.n, ew_ts)
        nparts = max(1, math.ceil(a.n / chunk))
        part = self._new((nparts,), a.dtype)
        self.emit(V.Instr(V.OP_REDUCE, dst=part.buf, a=a.buf, n=a.n, imm=kind))
        out = self._new((), a.dtype)
        self.emit(V.Instr(V.OP_REDUCE, dst=out.buf, a=part.buf, n=nparts,
                          imm=(1 << 3) | kind))
        return out

    def reduce_last(self, a: Tensor, kind: int) -> Tensor:
        a = self.materialize(a)
        seg = a.shape[-1]
        dst = self._new(a.shape[:-1], a.dtype)
        self.emit(V.Instr(V.OP_REDUCE_SEG, dst=dst.buf, a=a.buf, n=dst.n,
                          imm=(kind << 28) | seg))
        return dst

    def reduce_axis(self, a: Tensor, axis: int, kind: int) -> Tensor:
        a = self.materialize(a)
        if axis == len(a.shape) - 1:
            return self.reduce_last(a, kind)
        outer = _prod(a.shape[:axis])
        red = a.shape[axis]
        inner = _prod(a.shape[axis + 1:])
        dst = self._new(a.shape[:axis] + a.shape[axis + 1:], a.dtype)
        self.emit(V.Instr(V.OP_REDUCE_STRIDED, dst=dst.buf, a=a.buf,
                          n=outer * inner, imm=(kind << 28) | red, imm2=inner))
        return dst

    def argmax_last(self, a: Tensor, index_dtype="i32"):
        """(max value, first index of the max) over the last axis."""
        a = self.materialize(a)
        seg = a.shape[-1]
        idx = self._new(a.shape[:-1], index_dtype)
        val = self._new(a.shape[:-1], a.dtype)
        self.emit(V.Instr(V.OP_ARGMAX_SEG, dst=idx.buf, a=a.buf, b=val.buf,
                          n=idx.n, imm=seg))
        return val, idx

    def softmax_last(self, a: Tensor, out_dtype=None) -> Tensor:
        a = self.materialize(a)
        dst = self._new(a.shape, a.dtype if out_dtype is None else out_dtype)
        self.emit(V.Instr(V.OP_SOFTMAX, dst=dst.buf, a=a.buf,
                          n=a.n // a.shape[-1], imm=a.shape[-1]))
        return dst

    def layernorm_core(self, a: Tensor, eps: float) -> Tensor:
        a = self.materialize(a)
        dst = self._new(a.shape, a.dtype)
        self.emit(V.Instr(V.OP_LAYERNORM, dst=dst.buf, a=a.buf,
                          n=a.n // a.shape[-1], imm=a.shape[-1],
                          imm2=V.f32_bits(eps)))
        return dst

    def layernorm(self, a: Tensor, gamma: Tensor | None, beta: Tensor | None,
                  eps: float, gelu: bool = False, out_dtype=None) -> Tensor:
        """Fused row layernorm (two-pass variance) with optional per-column
        affine, tanh-GELU and output dtype conversion: one read, one write."""
        a = self.materialize(a)
        flags = V.LN_TWO_PASS | (V.LN_GELU if gelu else 0)
        if gamma is not None:
            flags |= V.LN_AFFINE
            gamma, beta = self.materialize(gamma), self.materialize(beta)
        off = self.add_aux([flags, beta.buf if gamma is not None else 0])
        dst = self._new(a.shape, a.dtype if out_dtype is None else out_dtype)
        self.emit(V.Instr(V.OP_LAYERNORM_AFFINE, dst=dst.buf, a=a.buf,
                          b=gamma.buf if gamma is not None else a.buf,
                          n=a.n // a.shape[-1], imm=a.shape[-1],
                          imm2=V.f32_bits(eps), aux=off,
                          reads_hint=(beta.buf,) if gamma is not None else ()))
        return dst

    # ---- contractions -------------------------------------------------------------
    def dot(self, a: Tensor, b: Tensor, out_dtype="f32", epilogue=None,
            residual: Tensor | None = None, tile: int = 0) -> Tensor:
        """C[G,M,N] = A[G,M,K] @ B[G,K,N]; leading dims of a 2-D-weight matmul
        fold into M.  ``a``/``b`` may be views (folded transposes).  The
        epilogue is a list of (kind, src, s, t) micro-ops applied before the
        store (src 0: unary, 1: residual per element, 2: residual per column,
        3: the constant s -- this build's extension, e.g. relu as (MAX, 3, 0, 0))."""
        if len(b.shape) == 2:
            G = 1
            K = a.shape[-1]
            M = _prod(a.shape[:-1])
            N = b.shape[1]
            out_shape = a.shape[:-1] + (N,)
        else:
            G = _prod(a.shape[:-2])
            M, K = a.shape[-2], a.shape[-1]
            N = b.shape[-1]
            if _prod(b.shape[:-2]) != G:
                raise GraphError("batch mismatch")
            out_shape = a.shape[:-1] + (N,)
        if b.shape[-2] != K:
            raise GraphError(f"contracting mismatch {a.shape} @ {b.shape}")
        if N > 0xFFFF or K > 0xFFFF:
            raise GraphError("N/K exceed the 16-bit packing of the DOT encoding")
        dst = self._new(out_shape, out_dtype)
        epi = 0
        if epilogue:
            words = [len(epilogue)]
            for kind, src, s, t in epilogue:
                words += [kind, src, V.f32_bits(s), V.f32_bits(t)]
            epi = self.add_aux(words) + 1
        ins = V.Instr(V.OP_DOT, dst=dst.buf, a=a.buf, b=b.buf, n=M,
                      imm=(N << 16) | K, imm2=G, aview=a.view, bview=b.view,
                      epi=epi, epi_res=residual.buf if residual is not None else 0,
                      mma_tile=tile)
        if a.view or b.view or epi:
            # mirror of the in-memory view/epilogue fields in an aux header so
            # re-parsed bytes keep them (lowering.py:2455-2466)
            ins.aux = self.add_aux([a.view, b.view, epi,
                                    residual.buf if residual is not None else 0])
        if residual is not None:
            ins.reads_hint = (residual.buf,)
        self.emit(ins)
        return dst

    def flash_attention(self, q: Tensor, k: Tensor, v: Tensor, scale: float,
                        causal: bool, out_dtype=None) -> Tensor:
        """softmax(scale * Q K^T [causal]) V over heads.  q: [..., T, hd],
        k/v: [..., C, hd] (same leading dims, flattened into H).  K is read as
        the matmul B operand [H, hd, C] through a transpose view, as the
        reference's fused op does (ops/attention.py:53-64)."""
        q, k, v = self.materialize(q), self.materialize(k), self.materialize(v)
        H = _prod(q.shape[:-2])
        T, hd = q.shape[-2], q.shape[-1]
        C = k.shape[-2]
        kt = self.view(k, (H, hd, C), (C * hd, 1, hd))   # [H,hd,C] <- [H,C,hd]
        desc = self.add_aux([H, T, C, hd, V.f32_bits(scale), int(causal),
                             0, kt.view, 0])
        dst = self._new(q.shape, q.dtype if out_dtype is None else out_dtype)
        self.emit(V.Instr(V.OP_FLASH_ATTN, dst=dst.buf, a=q.buf, b=k.buf, n=H,
                          imm=T, aux=desc, imm2=v.buf))
        return dst

    def decode_attention(self, q: Tensor, k: Tensor, v: Tensor, cache_kt: Tensor,
                         cache_v: Tensor, pos: Tensor, scale: float, krow: bool = False,
                         masked: bool = False) -> Tensor:
        """One decode step of attention per head (extension opcode
        OP_DECODE_ATTN): the keys are the cache prefix K^T[h, :, :pos] and the
        step's own key k[h], the values V[h, :pos] and v[h], so the step reads
        its new key/value straight from where they were computed and the cache
        update can run beside the next matmul.  q, k, v: [H, hd] (any shape of
        H * hd elements); cache_kt: [H, hd, C], or the key rows [H, C, hd] with
        ``krow``; cache_v: [H, C, hd]; pos: i32 scalar,
        clamped to [0, C].  All float operands share one dtype; the output
        [H, hd] has it too.  Equals the decomposed dot -> (mask beyond pos) ->
        softmax -> dot chain with pos's column of the cache holding k and v.
        ``masked``: that chain as a decoder writes it after storing k and v at
        pos: pos is clamped to [0, C - 1] like the store, and a negative pos
        leaves no key, so the output is NaN."""
        if cache_kt.view or cache_v.view:
            raise GraphError("decode_attention: caches must be plain buffers")
        q, k, v = self.materialize(q), self.materialize(k), self.materialize(v)
        if len(cache_kt.shape) != 3 or len(cache_v.shape) != 3:
            raise GraphError("decode_attention: caches are [H, hd, C] and [H, C, hd]")
        if krow:
            H, C, hd = cache_kt.shape
        else:
            H, hd, C = cache_kt.shape
        if cache_v.shape != (H, C, hd):
            raise GraphError(f"decode_attention: V cache {cache_v.shape} != {(H, C, hd)}")
        for name, t in (("q", q), ("k", k), ("v", v)):
            if t.n != H * hd:
                raise GraphError(f"decode_attention: {name} has {t.n} elements, want {H * hd}")
        dts = {t.dtype for t in (q, k, v, cache_kt, cache_v)}
        if len(dts) != 1 or next(iter(dts)) not in (V.DT_F32, V.DT_F16, V.DT_BF16):
            raise GraphError("decode_attention: q, k, v and the caches share one float dtype")
        if pos.n != 1 or pos.dtype != V.DT_I32:
            raise GraphError("decode_attention: pos is an i32 scalar")
        if hd % 8 or hd > 256 or C % 8 or C > 0xFFFF:
            raise GraphError("decode_attention: hd and C must be multiples of 8 (hd <= 256)")
        dst = self._new((H, hd), q.dtype)
        desc = self.add_aux([hd | int(krow) << 16 | int(masked) << 17, k.buf, v.buf, pos.buf,
                             V.f32_bits(scale)])
        self.emit(V.Instr(V.OP_DECODE_ATTN, dst=dst.buf, a=q.buf, b=cache_kt.buf, n=H,
                          imm=C, aux=desc, imm2=cache_v.buf,
                          reads_hint=(cache_v.buf, k.buf, v.buf, pos.buf)))
        return dst

    # ---- dynamic slices / gathers ------------------------------------------------
    def dynamic_slice(self, a: Tensor, starts, sizes) -> Tensor:
        a = self.materialize(a)
        rank = len(a.shape)
        st = _row_major_strides(a.shape)
        clamp = [a.shape[d] - sizes[d] for d in range(rank)]
        ids = [s.buf for s in starts]
        is64 = int(starts[0].dtype == V.DT_I64) if starts else 0
        off = self.add_aux([rank] + list(sizes) + st + clamp + [0] * rank + ids + [is64])
        dst = self._new(sizes, a.dtype)
        self.emit(V.Instr(V.OP_DYNAMIC_SLICE, dst=dst.buf, a=a.buf, n=dst.n,
                          aux=off, reads_hint=tuple(ids)))
        return dst

    def dynamic_update_slice(self, dst: Tensor, upd: Tensor, starts) -> None:
        """In place: dst[starts ...] = upd (the loop-carry form)."""
        upd = self.materialize(upd)
        rank = len(dst.shape)
        st = _row_major_strides(dst.shape)
        clamp = [dst.shape[d] - upd.shape[d] for d in range(rank)]
        ids = [s.buf for s in starts]
        is64 = int(starts[0].dtype == V.DT_I64) if starts else 0
        off = self.add_aux([rank] + list(upd.shape) + st + clamp + [0] * rank + ids + [is64])
        self.emit(V.Instr(V.OP_DYNAMIC_UPDATE_SLICE, dst=dst.buf, a=upd.buf,
                          n=upd.n, aux=off, reads_hint=tuple(ids)))

    def take_rows(self, table: Tensor, idx: Tensor) -> Tensor:
        """out[i, :] = table[clamp(idx[i]), :] (embedding lookup as a
        stablehlo.gather with one index component)."""
        table, idx = self.materialize(table), self.materialize(idx)
        rows, width = table.shape
        nidx = 1
        out_shape = tuple(idx.shape) + (width,)
        out_rank = len(out_shape)
        op_stride = [0] * (out_rank - 1) + [1]
        si_stride = _row_major_strides(idx.shape) + [0]
        words = [out_rank, nidx, 0, int(idx.dtype == V.DT_I64), 0, idx.buf]
        words += list(out_shape) + op_stride + si_stride + [width] + [rows - 1]
        off = self.add_aux(words)
        dst = self._new(out_shape, table.dtype)
        self.emit(V.Instr(V.OP_GATHER_INDEX, dst=dst.buf, a=table.buf, n=dst.n,
                          aux=off, reads_hint=(idx.buf,)))
        return dst

    def copy_into(self, dst: Tensor, src: Tensor) -> None:
        """dst <- src (elementwise copy; used for loop-carry updates)."""
        src = self.materialize(src)
        op = V.OP_COPY_F32 if src.dtype == V.DT_F32 else V.OP_CONVERT
        self.emit(V.Instr(op, dst=dst.buf, a=src.buf, n=src.n))

    # ---- control flow --------------------------------------------------------------
    def begin(self) -> None:
        self._stack.append([])

    def end(self) -> list:
        return self._stack.pop()

    def for_loop(self, trips: int, body: list) -> None:
        self.emit(V.Instr(V.OP_FOR, b=trips, n=0, imm=0))
        self._pending_region(self._last_list()[-1], [], body)

    def while_loop(self, cond: Tensor, cond_list: list, body: list) -> None:
        self.emit(V.Instr(V.OP_WHILE, dst=cond.buf))
        self._pending_region(self._last_list()[-1], cond_list, body)

    def if_(self, flag: Tensor, then_list: list, else_list: list) -> None:
        self.emit(V.Instr(V.OP_IF, dst=flag.buf))
        self._pending_region(self._last_list()[-1], then_list, else_list)

    def _last_list(self) -> list:
        return self._stack[-1] if self._stack else self.instrs

    def _pending_region(self, ins, first, second) -> None:
        self.regions.append((ins, first, second))

    # ---- build ----------------------------------------------------------------------
    def build(self) -> V.VMProgram:
        # Region sub-lists are appended after the root list; a region nested in
        # another's sub-list gets its ranges fixed the same way (BFS order).
        instrs = list(self.instrs)
        main_len = len(instrs)
        pending = list(self.regions)
        placed = set()
        while pending:
            progress = False
            for item in list(pending):
                ins, first, second = item
                if not any(ins is x for x in instrs):
                    continue
                pending.remove(item)
                progress = True
                a = len(instrs)
                instrs.extend(first)
                n = len(instrs)
                instrs.extend(second)
                if ins.op == V.OP_FOR:
                    ins.n, ins.imm = n, len(second)
                else:
                    ins.a, ins.b, ins.n, ins.imm = a, len(first), n, len(second)
                placed.add(id(ins))
            if not progress:
                raise GraphError("region instruction not reachable from root")
        bufs, off = [], 0
        for i, (n, dt) in enumerate(self.buffers):
            size = n * V.DT_SIZE[dt]
            if i in self.aliases:           # shares its parent's memory
                parent, byte_off = self.aliases[i]
                bufs.append(V.Buffer(bufs[parent].arena_byte_offset + byte_off, size, dt))
                continue
            bufs.append(V.Buffer(off, size, dt))
            off += max(ARENA_SLOT, -(-size // V.ARENA_ALIGN) * V.ARENA_ALIGN)
        return V.VMProgram(
            arena_bytes=off, buffers=bufs,
            inputs=[t.buf for t in self.inputs],
            outputs=[t.buf for t in self.outputs],
            input_shapes=[t.shape for t in self.inputs],
            output_shapes=[t.shape for t in self.outputs],
            consts=list(self.consts), instrs=instrs, main_len=main_len,
            aux=list(self.aux))


ARENA_SLOT = 64
