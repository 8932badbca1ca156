"""CPU oracle for the VMProgram megakernel VM -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker.  The product path (package
``pjrt_amd`` and ``libvmrt.so``) never imports or calls it.

It restates the reference's numpy validators and tile-op semantics:

* ``parse``          -- strict v3 reader (python/pjrt_ocl/vmreader.py:182-380),
                        written independently of the product writer so format
                        bugs on one side cannot hide on the other;
* ``execute``        -- tensor-level interpreter of the instruction list
                        (vmreader.py:389-470 + the ``interp`` handlers of
                        python/pjrt_ocl/ops/*.py);
* ``execute_schedule`` -- lane simulator over the schedule sections
                        (vmreader.py:475-773): per barrier phase it runs the
                        lanes forward and in reverse and requires identical
                        arenas, checks that every tile of every task is covered
                        exactly once and that control is uniform across lanes.

Per-op math follows the device kernels (pjrt_plugin/kernels/ops/*.cl):
fmax/fmin ignore NaN (ew.cl:24), integer shifts mask the count (ew.cl:420-458),
integer division by zero yields 0 (ew.cl:410), bool is one byte 0/1,
f16/bf16 are storage formats with f32 arithmetic (ew.cl:494-511) and
f32->bf16 rounds to nearest even (vm_common.cl:66-70).

Intentional differences from the reference kernels, each a fix the reference's
own tests (which compare against JAX) would agree with:
* u32 max/min/div compare unsigned (the reference's ew.cl:409-411 uses the
  signed view; its reduce.cl:33-34 already uses unsigned);
* f32->bf16 keeps NaN a NaN (the reference's bit formula can carry a NaN with
  low payload bits into the sign bit);
* the fused layernorm extension (LN_TWO_PASS) uses the two-pass variance that
  JAX's layernorm computes; the reference's fused core uses E[x^2]-mu^2
  (reduce.cl:447-473), which the oracle keeps for LAYERNORM_SEG without flags.

Parity status per function is listed in the module ``PINS`` table.
"""
from __future__ import annotations

import dataclasses
import math
import struct

import numpy as np

# --- format constants (independent restatement of docs/vmprogram.md) -----------
MAGIC, VERSION = 0x314D5056, 3
F32, I32, U32, BOOL, I64, F64, F16, BF16 = range(8)
NP = {F32: np.float32, I32: np.int32, U32: np.uint32, BOOL: np.uint8,
      I64: np.int64, F64: np.float64, F16: np.float16, BF16: np.uint16}
SIZE = {F32: 4, I32: 4, U32: 4, BOOL: 1, I64: 8, F64: 8, F16: 2, BF16: 2}
INTS = (I32, U32, I64)

NOP, BARRIER, WHILE, IF, FOR = (0xFFFFFFFF, 0xFFFFFFFE, 0xFFFFFFFD,
                                0xFFFFFFFC, 0xFFFFFFFB)
SENTINELS = (NOP, BARRIER, WHILE, IF, FOR)
FLAG_NONE = 0xFFFFFFFF     # an entry field that names no completion flag

# parity pins: how each semantic function is checked (see tests/test_oracle.py)
PINS = {
    "format": "golden bytes tests/test_lowering.py:109-171 + field layout 174-243",
    "ew_f32": "numpy float64 closed forms at rel 1e-6; integer-valued exact",
    "ew_int": "closed forms, bit-exact; shift masks ew.cl:420-458",
    "bf16": "bit formula == RNE computed in double over all 2^32 patterns (oracle/refcpu.c "
            "refcpu_bf16_rne_check, tests/test_refcpu.py); GPU convert == formula on 2^24 patterns",
    "gelu": "closed form, runtime_test.cc:256-262 (<=1e-5)",
    "control": "runtime_test.cc:136-215 known answers; _while_e2e_body.py closed forms",
    "reduce": "closed forms + identity table, bit-exact for int",
    "layernorm": "float64 two-pass closed form",
    "softmax": "float64 closed form",
    "dot": "integer-valued small-K inputs exact (test_ops_dot.py trick); float64",
    "flash": "float64 closed form of ops/attention.py:53-64",
    "decode_attn": "extension without a reference counterpart: brute-force loops on tiny "
                   "inputs, and equal to the decomposed dot / mask / softmax / dot chain "
                   "of pinned ops with the cache column at pos holding k, v",
    "gather/scatter/dyn": "brute force index loops on tiny inputs",
}


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    """RNE f32 -> bf16 bits; NaN stays NaN (quiet bit set)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    # u32 sums that wrap (negative NaN patterns only) lose only the bit the
    # 16-bit cast drops; NaNs are replaced below anyway
    r = (u >> 16) & np.uint32(1)
    r += u
    r += np.uint32(0x7FFF)
    r = (r >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    if np.any(nan):
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def _bits_f32(u):
    return np.frombuffer(struct.pack("<I", u & 0xFFFFFFFF), "<f4")[0]


def _i32(u):
    u &= 0xFFFFFFFF
    return u - (1 << 32) if u & 0x80000000 else u


class FormatError(ValueError):
    pass


@dataclasses.dataclass
class Task:
    top: int
    dt: int
    adt: int
    dst: int
    a: int
    b: int
    p: tuple


@dataclasses.dataclass
class Prog:
    arena_bytes: int
    bufs: list            # [(off, size, dtype)]
    inputs: list
    outputs: list
    in_shapes: list
    out_shapes: list
    consts: list
    instrs: list          # tuples (op, dst, a, b, n, imm, aux, imm2)
    main_len: int
    aux: list
    tasks: list | None = None
    streams: list | None = None
    root_lens: list | None = None
    n_lanes: int = 0
    n_flags: int = 0


def parse(data: bytes) -> Prog:
    data = bytes(data)
    if len(data) < 48:
        raise FormatError("short header")
    h = struct.unpack_from("<10IQ", data, 0)
    magic, ver, nb, ni, nc, main_len, nin, nout, naux, hpad, arena = h
    if magic != MAGIC:
        raise FormatError("bad magic")
    if ver != VERSION:
        raise FormatError(f"bad version {ver}")
    if hpad or main_len > ni:
        raise FormatError("bad header")
    pos = 48
    bufs = []
    for i in range(nb):
        off, size, dt, pad = struct.unpack_from("<QQII", data, pos)
        pos += 24
        if off % 64 or off + size > arena or dt > BF16 or pad:
            raise FormatError(f"bad buffer {i}")
        bufs.append((off, size, dt))

    def al():
        nonlocal pos
        pos += -pos % 8

    inputs = list(struct.unpack_from(f"<{nin}I", data, pos)); pos += 4 * nin; al()
    outputs = list(struct.unpack_from(f"<{nout}I", data, pos)); pos += 4 * nout; al()
    shapes = []
    for _ in range(nin + nout):
        rank, pad = struct.unpack_from("<II", data, pos)
        pos += 8
        if pad or rank > 16:
            raise FormatError("bad shape")
        shapes.append(tuple(struct.unpack_from(f"<{rank}Q", data, pos)))
        pos += 8 * rank
    aux = list(struct.unpack_from(f"<{naux}I", data, pos)); pos += 4 * naux; al()
    consts = []
    for _ in range(nc):
        bid, blen = struct.unpack_from("<II", data, pos)
        pos += 8
        if bid >= nb or blen > bufs[bid][1]:
            raise FormatError("bad const")
        consts.append((bid, data[pos:pos + blen]))
        pos += blen
        al()
    instrs = []
    for _ in range(ni):
        instrs.append(struct.unpack_from("<8I", data, pos))
        pos += 32
    p = Prog(arena, bufs, inputs, outputs, shapes[:nin], shapes[nin:], consts,
             instrs, main_len, aux)
    if pos < len(data):
        nt, ne, nf, nl = struct.unpack_from("<4I", data, pos)
        pos += 16
        if not 1 <= nl <= 4096:
            raise FormatError("bad n_lanes")
        tasks = []
        for _ in range(nt):
            w = struct.unpack_from("<12I", data, pos)
            pos += 48
            tasks.append(Task(w[0] & 0xFF, (w[0] >> 8) & 0xFF, (w[0] >> 16) & 0xFF,
                              w[1], w[2], w[3], tuple(w[4:])))
        lt = []
        for _ in range(nl):
            off, cnt, root, _ = struct.unpack_from("<4I", data, pos)
            pos += 16
            if off + cnt > ne or root > cnt:
                raise FormatError("bad lane table")
            lt.append((off, cnt, root))
        ents = []
        for _ in range(ne):
            ents.append(struct.unpack_from("<8I", data, pos))
            pos += 32
        if nf:
            # completion flags (this build's extension of the reserved WAIT /
            # SIGNAL fields): each flag signaled by at most one tile entry,
            # ranges inside [0, n_flags), no entry both waiting and signaling
            signaled = set()
            for e in ents:
                if e[0] in SENTINELS:
                    continue
                if e[4] and (e[3] == FLAG_NONE or e[3] + e[4] > nf or e[5] != FLAG_NONE):
                    raise FormatError("bad completion-flag wait")
                if e[5] != FLAG_NONE:
                    if e[5] >= nf or e[5] in signaled:
                        raise FormatError("bad completion-flag signal")
                    signaled.add(e[5])
        p.tasks = tasks
        p.streams = [ents[o:o + c] for o, c, _ in lt]
        p.root_lens = [r for _, _, r in lt]
        p.n_lanes = nl
        p.n_flags = nf
    if pos != len(data):
        raise FormatError("trailing bytes")
    return p


# --- memory -------------------------------------------------------------------------

class Mem:
    def __init__(self, prog: Prog):
        self.p = prog
        self.arena = np.zeros(prog.arena_bytes + 64, np.uint8)

    def view(self, bid, dt=None):
        off, size, bdt = self.p.bufs[bid]
        dt = bdt if dt is None else dt
        return self.arena[off:off + size].view(NP[dt])

    def load_f(self, bid, dt=None):
        """Buffer as float32 (f16/bf16 widened), the f32-compute view."""
        dt = self.p.bufs[bid][2] if dt is None else dt
        v = self.view(bid, dt)
        if dt == BF16:
            return bf16_to_f32(v)
        return v.astype(np.float32)

    def store_f(self, bid, sl, vals, dt=None):
        dt = self.p.bufs[bid][2] if dt is None else dt
        v = self.view(bid, dt)
        vals = np.asarray(vals, np.float32)
        if dt == BF16:
            v[sl] = f32_to_bf16(vals)
        elif dt == F16:
            v[sl] = vals.astype(np.float16)
        else:
            v[sl] = vals.astype(NP[dt])

    def aux_view(self, off, n):
        return [_i32(w) for w in self.p.aux[off:off + n]]


def _setup(prog: Prog, args) -> Mem:
    if len(args) != len(prog.inputs):
        raise ValueError(f"expected {len(prog.inputs)} args")
    m = Mem(prog)
    for bid, data in prog.consts:
        off = prog.bufs[bid][0]
        m.arena[off:off + len(data)] = np.frombuffer(data, np.uint8)
    for bid, arg in zip(prog.inputs, args):
        dt = prog.bufs[bid][2]
        flat = np.ascontiguousarray(arg).reshape(-1)
        if dt == BF16 and flat.dtype != np.uint16:
            flat = f32_to_bf16(flat.astype(np.float32))
        flat = flat.astype(NP[dt], copy=False)
        if flat.nbytes != prog.bufs[bid][1]:
            raise ValueError(f"arg for buffer {bid}: {flat.nbytes} bytes, want "
                             f"{prog.bufs[bid][1]}")
        m.view(bid)[:] = flat
    return m


def _outputs(prog: Prog, m: Mem):
    return [m.view(b).copy().reshape(s) for b, s in zip(prog.outputs, prog.out_shapes)]


# --- elementwise math (ew.cl:19-64, 394-490) ------------------------------------

def _sign(x):
    return np.where(x > 0, np.float32(1), np.where(x < 0, np.float32(-1), x)).astype(x.dtype)


def _round_afz(x):
    """Round half away from zero (C roundf).  |x| - floor(|x|) is exact, so the
    half-way test has no rounding error (floor(|x| + 0.5) would send
    0.49999997 to 1)."""
    ax = np.abs(x)
    fl = np.floor(ax)
    r = np.where(ax - fl >= 0.5, fl + 1, fl)
    return np.copysign(r, x).astype(x.dtype)


def gelu_f32(x):
    x = np.asarray(x, np.float32)
    inner = np.float32(0.7978845608) * (x + np.float32(0.044715) * x * x * x)
    return (np.float32(0.5) * x * (np.float32(1.0) + np.tanh(inner))).astype(np.float32)


def _float_bin(sub, x, y):
    with np.errstate(all="ignore"):
        if sub == 0: return x + y
        if sub == 1: return x * y
        if sub == 2: return x - y
        if sub == 3: return x / y
        if sub == 4: return np.fmax(x, y)
        if sub == 5: return np.fmin(x, y)
        if sub == 6: return np.power(x, y)
        if sub == 25: return np.arctan2(x, y)
        if sub == 26: return np.fmod(x, y)
    raise NotImplementedError(sub)


def _float_un(sub, x):
    with np.errstate(all="ignore"):
        if sub == 7: return x.copy()
        if sub == 8: return -x
        if sub == 9: return np.exp(x)
        if sub == 10: return np.log(x)
        if sub == 11: return np.sqrt(x)
        if sub == 12: return (1.0 / np.sqrt(x.astype(np.float64))).astype(x.dtype)
        if sub == 13: return np.tanh(x)
        if sub == 14: return np.abs(x)
        if sub == 15: return np.floor(x)
        if sub == 16: return np.ceil(x)
        if sub == 17: return _sign(x)
        if sub == 27: return np.log1p(x)
        if sub == 28: return np.expm1(x)
        if sub == 29: return np.cbrt(x)
        if sub == 30: return np.sin(x)
        if sub == 31: return np.cos(x)
        if sub == 32: return np.tan(x)
        if sub == 33: return np.rint(x)
        if sub == 34: return _round_afz(x)
        if sub == 41:
            if x.dtype == np.float64:
                return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))
            return gelu_f32(x)
    raise NotImplementedError(sub)


IS_BIN = set(range(0, 7)) | {25, 26}
IS_UN = set(range(7, 18)) | set(range(27, 35)) | {41}


def _int_op(sub, x, y, dt):
    """i32/u32/i64 elementwise, wrap-around arithmetic."""
    nbits = 64 if dt == I64 else 32
    ut = np.uint64 if nbits == 64 else np.uint32
    with np.errstate(all="ignore"):
        if sub == 0: return x + y
        if sub == 1: return x * y
        if sub == 2: return x - y
        if sub == 3:
            ys = np.where(y == 0, 1, y)
            if dt == U32:
                q = x // ys
            else:
                # C division truncates toward zero; numpy // floors.  Correct
                # the floor where the remainder is nonzero and signs differ
                # (no abs(), which overflows at the most negative value).
                q = x // ys
                fix = ((x % ys) != 0) & ((x < 0) != (ys < 0))
                q = (q + fix.astype(x.dtype)).astype(x.dtype)
            return np.where(y == 0, 0, q).astype(x.dtype)
        if sub == 4: return np.maximum(x, y)
        if sub == 5: return np.minimum(x, y)
        if sub == 7: return x.copy()
        if sub == 8: return (-x).astype(x.dtype)
        if sub == 14: return x if dt == U32 else np.abs(x).astype(x.dtype)
        if sub == 17:
            return (x > 0).astype(x.dtype) - (x < 0).astype(x.dtype) if dt != U32 \
                else (x > 0).astype(x.dtype)
        if sub == 35: return x & y
        if sub == 36: return x | y
        if sub == 37: return x ^ y
        if sub == 38: return ~x
        if sub in (42, 43, 44):
            cnt = (y.astype(ut) & ut(nbits - 1))
            if sub == 42:
                return (x.astype(ut) << cnt).astype(x.dtype)
            if sub == 43:
                return (x.astype(ut) >> cnt).astype(x.dtype)
            st = np.int64 if nbits == 64 else np.int32
            return (x.astype(st) >> cnt.astype(st)).astype(x.dtype)
    return x.copy()


def _cmp(pred, x, y):
    return {0: np.equal, 1: np.not_equal, 2: np.less, 3: np.less_equal,
            4: np.greater}.get(pred, np.greater_equal)(x, y).astype(np.uint8)


def _convert(x, adt, dt):
    """ew.cl:532-588: integer<->integer through 64-bit (low bits kept),
    otherwise a numeric cast with truncation toward zero; bool = (v != 0)."""
    if adt in INTS + (BOOL,) and dt in INTS:
        v = x.astype(np.uint32).astype(np.int64) if adt == U32 else x.astype(np.int64)
        if dt == I64:
            return v
        low = (v & 0xFFFFFFFF).astype(np.uint32)      # keep the low 32 bits
        return low.view(np.int32) if dt == I32 else low
    v = bf16_to_f32(x).astype(np.float64) if adt == BF16 else x.astype(np.float64)
    if dt == BOOL:
        return (v != 0).astype(np.uint8)
    if dt in INTS:
        # float -> int saturates to the target range and maps NaN to 0 (XLA's
        # convert semantics; the reference's C cast leaves out-of-range values
        # undefined).
        info = np.iinfo(NP[dt])
        with np.errstate(all="ignore"):
            tv = np.trunc(v)
            out = np.zeros(v.shape, NP[dt])
            ok = ~np.isnan(v)
            hi = ok & (tv >= float(info.max) + 1.0)
            lo = ok & (tv < float(info.min))
            mid = ok & ~hi & ~lo
            out[hi] = info.max
            out[lo] = info.min
            out[mid] = tv[mid].astype(np.int64).astype(NP[dt]) if dt != U32 else \
                tv[mid].astype(np.uint64).astype(np.uint32)
            return out
    if dt == BF16:
        return f32_to_bf16(v.astype(np.float32))
    if dt == F16:
        return v.astype(np.float32).astype(np.float16)
    return v.astype(NP[dt])


# --- reductions (reduce.cl:16-40, ops/reduce.py:56-160) --------------------------

def _red_float(arr, kind, axis=None):
    arr = arr.astype(np.float32)
    if kind == 0: return arr.sum(axis, dtype=np.float64).astype(np.float32)
    if kind == 1: return np.fmax.reduce(arr, axis=axis, initial=-np.inf)
    if kind == 2: return np.fmin.reduce(arr, axis=axis, initial=np.inf)
    if kind == 3: return arr.prod(axis, dtype=np.float64).astype(np.float32)
    raise NotImplementedError(kind)


def _red_int(arr, kind, dt, axis=None):
    if dt == BOOL:
        arr = (arr != 0).astype(np.int32)
        ident = {0: 0, 1: 0, 2: 1, 3: 1, 4: 1, 5: 0, 6: 0}
    else:
        info = np.iinfo(NP[dt])
        ident = {0: 0, 1: info.min, 2: info.max, 3: 1,
                 4: -1 if dt != U32 else info.max, 5: 0, 6: 0}
    with np.errstate(all="ignore"):
        init = np.array(ident[kind]).astype(arr.dtype)
        fn = {0: np.add, 1: np.maximum, 2: np.minimum, 3: np.multiply,
              4: np.bitwise_and, 5: np.bitwise_or, 6: np.bitwise_xor}[kind]
        r = fn.reduce(arr, axis=axis, initial=init)
    if dt == BOOL:
        return (np.asarray(r) & 1).astype(np.uint8)
    return np.asarray(r).astype(NP[dt])


def reduce_np(arr, kind, dt, axis=None):
    if dt in INTS or dt == BOOL:
        return _red_int(arr, kind, dt, axis)
    return _red_float(arr, kind, axis)


def layernorm_core(x, eps, two_pass: bool):
    """(x - mu) * rsqrt(var + eps) per row, float64 accumulation."""
    x64 = x.astype(np.float64)
    mu = x64.mean(-1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(-1, keepdims=True) if two_pass else \
        (x64 * x64).mean(-1, keepdims=True) - mu * mu
    return ((x64 - mu) / np.sqrt(var + eps)).astype(np.float32)


def softmax_rows(x):
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).astype(np.float32)


def attention(Q, Kb, Vb, scale, causal):
    """ops/attention.py:53-64 closed form; Q [H,T,hd], Kb [H,hd,C], Vb [H,C,hd]."""
    H, T, hd = Q.shape
    C = Kb.shape[2]
    s = np.einsum("htd,hdc->htc", Q.astype(np.float64), Kb.astype(np.float64)) * scale
    if causal:
        qpos = np.arange(T)[:, None] + (C - T)
        s = np.where(np.arange(C)[None, :] > qpos, -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("htc,hcd->htd", p, Vb.astype(np.float64)).astype(np.float32)


def decode_attention(q, Kt, Vc, k, v, pos, scale, krow=False, masked=False):
    """Extension OP_DECODE_ATTN (no reference counterpart; it is the per-step
    attention of the reference's decode idiom, DOT(q K^T) -> mask -> softmax ->
    DOT(P V), with the step's key/value appended to the cache prefix).
    q, k, v [H, hd]; Kt [H, hd, C] ([H, C, hd] with ``krow``); Vc [H, C, hd];
    pos clamped to [0, C].  ``masked``: the form a decoder writes with the step's
    key and value already stored at column pos and the keys after pos masked
    (tools/bench_decode.py:47-52 is the unmasked append form): pos is clamped
    to [0, C - 1] like the cache update's start, and a negative pos masks every
    key, so the row is NaN as the decomposed softmax makes it."""
    C = Kt.shape[1] if krow else Kt.shape[2]
    p = min(max(int(pos), 0), C - 1 if masked else C)
    kp = Kt[:, :p] if krow else Kt[:, :, :p].transpose(0, 2, 1)
    keys = np.concatenate([kp, k[:, None, :]], 1).astype(np.float64)
    vals = np.concatenate([Vc[:, :p], v[:, None, :]], 1).astype(np.float64)
    s = np.einsum("hd,hcd->hc", q.astype(np.float64), keys) * scale
    e = np.exp(s - s.max(-1, keepdims=True))
    e /= e.sum(-1, keepdims=True)
    out = np.einsum("hc,hcd->hd", e, vals)
    if masked and int(pos) < 0:
        out[:] = np.nan
    return out


def _round_to(y, dt):
    """f32 values as stored in dtype dt and read back as f32."""
    y = np.asarray(y, np.float32)
    if dt == BF16:
        return bf16_to_f32(f32_to_bf16(y))
    if dt == F16:
        return y.astype(np.float16).astype(np.float32)
    return y


def _epi_micro(kind, x, y, s, t):
    if kind in IS_BIN:
        return _float_bin(kind, x, y)
    if kind == 40:
        return x * s + t
    if kind in IS_UN:
        return _float_un(kind, x)
    return x


def _view_index(aux, view1, n):
    """Flat source index of each of the n elements of a strided view."""
    off = view1 - 1
    rank = aux[off]
    dims = [_i32(w) for w in aux[off + 1:off + 1 + rank]]
    st = [_i32(w) for w in aux[off + 1 + rank:off + 1 + 2 * rank]]
    src_off = _i32(aux[off + 1 + 2 * rank])
    idx = np.full(n, src_off, np.int64)
    rem = np.arange(n, dtype=np.int64)
    for e in range(rank - 1, -1, -1):
        idx += (rem % dims[e]) * st[e]
        rem //= dims[e]
    return idx


def _affine_index(aux, base_off, n):
    """[rank, dims, strides, off] descriptor -> flat offset of each element."""
    rank = aux[base_off]
    dims = [_i32(w) for w in aux[base_off + 1:base_off + 1 + rank]]
    st = [_i32(w) for w in aux[base_off + 1 + rank:base_off + 1 + 2 * rank]]
    off = _i32(aux[base_off + 1 + 2 * rank])
    idx = np.full(n, off, np.int64)
    rem = np.arange(n, dtype=np.int64)
    for e in range(rank - 1, -1, -1):
        idx += (rem % dims[e]) * st[e]
        rem //= dims[e]
    return idx


# --- task semantics over a tile range -----------------------------------------------------

class TaskRunner:
    """Executes tiles [lo, hi) of a task against ``Mem`` (the device contract:
    ops/*.cl; tile -> element mapping as scheduler.py:178-197)."""

    def __init__(self, m: Mem, ew_ts: int, mma_t: int):
        self.m = m
        self.ts = ew_ts
        self.mma_t = mma_t
        self.splits = {}            # (task, output tile) -> K-split tiles run so far

    def run(self, t: Task, lo: int, hi: int):
        fn = getattr(self, f"top{t.top}", None)
        if fn is None:
            raise NotImplementedError(f"tile op {t.top}")
        fn(t, lo, hi)

    def _range(self, n, lo, hi):
        return lo * self.ts, min(hi * self.ts, n)

    # 0: elementwise
    def top0(self, t, lo, hi):
        m = self.m
        sub, n = t.p[0], t.p[1]
        a0, a1 = self._range(n, lo, hi)
        if a0 >= a1:
            return
        sl = slice(a0, a1)
        dt, adt = t.dt, t.adt
        if sub == 20:       # CMP: operands as adt, bool out
            x = m.view(t.a, adt)[sl]; y = m.view(t.b, adt)[sl]
            if adt in (F16, BF16):
                x, y = m.load_f(t.a, adt)[sl], m.load_f(t.b, adt)[sl]
            m.view(t.dst, BOOL)[sl] = _cmp(t.p[2], x, y)
            return
        if sub == 21:       # SELECT: bool pred at p3
            pred = m.view(t.p[3], BOOL)[sl]
            x = m.view(t.a, dt)[sl]; y = m.view(t.b, dt)[sl]
            m.view(t.dst, dt)[sl] = np.where(pred != 0, x, y)
            return
        if sub == 23:
            m.view(t.dst, dt)[sl] = _convert(m.view(t.a, adt)[sl], adt, dt)
            return
        if sub == 24:
            m.view(t.dst, dt)[sl] = m.view(t.a, dt)[sl]
            return
        if sub == 39:
            m.view(t.dst, BOOL)[sl] = np.isfinite(m.load_f(t.a, adt)[sl]).astype(np.uint8)
            return
        if dt == BOOL:
            a = m.view(t.a, BOOL)[sl]
            if sub == 18:
                m.view(t.dst, BOOL)[sl] = np.uint8(t.p[2] != 0)
            elif sub == 38:
                m.view(t.dst, BOOL)[sl] = (a == 0).astype(np.uint8)
            elif sub in (35, 36, 37):
                b = m.view(t.b, BOOL)[sl] != 0
                a = a != 0
                r = a & b if sub == 35 else (a | b if sub == 36 else a ^ b)
                m.view(t.dst, BOOL)[sl] = r.astype(np.uint8)
            else:
                m.view(t.dst, BOOL)[sl] = a
            return
        if dt in INTS:
            d = m.view(t.dst, dt)
            if sub == 18:
                v = _i32(t.p[2])
                d[sl] = np.array(v).astype(NP[dt])
            elif sub == 19:
                d[sl] = np.arange(a0, a1).astype(NP[dt])
            else:
                x = m.view(t.a, dt)[sl]
                y = m.view(t.b, dt)[sl]
                d[sl] = _int_op(sub, x, y, dt)
            return
        if dt == F64:
            x = m.view(t.a, F64)[sl]
            d = m.view(t.dst, F64)
            if sub in IS_BIN:
                d[sl] = _float_bin(sub, x, m.view(t.b, F64)[sl])
            elif sub in IS_UN:
                d[sl] = _float_un(sub, x)
            elif sub == 18:
                d[sl] = np.float64(_bits_f32(t.p[2]))
            elif sub == 19:
                d[sl] = np.arange(a0, a1, dtype=np.float64)
            return
        # f32 / f16 / bf16: f32 arithmetic
        view_ok = sub in IS_BIN or sub in IS_UN
        if sub == 18:
            m.store_f(t.dst, sl, np.full(a1 - a0, _bits_f32(t.p[2]), np.float32), dt)
            return
        if sub == 19:
            m.store_f(t.dst, sl, np.arange(a0, a1, dtype=np.float32), dt)
            return
        if sub == 22:
            if lo == 0:
                r = np.float32(1.0 if m.load_f(t.a)[0] < m.load_f(t.b)[0] else 0.0)
                m.store_f(t.dst, slice(0, 1), [r], dt)
            return

        def rd(bid, view):
            if view_ok and view and dt == F32:
                idx = _view_index(self.m.p.aux, view, n)[a0:a1]
                return m.load_f(bid, dt)[idx]
            return m.load_f(bid, dt)[sl]

        x = rd(t.a, t.p[2])
        if sub in IS_BIN:
            r = _float_bin(sub, x, rd(t.b, t.p[3]))
        elif sub in IS_UN:
            r = _float_un(sub, x)
        elif sub == 40:
            s, tt = _bits_f32(t.p[2]), _bits_f32(t.p[3])
            x = m.load_f(t.a, dt)[sl]
            r = (x.astype(np.float64) * s + tt).astype(np.float32)
        else:
            raise NotImplementedError(f"EW subop {sub}")
        m.store_f(t.dst, sl, r, dt)

    # 1: matmul tiles (mma.cl:362-434 + epilogue 74-96)
    def _mma_operands(self, t):
        m = self.m
        M, N, K = t.p[0], t.p[1], t.p[2]
        G = max(1, t.p[3] & 0xFFFFFF)
        av, bv = t.p[4], t.p[5]
        A = m.load_f(t.a, t.adt)
        B = m.load_f(t.b, t.adt)
        A = (A[_view_index(m.p.aux, av, G * M * K)] if av else A[:G * M * K]).reshape(G, M, K)
        B = (B[_view_index(m.p.aux, bv, G * K * N)] if bv else B[:G * K * N]).reshape(G, K, N)
        return A, B, M, N, K, G

    def top1(self, t, lo, hi):
        """Matmul tiles.  A K-split task (p3 bits 28-31, this build's extension)
        has S tiles per output tile; the output tile is written, from the whole
        product, once all S of its tiles have run (in any order), which is when
        the device's last-arriving split writes it."""
        m = self.m
        A, B, M, N, K, G = self._mma_operands(t)
        code = (t.p[3] >> 24) & 0xF
        T = {1: 64, 2: 128, 3: 256}.get(code, self.mma_t)
        S = 1 << (t.p[3] >> 28)
        tn, tm = -(-N // T), -(-M // T)
        per = tn * tm
        if S > 1:
            done = []
            for tile in range(lo, hi):
                key = (id(t), tile // S)
                self.splits[key] = self.splits.get(key, 0) + 1
                if self.splits[key] == S:
                    del self.splits[key]
                    done.append(tile // S)
            lo, hi, tiles = 0, 0, done
        else:
            tiles = range(lo, hi)
        out = np.zeros((G, M, N), np.float32)
        have = self.m.load_f(t.dst, t.dt)[:G * M * N].reshape(G, M, N).copy()
        res = None
        if t.p[6] and t.p[7] is not None:
            try:
                res = self.m.load_f(t.p[7])
            except Exception:
                res = None
        for tile in tiles:
            g, loc = tile // per, tile % per
            tr, tc = loc // tn, loc % tn
            r0, r1 = tr * T, min(tr * T + T, M)
            c0, c1 = tc * T, min(tc * T + T, N)
            if r0 >= r1 or c0 >= c1:
                continue
            blk = (A[g, r0:r1].astype(np.float64) @ B[g, :, c0:c1].astype(np.float64)).astype(np.float32)
            if t.p[6]:
                blk = self._epilogue(t, blk, g, r0, r1, c0, c1, M, N, res)
            have[g, r0:r1, c0:c1] = blk
        self.m.store_f(t.dst, slice(0, G * M * N), have.reshape(-1), t.dt)

    # 20: skinny matmul (extension): tile g * ceil(N / CW) + nb is the column
    # strip [CW nb, CW nb + CW) of batch g over the whole K (p4 = CW).
    def top20(self, t, lo, hi):
        m = self.m
        M, N, K, G, CW = t.p[0], t.p[1], t.p[2], max(1, t.p[3]), t.p[4]
        ncb = -(-N // CW)
        if t.p[5]:
            # fused layernorm (extension): x is normalised while staged and
            # rounded to the layernorm's output dtype, its result never stored
            ln = m.p.tasks[t.p[5] - 1]
            A = _round_to(self._ln_rows(ln, 0, M), ln.dt).reshape(1, M, K)
        else:
            A = m.load_f(t.a, t.adt)[:G * M * K].reshape(G, M, K)
        B = m.load_f(t.b, t.adt)[:G * K * N].reshape(G, K, N)
        res = m.load_f(t.p[7]) if t.p[6] else None
        have = m.load_f(t.dst, t.dt)[:G * M * N].reshape(G, M, N).copy()
        for tile in range(lo, hi):
            nb, g = tile % ncb, tile // ncb
            c0, c1 = nb * CW, min(nb * CW + CW, N)
            blk = (A[g].astype(np.float64) @ B[g, :, c0:c1].astype(np.float64)).astype(np.float32)
            if t.p[6]:
                blk = self._epilogue(t, blk, g, 0, M, c0, c1, M, N, res)
            have[g, :, c0:c1] = blk
        m.store_f(t.dst, slice(0, G * M * N), have.reshape(-1), t.dt)

    def _epilogue(self, t, v, g, r0, r1, c0, c1, M, N, res):
        aux = self.m.p.aux
        off = t.p[6] - 1
        nm = aux[off]
        for k in range(nm):
            kind, src = aux[off + 1 + 4 * k], aux[off + 2 + 4 * k]
            s, tt = _bits_f32(aux[off + 3 + 4 * k]), _bits_f32(aux[off + 4 + 4 * k])
            if src == 1:
                y = res[:M * N * (g + 1)].reshape(-1, M, N)[g, r0:r1, c0:c1]
            elif src == 2:
                y = np.broadcast_to(res[c0:c1], v.shape)
            elif src == 3:          # this build's constant operand: y = s
                y = np.full(v.shape, np.float32(s), np.float32)
            else:
                y = v
            v = np.asarray(_epi_micro(kind, v, y, np.float32(s), np.float32(tt)), np.float32)
        return v

    # 2: strided gather (gather.cl:9-85)
    def top2(self, t, lo, hi):
        n = t.p[1]
        a0, a1 = self._range(n, lo, hi)
        if a0 >= a1:
            return
        esz = SIZE[t.dt]
        dtn = {1: BOOL, 2: BF16, 4: U32, 8: I64}[esz]
        idx = _affine_index(self.m.p.aux, t.p[0], n)[a0:a1]
        self.m.view(t.dst, dtn)[a0:a1] = self.m.view(t.a, dtn)[idx]

    # 3/4: two-phase full reduce
    def top3(self, t, lo, hi):
        n, chunk, kind = t.p[0], t.p[1], t.p[2]
        src = self.m.view(t.a, t.dt)
        out = self.m.view(t.dst, t.dt)
        for tile in range(lo, hi):
            s0, s1 = tile * chunk, min(tile * chunk + chunk, n)
            if s0 < s1:
                out[tile] = reduce_np(src[s0:s1], kind, t.dt)

    def top4(self, t, lo, hi):
        if lo <= 0 < hi:
            n, kind = t.p[0], t.p[1]
            self.m.view(t.dst, t.dt)[0] = reduce_np(self.m.view(t.a, t.dt)[:n], kind, t.dt)

    # 5: iota along a dimension (iota.cl:4-29)
    def top5(self, t, lo, hi):
        n = t.p[1]
        a0, a1 = self._range(n, lo, hi)
        aux = self.m.p.aux
        rank = aux[t.p[0]]
        dims = aux[t.p[0] + 1:t.p[0] + 1 + rank]
        dim = aux[t.p[0] + 1 + rank]
        coord = (np.arange(a0, a1) // int(np.prod(dims[dim + 1:], dtype=np.int64))) % dims[dim]
        d = self.m
        if t.dt in INTS:
            d.view(t.dst, t.dt)[a0:a1] = coord.astype(NP[t.dt])
        else:
            d.store_f(t.dst, slice(a0, a1), coord.astype(np.float32), t.dt)

    # 6: strided scatter (scatter.cl:9-60)
    def top6(self, t, lo, hi):
        n = t.p[1]
        a0, a1 = self._range(n, lo, hi)
        esz = SIZE[t.dt]
        dtn = {1: BOOL, 2: BF16, 4: U32, 8: I64}[esz]
        idx = _affine_index(self.m.p.aux, t.p[0], n)[a0:a1]
        self.m.view(t.dst, dtn)[idx] = self.m.view(t.a, dtn)[a0:a1]

    def _dyn(self, t):
        aux = self.m.p.aux
        x = t.p[0]
        rank = aux[x]
        dims = [_i32(w) for w in aux[x + 1:x + 1 + rank]]
        st = [_i32(w) for w in aux[x + 1 + rank:x + 1 + 2 * rank]]
        cmax = [_i32(w) for w in aux[x + 1 + 2 * rank:x + 1 + 3 * rank]]
        ids = aux[x + 1 + 4 * rank:x + 1 + 5 * rank]
        is64 = aux[x + 1 + 5 * rank]
        base = 0
        for d in range(rank):
            s = int(self.m.view(ids[d], I64 if is64 else I32)[0])
            base += min(max(s, 0), cmax[d]) * st[d]
        idx = np.full(int(np.prod(dims)) if rank else 1, base, np.int64)
        rem = np.arange(idx.size, dtype=np.int64)
        for e in range(rank - 1, -1, -1):
            idx += (rem % dims[e]) * st[e]
            rem //= dims[e]
        return idx

    # 7/8: dynamic slice / update (dynslice.cl:1-166)
    def top7(self, t, lo, hi):
        n = t.p[1]
        a0, a1 = self._range(n, lo, hi)
        dtn = {1: BOOL, 2: BF16, 4: U32, 8: I64}[SIZE[t.dt]]
        idx = self._dyn(t)[a0:a1]
        self.m.view(t.dst, dtn)[a0:a1] = self.m.view(t.a, dtn)[idx]

    def top8(self, t, lo, hi):
        n = t.p[1]
        a0, a1 = self._range(n, lo, hi)
        dtn = {1: BOOL, 2: BF16, 4: U32, 8: I64}[SIZE[t.dt]]
        idx = self._dyn(t)[a0:a1]
        self.m.view(t.dst, dtn)[idx] = self.m.view(t.a, dtn)[a0:a1]

    # 10: segmented reduce, GEMV dot mode (reduce.cl:165-281)
    def top10(self, t, lo, hi):
        n_out, seg, kind, dot = t.p[0], t.p[1], t.p[2], t.p[3]
        r0, r1 = lo, min(hi, n_out)
        if r0 >= r1:
            return
        if dot:
            A = self.m.load_f(t.a, t.adt)[r0 * seg:r1 * seg].reshape(-1, seg)
            x = self.m.load_f(t.b, t.adt)[:seg]
            r = (A.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
            self.m.store_f(t.dst, slice(r0, r1), r, t.dt)
            return
        if t.dt in INTS or t.dt == BOOL:
            src = self.m.view(t.a, t.dt)[r0 * seg:r1 * seg].reshape(-1, seg)
            self.m.view(t.dst, t.dt)[r0:r1] = reduce_np(src, kind, t.dt, axis=1)
        else:
            src = self.m.load_f(t.a, t.adt)[r0 * seg:r1 * seg].reshape(-1, seg)
            self.m.store_f(t.dst, slice(r0, r1), _red_float(src, kind, 1), t.dt)

    # 11: softmax rows
    def top11(self, t, lo, hi):
        n_out, seg = t.p[0], t.p[1]
        r0, r1 = lo, min(hi, n_out)
        if r0 < r1:
            x = self.m.load_f(t.a, t.adt)[r0 * seg:r1 * seg].reshape(-1, seg)
            self.m.store_f(t.dst, slice(r0 * seg, r1 * seg), softmax_rows(x).reshape(-1), t.dt)

    # 12: layernorm rows (+ extension flags in p3)
    def top12(self, t, lo, hi):
        n_out, seg, c = t.p[0], t.p[1], t.p[5]
        r0, r1 = lo, min(hi, n_out)
        if r0 >= r1:
            return
        if c:
            # row interleave (extension p5): logical row i is (i % c) * (n_out / c) + i / c
            for i in range(r0, r1):
                r = (i % c) * (n_out // c) + i // c
                y = self._ln_rows(t, r, r + 1)
                self.m.store_f(t.dst, slice(r * seg, (r + 1) * seg), y.reshape(-1), t.dt)
            return
        y = self._ln_rows(t, r0, r1)
        self.m.store_f(t.dst, slice(r0 * seg, r1 * seg), y.reshape(-1), t.dt)

    def _ln_rows(self, t, r0, r1):
        """Layernorm rows [r0, r1) of a LAYERNORM_SEG task in f32, before the
        store's conversion to the task's output dtype."""
        seg, flags = t.p[1], t.p[3]
        eps = float(_bits_f32(t.p[2]))
        x = self.m.load_f(t.a, t.adt)[r0 * seg:r1 * seg].reshape(-1, seg)
        y = layernorm_core(x, eps, two_pass=bool(flags & 4))
        if flags & 1:
            g = self.m.load_f(t.b)[:seg].astype(np.float64)
            b = self.m.load_f(t.p[4])[:seg].astype(np.float64)
            y = (y.astype(np.float64) * g + b).astype(np.float32)
        if flags & 2:
            y = gelu_f32(y)
        return y

    # 13: map region (region.cl:43-98)
    def top13(self, t, lo, hi):
        n = t.p[1]
        a0, a1 = self._range(n, lo, hi)
        if a0 >= a1:
            return
        aux = self.m.p.aux
        d = t.p[0]
        n_in, out_slot, n_micro = aux[d], aux[d + 1], aux[d + 2]
        handles = [t.a, t.b] + list(t.p[2:8])
        R = {}
        for k in range(n_in):
            R[aux[d + 3 + k]] = self.m.load_f(handles[k])[a0:a1]
        o = d + 3 + n_in
        for _ in range(n_micro):
            kind, ds, as_, bs = aux[o:o + 4]
            s, tt = _bits_f32(aux[o + 4]), _bits_f32(aux[o + 5])
            x = R[as_]
            y = R.get(bs, x)
            R[ds] = np.asarray(_epi_micro(kind, x, y, np.float32(s), np.float32(tt)), np.float32)
            o += 6
        self.m.store_f(t.dst, slice(a0, a1), R[out_slot], t.dt)

    # 14: flash attention, one (head, query row) per tile (attention.cl:49-159)
    def top14(self, t, lo, hi):
        aux = self.m.p.aux
        d = t.p[3]
        H, T, C, hd = aux[d:d + 4]
        scale = float(_bits_f32(aux[d + 4]))
        causal, qv, kv, vv = aux[d + 5:d + 9]
        Q = self.m.load_f(t.a, t.adt)
        K = self.m.load_f(t.b, t.adt)
        Vv = self.m.load_f(t.p[0], t.adt)
        Q = (Q[_view_index(aux, qv, H * T * hd)] if qv else Q[:H * T * hd]).reshape(H, T, hd)
        K = (K[_view_index(aux, kv, H * hd * C)] if kv else K[:H * hd * C]).reshape(H, hd, C)
        Vv = (Vv[_view_index(aux, vv, H * C * hd)] if vv else Vv[:H * C * hd]).reshape(H, C, hd)
        out = self.m.load_f(t.dst, t.dt)[:H * T * hd].reshape(H, T, hd).copy()
        # tile = head * Tp + row, each head's rows padded to Tp = whole 256-row
        # blocks (tiles past T are empty)
        Tp = -(-T // 256) * 256
        tiles = [tile for tile in range(lo, min(hi, H * Tp)) if tile % Tp < T]
        heads = sorted({tile // Tp for tile in tiles})
        for g in heads:
            O = attention(Q[g:g + 1], K[g:g + 1], Vv[g:g + 1], scale, causal)[0]
            for tile in tiles:
                if tile // Tp == g:
                    out[g, tile % Tp] = O[tile % Tp]
        self.m.store_f(t.dst, slice(0, H * T * hd), out.reshape(-1), t.dt)

    # 21: decode-step attention (extension): tile = head * S + split, p4 = H | S << 16;
    # a head's result is complete once its last split has run
    def top21(self, t, lo, hi):
        H, S, hd, C = t.p[4] & 0xFFFF, max(1, t.p[4] >> 16), t.p[5] & 0xFFFF, t.p[6]
        krow, masked = bool(t.p[5] >> 16 & 1), bool(t.p[5] >> 17 & 1)
        heads = [tile // S for tile in range(lo, min(hi, H * S)) if tile % S == S - 1]
        if not heads:
            return
        h0, h1 = heads[0], heads[-1] + 1
        ld = lambda bid, n: self.m.load_f(bid, t.adt)[:n]
        q = ld(t.a, H * hd).reshape(H, hd)
        Kt = ld(t.b, H * hd * C).reshape((H, C, hd) if krow else (H, hd, C))
        Vc = ld(t.p[0], H * C * hd).reshape(H, C, hd)
        k = ld(t.p[1], H * hd).reshape(H, hd)
        v = ld(t.p[2], H * hd).reshape(H, hd)
        pos = int(self.m.view(t.p[3], I32)[0])
        sl = slice(h0, h1)
        o = decode_attention(q[sl], Kt[sl], Vc[sl], k[sl], v[sl], pos, float(_bits_f32(t.p[7])), krow, masked)
        self.m.store_f(t.dst, slice(h0 * hd, h1 * hd), o.reshape(-1).astype(np.float32), t.dt)

    # 15: strided partial-axis reduce
    def top15(self, t, lo, hi):
        n_out, red, inner, kind = t.p[0], t.p[1], t.p[2], t.p[3]
        a0, a1 = lo * self.ts, min(hi * self.ts, n_out)
        if a0 >= a1:
            return
        outer = n_out // inner
        if t.dt in INTS or t.dt == BOOL:
            src = self.m.view(t.a, t.dt)[:outer * red * inner].reshape(outer, red, inner)
            r = reduce_np(src, kind, t.dt, axis=1).reshape(-1)
            self.m.view(t.dst, t.dt)[a0:a1] = r[a0:a1]
        else:
            src = self.m.load_f(t.a, t.adt)[:outer * red * inner].reshape(outer, red, inner)
            r = _red_float(src, kind, 1).reshape(-1)
            self.m.store_f(t.dst, slice(a0, a1), r[a0:a1], t.dt)

    # 16: data-dependent gather (gather.cl:108+)
    def top16(self, t, lo, hi):
        n = t.p[1]
        a0, a1 = self._range(n, lo, hi)
        if a0 >= a1:
            return
        aux = [_i32(w) for w in self.m.p.aux]
        x = t.p[0]
        out_rank, nidx, vstride, is64, _, idx_buf = aux[x:x + 6]
        od = aux[x + 6:x + 6 + out_rank]
        ops = aux[x + 6 + out_rank:x + 6 + 2 * out_rank]
        sis = aux[x + 6 + 2 * out_rank:x + 6 + 3 * out_rank]
        ios = aux[x + 6 + 3 * out_rank:x + 6 + 3 * out_rank + nidx]
        cm = aux[x + 6 + 3 * out_rank + nidx:x + 6 + 3 * out_rank + 2 * nidx]
        idxv = self.m.view(idx_buf, I64 if is64 else I32)
        i = np.arange(a0, a1, dtype=np.int64)
        off = np.zeros_like(i)
        si = np.zeros_like(i)
        rem = i.copy()
        for e in range(out_rank - 1, -1, -1):
            c = rem % od[e]
            rem //= od[e]
            off += c * ops[e]
            si += c * sis[e]
        for k in range(nidx):
            s = idxv[si + k * vstride].astype(np.int64)
            off += np.clip(s, 0, cm[k]) * ios[k]
        dtn = {1: BOOL, 2: BF16, 4: U32, 8: I64}[SIZE[t.dt]]
        self.m.view(t.dst, dtn)[a0:a1] = self.m.view(t.a, dtn)[off]

    # 19: argmax over the last axis (extension); tile = row * S + split with
    # S = p3 (a row's result is complete once its last split has run)
    def top19(self, t, lo, hi):
        n_out, seg, S = t.p[0], t.p[1], max(1, t.p[3])
        rows = [tile // S for tile in range(lo, min(hi, n_out * S)) if tile % S == S - 1]
        if not rows:
            return
        r0, r1 = rows[0], rows[-1] + 1
        x = self.m.load_f(t.a, t.adt)[r0 * seg:r1 * seg].reshape(-1, seg)
        nan = np.isnan(x)
        idx = np.where(nan.any(1), nan.argmax(1), np.nanargmax(np.where(nan, -np.inf, x), 1))
        self.m.view(t.dst, t.dt)[r0:r1] = idx.astype(NP[t.dt])
        vals = x[np.arange(x.shape[0]), idx]
        bdt = self.m.p.bufs[t.b][2]
        self.m.store_f(t.b, slice(r0, r1), vals, bdt)


# --- tensor-level interpreter (validator a) -------------------------------------------------

def _instr_task(prog: Prog, ins, ew_ts: int, mma_t: int):
    """Minimal instruction -> task restatement for the interpreter (same field
    meanings as every reference ``*_to_task``; independent of the product
    scheduler)."""
    op, dst, a, b, n, imm, aux, imm2 = ins
    bufs = prog.bufs
    dt = bufs[dst][2]
    adt = bufs[a][2] if a < len(bufs) else dt
    BIN = {1: 0, 2: 1, 3: 2, 8: 3, 9: 4, 10: 5, 11: 6, 40: 25, 41: 26, 42: 35,
           43: 36, 44: 37, 61: 42, 62: 43, 63: 44}
    UN = {12: 7, 13: 8, 14: 9, 15: 10, 16: 11, 17: 12, 18: 13, 19: 14, 20: 15,
          21: 16, 22: 17, 32: 27, 33: 28, 34: 29, 35: 30, 36: 31, 37: 32,
          38: 33, 39: 34, 45: 38, 56: 41}
    p = [0] * 8
    if op in BIN:
        top, p[:4] = 0, [BIN[op], n, imm, imm2]
    elif op in UN:
        top, p[:3], b = 0, [UN[op], n, imm], a
    elif op == 4:
        top, p[:3] = 0, [18, n, imm]
    elif op == 5:
        top, p[:2] = 0, [19, n]
    elif op == 6:
        top, p[:2] = 0, [22, 1]
    elif op == 23:
        top, p[:3] = 0, [20, n, imm]
    elif op == 24:
        top, p[:4] = 0, [21, n, 0, imm]
    elif op == 30:
        top, p[:2] = 0, [23, n]
    elif op == 31:
        top, p[:2] = 0, [24, n]
    elif op == 46:
        top, p[:2] = 0, [39, n]
    elif op == 51:
        top, p[:4] = 0, [40, n, imm, imm2]
    elif op == 25:
        top, p[:2] = 2, [aux, n]
    elif op == 28:
        top, p[:2] = 5, [aux, n]
    elif op == 47:
        top, p[:2] = 6, [aux, n]
    elif op == 48:
        top, p[:2] = 7, [aux, n]
    elif op == 49:
        top, p[:2] = 8, [aux, n]
    elif op == 60:
        top, p[:2] = 16, [aux, n]
    elif op == 26:
        phase, kind = (imm >> 3) & 1, imm & 7
        if phase == 0:
            top, p[:3] = 3, [n, max(ew_ts, math.ceil(n / 256)) if n else 1, kind]
        else:
            top, p[:2] = 4, [n, kind]
    elif op == 52:
        top, p[:3] = 10, [n, imm & 0x0FFFFFFF, imm >> 28]
    elif op == 59:
        top, p[:4] = 15, [n, imm & 0x0FFFFFFF, imm2, imm >> 28]
    elif op == 54:
        top, p[:2] = 11, [n, imm]
    elif op == 55:
        top, p[:3] = 12, [n, imm, imm2]
    elif op == 66:
        flags, beta = prog.aux[aux], prog.aux[aux + 1]
        top, p[:5] = 12, [n, imm, imm2, flags, beta]
    elif op == 67:
        top, p[:3] = 19, [n, imm, imm2]
    elif op == 57:
        dsc = aux
        n_in, n_micro = prog.aux[dsc], prog.aux[dsc + 2]
        tail = dsc + 3 + n_in + 6 * n_micro
        inp = [prog.aux[tail + k] for k in range(n_in)]
        f = [inp[k] if k < n_in else inp[0] for k in range(8)]
        a, b = f[0], f[1]
        top, p = 13, [aux, n] + f[2:]
    elif op == 58:
        top, p[:4] = 14, [imm2, n, imm, aux]
    elif op == 68:
        hd, kb, vb, posb, sbits = prog.aux[aux:aux + 5]
        top, p = 21, [imm2, kb, vb, posb, n, hd, imm, sbits]
    elif op == 27:
        M, N, K, G = n, imm >> 16, imm & 0xFFFF, max(1, imm2)
        views = prog.aux[aux:aux + 4] if aux else [0, 0, 0, 0]
        if N == 1 and G == 1 and not any(views[:3]):
            top, p[:4] = 10, [M, K, 0, 1]
        else:
            top, p = 1, [M, N, K, G, views[0], views[1], views[2], views[3]]
    else:
        raise NotImplementedError(f"opcode {op}")
    return Task(top, dt, adt, dst, a, b, tuple(p))


def _whole_tiles(t: Task, ew_ts: int, mma_t: int) -> int:
    p = t.p
    if t.top in (0, 2, 5, 6, 7, 8, 9, 13, 16, 17, 18):
        return max(1, -(-p[1] // ew_ts))
    if t.top == 15:
        return max(1, -(-p[0] // ew_ts))
    if t.top == 1:
        T = {1: 64, 2: 128, 3: 256}.get((p[3] >> 24) & 0xF, mma_t)
        return -(-p[0] // T) * -(-p[1] // T) * max(1, p[3] & 0xFFFFFF) << (p[3] >> 28)
    if t.top == 3:
        return max(1, -(-p[0] // p[1]))
    if t.top == 4:
        return 1
    if t.top in (10, 11, 12):
        return max(1, p[0])
    if t.top == 19:
        return max(1, p[0]) * max(1, p[3])
    if t.top == 14:
        return max(1, p[1] * (-(-p[2] // 256) * 256))        # each head's rows padded to 256-row blocks
    if t.top == 20:
        return max(1, p[3]) * -(-p[1] // p[4])
    if t.top == 21:
        return max(1, (p[4] & 0xFFFF) * max(1, p[4] >> 16))
    raise NotImplementedError(t.top)


def _cond_true(m: Mem, bid: int) -> bool:
    dt = m.p.bufs[bid][2]
    v = m.view(bid, dt)[0]
    if dt == BF16:
        return bool(bf16_to_f32(v) != 0)
    return bool(v != 0)


def execute(data_or_prog, args, ew_ts: int = 4096, mma_t: int = 128):
    """Validator (a): interpret the tensor instruction list."""
    prog = data_or_prog if isinstance(data_or_prog, Prog) else parse(data_or_prog)
    m = _setup(prog, args)
    tr = TaskRunner(m, ew_ts, mma_t)

    def run(start, length, depth=0):
        if depth > 8:
            raise FormatError("region nesting exceeds 8")
        for pc in range(start, start + length):
            ins = prog.instrs[pc]
            op = ins[0]
            if op == 0:
                continue
            if op == 7:                       # WHILE: cond [a,a+b), body [n,n+imm)
                while True:
                    run(ins[2], ins[3], depth + 1)
                    if not _cond_true(m, ins[1]):
                        break
                    run(ins[4], ins[5], depth + 1)
            elif op == 53:                    # FOR: body [n,n+imm) x b
                for _ in range(ins[3]):
                    run(ins[4], ins[5], depth + 1)
            elif op == 29:                    # IF
                if _cond_true(m, ins[1]):
                    run(ins[2], ins[3], depth + 1)
                else:
                    run(ins[4], ins[5], depth + 1)
            else:
                t = _instr_task(prog, ins, ew_ts, mma_t)
                tr.run(t, 0, _whole_tiles(t, ew_ts, mma_t))

    run(0, prog.main_len)
    return _outputs(prog, m)


# --- schedule lane simulator (validator b) --------------------------------------------------

def check_coverage(prog: Prog, ew_ts: int, mma_t: int) -> None:
    """Every tile of every task runs exactly once, except the layernorm tasks a
    GEMV stages as its prologue (task p5), which no lane runs."""
    prologue = {t.p[5] - 1 for t in prog.tasks if t.top == 20 and t.p[5]}
    per = {}
    for s in prog.streams:
        for e in s:
            if e[0] in SENTINELS:
                continue
            per.setdefault(e[0], []).append((e[1], e[2]))
    for tid, t in enumerate(prog.tasks):
        if tid in prologue:
            if tid in per or t.top != 12:
                raise AssertionError(f"task {tid}: a GEMV prologue must be a layernorm that no lane runs")
            continue
        nt = _whole_tiles(t, ew_ts, mma_t)
        rs = sorted(per.get(tid, []))
        cur = 0
        for lo, hi in rs:
            if not 0 <= lo <= hi <= nt or lo != cur:
                raise AssertionError(f"task {tid}: tiles not covered exactly once "
                                     f"({rs}, n_tiles={nt})")
            cur = hi
        if cur != nt:
            raise AssertionError(f"task {tid}: covers {cur}/{nt} tiles")


def execute_schedule(data_or_prog, args, ew_ts: int = 4096, mma_t: int = 128,
                     check_order: bool = True):
    prog = data_or_prog if isinstance(data_or_prog, Prog) else parse(data_or_prog)
    if prog.streams is None:
        raise ValueError("no schedule sections")
    check_coverage(prog, ew_ts, mma_t)
    m = _setup(prog, args)
    tr = TaskRunner(m, ew_ts, mma_t)

    def run_batch(batch):
        if not batch:
            return
        by_lane = {}
        for lane, e in batch:
            by_lane.setdefault(lane, []).append(e)
        order = list(by_lane)
        base = m.arena.copy()

        def go(lanes):
            # each lane runs its entries in stream order; with completion flags
            # an entry that waits runs only once every flag of its range was
            # signaled in this phase, so lanes take turns, in `lanes` order,
            # each going as far as it can
            m.arena[:] = base
            pos = dict.fromkeys(lanes, 0)
            signaled = set()
            while True:
                moved = False
                for ln in lanes:
                    es = by_lane[ln]
                    while pos[ln] < len(es):
                        e = es[pos[ln]]
                        if prog.n_flags and e[4] and not all(f in signaled for f in range(e[3], e[3] + e[4])):
                            break
                        tr.run(prog.tasks[e[0]], e[1], e[2])
                        if prog.n_flags and e[5] != FLAG_NONE:
                            signaled.add(e[5])
                        pos[ln] += 1
                        moved = True
                if all(pos[ln] == len(by_lane[ln]) for ln in lanes):
                    return m.arena.copy()
                if not moved:
                    raise AssertionError("completion flags: a wait that no entry of its phase signals")

        fwd = go(order)
        if check_order and len(order) > 1:
            rev = go(order[::-1])
            if not np.array_equal(fwd, rev):
                raise AssertionError("phase is lane-order dependent (cross-lane race)")
        m.arena[:] = fwd

    n = prog.n_lanes
    streams = prog.streams
    stacks = [[[0, prog.root_lens[l], -1, 0]] for l in range(n)]

    def advance(l, batch):
        st = streams[l]
        while True:
            f = stacks[l][-1]
            if f[0] >= f[1]:
                if f[2] == -1:
                    return "DONE"
                w = st[f[2]]
                if w[0] == IF:
                    stacks[l].pop()
                    stacks[l][-1][0] += 1
                    continue
                if w[0] == FOR:
                    return "FOR"
                return "WCOND" if f[3] == 0 else "WBODY"
            e = st[f[0]]
            if e[0] == BARRIER:
                return "BAR"
            if e[0] in (WHILE, FOR, IF):
                if len(stacks[l]) > 8:
                    raise FormatError("frame depth exceeds 8")
            if e[0] == WHILE:
                stacks[l].append([e[1], e[1] + e[2], f[0], 0])
                continue
            if e[0] == FOR:
                if e[3] == 0:
                    f[0] += 1
                    continue
                stacks[l].append([e[1], e[1] + e[2], f[0], e[3]])
                continue
            if e[0] == IF:
                c = _cond_true(m, e[5])
                s0, ln = (e[1], e[2]) if c else (e[3], e[4])
                if ln == 0:
                    f[0] += 1
                    continue
                stacks[l].append([s0, s0 + ln, f[0], 2])
                continue
            if e[0] != NOP:
                batch.append((l, e))
            f[0] += 1

    while True:
        batch = []
        toks = [advance(l, batch) for l in range(n)]
        if all(t == "DONE" for t in toks):
            run_batch(batch)
            break
        if len(set(toks)) != 1:
            raise AssertionError(f"non-uniform control across lanes: {set(toks)}")
        run_batch(batch)
        k = toks[0]
        for l in range(n):
            f = stacks[l][-1]
            if k == "BAR":
                f[0] += 1
                continue
            w = streams[l][f[2]]
            if k == "WCOND":
                if _cond_true(m, w[5]):
                    f[0], f[1], f[3] = w[3], w[3] + w[4], 1
                else:
                    stacks[l].pop()
                    stacks[l][-1][0] += 1
            elif k == "WBODY":
                f[0], f[1], f[3] = w[1], w[1] + w[2], 0
            else:
                f[3] -= 1
                if f[3] > 0:
                    f[0], f[1] = w[1], w[1] + w[2]
                else:
                    stacks[l].pop()
                    stacks[l][-1][0] += 1
    return _outputs(prog, m)
