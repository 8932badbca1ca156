"""VMProgram v3: the bytecode contract between the Python lowering/scheduler and
the MI355X runtime (``libvmrt.so``).

The byte layout is the reference plugin's format so that programs produced by
either side run on the other (reference: python/pjrt_ocl/lowering.py:207-331,
python/pjrt_ocl/scheduler.py:99-106,226-248, pjrt_plugin/src/runtime.cc:90-251,
docs/vmprogram.md).  All integers are little-endian; every section starts on an
8-byte boundary.

    header (48 B)   magic 0x314D5056, version 3, n_buffers, n_instrs, n_consts,
                    main_len, n_inputs, n_outputs, n_aux, pad=0, arena_bytes u64
    buffers         n_buffers x {arena_byte_offset u64, size_bytes u64,
                    dtype u32, pad u32}; offsets 64-byte aligned
    io maps         inputs u32[n_inputs], pad8, outputs u32[n_outputs], pad8
    io shapes       per io buffer (inputs then outputs): {rank u32, pad u32,
                    dims u64[rank]}
    aux pool        n_aux x u32 (signed words are two's complement), pad8
    const pool      n_consts x {buffer_id u32, byte_len u32, data, pad8}
    instructions    n_instrs x {op, dst, a, b, n, imm, aux, imm2} (u32 each);
                    root list = [0, main_len)
    schedule hdr    {n_tasks, n_entries, n_flags, n_lanes}
    tasks           n_tasks x 12 u32: {tile_op | dtype<<8 | adtype<<16, dst, a,
                    b, p0..p7}
    lane table      n_lanes x {entry_off, entry_count, root_len, pad}
    entries         n_entries x {task, tile_lo, tile_hi, wait_flag,
                    wait_count, signal_flag, slots, pad}

Extensions of this build (absent from the reference, chosen so that a program
which does not use them is byte-for-byte a reference program):

* tensor opcode ``OP_LAYERNORM_AFFINE`` (66) and the ``LAYERNORM_SEG`` task
  flags in ``p3`` (affine gamma/beta, tanh-GELU epilogue, output convert);
  ``LAYERNORM_SEG`` p5: row interleave c (logical row i is row
  (i % c) * (n / c) + i / c; 0 = none);
* ``MMA`` task ``p3`` bits 24..27 select a per-task output tile edge
  (0 = the runtime default advertised as PJRT_OCL_MMA_T);
* tensor opcode ``OP_ARGMAX_SEG`` (67) / tile op ``TOP_ARGMAX_SEG`` (19):
  the variadic (value, index) reduce that ``jnp.argmax`` lowers to, which the
  reference rejects (python/pjrt_ocl/ops/reduce.py:165-168); task p3 S splits
  a row over S tiles (tile = row * S + split) combined by the last split
  through the task's scratch;
* tile op ``TOP_GEMV`` (20): the scheduler's column-strip form of an ``OP_DOT``
  with at most 8 rows (decode-time matmuls); p0 M, p1 N, p2 K, p3 G, p4 strip
  width, p5 layernorm prologue (index + 1 of a ``LAYERNORM_SEG`` task that no
  lane runs: the GEMV normalises its x rows while staging them), p6 epilogue +
  1, p7 residual;
* tensor opcode ``OP_DECODE_ATTN`` (68) / tile op ``TOP_DECODE_ATTN`` (21): one
  decode step of attention per head, over a cache prefix of runtime length plus
  the step's own key/value: ``out[h] = softmax(scale q[h] . [K^T[h, :, :pos],
  k[h]]) [V[h, :pos]; v[h]]``.  Instr: dst out, a q, b K^T cache [H, hd, C],
  n H, imm C, imm2 V cache [H, C, hd], aux -> [hd, k, v, pos buffer, scale
  bits].  Task: p0 V, p1 k, p2 v, p3 pos, p4 H | S << 16, p5 hd | krow << 16
  | masked << 17, p6 C, p7 scale bits; tile = head * S + split, each split at
  most 64 cache keys, combined by the last split through the task's scratch.
  ``pos`` (i32 scalar) is clamped to [0, C].  ``krow``: the key cache holds
  rows [H, C, hd] instead of K^T.  ``masked``: the
  decoder's form that stores k, v at pos before attending over keys <= pos:
  pos is clamped to [0, C - 1] and a negative pos gives a NaN output.

Task scratch: the loader gives each task that needs it (a split decode
attention or argmax) its own zeroed region of device memory; the last split of
a head / row resets its arrival counter, so the region is zero again for the
next run.

Matmul epilogue source 3: a micro-op (kind, 3, s, t) takes the constant s as
its operand, e.g. relu as (SUB_MAX, 3, 0, 0) in the matmul's store.
"""
from __future__ import annotations

import dataclasses
import struct

import numpy as np

MAGIC = 0x314D5056          # b"VPM1" little-endian
VERSION = 3
ARENA_ALIGN = 64
SECTION_ALIGN = 8

# ---- dtypes (lowering.py:59-81) ---------------------------------------------
DT_F32, DT_I32, DT_U32, DT_BOOL, DT_I64, DT_F64, DT_F16, DT_BF16 = range(8)
DT_MAX = DT_BF16
DT_NAMES = {DT_F32: "f32", DT_I32: "i32", DT_U32: "u32", DT_BOOL: "bool",
            DT_I64: "i64", DT_F64: "f64", DT_F16: "f16", DT_BF16: "bf16"}
DT_BY_NAME = {v: k for k, v in DT_NAMES.items()}
DT_SIZE = {DT_F32: 4, DT_I32: 4, DT_U32: 4, DT_BOOL: 1, DT_I64: 8, DT_F64: 8,
           DT_F16: 2, DT_BF16: 2}
# numpy storage dtype for each element type; bf16 is carried as its raw 16-bit
# pattern (uint16) because numpy has no bfloat16 (see f32_to_bf16/bf16_to_f32).
DT_NUMPY = {DT_F32: np.dtype("<f4"), DT_I32: np.dtype("<i4"),
            DT_U32: np.dtype("<u4"), DT_BOOL: np.dtype("u1"),
            DT_I64: np.dtype("<i8"), DT_F64: np.dtype("<f8"),
            DT_F16: np.dtype("<f2"), DT_BF16: np.dtype("<u2")}
FLOAT_DTYPES = frozenset({DT_F32, DT_F64, DT_F16, DT_BF16})


def f32_to_bf16(x) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit pattern (uint16), the rule the
    device uses: (u + 0x7fff + ((u >> 16) & 1)) >> 16 (vm_common.cl:66-70)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    # u32 arithmetic: a sum that wraps past 2^32 (negative NaN patterns only)
    # loses just the bit that the cast to 16 bits drops anyway
    r = (u >> 16) & np.uint32(1)
    r += u
    r += np.uint32(0x7FFF)
    r >>= 16
    return r.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


def bits_f32(u: int) -> float:
    return struct.unpack("<f", struct.pack("<I", u & 0xFFFFFFFF))[0]


# ---- tensor opcodes (lowering.py:85-167) --------------------------------------
OP_NOP, OP_ADD_F32, OP_MUL_F32, OP_SUB_F32, OP_FILL_F32, OP_IOTA_F32, \
    OP_LTS_F32, OP_WHILE = range(8)
OP_DIV_F32, OP_MAX_F32, OP_MIN_F32, OP_POW_F32, OP_COPY_F32, OP_NEG_F32, \
    OP_EXP_F32, OP_LOG_F32, OP_SQRT_F32, OP_RSQRT_F32, OP_TANH_F32, \
    OP_ABS_F32, OP_FLOOR_F32, OP_CEIL_F32, OP_SIGN_F32 = range(8, 23)
OP_CMP_F32 = 23
OP_SELECT_F32 = 24
OP_GATHER_STRIDED = 25
OP_REDUCE = 26
OP_DOT = 27
OP_IOTA_DIM = 28
OP_IF = 29
OP_CONVERT = 30
OP_BITCAST = 31
OP_LOG1P_F32, OP_EXPM1_F32, OP_CBRT_F32, OP_SIN_F32, OP_COS_F32, \
    OP_TAN_F32, OP_ROUND_NEAREST_EVEN_F32, OP_ROUND_NEAREST_AFZ_F32, \
    OP_ATAN2_F32, OP_REMAINDER_F32 = range(32, 42)
OP_AND, OP_OR, OP_XOR, OP_NOT, OP_IS_FINITE = range(42, 47)
OP_SCATTER = 47
OP_DYNAMIC_SLICE = 48
OP_DYNAMIC_UPDATE_SLICE = 49
OP_REDUCE_WINDOW = 50
OP_AFFINE_F32 = 51
OP_REDUCE_SEG = 52
OP_FOR = 53
OP_SOFTMAX = 54
OP_LAYERNORM = 55
OP_GELU = 56
OP_MAP_REGION = 57
OP_FLASH_ATTN = 58
OP_REDUCE_STRIDED = 59
OP_GATHER_INDEX = 60
OP_SHL, OP_SHR_L, OP_SHR_A = 61, 62, 63
OP_CONV = 64
OP_SCATTER_INDEX = 65
# extensions (see module docstring)
OP_LAYERNORM_AFFINE = 66
OP_ARGMAX_SEG = 67
OP_DECODE_ATTN = 68
OP_MAX = OP_DECODE_ATTN

REGION_OPS = frozenset({OP_WHILE, OP_IF, OP_FOR})

# ---- tile ops (scheduler.py:47-71, vm_common.cl:74-117) ------------------------
TOP_EW, TOP_MMA, TOP_GATHER, TOP_RED_PART, TOP_RED_COMB, TOP_IOTA_DIM, \
    TOP_SCATTER, TOP_DYN_GATHER, TOP_DYN_SCATTER, TOP_RED_WINDOW, \
    TOP_RED_SEG, TOP_SOFTMAX_SEG, TOP_LAYERNORM_SEG, TOP_MAP_REGION, \
    TOP_FLASH_ATTN, TOP_RED_STRIDED, TOP_GATHER_INDEX, TOP_CONV, \
    TOP_SCATTER_INDEX = range(19)
TOP_ARGMAX_SEG = 19          # extension
TOP_GEMV = 20                # extension
TOP_DECODE_ATTN = 21         # extension
TOP_MAX = TOP_DECODE_ATTN

# ---- EW subops (vm_common.cl:118-146) ------------------------------------------
SUB_ADD, SUB_MUL, SUB_SUB, SUB_DIV, SUB_MAX, SUB_MIN, SUB_POW, SUB_COPY, \
    SUB_NEG, SUB_EXP, SUB_LOG, SUB_SQRT, SUB_RSQRT, SUB_TANH, SUB_ABS, \
    SUB_FLOOR, SUB_CEIL, SUB_SIGN, SUB_FILL, SUB_IOTA_FLAT, SUB_CMP, \
    SUB_SELECT, SUB_LTS, SUB_CONVERT, SUB_BITCAST, SUB_ATAN2, \
    SUB_REMAINDER, SUB_LOG1P, SUB_EXPM1, SUB_CBRT, SUB_SIN, SUB_COS, \
    SUB_TAN, SUB_RINT, SUB_ROUND, SUB_AND, SUB_OR, SUB_XOR, SUB_NOT, \
    SUB_ISFINITE, SUB_AFFINE, SUB_GELU, SUB_SHL, SUB_SHR_L, SUB_SHR_A = range(45)


def sub_is_bin(sub: int) -> bool:
    """Float binary subops (carry a/b view offsets in p2/p3)."""
    return sub <= SUB_POW or SUB_ATAN2 <= sub <= SUB_REMAINDER


def sub_is_un(sub: int) -> bool:
    """Float unary subops (carry an a view offset in p2)."""
    return (SUB_COPY <= sub <= SUB_SIGN or SUB_LOG1P <= sub <= SUB_ROUND
            or sub == SUB_GELU)


# compare predicates and reduce kinds
CMP_EQ, CMP_NE, CMP_LT, CMP_LE, CMP_GT, CMP_GE = range(6)
RED_SUM, RED_MAX, RED_MIN, RED_PROD, RED_AND, RED_OR, RED_XOR = range(7)

# LAYERNORM_SEG task p3 flags (extension; 0 = the reference's core op)
LN_AFFINE = 1     # y = y * gamma[col] + beta[col]; gamma = task.b, beta = task.p4
LN_GELU = 2       # y = gelu_tanh(y)
LN_TWO_PASS = 4   # variance as mean((x - mu)^2) instead of E[x^2] - mu^2

# MMA task p3: batch count in bits 0..23, tile-edge code in bits 24..27
MMA_TILE_CODES = {0: 0, 64: 1, 128: 2, 256: 3}
MMA_CODE_TILE = {1: 64, 2: 128, 3: 256}
# TOP_MMA p3 bits 28-31: log2 of the K split (extension), at most 5
MMA_SPLIT_SHIFT = 28
MMA_MAX_SPLIT_LOG2 = 5

# ---- entry sentinels (scheduler.py:80-85) ---------------------------------------
ENT_NOP = 0xFFFFFFFF
ENT_BARRIER = 0xFFFFFFFE
ENT_WHILE = 0xFFFFFFFD
ENT_IF = 0xFFFFFFFC
ENT_FOR = 0xFFFFFFFB
FLAG_NONE = 0xFFFFFFFF
CONTROL_SENTINELS = frozenset({ENT_NOP, ENT_BARRIER, ENT_WHILE, ENT_IF, ENT_FOR})

HEADER = struct.Struct("<IIIIIIIIIIQ")
BUFENT = struct.Struct("<QQII")
CONSTHDR = struct.Struct("<II")
INSTR = struct.Struct("<8I")
SCHED_HDR = struct.Struct("<IIII")
TASK = struct.Struct("<12I")
LANETAB = struct.Struct("<IIII")
ENTRY = struct.Struct("<8I")


class FormatError(ValueError):
    """Malformed VMProgram bytes."""


@dataclasses.dataclass
class Buffer:
    arena_byte_offset: int
    size_bytes: int
    dtype: int = DT_F32

    @property
    def n_elems(self) -> int:
        return self.size_bytes // DT_SIZE[self.dtype]


@dataclasses.dataclass
class Instr:
    op: int
    dst: int = 0
    a: int = 0
    b: int = 0
    n: int = 0
    imm: int = 0
    aux: int = 0
    imm2: int = 0
    # Not serialized: extra read buffer ids for dependency analysis (runtime
    # start scalars, matmul residual, region inputs), and in-memory-only task
    # fields the scheduler forwards (matmul views/epilogue).
    reads_hint: tuple = ()
    aview: int = 0
    bview: int = 0
    epi: int = 0
    epi_res: int = 0
    region_inputs: tuple = ()
    disjoint: int = 0
    mma_tile: int = 0


@dataclasses.dataclass
class Task:
    tile_op: int
    dst: int = 0
    a: int = 0
    b: int = 0
    p0: int = 0
    p1: int = 0
    p2: int = 0
    p3: int = 0
    p4: int = 0
    p5: int = 0
    p6: int = 0
    p7: int = 0
    dtype: int = DT_F32
    adtype: int = DT_F32

    @property
    def params(self):
        return (self.p0, self.p1, self.p2, self.p3, self.p4, self.p5, self.p6,
                self.p7)


@dataclasses.dataclass
class Entry:
    task: int
    tile_lo: int = 0
    tile_hi: int = 0
    wait_flag: int = FLAG_NONE
    wait_count: int = 0
    signal_flag: int = FLAG_NONE
    slots: int = 0
    pad: int = 0


def barrier_entry() -> Entry:
    return Entry(ENT_BARRIER)


@dataclasses.dataclass
class Schedule:
    n_lanes: int
    tasks: list
    lane_streams: list                 # list[list[Entry]], len == n_lanes
    root_lens: list | None = None      # None: every stream is all root
    n_flags: int = 0

    def root_len(self, lane: int) -> int:
        if self.root_lens is None:
            return len(self.lane_streams[lane])
        return self.root_lens[lane]


@dataclasses.dataclass
class VMProgram:
    arena_bytes: int
    buffers: list
    inputs: list
    outputs: list
    input_shapes: list
    output_shapes: list
    consts: list                       # [(buffer_id, bytes)]
    instrs: list
    main_len: int
    aux: list = dataclasses.field(default_factory=list)
    schedule: Schedule | None = None
    # Buffer id -> lowest id of its group of true aliases (views of the same
    # data), kept by passes.reuse_arena from the layout before packing: after
    # packing, buffers with disjoint lifetimes share bytes too, and ordering
    # those like one buffer would serialise unrelated work.  Not serialized;
    # None: groups follow arena overlap.
    alias_groups: list | None = dataclasses.field(default=None, compare=False, repr=False)
    # [(input index, output index)]: a donated input whose memory the output may
    # take (the lowering's donation_aliases).  Not serialized.
    io_aliases: list = dataclasses.field(default_factory=list, compare=False, repr=False)


def _pad8(out: bytearray) -> None:
    out += b"\0" * (-len(out) % SECTION_ALIGN)


def serialize(prog: VMProgram, schedule: Schedule | None = None) -> bytes:
    """Write v3 bytes: the tensor sections, then the schedule sections when a
    schedule is given (``prog.schedule`` is used when ``schedule`` is None)."""
    sched = schedule if schedule is not None else prog.schedule
    if len(prog.inputs) != len(prog.input_shapes):
        raise FormatError("inputs / input_shapes length mismatch")
    if len(prog.outputs) != len(prog.output_shapes):
        raise FormatError("outputs / output_shapes length mismatch")
    out = bytearray()
    out += HEADER.pack(MAGIC, VERSION, len(prog.buffers), len(prog.instrs),
                       len(prog.consts), prog.main_len, len(prog.inputs),
                       len(prog.outputs), len(prog.aux), 0, prog.arena_bytes)
    for b in prog.buffers:
        if b.arena_byte_offset % ARENA_ALIGN:
            raise FormatError(f"buffer offset {b.arena_byte_offset} not aligned")
        out += BUFENT.pack(b.arena_byte_offset, b.size_bytes, b.dtype, 0)
    for ids in (prog.inputs, prog.outputs):
        for i in ids:
            out += struct.pack("<I", i)
        _pad8(out)
    for shape in list(prog.input_shapes) + list(prog.output_shapes):
        out += struct.pack("<II", len(shape), 0)
        for d in shape:
            out += struct.pack("<Q", int(d))
    if prog.aux:
        out += np.asarray([w & 0xFFFFFFFF for w in prog.aux],
                          dtype="<u4").tobytes()
    _pad8(out)
    for buf_id, data in prog.consts:
        out += CONSTHDR.pack(buf_id, len(data))
        out += bytes(data)
        _pad8(out)
    for ins in prog.instrs:
        out += INSTR.pack(ins.op, ins.dst, ins.a, ins.b, ins.n & 0xFFFFFFFF,
                          ins.imm & 0xFFFFFFFF, ins.aux, ins.imm2 & 0xFFFFFFFF)
    if sched is not None:
        out += serialize_schedule(sched)
    return bytes(out)


def serialize_schedule(sched: Schedule) -> bytes:
    if len(sched.lane_streams) != sched.n_lanes:
        raise FormatError("lane_streams length != n_lanes")
    out = bytearray()
    n_entries = sum(len(s) for s in sched.lane_streams)
    out += SCHED_HDR.pack(len(sched.tasks), n_entries, sched.n_flags,
                          sched.n_lanes)
    for t in sched.tasks:
        out += TASK.pack(t.tile_op | (t.dtype << 8) | (t.adtype << 16),
                         t.dst, t.a, t.b, *(p & 0xFFFFFFFF for p in t.params))
    off = 0
    for lane, stream in enumerate(sched.lane_streams):
        out += LANETAB.pack(off, len(stream), sched.root_len(lane), 0)
        off += len(stream)
    for stream in sched.lane_streams:
        for e in stream:
            out += ENTRY.pack(e.task, e.tile_lo, e.tile_hi, e.wait_flag,
                              e.wait_count, e.signal_flag, e.slots, e.pad)
    return bytes(out)


def parse(data: bytes) -> VMProgram:
    """Strict v3 parse with the validation the runtime applies (bounds,
    alignment, dtype and tile-op ranges, uniform top-level barrier counts,
    control sub-ranges inside the owning lane stream, no trailing bytes)."""
    data = bytes(data)
    if len(data) < HEADER.size:
        raise FormatError(f"truncated header ({len(data)} bytes)")
    (magic, version, n_buffers, n_instrs, n_consts, main_len, n_inputs,
     n_outputs, n_aux, hpad, arena_bytes) = HEADER.unpack_from(data, 0)
    if magic != MAGIC:
        raise FormatError(f"bad magic {magic:#010x}")
    if version != VERSION:
        raise FormatError(f"unsupported version {version} (want {VERSION})")
    if hpad != 0:
        raise FormatError("header pad nonzero")
    if main_len > n_instrs:
        raise FormatError("main_len > n_instrs")
    pos = HEADER.size

    def need(nbytes: int, what: str) -> None:
        if pos + nbytes > len(data):
            raise FormatError(f"truncated {what}")

    buffers = []
    need(BUFENT.size * n_buffers, "buffer table")
    for i in range(n_buffers):
        off, size, dt, pad = BUFENT.unpack_from(data, pos)
        pos += BUFENT.size
        if off % ARENA_ALIGN or off + size > arena_bytes:
            raise FormatError(f"buffer {i} outside arena / misaligned")
        if dt > DT_MAX:
            raise FormatError(f"buffer {i} unsupported dtype {dt}")
        if pad:
            raise FormatError(f"buffer {i} pad nonzero")
        buffers.append(Buffer(off, size, dt))

    def ids(count: int, what: str) -> list:
        nonlocal pos
        need(4 * count, what)
        v = list(struct.unpack_from(f"<{count}I", data, pos))
        pos += 4 * count
        pos += -pos % SECTION_ALIGN
        if any(i >= n_buffers for i in v):
            raise FormatError(f"bad {what} map")
        return v

    inputs = ids(n_inputs, "input")
    outputs = ids(n_outputs, "output")

    def shape() -> tuple:
        nonlocal pos
        need(8, "io shape")
        rank, pad = struct.unpack_from("<II", data, pos)
        pos += 8
        if rank > 16 or pad:
            raise FormatError("bad io shape entry")
        need(8 * rank, "io shape dims")
        dims = struct.unpack_from(f"<{rank}Q", data, pos)
        pos += 8 * rank
        return tuple(dims)

    input_shapes = [shape() for _ in range(n_inputs)]
    output_shapes = [shape() for _ in range(n_outputs)]

    need(4 * n_aux, "aux pool")
    aux = list(struct.unpack_from(f"<{n_aux}I", data, pos)) if n_aux else []
    pos += 4 * n_aux
    pos += -pos % SECTION_ALIGN

    consts = []
    for _ in range(n_consts):
        need(CONSTHDR.size, "const entry")
        bid, blen = CONSTHDR.unpack_from(data, pos)
        pos += CONSTHDR.size
        if bid >= n_buffers or blen > buffers[bid].size_bytes:
            raise FormatError("bad const entry")
        need(blen, "const data")
        consts.append((bid, data[pos:pos + blen]))
        pos += blen
        pos += -pos % SECTION_ALIGN

    instrs = []
    need(INSTR.size * n_instrs, "instructions")
    for i in range(n_instrs):
        op, dst, a, b, n, imm, aux_off, imm2 = INSTR.unpack_from(data, pos)
        pos += INSTR.size
        if op > OP_MAX:
            raise FormatError(f"instr {i}: unknown opcode {op}")
        if aux_off > n_aux:
            raise FormatError(f"instr {i}: aux offset out of range")
        if op in (OP_WHILE, OP_IF):
            if a + b > n_instrs or n + imm > n_instrs or dst >= n_buffers:
                raise FormatError(f"instr {i}: region out of range")
        elif op == OP_FOR:
            if n + imm > n_instrs:
                raise FormatError(f"instr {i}: FOR body out of range")
        instrs.append(Instr(op, dst, a, b, n, imm, aux_off, imm2))

    prog = VMProgram(arena_bytes, buffers, inputs, outputs, input_shapes,
                     output_shapes, consts, instrs, main_len, aux)
    if pos < len(data):
        prog.schedule, pos = _parse_schedule(data, pos, n_buffers, n_aux)
    if pos != len(data):
        raise FormatError(f"trailing bytes: parsed {pos} of {len(data)}")
    return prog


def _parse_schedule(data: bytes, pos: int, n_buffers: int, n_aux: int):
    if pos + SCHED_HDR.size > len(data):
        raise FormatError("truncated schedule header")
    n_tasks, n_entries, n_flags, n_lanes = SCHED_HDR.unpack_from(data, pos)
    pos += SCHED_HDR.size
    if not 1 <= n_lanes <= 4096:
        raise FormatError(f"bad n_lanes {n_lanes}")
    if pos + TASK.size * n_tasks + LANETAB.size * n_lanes + \
            ENTRY.size * n_entries != len(data):
        raise FormatError("schedule section size mismatch (truncated/trailing)")
    tasks = []
    for i in range(n_tasks):
        w = TASK.unpack_from(data, pos)
        pos += TASK.size
        top, dt, adt = w[0] & 0xFF, (w[0] >> 8) & 0xFF, (w[0] >> 16) & 0xFF
        if top > TOP_MAX:
            raise FormatError(f"task {i}: unknown tile_op {top}")
        if dt > DT_MAX or adt > DT_MAX:
            raise FormatError(f"task {i}: unknown dtype")
        if max(w[1], w[2], w[3]) >= n_buffers:
            raise FormatError(f"task {i}: buffer id out of range")
        tasks.append(Task(top, w[1], w[2], w[3], *w[4:], dtype=dt, adtype=adt))
    lanes = []
    for i in range(n_lanes):
        off, cnt, root, _ = LANETAB.unpack_from(data, pos)
        pos += LANETAB.size
        if off + cnt > n_entries or root > cnt:
            raise FormatError(f"lane {i}: bad stream range")
        lanes.append((off, cnt, root))
    entries = []
    for i in range(n_entries):
        e = Entry(*ENTRY.unpack_from(data, pos))
        pos += ENTRY.size
        if e.task not in CONTROL_SENTINELS and e.task >= n_tasks:
            raise FormatError(f"entry {i}: task index out of range")
        entries.append(e)
    streams = [entries[off:off + cnt] for off, cnt, _ in lanes]
    ref = None
    for lane, (stream, (_, cnt, _)) in enumerate(zip(streams, lanes)):
        nbar = 0
        for e in stream:
            if e.task == ENT_BARRIER:
                nbar += 1
            elif e.task in (ENT_WHILE, ENT_IF):
                if e.signal_flag >= n_buffers:
                    raise FormatError("control cond buffer out of range")
                if e.tile_lo + e.tile_hi > cnt or e.wait_flag + e.wait_count > cnt:
                    raise FormatError("control sub-range outside lane stream")
            elif e.task == ENT_FOR:
                if e.tile_lo + e.tile_hi > cnt:
                    raise FormatError("control sub-range outside lane stream")
        if ref is None:
            ref = nbar
        elif nbar != ref:
            raise FormatError("non-uniform barrier counts across lanes")
    sched = Schedule(n_lanes, tasks, streams, [r for _, _, r in lanes], n_flags)
    return sched, pos


def dtype_of(prog: VMProgram, buf_id: int) -> int:
    return prog.buffers[buf_id].dtype
