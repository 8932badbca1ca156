"""Tensor VMProgram -> v3 schedule sections (tasks + per-lane entry streams).

Contract with the device (reference: python/pjrt_ocl/scheduler.py:178-197,
312-433, 451-715; docs/vmprogram.md "v2.1"):

* one TASK per compute instruction; a task is cut into tiles whose count the
  kernel recomputes identically (``n_tiles``);
* lane streams hold ENTRIES ``(task, tile_lo, tile_hi)``; a global BARRIER is
  emitted only where a dependency crosses lanes -- two elementwise ops over the
  same element count chain on one lane (tile T of both stays on the lane that
  owns T), every other dependency needs a barrier;
* the tiles of each unit of a phase are split into contiguous chunks in
  proportion to the unit's share of the phase cost, then list-scheduled
  (longest first) onto the least-loaded lane;
* WHILE / FOR / IF become a uniform control entry in every lane; their
  sub-lists are scheduled after the root so they live at stream index
  >= root_len, and the kernel supplies the loop barriers.

The device parameters come from the runtime through the environment the plugin
gives the lowering subprocess: PJRT_OCL_NLANES, PJRT_OCL_EW_TS, PJRT_OCL_MMA_T,
PJRT_OCL_COST_TABLE, PJRT_OCL_FUSE (same variable names as the reference,
plugin.cc:770-780).
"""
from __future__ import annotations

import dataclasses
import json
import math
import os

from . import vmprogram as V

# --- device configuration -----------------------------------------------------

# Defaults for one MI355X when no environment is given: one lane per CU.
DEFAULT_NLANES = 256
DEFAULT_EW_TS = 4096
DEFAULT_MMA_T = 128

_COST_KEYS = {
    V.TOP_EW: "ew_tile_us", V.TOP_MMA: "mma_tile_us",
    V.TOP_GATHER: "gather_tile_us", V.TOP_GATHER_INDEX: "gather_tile_us",
    V.TOP_RED_PART: "reduce_tile_us", V.TOP_RED_COMB: "reduce_tile_us",
}
# terms of the phase work model a measured cost table may set (vmrt_calibrate)
_MODEL_KEYS = ("tile_us", "lane_gbs", "lane_mma_tflops", "barrier_us", "barrier_us_per_lane")


def load_cost_table(spec: str) -> dict:
    """A cost table from PJRT_OCL_COST_TABLE: a JSON file path (the reference's
    form, runtime.cc:2500-2515) or the JSON object itself; unknown keys and
    unreadable tables are ignored (unit costs then)."""
    try:
        if spec.lstrip().startswith("{"):
            raw = json.loads(spec)
        else:
            with open(spec) as f:
                raw = json.load(f)
        keys = set(_COST_KEYS.values()) | set(_MODEL_KEYS)
        return {k: float(raw[k]) for k in keys if k in raw and float(raw[k]) > 0}
    except (OSError, ValueError, TypeError):
        return {}


class ScheduleError(NotImplementedError):
    """Program valid but outside the scheduler's coverage (service exit 2)."""


@dataclasses.dataclass
class DeviceConfig:
    nlanes: int = DEFAULT_NLANES
    ew_ts: int = DEFAULT_EW_TS
    mma_t: int = DEFAULT_MMA_T
    costs: dict = dataclasses.field(default_factory=dict)
    fuse: bool = True
    # Per-task MMA tile selection (extension): pick the largest tile edge that
    # still gives every lane work; False keeps every MMA at the default edge.
    mma_autotile: bool = True
    # Matmuls whose tiles leave most lanes idle split K over more lanes
    # (extension; ``mma_split_log2``).
    mma_splitk: bool = True
    # Matmuls of at most 8 rows as column-strip TOP_GEMV tasks (extension), and
    # the narrowest strip width they may use.
    gemv: bool = True
    gemv_min_strip: int = 0          # 0: by lane count (gemv_strip_floor)
    # A layernorm whose only reader is a TOP_GEMV runs inside that GEMV's x
    # staging (extension; saves the phase between them).
    ln_gemv: bool = True
    # Phases that leave lanes idle keep lane 0, the grid barrier's master, idle
    # too, so it polls the arrivals while the others compute.
    idle_master: bool | None = None  # None: by lane count (master_idle)
    # A program may run on half the lanes when the work model below says the
    # saved per-phase overhead outweighs the halved bandwidth (extension).
    fit_lanes: bool = True
    # A decode attention whose q, k and v come from TOP_GEMV strips of the
    # phase before it joins that phase: its tiles wait for completion flags
    # that the strips of their head signal, instead of a grid barrier
    # (extension of the entries' WAIT / SIGNAL fields; ``_flag_edges``).
    counters: bool = True
    # A streaming layernorm's lanes take rows nlanes apart (``row_interleave``).
    ln_interleave: bool = True

    @classmethod
    def from_env(cls, environ=None) -> "DeviceConfig":
        env = os.environ if environ is None else environ

        def geti(name, default):
            try:
                v = int(env.get(name, "") or default)
            except ValueError:
                v = default
            return v

        spec = env.get("PJRT_OCL_COST_TABLE", "")
        costs = load_cost_table(spec) if spec else {}
        return cls(nlanes=max(1, min(4096, geti("PJRT_OCL_NLANES", DEFAULT_NLANES))),
                   ew_ts=max(64, geti("PJRT_OCL_EW_TS", DEFAULT_EW_TS)),
                   mma_t=geti("PJRT_OCL_MMA_T", DEFAULT_MMA_T),
                   costs=costs,
                   fuse=env.get("PJRT_OCL_FUSE", "1") != "0",
                   mma_autotile=env.get("PJRT_AMD_MMA_AUTOTILE", "1") != "0",
                   mma_splitk=env.get("PJRT_AMD_MMA_SPLITK", "1") != "0",
                   gemv=env.get("PJRT_AMD_GEMV", "1") != "0",
                   gemv_min_strip=max(0, min(256, geti("PJRT_AMD_GEMV_STRIP", 0))),
                   ln_gemv=env.get("PJRT_AMD_LN_GEMV", "1") != "0",
                   idle_master=(env["PJRT_AMD_IDLE_MASTER"] != "0") if env.get("PJRT_AMD_IDLE_MASTER") else None,
                   fit_lanes=env.get("PJRT_AMD_FIT_LANES", "1") != "0",
                   counters=env.get("PJRT_AMD_COUNTERS", "1") != "0",
                   ln_interleave=env.get("PJRT_AMD_LN_INTERLEAVE", "1") != "0")


# --- instruction -> task ------------------------------------------------------

_BIN_SUB = {
    V.OP_ADD_F32: V.SUB_ADD, V.OP_MUL_F32: V.SUB_MUL, V.OP_SUB_F32: V.SUB_SUB,
    V.OP_DIV_F32: V.SUB_DIV, V.OP_MAX_F32: V.SUB_MAX, V.OP_MIN_F32: V.SUB_MIN,
    V.OP_POW_F32: V.SUB_POW, V.OP_ATAN2_F32: V.SUB_ATAN2,
    V.OP_REMAINDER_F32: V.SUB_REMAINDER, V.OP_AND: V.SUB_AND,
    V.OP_OR: V.SUB_OR, V.OP_XOR: V.SUB_XOR, V.OP_SHL: V.SUB_SHL,
    V.OP_SHR_L: V.SUB_SHR_L, V.OP_SHR_A: V.SUB_SHR_A,
}
_UN_SUB = {
    V.OP_COPY_F32: V.SUB_COPY, V.OP_NEG_F32: V.SUB_NEG, V.OP_EXP_F32: V.SUB_EXP,
    V.OP_LOG_F32: V.SUB_LOG, V.OP_SQRT_F32: V.SUB_SQRT,
    V.OP_RSQRT_F32: V.SUB_RSQRT, V.OP_TANH_F32: V.SUB_TANH,
    V.OP_ABS_F32: V.SUB_ABS, V.OP_FLOOR_F32: V.SUB_FLOOR,
    V.OP_CEIL_F32: V.SUB_CEIL, V.OP_SIGN_F32: V.SUB_SIGN,
    V.OP_LOG1P_F32: V.SUB_LOG1P, V.OP_EXPM1_F32: V.SUB_EXPM1,
    V.OP_CBRT_F32: V.SUB_CBRT, V.OP_SIN_F32: V.SUB_SIN, V.OP_COS_F32: V.SUB_COS,
    V.OP_TAN_F32: V.SUB_TAN, V.OP_ROUND_NEAREST_EVEN_F32: V.SUB_RINT,
    V.OP_ROUND_NEAREST_AFZ_F32: V.SUB_ROUND, V.OP_NOT: V.SUB_NOT,
    V.OP_GELU: V.SUB_GELU,
}


def red_chunk(n: int, ew_ts: int) -> int:
    """Elements per REDUCE_PART tile (ops/reduce.py:81-87): at least one EW tile
    and at most 256 partials."""
    if n <= 0:
        return 1
    return max(ew_ts, math.ceil(n / 256))


def mma_tile_edge(task: V.Task, cfg: DeviceConfig) -> int:
    code = (task.p3 >> 24) & 0xF
    return V.MMA_CODE_TILE.get(code, cfg.mma_t)


def n_tiles(task: V.Task, cfg: DeviceConfig) -> int:
    """Tile count of a task; the kernel decodes tile indices the same way."""
    top = task.tile_op
    if top in (V.TOP_EW, V.TOP_GATHER, V.TOP_IOTA_DIM, V.TOP_SCATTER,
               V.TOP_DYN_GATHER, V.TOP_DYN_SCATTER, V.TOP_RED_WINDOW,
               V.TOP_MAP_REGION, V.TOP_GATHER_INDEX, V.TOP_CONV,
               V.TOP_SCATTER_INDEX):
        return max(1, math.ceil(task.p1 / cfg.ew_ts))
    if top == V.TOP_RED_STRIDED:
        return max(1, math.ceil(task.p0 / cfg.ew_ts))
    if top == V.TOP_MMA:
        t = mma_tile_edge(task, cfg)
        g = max(1, task.p3 & 0xFFFFFF)
        return math.ceil(task.p0 / t) * math.ceil(task.p1 / t) * g << (task.p3 >> V.MMA_SPLIT_SHIFT)
    if top == V.TOP_RED_PART:
        return max(1, math.ceil(task.p0 / task.p1)) if task.p1 else 1
    if top == V.TOP_RED_COMB:
        return 1
    if top in (V.TOP_RED_SEG, V.TOP_SOFTMAX_SEG, V.TOP_LAYERNORM_SEG):
        return max(1, task.p0)
    if top == V.TOP_ARGMAX_SEG:
        return max(1, task.p0) * max(1, task.p3)
    if top == V.TOP_FLASH_ATTN:
        return max(1, task.p1 * attn_rows_padded(task.p2))
    if top == V.TOP_GEMV:
        return max(1, task.p3) * -(-task.p1 // task.p4)
    if top == V.TOP_DECODE_ATTN:
        return max(1, (task.p4 & 0xFFFF) * max(1, task.p4 >> 16))
    raise ScheduleError(f"n_tiles: unknown tile_op {top}")


# Flash attention tiles: one per query row, each head's rows padded to whole
# 256-row blocks (the matrix-core kernel's block), so that chunks of whole blocks
# never split one between lanes; tiles past a head's T are empty.
ATTN_BLOCK_ROWS = 256


def attn_rows_padded(T: int) -> int:
    return -(-T // ATTN_BLOCK_ROWS) * ATTN_BLOCK_ROWS


# --- skinny matmuls (TOP_GEMV) ------------------------------------------------------

GEMV_MAX_M = 8
GEMV_LDS_FLOATS = 147456 // 4   # the kernel's LDS: x rows + row-phase sums
_EPI_INLINE = {V.SUB_AFFINE, V.SUB_GELU, V.SUB_COPY, V.SUB_ADD, V.SUB_MUL, V.SUB_SUB, V.SUB_DIV,
               V.SUB_MAX, V.SUB_MIN}


# Defaults that depend on the lane count, measured on the decode loop (C5,
# alternating runs): on 256 lanes 8-column strips and an idle lane 0 were
# faster (1035 -> 1042 and 1006 -> 1015 tokens/s); on 128 lanes 16-column
# strips with lane 0 taking tiles are (1178 -> 1197).
def gemv_strip_floor(cfg) -> int:
    """Narrowest GEMV strip the scheduler may use."""
    if cfg.gemv_min_strip:
        return max(8, cfg.gemv_min_strip)
    return 8 if cfg.nlanes > 128 else 16


def master_idle(cfg) -> bool:
    """Whether phases that leave lanes idle keep lane 0 idle too."""
    return cfg.idle_master if cfg.idle_master is not None else cfg.nlanes > 128


def gemv_strip(N: int, G: int, nlanes: int, min_strip: int = 8) -> int:
    """Columns per TOP_GEMV tile: the narrowest strip (min_strip, ... 256, powers
    of two) that gives no lane a second tile.  A tile's time is latency, not
    bytes: measured on MI355X with K = 768, a strip width that gave lanes two
    tiles cost a whole tile (N = 2304: 9.2 against 15.3 us per one-phase
    launch), and the 32000-column LM head takes 128 (16.4 against 21.0 us at
    64).  Within one tile per lane the narrowest strip wins in the decoder
    (C5, strips XCD-grouped: 1042 against 1035 tokens/s with 8 against 16
    columns for N = 768)."""
    cw = 8
    while cw < min_strip:
        cw *= 2
    while cw < 256 and G * -(-N // cw) > nlanes:
        cw *= 2
    return cw


def gemv_eligible(M, N, K, G, aview, bview, epi, adt, dt, prog) -> bool:
    if not (1 <= M <= GEMV_MAX_M and N % 8 == 0 and N >= 8 and K >= 1) or aview or bview:
        return False
    if (M * K + 3) // 4 * 4 + 4096 * M > GEMV_LDS_FLOATS:
        return False
    if adt not in (V.DT_BF16, V.DT_F16, V.DT_F32) or dt not in (V.DT_F32, V.DT_BF16, V.DT_F16):
        return False
    if epi:
        nm = prog.aux[epi - 1]
        if any(prog.aux[epi + 4 * k] not in _EPI_INLINE for k in range(nm)):
            return False
    return True


def row_interleave(n_rows: int, cfg: DeviceConfig) -> int:
    """LAYERNORM_SEG p5 (extension): with n_rows a multiple of the lane count,
    logical row i is row (i % c) * (n_rows / c) + i / c for c = n_rows / nlanes,
    so each lane's contiguous chunk of logical rows is a stride-nlanes set of
    real rows and the lanes stream neighbouring rows together (C2, alternating
    runs on one MI355X: 38.7 against 39.6 us).  0: rows as they are."""
    if not cfg.ln_interleave or cfg.nlanes <= 1 or n_rows < 2 * cfg.nlanes or n_rows % cfg.nlanes:
        return 0
    return n_rows // cfg.nlanes


def argmax_splits(n_out: int, seg: int, cfg: DeviceConfig) -> int:
    """Splits per row of an argmax (p3): rows of 8192 elements or more are cut
    into runs of about 4096 on separate CUs (one 32000-element row took ~21 us
    on one CU), as long as every split has a lane."""
    if seg < 8192 or n_out <= 0:
        return 1
    return max(1, min(-(-seg // 4096), cfg.nlanes // n_out, 256))


def decode_splits(H: int, C: int, cfg: DeviceConfig) -> int:
    """Key splits per head of a decode attention: one per 64 cache keys (the
    tile kernel's register window), whatever the lane count.  A split's reads
    are all issued before its first wait, so a tile costs about one memory
    round trip; one CU streaming a 640-key head took ~19 us."""
    return max(1, -(-C // 64))


def _dot_fields(ins: V.Instr, prog: V.VMProgram):
    """(M, N, K, G, aview, bview, epi, epi_res) of an OP_DOT, the view /
    epilogue fields taken from the in-memory instruction or its aux mirror."""
    M, N, K, G = ins.n, ins.imm >> 16, ins.imm & 0xFFFF, max(1, ins.imm2)
    aview, bview, epi, epi_res = ins.aview, ins.bview, ins.epi, ins.epi_res
    if ins.aux and not (aview or bview or epi):
        aview, bview, epi, epi_res = prog.aux[ins.aux:ins.aux + 4]
    return M, N, K, G, aview, bview, epi, epi_res


def _gemv_form(ins: V.Instr, prog: V.VMProgram, cfg: DeviceConfig) -> bool:
    """An OP_DOT the scheduler maps to TOP_GEMV."""
    M, N, K, G, aview, bview, epi, _ = _dot_fields(ins, prog)
    if N == 1 and G == 1 and not aview and not bview and not epi:
        return False                     # the reference's dot-mode segmented reduce
    bufs = prog.buffers
    return cfg.gemv and gemv_eligible(M, N, K, G, aview, bview, epi, bufs[ins.a].dtype,
                                      bufs[ins.dst].dtype, prog)


def _instr_lists(prog: V.VMProgram):
    """Every instruction list of the program: the root list and each region's
    sub-lists, as index ranges."""
    out, todo = [], [range(prog.main_len)]
    while todo:
        r = todo.pop()
        out.append(r)
        for i in r:
            ins = prog.instrs[i]
            if ins.op == V.OP_FOR:
                todo.append(range(ins.n, ins.n + ins.imm))
            elif ins.op in (V.OP_WHILE, V.OP_IF):
                todo += [range(ins.a, ins.a + ins.b), range(ins.n, ins.n + ins.imm)]
    return out


def ln_gemv_pairs(prog: V.VMProgram, cfg: DeviceConfig) -> dict:
    """{dot index: layernorm index} for each OP_LAYERNORM_AFFINE whose result is
    read by exactly one instruction, an OP_DOT mapped to TOP_GEMV with M = the
    layernorm's rows and K = its row length, later in the same instruction list
    with no write to the layernorm's inputs and no region in between.  The GEMV
    then normalises x while staging it (task p5 = layernorm task + 1) and the
    layernorm gets no tile of its own; its result buffer is never written."""
    if not cfg.ln_gemv:
        return {}
    grp = overlap_groups(prog)
    gsize: dict = {}
    for g in grp:
        gsize[g] = gsize.get(g, 0) + 1
    readers: dict = {}
    writers: dict = {}
    for i, ins in enumerate(prog.instrs):
        if ins.op in V.REGION_OPS or ins.op == V.OP_NOP:
            continue
        for b in instr_reads(ins, prog):
            readers.setdefault(b, []).append(i)
        for b in instr_writes(ins, prog):
            writers.setdefault(b, []).append(i)
    io = set(prog.inputs) | set(prog.outputs)
    pairs = {}
    for lst in _instr_lists(prog):
        idx = list(lst)
        for p, i in enumerate(idx):
            ln = prog.instrs[i]
            if ln.op != V.OP_LAYERNORM_AFFINE:
                continue
            h = ln.dst
            gh = grp[h] if h < len(grp) else h
            if h in io or gsize.get(gh, 1) != 1 or writers.get(gh, []) != [i]:
                continue
            rd = readers.get(gh, [])
            if len(rd) != 1 or rd[0] not in lst:
                continue
            j = rd[0]
            dot = prog.instrs[j]
            if dot.op != V.OP_DOT or dot.a != h or j < i or not _gemv_form(dot, prog, cfg):
                continue
            M, N, K, G, aview, _, _, _ = _dot_fields(dot, prog)
            if G != 1 or aview or M != ln.n or K != ln.imm:
                continue
            ins_reads = instr_reads(ln, prog)
            between = idx[p + 1:idx.index(j)]
            if any(prog.instrs[k].op in V.REGION_OPS or instr_writes(prog.instrs[k], prog) & ins_reads
                   for k in between):
                continue
            pairs[j] = i
    return pairs


def instr_to_task(ins: V.Instr, prog: V.VMProgram, cfg: DeviceConfig) -> V.Task:
    """One compute instruction -> its task (field meanings: the task table of
    docs/vmprogram.md and each reference ops/*.py ``*_to_task``)."""
    op = ins.op
    bufs = prog.buffers
    if op in _BIN_SUB:
        t = V.Task(V.TOP_EW, ins.dst, ins.a, ins.b, _BIN_SUB[op], ins.n,
                   ins.imm, ins.imm2)
    elif op in _UN_SUB:
        t = V.Task(V.TOP_EW, ins.dst, ins.a, ins.a, _UN_SUB[op], ins.n,
                   ins.imm, 0)
    elif op == V.OP_FILL_F32:
        t = V.Task(V.TOP_EW, ins.dst, ins.dst, ins.dst, V.SUB_FILL, ins.n, ins.imm)
    elif op == V.OP_IOTA_F32:
        t = V.Task(V.TOP_EW, ins.dst, ins.dst, ins.dst, V.SUB_IOTA_FLAT, ins.n)
    elif op == V.OP_LTS_F32:
        t = V.Task(V.TOP_EW, ins.dst, ins.a, ins.b, V.SUB_LTS, 1)
    elif op == V.OP_CMP_F32:
        t = V.Task(V.TOP_EW, ins.dst, ins.a, ins.b, V.SUB_CMP, ins.n, ins.imm)
    elif op == V.OP_SELECT_F32:
        t = V.Task(V.TOP_EW, ins.dst, ins.a, ins.b, V.SUB_SELECT, ins.n, 0, ins.imm)
    elif op == V.OP_CONVERT:
        t = V.Task(V.TOP_EW, ins.dst, ins.a, ins.a, V.SUB_CONVERT, ins.n)
    elif op == V.OP_BITCAST:
        t = V.Task(V.TOP_EW, ins.dst, ins.a, ins.a, V.SUB_BITCAST, ins.n)
    elif op == V.OP_IS_FINITE:
        t = V.Task(V.TOP_EW, ins.dst, ins.a, ins.a, V.SUB_ISFINITE, ins.n)
    elif op == V.OP_AFFINE_F32:
        t = V.Task(V.TOP_EW, ins.dst, ins.a, ins.a, V.SUB_AFFINE, ins.n,
                   ins.imm, ins.imm2)
    elif op == V.OP_GATHER_STRIDED:
        t = V.Task(V.TOP_GATHER, ins.dst, ins.a, ins.a, ins.aux, ins.n)
    elif op == V.OP_IOTA_DIM:
        t = V.Task(V.TOP_IOTA_DIM, ins.dst, ins.dst, ins.dst, ins.aux, ins.n)
    elif op == V.OP_SCATTER:
        t = V.Task(V.TOP_SCATTER, ins.dst, ins.a, ins.a, ins.aux, ins.n)
    elif op == V.OP_DYNAMIC_SLICE:
        t = V.Task(V.TOP_DYN_GATHER, ins.dst, ins.a, ins.a, ins.aux, ins.n)
    elif op == V.OP_DYNAMIC_UPDATE_SLICE:
        t = V.Task(V.TOP_DYN_SCATTER, ins.dst, ins.a, ins.a, ins.aux, ins.n)
    elif op == V.OP_GATHER_INDEX:
        t = V.Task(V.TOP_GATHER_INDEX, ins.dst, ins.a, ins.a, ins.aux, ins.n)
    elif op == V.OP_REDUCE:
        phase, kind = (ins.imm >> 3) & 1, ins.imm & 7
        if phase == 0:
            t = V.Task(V.TOP_RED_PART, ins.dst, ins.a, ins.a, ins.n,
                       red_chunk(ins.n, cfg.ew_ts), kind)
        else:
            t = V.Task(V.TOP_RED_COMB, ins.dst, ins.a, ins.a, ins.n, kind)
    elif op == V.OP_REDUCE_SEG:
        t = V.Task(V.TOP_RED_SEG, ins.dst, ins.a, ins.a, ins.n,
                   ins.imm & 0x0FFFFFFF, ins.imm >> 28)
    elif op == V.OP_REDUCE_STRIDED:
        t = V.Task(V.TOP_RED_STRIDED, ins.dst, ins.a, ins.a, ins.n,
                   ins.imm & 0x0FFFFFFF, ins.imm2, ins.imm >> 28)
    elif op == V.OP_SOFTMAX:
        t = V.Task(V.TOP_SOFTMAX_SEG, ins.dst, ins.a, ins.a, ins.n, ins.imm)
    elif op == V.OP_LAYERNORM:
        t = V.Task(V.TOP_LAYERNORM_SEG, ins.dst, ins.a, ins.a, ins.n, ins.imm,
                   ins.imm2, 0, 0, row_interleave(ins.n, cfg))
    elif op == V.OP_LAYERNORM_AFFINE:
        # aux -> [flags, beta buffer id]; gamma rides in b.
        flags, beta = prog.aux[ins.aux], prog.aux[ins.aux + 1]
        t = V.Task(V.TOP_LAYERNORM_SEG, ins.dst, ins.a,
                   ins.b if flags & V.LN_AFFINE else ins.a, ins.n, ins.imm,
                   ins.imm2, flags, beta if flags & V.LN_AFFINE else ins.a,
                   row_interleave(ins.n, cfg))
    elif op == V.OP_ARGMAX_SEG:
        # dst = index output, b = value output (may alias a scratch), p2 = kind
        t = V.Task(V.TOP_ARGMAX_SEG, ins.dst, ins.a, ins.b, ins.n, ins.imm,
                   ins.imm2, argmax_splits(ins.n, ins.imm, cfg))
    elif op == V.OP_MAP_REGION:
        inp = list(ins.region_inputs) or _region_inputs_from_aux(ins, prog)
        f = [inp[k] if k < len(inp) else inp[0] for k in range(8)]
        t = V.Task(V.TOP_MAP_REGION, ins.dst, f[0], f[1], ins.aux, ins.n,
                   f[2], f[3], f[4], f[5], f[6], f[7])
    elif op == V.OP_FLASH_ATTN:
        t = V.Task(V.TOP_FLASH_ATTN, ins.dst, ins.a, ins.b, ins.imm2, ins.n,
                   ins.imm, ins.aux)
    elif op == V.OP_DECODE_ATTN:
        hd, kb, vb, posb, sbits = prog.aux[ins.aux:ins.aux + 5]
        S = decode_splits(ins.n, ins.imm, cfg)
        t = V.Task(V.TOP_DECODE_ATTN, ins.dst, ins.a, ins.b, ins.imm2, kb, vb,
                   posb, ins.n | (S << 16), hd, ins.imm, sbits)
    elif op == V.OP_DOT:
        M, N, K, G = ins.n, ins.imm >> 16, ins.imm & 0xFFFF, max(1, ins.imm2)
        aview, bview, epi, epi_res = ins.aview, ins.bview, ins.epi, ins.epi_res
        if ins.aux and not (aview or bview or epi):
            aview, bview, epi, epi_res = prog.aux[ins.aux:ins.aux + 4]
        adt, dt = bufs[ins.a].dtype, bufs[ins.dst].dtype
        if N == 1 and G == 1 and not aview and not bview and not epi:
            # GEMV: one matrix row per tile through the segmented reduce in dot
            # mode (ops/dot.py:166-183).
            t = V.Task(V.TOP_RED_SEG, ins.dst, ins.a, ins.b, M, K, 0, 1)
        elif _gemv_form(ins, prog, cfg):
            t = V.Task(V.TOP_GEMV, ins.dst, ins.a, ins.b, M, N, K, G,
                       gemv_strip(N, G, cfg.nlanes, gemv_strip_floor(cfg)), 0, epi,
                       epi_res if epi else 0)
        else:
            code = V.MMA_TILE_CODES.get(ins.mma_tile, 0)
            if not code and cfg.mma_autotile:
                code = V.MMA_TILE_CODES[_auto_mma_tile(M, N, G, cfg, adt, K, bool(aview or bview))]
            edge = V.MMA_CODE_TILE.get(code, cfg.mma_t)
            split = mma_split_log2(M, N, K, G, edge, adt, cfg)
            t = V.Task(V.TOP_MMA, ins.dst, ins.a, ins.b, M, N, K,
                       G | (code << 24) | (split << V.MMA_SPLIT_SHIFT), aview, bview, epi,
                       epi_res if epi else 0)
    else:
        raise ScheduleError(f"scheduler: no task mapping for opcode {op}")
    t.dtype = bufs[ins.dst].dtype
    t.adtype = bufs[ins.a].dtype if ins.a < len(bufs) else t.dtype
    return t


def _auto_mma_tile(M: int, N: int, G: int, cfg: DeviceConfig, adt: int = V.DT_F32, K: int = 0,
                   views: bool = False) -> int:
    """Largest output tile edge whose tile count still covers the lanes (big
    tiles raise MFMA arithmetic intensity; small matmuls need the parallelism).
    A 16-bit matmul the 256-wide fast tile takes (no operand view; K and N
    multiples of 8) keeps 256 down to an eighth of the lanes: measured on MI355X,
    bf16 1536^3 0.045 ms against 0.113 with the general tile the count rule picks,
    3072^3 0.073 against 0.248, 2048^3 0.054 against 0.068; at 1024^3 (16 tiles)
    the general tiles win, 0.030 against 0.034.  A long K (>= 4096) with at most
    a sixth of the lanes' worth of 256-wide tiles takes 128-wide tiles instead,
    which the K split then spreads over the lanes (one 256 x 256 x 4096 tile is
    ~90 us of one CU's matrix cores): bf16 256x4096x4096 0.058 ms against 0.095,
    512x2048x4096 0.058 against 0.095, 128x4096x4096 0.051 against 0.059,
    512x4096x4096 0.079 against 0.088, 512x4096x11008 0.154 against 0.207; with
    48 or more 256-wide tiles (768x4096x4096, 384x8192x4096) or K <= 3072 the
    rules above win.  Where the 64-wide tiles fit the lanes in one round they
    take it (their 128-deep K slabs and transposed B reads): 256x4096x4096
    0.042 ms against 0.053 with 128, 128x4096x4096 0.036 against 0.049; with
    more than a round of them (512x4096x11008) 128 stays ahead, 0.125 against
    0.186."""
    t256 = math.ceil(M / 256) * math.ceil(N / 256) * G
    fast16 = adt in (V.DT_BF16, V.DT_F16) and not views and K >= 8 and K % 8 == 0 and N % 8 == 0
    if fast16 and K >= 4096 and t256 * 6 < cfg.nlanes:
        return 64 if math.ceil(M / 64) * math.ceil(N / 64) * G <= cfg.nlanes else 128
    if fast16 and t256 * 8 >= cfg.nlanes:
        return 256
    for t in (256, 128, 64):
        if math.ceil(M / t) * math.ceil(N / t) * G >= cfg.nlanes:
            return t
    return 64


def mma_split_log2(M: int, N: int, K: int, G: int, edge: int, adt: int, cfg: DeviceConfig) -> int:
    """log2 of the K split of a matmul (extension; 0 = none).  A matmul whose
    output tiles leave at least half the lanes idle and whose K spans at least
    four slabs of the general tile (16 f32 or 32 16-bit k) is cut along K into S
    splits: the largest power of two, at most 32, that keeps every split at two
    slabs or more and the split tiles within the lanes.  Each split's tile waits
    on its own loads only once per slab, so the loads of a deep, narrow product
    (config 1's [256, 512] x [512, 64]: four 64 x 64 tiles) no longer run one
    slab after another on a few lanes.  256-wide tiles are never split (they
    cover large outputs, and their combine would hold 64 float4 per thread)."""
    if not cfg.mma_splitk:
        return 0
    tiles = math.ceil(M / edge) * math.ceil(N / edge) * max(1, G)
    slab = 16 if adt == V.DT_F32 else 32
    if tiles * 2 > cfg.nlanes or K < 4 * slab:
        return 0
    if edge == 256:
        return 0
    lg = 0
    while (lg < V.MMA_MAX_SPLIT_LOG2 and tiles << (lg + 1) <= cfg.nlanes
           and math.ceil(K / (1 << (lg + 1))) >= 2 * slab):
        lg += 1
    return lg


def _region_inputs_from_aux(ins: V.Instr, prog: V.VMProgram) -> list:
    desc = ins.aux
    n_in, n_micro = prog.aux[desc], prog.aux[desc + 2]
    tail = desc + 3 + n_in + 6 * n_micro
    return [prog.aux[tail + k] for k in range(n_in)]


def overlap_groups(prog: V.VMProgram) -> list:
    """Buffer id -> the lowest id of its group of arena-overlapping buffers, so
    that accesses to aliasing buffers (a contiguous slice kept as a buffer of its
    own) are ordered like accesses to one buffer.  A program whose arena was
    packed by liveness carries the groups of its layout before packing
    (``alias_groups``): buffers the packing placed on the same bytes are
    separated by a grid barrier by construction, not ordered as one buffer."""
    bufs = prog.buffers
    alias = getattr(prog, "alias_groups", None)
    if alias is not None and len(alias) == len(bufs):
        return alias
    cached = getattr(prog, "_overlap_groups", None)
    if cached is not None and len(cached) == len(bufs):
        return cached
    group = list(range(len(bufs)))
    members, end = [], -1
    for i in sorted(range(len(bufs)), key=lambda k: (bufs[k].arena_byte_offset, k)):
        b = bufs[i]
        if b.size_bytes <= 0:
            continue
        if members and b.arena_byte_offset < end:
            members.append(i)
            end = max(end, b.arena_byte_offset + b.size_bytes)
        else:
            if len(members) > 1:
                root = min(members)
                for m in members:
                    group[m] = root
            members, end = [i], b.arena_byte_offset + b.size_bytes
    if len(members) > 1:
        root = min(members)
        for m in members:
            group[m] = root
    try:
        prog._overlap_groups = group
    except AttributeError:
        pass
    return group


def instr_reads(ins: V.Instr, prog: V.VMProgram) -> set:
    grp = overlap_groups(prog)
    return {grp[b] if 0 <= b < len(grp) else b for b in _instr_reads(ins, prog)}


def instr_writes(ins: V.Instr, prog: V.VMProgram) -> set:
    grp = overlap_groups(prog)
    return {grp[b] if 0 <= b < len(grp) else b for b in _instr_writes(ins, prog)}


def _instr_reads(ins: V.Instr, prog: V.VMProgram) -> set:
    op = ins.op
    if op in (V.OP_NOP, V.OP_FILL_F32, V.OP_IOTA_F32, V.OP_IOTA_DIM):
        return set()
    if op in _UN_SUB or op in (V.OP_CONVERT, V.OP_BITCAST, V.OP_IS_FINITE,
                               V.OP_AFFINE_F32, V.OP_GATHER_STRIDED,
                               V.OP_REDUCE, V.OP_REDUCE_SEG,
                               V.OP_REDUCE_STRIDED, V.OP_SOFTMAX,
                               V.OP_LAYERNORM, V.OP_SCATTER):
        r = {ins.a}
    elif op == V.OP_SELECT_F32:
        r = {ins.a, ins.b, ins.imm}
    elif op == V.OP_LAYERNORM_AFFINE:
        flags = prog.aux[ins.aux]
        r = {ins.a} | ({ins.b, prog.aux[ins.aux + 1]} if flags & V.LN_AFFINE else set())
    elif op == V.OP_ARGMAX_SEG:
        r = {ins.a}
    elif op == V.OP_FLASH_ATTN:
        r = {ins.a, ins.b, ins.imm2}
    elif op == V.OP_DECODE_ATTN:
        r = {ins.a, ins.b, ins.imm2} | set(prog.aux[ins.aux + 1:ins.aux + 4])
    elif op == V.OP_MAP_REGION:
        r = set(ins.region_inputs or _region_inputs_from_aux(ins, prog))
    elif op in (V.OP_DYNAMIC_SLICE, V.OP_DYNAMIC_UPDATE_SLICE, V.OP_GATHER_INDEX):
        r = {ins.a}
    elif op == V.OP_DOT:
        r = {ins.a, ins.b}
        epi, epi_res = ins.epi, ins.epi_res
        if ins.aux and not (ins.aview or ins.bview or ins.epi):
            epi, epi_res = prog.aux[ins.aux + 2], prog.aux[ins.aux + 3]
        # the residual / bias is read when a micro-op takes it as its source
        # (buffer 0 is a valid residual: the test is the epilogue's, not the id)
        if epi and any(prog.aux[epi + 1 + 4 * k] in (1, 2) for k in range(prog.aux[epi - 1])):
            r.add(epi_res)
    else:
        r = {ins.a, ins.b}
    if op in (V.OP_SCATTER, V.OP_DYNAMIC_UPDATE_SLICE):
        r.add(ins.dst)        # partial writes keep the rest of dst
    return r | set(ins.reads_hint)


def _instr_writes(ins: V.Instr, prog: V.VMProgram) -> set:
    if ins.op == V.OP_NOP:
        return set()
    if ins.op == V.OP_ARGMAX_SEG:
        return {ins.dst, ins.b}
    return {ins.dst}


# --- cost model ----------------------------------------------------------------

_HBM_GBS = 5000.0          # effective GB/s assumed before calibration
_MFMA_TFLOPS = 1200.0


def task_cost(task: V.Task, cfg: DeviceConfig, prog: V.VMProgram) -> float:
    """Estimated microseconds for the whole task (calibrated per-tile costs
    override the analytic model when a cost table is present)."""
    tiles = n_tiles(task, cfg)
    key = _COST_KEYS.get(task.tile_op)
    if key and key in cfg.costs:
        return tiles * cfg.costs[key]
    dsz = V.DT_SIZE.get(task.dtype, 4)
    asz = V.DT_SIZE.get(task.adtype, 4)
    top = task.tile_op
    if top == V.TOP_MMA:
        M, N, K, G = task.p0, task.p1, task.p2, max(1, task.p3 & 0xFFFFFF)
        flops = 2.0 * M * N * K * G
        byts = (M * K + K * N) * G * asz + M * N * G * dsz
        return max(flops / (_MFMA_TFLOPS * 1e6), byts / (_HBM_GBS * 1e3)) + 1.0
    if top == V.TOP_GEMV:
        M, N, K, G = task.p0, task.p1, task.p2, max(1, task.p3)
        return (K * N * asz + M * N * dsz) * G / (_HBM_GBS * 1e3) + 2.0
    if top == V.TOP_FLASH_ATTN:
        H, T = task.p1, task.p2
        hd = prog.aux[task.p3 + 3] if task.p3 + 3 < len(prog.aux) else 128
        C = prog.aux[task.p3 + 2] if task.p3 + 2 < len(prog.aux) else T
        return 4.0 * H * T * C * hd / (_MFMA_TFLOPS * 1e6) + 1.0
    if top == V.TOP_DECODE_ATTN:
        # each tile streams its share of a head's two cache slices (~15 GB/s per CU)
        H, S = task.p4 & 0xFFFF, max(1, task.p4 >> 16)
        return H * S * (2.0 * (task.p5 & 0xFFFF) * task.p6 * asz / S / 15e3 + 3.0)
    if top in (V.TOP_RED_SEG, V.TOP_SOFTMAX_SEG, V.TOP_LAYERNORM_SEG,
               V.TOP_ARGMAX_SEG):
        n = task.p0 * task.p1
        return n * (asz + (dsz if top != V.TOP_RED_SEG else 0)) / (_HBM_GBS * 1e3) + 0.5
    n = max(task.p0, task.p1) if top != V.TOP_EW else task.p1
    return n * (asz * 2 + dsz) / (_HBM_GBS * 1e3) + 0.3


# Work model of lane_fit: chip rates split evenly over 256 CUs, one tile's
# latency, and the grid barrier's cost (base + per lane).
_LANE_GBS = 8000.0 / 256
_LANE_TFLOPS = {V.DT_F32: 150.0 / 256}
_LANE_TFLOPS_MMA = 2500.0 / 256
_TILE_US = 2.0
_BAR_US = 2.3
_BAR_US_PER_LANE = 1.8 / 128


def task_work(task: V.Task, prog: V.VMProgram) -> tuple:
    """(HBM bytes, flops) one task moves and computes, algorithmically."""
    dsz = V.DT_SIZE.get(task.dtype, 4)
    asz = V.DT_SIZE.get(task.adtype, 4)
    top = task.tile_op
    if top == V.TOP_MMA:
        M, N, K, G = task.p0, task.p1, task.p2, max(1, task.p3 & 0xFFFFFF)
        return (M * K + K * N) * G * asz + M * N * G * dsz, 2.0 * M * N * K * G
    if top == V.TOP_GEMV:
        M, N, K, G = task.p0, task.p1, task.p2, max(1, task.p3)
        return (K * N + M * K) * G * asz + M * N * G * dsz, 2.0 * M * N * K * G
    if top == V.TOP_FLASH_ATTN:
        H, T = task.p1, task.p2
        hd = prog.aux[task.p3 + 3] if task.p3 + 3 < len(prog.aux) else 128
        C = prog.aux[task.p3 + 2] if task.p3 + 2 < len(prog.aux) else T
        return 2 * H * C * hd * asz, 4.0 * H * T * C * hd
    if top == V.TOP_DECODE_ATTN:
        return 2 * (task.p4 & 0xFFFF) * (task.p5 & 0xFFFF) * task.p6 * asz, 0.0
    if top in (V.TOP_RED_SEG, V.TOP_SOFTMAX_SEG, V.TOP_LAYERNORM_SEG, V.TOP_ARGMAX_SEG):
        return task.p0 * task.p1 * (asz + (dsz if top != V.TOP_RED_SEG else 0)), 0.0
    n = max(task.p0, task.p1) if top != V.TOP_EW else task.p1
    return n * (asz * 2 + dsz), 0.0


def model_terms(cfg: DeviceConfig) -> tuple:
    """(tile latency us, per-lane GB/s, per-lane MFMA TFLOP/s, barrier us, barrier
    us per lane): measured values from the cost table, else the constants above
    (fitted on one MI355X)."""
    c = cfg.costs
    return (c.get("tile_us", _TILE_US), c.get("lane_gbs", _LANE_GBS), c.get("lane_mma_tflops", _LANE_TFLOPS_MMA),
            c.get("barrier_us", _BAR_US), c.get("barrier_us_per_lane", _BAR_US_PER_LANE))


def phase_us(tasks: list, n_lanes: int, cfg: DeviceConfig, prog: V.VMProgram) -> float:
    """Estimated microseconds of one phase on ``n_lanes`` lanes."""
    tile_us, lane_gbs, lane_mma, _, _ = model_terms(cfg)
    byts = flops = 0.0
    tiles = 0
    for t in tasks:
        b, f = task_work(t, prog)
        rate = lane_mma if t.adtype != V.DT_F32 else _LANE_TFLOPS[V.DT_F32]
        byts += b
        flops += f / rate
        tiles += n_tiles(t, cfg)
    rounds = -(-tiles // n_lanes) if tiles else 0
    return rounds * tile_us + max(byts / (n_lanes * lane_gbs * 1e3), flops / (n_lanes * 1e6))


# --- phases ---------------------------------------------------------------------

_VIEW_BIN = frozenset({V.OP_ADD_F32, V.OP_MUL_F32, V.OP_SUB_F32, V.OP_DIV_F32, V.OP_MAX_F32,
                       V.OP_MIN_F32, V.OP_POW_F32, V.OP_ATAN2_F32, V.OP_REMAINDER_F32})


def viewed_reads(ins: V.Instr) -> set:
    """Buffers a float elementwise instruction reads through a strided view
    (operand a's view in imm, b's in imm2 for the binary ops)."""
    out = set()
    if ins.op in _VIEW_BIN:
        if ins.imm:
            out.add(ins.a)
        if ins.imm2:
            out.add(ins.b)
    elif ins.op in _UN_SUB and ins.op != V.OP_AFFINE_F32 and ins.imm:
        out.add(ins.a)
    return out


def _phases(prog, indices, tasks_of, fuse, extra_reads=None):
    """Split ``indices`` (program order) into barrier-separated phases: an
    instruction with a cross-lane dependency (RAW, WAW or WAR through a shared
    buffer) on an earlier one runs in a later phase; a lane-local one (an
    elementwise chain) may share its phase.
    ``extra_reads``: {index: buffers} read beyond the instruction's own operands
    (a GEMV staging a fused layernorm reads the layernorm's inputs)."""
    instrs = prog.instrs
    extra_reads = extra_reads or {}

    def reads(k):
        r = instr_reads(instrs[k], prog)
        return r | extra_reads[k] if k in extra_reads else r
    phases = []
    readers: dict = {}
    writers: dict = {}

    def is_map(i):
        return tasks_of(i).tile_op == V.TOP_EW

    def cross(j, i):
        a, b = instrs[i], instrs[j]
        wa, wb = instr_writes(a, prog), instr_writes(b, prog)
        if a.disjoint and a.disjoint == b.disjoint:
            wa, wb = wa - wb, wb - instr_writes(a, prog)
        dep = (reads(j) & wa) or (wb & wa) or (reads(i) & wb)
        if not dep:
            return False
        if not fuse:
            return True
        # lane-local: both elementwise over the same count, no shared writes,
        # and no dependency through a strided view (a viewed operand reads
        # elements of other tiles, which other lanes produce or still read)
        if not (is_map(i) and is_map(j) and a.n == b.n and wa.isdisjoint(wb)):
            return True
        grp = overlap_groups(prog)
        return bool(({grp[x] for x in viewed_reads(b)} & wa) or ({grp[x] for x in viewed_reads(a)} & wb))

    # each instruction goes to the earliest phase its dependencies allow (as
    # soon as possible, not merely after the phase in progress): an
    # independent op written late, such as a bias added to a residual for the
    # next matmul's epilogue, runs beside earlier work instead of opening a
    # phase of its own
    level: dict = {}
    for j in indices:
        ins = instrs[j]
        cand = set()
        for b in reads(j):
            cand.update(writers.get(b, ()))
        for b in instr_writes(ins, prog):
            cand.update(writers.get(b, ()))
            cand.update(readers.get(b, ()))
        lv = 0
        for i in cand:
            lv = max(lv, level[i] + 1 if cross(j, i) else level[i])
        level[j] = lv
        while len(phases) <= lv:
            phases.append([])
        phases[lv].append(j)
        for b in reads(j):
            readers.setdefault(b, []).append(j)
        for b in instr_writes(ins, prog):
            writers.setdefault(b, []).append(j)
    return phases


# --- packing --------------------------------------------------------------------

def _tile_quantum(task: V.Task, cfg: DeviceConfig, prog: V.VMProgram) -> int:
    """Preferred chunk granularity in tiles (chunk boundaries on multiples of
    it keep the kernel's multi-row blocks whole)."""
    if task.tile_op == V.TOP_FLASH_ATTN:
        # the matrix-core kernel works on 256-row blocks of one head, and each
        # head's tiles are padded to whole blocks (attn_rows_padded)
        return ATTN_BLOCK_ROWS
    return 1


def xcd_lane_order(n_lanes: int, n_xcd: int = 8) -> list:
    """Lanes grouped by XCD: workgroup (lane) i runs on XCD i % n_xcd, so this
    order lists XCD 0's lanes first, then XCD 1's, ...  Consecutive chunks
    placed in this order share an XCD and its L2."""
    if n_lanes % n_xcd:
        return list(range(n_lanes))
    return [x + n_xcd * j for x in range(n_xcd) for j in range(n_lanes // n_xcd)]


def pack_units(units, n_lanes: int, idle_master: bool = False, loads=None):
    """units: [(task_ids, tiles, cost, quantum[, xcd_grouped])] -> [(lane, Entry)].

    Each unit is cut into k = min(tiles/quantum, ceil(n_lanes * cost share))
    contiguous chunks, and the chunks are placed longest-first on the
    least-loaded lane; a unit's whole chain runs over each of its chunks.  Ties
    between equally loaded lanes go to the lowest lane, or, for an xcd_grouped
    unit (neighbouring chunks read the same operands), to the first lane in
    XCD-grouped order, so neighbouring chunks land on one XCD.  ``idle_master``:
    a phase with fewer chunks than lanes keeps lane 0 free (C5: 1006 -> 1015
    tokens/s in alternating runs).  ``loads``: the lanes' work so far in the
    phase (updated in place), when this call adds to a phase already packed."""
    out = []
    if not units:
        return out
    total = sum(u[2] for u in units) or 1.0
    chunks = []
    for uid, unit in enumerate(units):
        tids, tiles, cost, q = unit[:4]
        grouped = len(unit) > 4 and bool(unit[4])
        blocks = max(1, math.ceil(tiles / q))
        k = min(blocks, max(1, math.ceil(n_lanes * cost / total)))
        for j in range(k):
            lo = min(tiles, (blocks * j // k) * q)
            hi = min(tiles, (blocks * (j + 1) // k) * q)
            if hi > lo:
                chunks.append((cost * (hi - lo) / tiles, uid, tids, lo, hi, grouped))
    chunks.sort(key=lambda c: (-c[0], c[1], c[3]))
    if loads is None:
        loads = [0.0] * n_lanes
    plain, grouped_order = range(n_lanes), xcd_lane_order(n_lanes)
    if idle_master and 1 < len(chunks) < n_lanes:
        # a phase that leaves lanes idle leaves lane 0 (the grid barrier's
        # master, which polls the other lanes' arrivals) idle too, so it is
        # already polling when the last tile ends
        plain = range(1, n_lanes)
        grouped_order = [l for l in grouped_order if l != 0]
    # heap-free least-loaded search: lanes are few (<= 4096) and chunks are
    # bounded by n_lanes per unit, so the linear scan stays cheap.
    for cost, _uid, tids, lo, hi, grouped in chunks:
        lane = min(grouped_order if grouped else plain, key=loads.__getitem__)
        for tid in tids:
            out.append((lane, V.Entry(tid, lo, hi)))
        loads[lane] += cost
    return out


# --- the scheduler ------------------------------------------------------------------

@dataclasses.dataclass
class _Region:
    entries: list           # control entry of each lane, patched after scheduling
    first: list             # WHILE: cond, FOR: [], IF: then
    second: list            # WHILE/FOR: body, IF: else
    op: int
    weight: float = 1.0     # executions per launch (FOR trips, nested)


class _Scheduler:
    def __init__(self, prog: V.VMProgram, cfg: DeviceConfig):
        self.prog = prog
        self.cfg = cfg
        self.n = cfg.nlanes
        self.lanes = [[] for _ in range(self.n)]
        self.tasks: list = []
        self.task_of: dict = {}
        self.regions: list = []
        # layernorms staged inside their GEMV: {dot index: layernorm index}
        self.ln_pro = ln_gemv_pairs(prog, cfg)
        self.ln_fused = set(self.ln_pro.values())
        self.extra_reads = {j: instr_reads(prog.instrs[i], prog) for j, i in self.ln_pro.items()}
        # estimated microseconds per launch (work model of lane_fit)
        self.weight = 1.0
        self.est = 0.0
        self.n_flags = 0          # completion flags handed out (``emit_flagged``)

    def task_id(self, i: int) -> int:
        tid = self.task_of.get(i)
        if tid is None:
            tid = len(self.tasks)
            self.task_of[i] = tid
            t = instr_to_task(self.prog.instrs[i], self.prog, self.cfg)
            self.tasks.append(t)
            if i in self.ln_pro:
                # the layernorm's task is a descriptor only: no lane runs it
                t.p5 = self.task_id(self.ln_pro[i]) + 1
        return tid

    def task(self, i: int) -> V.Task:
        return self.tasks[self.task_id(i)]

    def barrier(self):
        for s in self.lanes:
            s.append(V.barrier_entry())
        _, _, _, bar, bar_lane = model_terms(self.cfg)
        self.est += self.weight * (bar + bar_lane * self.n)

    def levels(self, indices):
        out, seg = [], []

        def flush():
            if seg:
                for ph in _phases(self.prog, list(seg), self.task, self.cfg.fuse, self.extra_reads):
                    out.append(("compute", ph))
                seg.clear()

        for i in indices:
            op = self.prog.instrs[i].op
            if op in V.REGION_OPS:
                flush()
                out.append(("region", i))
            elif op != V.OP_NOP and i not in self.ln_fused:
                seg.append(i)
        flush()
        return out

    def chains(self, map_idx):
        parent = {i: i for i in map_idx}

        def find(x):
            while parent[x] != x:
                parent[x] = parent[parent[x]]
                x = parent[x]
            return x

        writer = {}
        for i in map_idx:
            for b in instr_writes(self.prog.instrs[i], self.prog):
                writer[b] = i
        for j in map_idx:
            for b in instr_reads(self.prog.instrs[j], self.prog):
                w = writer.get(b)
                if w is not None and w != j:
                    parent[find(w)] = find(j)
        comps: dict = {}
        for i in map_idx:
            comps.setdefault(find(i), []).append(i)
        return [sorted(v) for v in comps.values()]

    def reads(self, i):
        r = instr_reads(self.prog.instrs[i], self.prog)
        return r | self.extra_reads[i] if i in self.extra_reads else r

    def phase_units(self, indices):
        shaped, maps = [], []
        for i in sorted(indices):
            (maps if self.task(i).tile_op == V.TOP_EW else shaped).append(i)
        units = []
        for i in shaped:
            t = self.task(i)
            units.append(([self.task_id(i)], n_tiles(t, self.cfg),
                          task_cost(t, self.cfg, self.prog),
                          _tile_quantum(t, self.cfg, self.prog),
                          # neighbouring strips share weight lines (a 16-column
                          # bf16 strip is a quarter of a 128-byte line): on one
                          # XCD they share its L2 (C5: 1014 -> 1036 tokens/s)
                          t.tile_op in (V.TOP_FLASH_ATTN, V.TOP_GEMV)))
        for comp in self.chains(maps):
            tids = [self.task_id(i) for i in comp]
            t0 = self.tasks[tids[0]]
            cost = sum(task_cost(self.tasks[t], self.cfg, self.prog) for t in tids)
            units.append((tids, n_tiles(t0, self.cfg), cost, 1))
        return units

    def emit_phase(self, indices):
        for lane, e in pack_units(self.phase_units(indices), self.n, master_idle(self.cfg)):
            self.lanes[lane].append(e)
        self.est += self.weight * phase_us([self.task(i) for i in indices if i not in self.ln_fused],
                                           self.n, self.cfg, self.prog)

    # -- completion flags: a consumer phase joined to its producer phase ---------------

    def _flag_edges(self, prod, cons):
        """Phase ``cons`` can join phase ``prod`` with completion flags when every
        instruction in it is a decode attention whose only dependencies on
        ``prod`` are reads of its q, k and v from the output of TOP_GEMV tasks
        there (no write-after-read or write-after-write, caches and position
        written earlier).  Returns {consumer: (GEMV indices, per head the byte
        ranges of its q, k and v)}, or None."""
        prog, bufs = self.prog, self.prog.buffers
        if not self.cfg.counters:
            return None
        grp = overlap_groups(prog)
        edges = {}
        for j in cons:
            ins = prog.instrs[j]
            if ins.op != V.OP_DECODE_ATTN:
                return None
            hd = prog.aux[ins.aux] & 0xFFFF
            kb, vb, posb = prog.aux[ins.aux + 1:ins.aux + 4]
            qkv = {grp[ins.a], grp[kb], grp[vb]}
            if qkv & {grp[ins.b], grp[ins.imm2], grp[posb]}:
                return None
            wj, rj = instr_writes(ins, prog), self.reads(j)
            # the arena bytes the consumer writes must not be bytes any producer
            # reads or writes, aliases and arena packing included
            dst = bufs[ins.dst]
            wbytes = (dst.arena_byte_offset, dst.arena_byte_offset + dst.size_bytes)
            gemvs = []
            for i in prod:
                wi, ri = instr_writes(prog.instrs[i], prog), self.reads(i)
                if wj & (wi | ri):
                    return None
                for b in self.raw_operands(i):
                    B = bufs[b]
                    if B.size_bytes and B.arena_byte_offset < wbytes[1] and wbytes[0] < B.arena_byte_offset + B.size_bytes:
                        return None
                raw = rj & wi
                if not raw:
                    continue
                if raw - qkv or self.task(i).tile_op != V.TOP_GEMV:
                    return None
                gemvs.append(i)
            if not gemvs:
                return None
            es = V.DT_SIZE[bufs[ins.a].dtype]
            heads = [[(bufs[b].arena_byte_offset + h * hd * es, bufs[b].arena_byte_offset + (h + 1) * hd * es)
                      for b in (ins.a, kb, vb)] for h in range(ins.n)]
            edges[j] = (gemvs, heads)
        return edges

    def raw_operands(self, i):
        """Buffer ids (not alias groups) instruction ``i`` reads or writes,
        with the inputs of a layernorm staged in it."""
        ins = self.prog.instrs[i]
        ids = _instr_reads(ins, self.prog) | _instr_writes(ins, self.prog)
        if i in self.ln_pro:
            ids |= _instr_reads(self.prog.instrs[self.ln_pro[i]], self.prog)
        return {b for b in ids if 0 <= b < len(self.prog.buffers)}

    def joined_levels(self, lv) -> set:
        """Levels k whose phase joins level k - 1's with completion flags
        (``_flag_edges``); a joined level is not joined onward.  The arena
        packing gives such a level the phase time of the one before it."""
        out, k = set(), 1
        while k < len(lv):
            if lv[k - 1][0] == "compute" and lv[k][0] == "compute" and self._flag_edges(lv[k - 1][1], lv[k][1]):
                out.add(k)
                k += 2
            else:
                k += 1
        return out

    def _gemv_bytes(self, i, lo, hi):
        """Arena byte ranges TOP_GEMV tiles [lo, hi) of instruction ``i`` write."""
        t, dst = self.task(i), self.prog.buffers[self.prog.instrs[i].dst]
        M, N, w = t.p0, t.p1, t.p4
        es, ncb = V.DT_SIZE[dst.dtype], -(-N // w)
        out = []
        for tile in range(lo, hi):
            g, nb = divmod(tile, ncb)
            for m in range(M):
                a = dst.arena_byte_offset + ((g * M + m) * N + nb * w) * es
                out.append((a, a + min(w, N - nb * w) * es))
        return out

    def emit_flagged(self, prod, cons, edges) -> bool:
        """One phase for ``prod`` and ``cons`` (see ``_flag_edges``).  The
        producer phase is packed as usual; every chunk of a GEMV that some head
        reads signals a flag of its own, numbered head by head, so the strips
        of a head hold consecutive flags; the decode attention is packed after
        them onto the least-loaded lanes, each chunk waiting for the flags of
        the heads it covers.  Every lane runs its producer entries before its
        consumer entries, so every wait ends.  False (nothing emitted) when a
        producer chunk serves more than one head."""
        loads = [0.0] * self.n
        placed = pack_units(self.phase_units(prod), self.n, master_idle(self.cfg), loads)
        by_tid = {}
        for j, (gemvs, _) in edges.items():
            for i in gemvs:
                by_tid.setdefault(self.task_id(i), set()).add(i)
        members = {}
        for _lane, e in placed:
            if e.task not in by_tid:
                continue
            served = set()
            for i in by_tid[e.task]:
                wr = self._gemv_bytes(i, e.tile_lo, e.tile_hi)
                for j, (gemvs, heads) in edges.items():
                    if i not in gemvs:
                        continue
                    for h, rngs in enumerate(heads):
                        if any(a < d and c < b for a, b in wr for c, d in rngs):
                            served.add((j, h))
            if len(served) > 1:
                return False
            if served:
                members.setdefault(served.pop(), []).append(e)
        base, f = {}, self.n_flags
        for j in sorted(edges):
            for h in range(len(edges[j][1])):
                base[(j, h)] = f
                for e in sorted(members.get((j, h), []), key=lambda e: (e.task, e.tile_lo)):
                    e.signal_flag = f
                    f += 1
        end = {g: base[g] + len(members.get(g, [])) for g in base}
        waits = pack_units(self.phase_units(cons), self.n, master_idle(self.cfg), loads)
        for _lane, e in waits:
            j = next(j for j in edges if self.task_id(j) == e.task)
            S = max(1, self.tasks[e.task].p4 >> 16)
            lo, hi = base[(j, e.tile_lo // S)], end[(j, (e.tile_hi - 1) // S)]
            if hi > lo:
                e.wait_flag, e.wait_count = lo, hi - lo
        for lane, e in placed + waits:
            self.lanes[lane].append(e)
        self.n_flags = f
        self.est += self.weight * phase_us([self.task(i) for i in list(prod) + list(cons) if i not in self.ln_fused],
                                           self.n, self.cfg, self.prog)
        return True

    def schedule_range(self, indices, trailing_barrier: bool):
        lv = self.levels(indices)
        k = 0
        while k < len(lv):
            kind, payload = lv[k]
            if kind == "compute":
                joined = False
                if k + 1 < len(lv) and lv[k + 1][0] == "compute":
                    edges = self._flag_edges(payload, lv[k + 1][1])
                    joined = bool(edges) and self.emit_flagged(payload, lv[k + 1][1], edges)
                if joined:
                    k += 1
                else:
                    self.emit_phase(payload)
            else:
                self.emit_region(payload)
            if trailing_barrier or k != len(lv) - 1:
                self.barrier()
            k += 1

    def emit_region(self, i):
        ins = self.prog.instrs[i]
        ents = []
        for s in self.lanes:
            if ins.op == V.OP_FOR:
                e = V.Entry(V.ENT_FOR, 0, 0, ins.b, 0, V.FLAG_NONE)
            elif ins.op == V.OP_IF:
                e = V.Entry(V.ENT_IF, 0, 0, 0, 0, ins.dst)
            else:
                e = V.Entry(V.ENT_WHILE, 0, 0, 0, 0, ins.dst)
            s.append(e)
            ents.append(e)
        if ins.op == V.OP_FOR:
            first, second = [], list(range(ins.n, ins.n + ins.imm))
        else:
            first = list(range(ins.a, ins.a + ins.b))
            second = list(range(ins.n, ins.n + ins.imm))
        w = self.weight * (max(1, ins.b) if ins.op == V.OP_FOR else 1)
        self.regions.append(_Region(ents, first, second, ins.op, w))

    def schedule_region(self, r: _Region):
        self.weight = r.weight
        s0 = [len(s) for s in self.lanes]
        if r.op != V.OP_FOR:
            self.schedule_range(r.first, trailing_barrier=False)
        s1 = [len(s) for s in self.lanes]
        self.schedule_range(r.second, trailing_barrier=False)
        s2 = [len(s) for s in self.lanes]
        for lane, e in enumerate(r.entries):
            if r.op == V.OP_FOR:
                e.tile_lo, e.tile_hi = s1[lane], s2[lane] - s1[lane]
            else:
                # WHILE: cond [tile_lo, +tile_hi), body [wait_flag, +wait_count)
                # IF:    then [tile_lo, +tile_hi), else [wait_flag, +wait_count)
                e.tile_lo, e.tile_hi = s0[lane], s1[lane] - s0[lane]
                e.wait_flag, e.wait_count = s1[lane], s2[lane] - s1[lane]


def lane_fit(prog: V.VMProgram, cfg: DeviceConfig) -> int:
    """Lane count to schedule ``prog`` on (extension): the advertised count, or
    half of it when the work model estimates the launch faster there.  A phase
    of bytes B and flops F costs max(B / (L bw), F / (L flops)) per lane share
    plus one tile latency per round of tiles, and each grid barrier a per-lane
    overhead fitted to the decode loop (C5, one FOR trip per token: 935 us per
    token on 256 lanes, 845 on 128 -- the saved barrier time is larger than
    the halved bandwidth of its 240 MB).  Bandwidth- and MFMA-bound programs
    (C2-C4) keep every lane."""
    return _fit(prog, cfg)[0]


def _fit(prog: V.VMProgram, cfg: DeviceConfig):
    """(lanes, schedule) of lane_fit; the schedule is None when only one lane
    count was a candidate."""
    n = cfg.nlanes
    if not cfg.fit_lanes or n < 128 or n % 16:
        return n, None
    best, best_sc = n, None
    for lanes in (n, n // 2):
        sc = _schedule(prog, dataclasses.replace(cfg, nlanes=lanes, fit_lanes=False))
        if best_sc is None or sc.est < best_sc.est:
            best, best_sc = lanes, sc
    return best, best_sc


def _schedule(prog: V.VMProgram, cfg: DeviceConfig) -> _Scheduler:
    sc = _Scheduler(prog, cfg)
    # No barrier after the last root level: nothing reads it before the launch
    # completes, so a one-phase program needs no grid barrier at all.
    sc.schedule_range(list(range(prog.main_len)), trailing_barrier=False)
    if not any(sc.lanes):
        sc.barrier()
    root_lens = [len(s) for s in sc.lanes]
    while sc.regions:
        sc.schedule_region(sc.regions.pop(0))
    sc.root_lens = root_lens
    return sc


def schedule_program(prog: V.VMProgram, cfg: DeviceConfig | None = None) -> V.Schedule:
    cfg = cfg or DeviceConfig.from_env()
    lanes, sc = _fit(prog, cfg)
    if sc is None:
        sc = _schedule(prog, dataclasses.replace(cfg, nlanes=lanes, fit_lanes=False))
    return V.Schedule(lanes, sc.tasks, sc.lanes, sc.root_lens, sc.n_flags)


def schedule_bytes(prog: V.VMProgram, cfg: DeviceConfig | None = None) -> bytes:
    sched = schedule_program(prog, cfg)
    return V.serialize(prog, sched)
