"""Program fixtures shared by the CPU and GPU tests.

* ``raw_*``: hand-encoded v3 blobs written with plain struct packing (no
  product code), restating the reference's C++ known-answer programs
  (pjrt_plugin/src/runtime_test.cc:136-215);
* ``while_*``: the closed-form control-flow cases of
  tests/_while_e2e_body.py:16-84, built with the graph builder.
"""
from __future__ import annotations

import struct

import numpy as np

from pjrt_amd import graph as G
from pjrt_amd import vmprogram as V

NOPE, BARR, WHIL = 0xFFFFFFFF, 0xFFFFFFFE, 0xFFFFFFFD
FLAGN = 0xFFFFFFFF


class RawBuilder:
    """Minimal v3 writer over raw structs (runtime_test.cc:31-110 layout)."""

    def __init__(self, n_lanes):
        self.n_lanes = n_lanes
        self.bufs = []
        self.arena = 0
        self.inputs, self.outputs = [], []
        self.in_dims, self.out_dims = [], []
        self.consts = []
        self.tasks = []
        self.lanes = [[] for _ in range(n_lanes)]
        self.root_lens = [0] * n_lanes

    def buf(self, elems, esz=4, dtype=0):
        self.bufs.append((self.arena, elems * esz, dtype))
        self.arena = (self.arena + elems * esz + 63) & ~63
        return len(self.bufs) - 1

    def task(self, tile_op, dst, a, b, *p):
        p = list(p) + [0] * (8 - len(p))
        self.tasks.append((tile_op, dst, a, b, *p))
        return len(self.tasks) - 1

    def ent(self, lane, e):
        e = list(e) + [0] * (8 - len(e))
        self.lanes[lane].append(e)

    def barrier_all(self):
        for l in self.lanes:
            l.append([BARR, 0, 0, FLAGN, 0, FLAGN, 0, 0])

    def bytes(self):
        b = bytearray()

        def a8():
            b.extend(b"\0" * (-len(b) % 8))

        n_ent = sum(len(l) for l in self.lanes)
        b += struct.pack("<10IQ", 0x314D5056, 3, len(self.bufs), 0, len(self.consts),
                         0, len(self.inputs), len(self.outputs), 0, 0, self.arena)
        for off, size, dt in self.bufs:
            b += struct.pack("<QQII", off, size, dt, 0)
        for i in self.inputs:
            b += struct.pack("<I", i)
        a8()
        for i in self.outputs:
            b += struct.pack("<I", i)
        a8()
        for d in self.in_dims + self.out_dims:
            b += struct.pack("<II", len(d), 0) + b"".join(struct.pack("<Q", x) for x in d)
        for bid, vals in self.consts:
            raw = np.asarray(vals, np.float32).tobytes()
            b += struct.pack("<II", bid, len(raw)) + raw
            a8()
        b += struct.pack("<4I", len(self.tasks), n_ent, 0, self.n_lanes)
        for t in self.tasks:
            b += struct.pack("<12I", *t)
        off = 0
        for l, s in enumerate(self.lanes):
            b += struct.pack("<4I", off, len(s), self.root_lens[l] or len(s), 0)
            off += len(s)
        for s in self.lanes:
            for e in s:
                b += struct.pack("<8I", *e)
        return bytes(b)


def raw_two_level_ew(ew_ts: int, lanes: int = 4):
    """c = (a + b) * a over ``lanes`` tiles, two phases (runtime_test.cc A)."""
    n = lanes * ew_ts
    rb = RawBuilder(lanes)
    ba, bb, bt, bc = rb.buf(n), rb.buf(n), rb.buf(n), rb.buf(n)
    rb.inputs, rb.outputs = [ba, bb], [bc]
    rb.in_dims, rb.out_dims = [[n], [n]], [[n]]
    t0 = rb.task(0, bt, ba, bb, 0, n)
    t1 = rb.task(0, bc, bt, ba, 1, n)
    for l in range(lanes):
        rb.ent(l, [t0, l, l + 1, FLAGN, 0, FLAGN])
    rb.barrier_all()
    for l in range(lanes):
        rb.ent(l, [t1, l, l + 1, FLAGN, 0, FLAGN])
    rb.barrier_all()
    a = (np.arange(n) % 251).astype(np.float32)
    b = (np.arange(n) % 83 + 1).astype(np.float32)
    return rb.bytes(), [a, b], [(a + b) * a]


def raw_while_doubling(ew_ts: int):
    """while (i < 10) { x += x; i += 1 } on 2 lanes (runtime_test.cc B):
    x * 1024 exactly."""
    n = 2 * ew_ts
    rb = RawBuilder(2)
    bx, bi, bk, bone, bcond = rb.buf(n), rb.buf(1), rb.buf(1), rb.buf(1), rb.buf(1)
    rb.inputs, rb.outputs = [bx], [bx]
    rb.in_dims, rb.out_dims = [[n]], [[n]]
    rb.consts = [(bi, [0.0]), (bk, [10.0]), (bone, [1.0])]
    tdbl = rb.task(0, bx, bx, bx, 0, n)
    tinc = rb.task(0, bi, bi, bone, 0, 1)
    tlts = rb.task(0, bcond, bi, bk, 22, 1)
    wh = [WHIL, 1, 1, 2, 2, bcond, 0, 0]
    rb.ent(0, wh)
    rb.ent(0, [tlts, 0, 1, FLAGN, 0, FLAGN])
    rb.ent(0, [tdbl, 0, 1, FLAGN, 0, FLAGN])
    rb.ent(0, [tinc, 0, 1, FLAGN, 0, FLAGN])
    rb.ent(1, wh)
    rb.ent(1, [NOPE, 0, 0, FLAGN, 0, FLAGN])
    rb.ent(1, [tdbl, 1, 2, FLAGN, 0, FLAGN])
    rb.ent(1, [NOPE, 0, 0, FLAGN, 0, FLAGN])
    rb.root_lens = [1, 1]
    x = (np.arange(n) % 13 + 1).astype(np.float32)
    return rb.bytes(), [x], [x * 1024.0]


def raw_region_gelu(ew_ts: int, lanes: int = 8):
    """Hand-emitted GELU micro-program through MAP_REGION (runtime_test.cc C)."""
    fb = V.f32_bits
    n = lanes * ew_ts
    rb = RawBuilder(lanes)
    bx, by = rb.buf(n), rb.buf(n)
    rb.inputs, rb.outputs = [bx], [by]
    rb.in_dims, rb.out_dims = [[n]], [[n]]
    MUL, ADD, TANH, AFF = 1, 0, 13, 40
    aux = [1, 0, 8, 0,
           MUL, 1, 0, 0, 0, 0,
           MUL, 1, 1, 0, 0, 0,
           AFF, 1, 1, 0, fb(0.044715), fb(0.0),
           ADD, 1, 1, 0, 0, 0,
           AFF, 1, 1, 0, fb(0.7978845608), fb(0.0),
           TANH, 1, 1, 0, 0, 0,
           AFF, 1, 1, 0, fb(0.5), fb(0.5),
           MUL, 0, 0, 1, 0, 0]
    # desc layout: [n_in, out_slot, n_micro, in_slot[n_in], micro...]
    treg = rb.task(13, by, bx, bx, 0, n)
    for l in range(lanes):
        rb.ent(l, [treg, l, l + 1, FLAGN, 0, FLAGN])
    blob = bytearray(rb.bytes())
    # splice the aux pool in: header n_aux and the section before consts
    hdr = list(struct.unpack_from("<10IQ", blob, 0))
    hdr[8] = len(aux)
    struct.pack_into("<10IQ", blob, 0, *hdr)
    pos = 48 + 24 * len(rb.bufs) + 8 + 8 + 16 + 16
    aux_bytes = struct.pack(f"<{len(aux)}I", *aux)
    aux_bytes += b"\0" * (-len(aux_bytes) % 8)
    blob[pos:pos] = aux_bytes
    x = (-4.0 + 8.0 * (np.arange(n) % 101) / 100.0).astype(np.float32)
    g = 0.5 * x.astype(np.float64) * (1 + np.tanh(0.7978845608 * (x + 0.044715 * x.astype(np.float64) ** 3)))
    return bytes(blob), [x], [g.astype(np.float32)]


# --- while / fori closed forms (tests/_while_e2e_body.py) ---------------------------

def while_double():
    """(i, v) = while i < 10: (i + 1, v * 2) from (0, 1.0) -> (10, 1024)."""
    g = G.Graph()
    v0 = g.input((), "f32")
    i = g.fill((), 0, "i32")
    v = g.fill((), 0.0)
    g.copy_into(v, v0)
    ten, one, two = g.scalar(10, "i32"), g.scalar(1, "i32"), g.scalar(2.0)
    g.begin()
    cond = g.compare(i, ten, "LT")
    cl = g.end()
    g.begin()
    i2 = g.add(i, one)
    v2 = g.mul(v, two)
    g.copy_into(i, i2)
    g.copy_into(v, v2)
    body = g.end()
    g.while_loop(cond, cl, body)
    g.output(i, v)
    return g.build(), [np.float32(1.0)], [np.int32(10), np.float32(1024.0)]


def fori_add():
    """fori_loop(0, 5, a + 3) from 2.0 -> 17."""
    g = G.Graph()
    x = g.input((), "f32")
    a = g.fill((), 0.0)
    g.copy_into(a, x)
    three = g.scalar(3.0)
    g.begin()
    t = g.add(a, three)
    g.copy_into(a, t)
    body = g.end()
    g.for_loop(5, body)
    g.output(a)
    return g.build(), [np.float32(2.0)], [np.float32(17.0)]


def fori_vec(n=40000):
    """vector carry over several tiles: v + 3."""
    g = G.Graph()
    x = g.input((n,), "f32")
    a = g.fill((n,), 0.0)
    g.copy_into(a, x)
    one = g.const(np.ones(n, np.float32))
    g.begin()
    t = g.add(a, one)
    g.copy_into(a, t)
    body = g.end()
    g.for_loop(3, body)
    g.output(a)
    vin = np.arange(n, dtype=np.float32)
    return g.build(), [vin], [vin + 3.0]


def while_multilevel():
    """a *= 3 three times via b = 2a, d = b + a: 1 -> 27."""
    g = G.Graph()
    x = g.input((), "f32")
    k = g.fill((), 0, "i32")
    a = g.fill((), 0.0)
    g.copy_into(a, x)
    three, one, two = g.scalar(3, "i32"), g.scalar(1, "i32"), g.scalar(2.0)
    g.begin()
    c = g.compare(k, three, "LT")
    cl = g.end()
    g.begin()
    b = g.mul(a, two)
    d = g.add(b, a)
    k2 = g.add(k, one)
    g.copy_into(a, d)
    g.copy_into(k, k2)
    body = g.end()
    g.while_loop(c, cl, body)
    g.output(a)
    return g.build(), [np.float32(1.0)], [np.float32(27.0)]


def while_zero():
    g = G.Graph()
    x = g.input((), "f32")
    i = g.fill((), 0, "i32")
    v = g.fill((), 0.0)
    g.copy_into(v, x)
    zero, one, two = g.scalar(0, "i32"), g.scalar(1, "i32"), g.scalar(2.0)
    g.begin()
    c = g.compare(i, zero, "LT")
    cl = g.end()
    g.begin()
    i2 = g.add(i, one)
    v2 = g.mul(v, two)
    g.copy_into(i, i2)
    g.copy_into(v, v2)
    body = g.end()
    g.while_loop(c, cl, body)
    g.output(i, v)
    return g.build(), [np.float32(7.0)], [np.int32(0), np.float32(7.0)]


def while_nested():
    """outer 4 x (inner 3 x s += 1) from 0 -> 12."""
    g = G.Graph()
    x = g.input((), "f32")
    k = g.fill((), 0, "i32")
    d = g.fill((), 0, "i32")
    s = g.fill((), 0.0)
    g.copy_into(s, x)
    four, three, one = g.scalar(4, "i32"), g.scalar(3, "i32"), g.scalar(1, "i32")
    onef = g.scalar(1.0)
    zero = g.scalar(0, "i32")
    # inner while
    g.begin()
    ci = g.compare(d, three, "LT")
    inner_cond = g.end()
    g.begin()
    d2 = g.add(d, one)
    s2 = g.add(s, onef)
    g.copy_into(d, d2)
    g.copy_into(s, s2)
    inner_body = g.end()
    # outer
    g.begin()
    co = g.compare(k, four, "LT")
    outer_cond = g.end()
    g.begin()
    g.copy_into(d, zero)
    g.while_loop(ci, inner_cond, inner_body)
    k2 = g.add(k, one)
    g.copy_into(k, k2)
    outer_body = g.end()
    g.while_loop(co, outer_cond, outer_body)
    g.output(s)
    return g.build(), [np.float32(0.0)], [np.float32(12.0)]


def while_then():
    """y = while i < 5: y + 2 from 1; out y*y = 121."""
    g = G.Graph()
    x = g.input((), "f32")
    i = g.fill((), 0, "i32")
    y = g.fill((), 0.0)
    g.copy_into(y, x)
    five, one, two = g.scalar(5, "i32"), g.scalar(1, "i32"), g.scalar(2.0)
    g.begin()
    c = g.compare(i, five, "LT")
    cl = g.end()
    g.begin()
    i2 = g.add(i, one)
    y2 = g.add(y, two)
    g.copy_into(i, i2)
    g.copy_into(y, y2)
    body = g.end()
    g.while_loop(c, cl, body)
    out = g.mul(y, y)
    g.output(out)
    return g.build(), [np.float32(1.0)], [np.float32(121.0)]


def scan_stack(n=5000, T=6):
    """scan(c + x_t) stacking c * 2 into ys via dynamic_update_slice."""
    g = G.Graph()
    c0 = g.input((n,), "f32")
    xs = g.input((T, n), "f32")
    c = g.fill((n,), 0.0)
    g.copy_into(c, c0)
    ys = g.fill((T, n), 0.0)
    t = g.fill((), 0, "i32")
    zero = g.scalar(0, "i32")
    one = g.scalar(1, "i32")
    two = g.const(np.full(n, 2.0, np.float32))
    g.begin()
    xt = g.dynamic_slice(xs, [t, zero], [1, n])
    c2 = g.add(c, g.reshape(xt, (n,)))
    g.copy_into(c, c2)
    y = g.mul(c, two)
    g.dynamic_update_slice(ys, g.reshape(y, (1, n)), [t, zero])
    t2 = g.add(t, one)
    g.copy_into(t, t2)
    body = g.end()
    g.for_loop(T, body)
    g.output(c, ys)
    xs8 = np.arange(n * T, dtype=np.float32).reshape(T, n)
    cr = np.zeros(n, np.float32)
    ysr = np.empty_like(xs8)
    for k in range(T):
        cr = cr + xs8[k]
        ysr[k] = cr * 2.0
    return g.build(), [np.zeros(n, np.float32), xs8], [cr, ysr]


WHILE_CASES = {
    "while_double": while_double, "fori_add": fori_add, "fori_vec": fori_vec,
    "while_multilevel": while_multilevel, "while_zero": while_zero,
    "while_nested": while_nested, "while_then": while_then,
    "scan_stack": scan_stack,
}
