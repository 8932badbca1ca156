"""VMProgram v3 byte format: golden layout and reader rejections.

Golden bytes restate tests/test_lowering.py:93-171 of the reference (the
hand-built ``b3 = (b0 + b1) - const`` program) field for field."""
import struct

import numpy as np
import pytest

from pjrt_amd import scheduler as S
from pjrt_amd import vmprogram as V
from oracle import vmref

GOLDEN_CFG = S.DeviceConfig(nlanes=8, ew_ts=16384, mma_t=64)


def hand_built():
    const = np.array([1.0, 2.0, 3.0], dtype=np.float32)
    return V.VMProgram(
        arena_bytes=256,
        buffers=[V.Buffer(0, 12), V.Buffer(64, 12), V.Buffer(128, 12), V.Buffer(192, 12)],
        inputs=[0, 1], outputs=[3],
        input_shapes=[(3,), (3,)], output_shapes=[(3,)],
        consts=[(2, const.tobytes())],
        instrs=[V.Instr(V.OP_ADD_F32, dst=3, a=0, b=1, n=3),
                V.Instr(V.OP_SUB_F32, dst=3, a=3, b=2, n=3)],
        main_len=2)


def test_golden_layout_exact_bytes():
    prog = hand_built()
    blob = V.serialize(prog, S.schedule_program(prog, GOLDEN_CFG))
    exp = bytearray()
    exp += struct.pack("<IIIIIIIIIIQ", 0x314D5056, 3, 4, 2, 1, 2, 2, 1, 0, 0, 256)
    for off in (0, 64, 128, 192):
        exp += struct.pack("<QQII", off, 12, 0, 0)
    exp += struct.pack("<II", 0, 1)
    exp += struct.pack("<I", 3) + b"\0" * 4
    for _ in range(3):
        exp += struct.pack("<IIQ", 1, 0, 3)
    exp += struct.pack("<II", 2, 12)
    exp += np.array([1.0, 2.0, 3.0], dtype="<f4").tobytes() + b"\0" * 4
    exp += struct.pack("<8I", 1, 3, 0, 1, 3, 0, 0, 0)
    exp += struct.pack("<8I", 3, 3, 3, 2, 3, 0, 0, 0)
    tensor_len = 48 + 4 * 24 + 16 + 48 + 24 + 2 * 32
    assert tensor_len == 296
    assert blob[:tensor_len] == bytes(exp)

    pos = tensor_len
    n_tasks, n_entries, n_flags, n_lanes = struct.unpack_from("<IIII", blob, pos)
    assert (n_tasks, n_flags, n_lanes) == (2, 0, 8)
    # add then sub (WAW on buffer 3) -> two phases; lane 0: E, BAR, E; others BAR
    assert n_entries == 3 + 7
    pos += 16
    assert struct.unpack_from("<12I", blob, pos) == (V.TOP_EW, 3, 0, 1, V.SUB_ADD, 3,
                                                      0, 0, 0, 0, 0, 0)
    pos += 48 * n_tasks
    assert struct.unpack_from("<II", blob, pos) == (0, 3)
    pos += 16 * n_lanes
    assert struct.unpack_from("<8I", blob, pos) == (0, 0, 1, V.FLAG_NONE, 0,
                                                     V.FLAG_NONE, 0, 0)
    assert struct.unpack_from("<8I", blob, pos + 32) == (V.ENT_BARRIER, 0, 0, V.FLAG_NONE,
                                                          0, V.FLAG_NONE, 0, 0)
    assert len(blob) == tensor_len + 16 + 48 * n_tasks + 16 * n_lanes + 32 * n_entries


def test_roundtrip_and_independent_reader_agree():
    prog = hand_built()
    blob = V.serialize(prog, S.schedule_program(prog, GOLDEN_CFG))
    p2 = V.parse(blob)
    assert V.serialize(p2) == blob
    o = vmref.parse(blob)
    assert o.bufs == [(b.arena_byte_offset, b.size_bytes, b.dtype) for b in p2.buffers]
    assert len(o.tasks) == len(p2.schedule.tasks)
    assert [len(s) for s in o.streams] == [len(s) for s in p2.schedule.lane_streams]


def test_golden_semantics_both_validators():
    prog = hand_built()
    blob = V.serialize(prog, S.schedule_program(prog, GOLDEN_CFG))
    a = np.array([1.5, -2.0, 10.0], np.float32)
    b = np.array([0.5, 4.0, -1.0], np.float32)
    want = a + b - np.array([1, 2, 3], np.float32)
    (x,) = vmref.execute(blob, [a, b])
    (y,) = vmref.execute_schedule(blob, [a, b], ew_ts=16384)
    np.testing.assert_array_equal(x, want)
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("reader", ["product", "oracle"])
def test_reader_rejections(reader):
    parse = V.parse if reader == "product" else vmref.parse
    prog = hand_built()
    good = V.serialize(prog, S.schedule_program(prog, GOLDEN_CFG))
    blob = bytearray(good)
    blob[0] ^= 0xFF
    with pytest.raises(ValueError, match="magic"):
        parse(bytes(blob))
    blob = bytearray(good)
    struct.pack_into("<I", blob, 4, 2)
    with pytest.raises(ValueError, match="version"):
        parse(bytes(blob))
    with pytest.raises(ValueError, match="trailing|mismatch"):
        parse(good + b"\0" * 8)
    with pytest.raises(ValueError):
        parse(good[:40])


def test_product_reader_rejects_bad_schedules():
    prog = hand_built()
    sched = S.schedule_program(prog, GOLDEN_CFG)
    # non-uniform barriers: drop lane 3's barrier
    sched.lane_streams[3] = []
    sched.root_lens[3] = 0
    with pytest.raises(V.FormatError, match="non-uniform"):
        V.parse(V.serialize(prog, sched))
    sched = S.schedule_program(prog, GOLDEN_CFG)
    sched.root_lens[0] = 99
    with pytest.raises(V.FormatError, match="lane"):
        V.parse(V.serialize(prog, sched))
    sched = S.schedule_program(prog, GOLDEN_CFG)
    sched.lane_streams[0][0].task = 77
    with pytest.raises(V.FormatError, match="task index"):
        V.parse(V.serialize(prog, sched))
    sched = S.schedule_program(prog, GOLDEN_CFG)
    sched.tasks[0].tile_op = 40
    with pytest.raises(V.FormatError, match="tile_op"):
        V.parse(V.serialize(prog, sched))
    bad = hand_built()
    bad.buffers[1] = V.Buffer(32, 12)
    with pytest.raises(V.FormatError):
        V.parse(V.serialize(bad))


def test_bf16_rne_closed_form():
    # f32 -> bf16 round-to-nearest-even: (u + 0x7fff + lsb) >> 16
    u = np.array([0x3F800000, 0x3F808000, 0x3F818000, 0x3F807FFF, 0x3F80C000,
                  0x7F7FFFFF, 0xFF800000, 0x00000001], np.uint32)
    got = V.f32_to_bf16(u.view(np.float32))
    want = [0x3F80, 0x3F80, 0x3F82, 0x3F80, 0x3F81, 0x7F80, 0xFF80, 0x0000]
    assert got.tolist() == want
    # ties to even on both sides
    assert vmref.f32_to_bf16(u.view(np.float32)).tolist() == want
    # NaN stays NaN
    nan = np.array([0x7FC00000, 0x7FFFFFFF, 0xFFC00001], np.uint32).view(np.float32)
    back = vmref.bf16_to_f32(vmref.f32_to_bf16(nan))
    assert np.isnan(back).all()
