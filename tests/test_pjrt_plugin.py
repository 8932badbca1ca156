"""The PJRT plugin (libpjrt_amd.so, include/pjrt_amd.h) through its C API table,
driven by ctypes the way jaxlib drives it (no jax in this image: the jax e2e
path itself -- jax.devices() / jax.jit -- is not runnable here).

CPU: the table (version 0.112, every slot populated, UNIMPLEMENTED stubs named
after their call, the four calls jaxlib cannot take as stubs), the lowering
service's one-shot and server contracts.  GPU: Client_Create ->
BufferFromHostBuffer -> Compile (StableHLO text through the lowering service) ->
Execute -> ToHostBuffer, against numpy and the CPU oracle."""
import ctypes as C
import json
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

import hlo_programs as H
import pjrt_ctypes as P

pytestmark = []


def plugin():
    if not os.path.isfile(P.PLUGIN):
        pytest.skip("libpjrt_amd.so not built (make -C pjrt-ocl_amd/csrc)")
    return P.Plugin()


# --- CPU: the table ------------------------------------------------------------------------

def test_api_version_and_every_slot_populated():
    p = plugin()
    assert (p.api.version.major, p.api.version.minor) == (0, 112)
    assert p.api.struct_size == C.sizeof(P.Api)
    assert len(P.SLOTS) == 138
    assert all(p.api.slots[k] for k in range(len(P.SLOTS)))


def test_unimplemented_slots_name_their_call():
    p = plugin()
    for name in ("PJRT_Executable_Serialize", "PJRT_Buffer_CopyToDevice", "PJRT_TopologyDescription_Create"):
        args = P.ErrDestroy()
        err = p.raw(name, args)
        code, msg = p.error_info(err)
        p.destroy_error(err)
        assert code == 12 and name in msg


def test_plugin_attributes_advertise_stablehlo_version():
    p = plugin()
    a = p.call("PJRT_Plugin_Attributes", P.PluginAttrs())
    assert a.num_attributes == 1
    nv = a.attributes[0]
    assert C.string_at(nv.name, nv.name_size) == b"stablehlo_current_version"
    assert nv.type == 2 and nv.value_size == 3
    vals = C.cast(C.c_void_p(nv.value), C.POINTER(C.c_int64))
    assert [vals[k] for k in range(3)] == [1, 17, 0]


def test_calls_jaxlib_cannot_take_as_stubs():
    """Error_ForEachPayload, LoadedExecutable_AddressableDeviceLogicalIds and
    GetDeviceAssignment need no device (plugin.cc:851-861): the assignment is the
    9-byte DeviceAssignmentProto of one replica on device 0."""
    p = plugin()
    assert p.raw("PJRT_Error_ForEachPayload", P.ErrPayload()) == 0
    ids = p.call("PJRT_LoadedExecutable_AddressableDeviceLogicalIds", P.LogicalIds())
    assert ids.num_ids == 1 and list(ids.ids[0]) == [0, 0]
    da = p.call("PJRT_LoadedExecutable_GetDeviceAssignment", P.DeviceAssign())
    raw = C.string_at(da.bytes, da.bytes_size)
    assert raw == bytes([0x08, 0x01, 0x10, 0x01, 0x1A, 0x03, 0x0A, 0x01, 0x00])


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is visible")
def test_client_create_without_a_device_is_an_error():
    p = plugin()
    with pytest.raises(P.PjrtError) as e:
        p.create_client()
    assert e.value.code in (5, 13)


# --- CPU: the lowering service -------------------------------------------------------------

def _service(args, data, env=None):
    return subprocess.run([sys.executable, P.LOWER_SERVICE] + args, input=data, capture_output=True, timeout=120,
                          env={**os.environ, **(env or {})})


def test_lower_service_one_shot_contract():
    r = _service([], H.mlp(16, 8, 32, 4).encode(), {"PJRT_OCL_NLANES": "8"})
    assert r.returncode == 0, r.stderr
    from pjrt_amd import vmprogram as V
    prog = V.parse(r.stdout)
    assert prog.schedule.n_lanes == 8 and len(prog.inputs) == 5
    bad = _service([], H.mlp().replace("stablehlo.maximum", "stablehlo.cholesky").encode())
    assert bad.returncode == 2 and bad.stdout == b""
    err = json.loads(bad.stderr)
    assert err["error"] == "LoweringError" and "cholesky" in err["message"]
    empty = _service([], b"")
    assert empty.returncode == 3 and json.loads(empty.stderr)["error"] == "ValueError"


def test_lower_service_reports_donation_aliases():
    code = H.donated_chain(64).encode()
    req = struct.pack("<IIIIQ", 4, 256, 64, 0, len(code)) + code + struct.pack("<IIIIQ", 0, 0, 0, 0, 0xFFFFFFFFFFFFFFFF)
    r = _service(["--serve"], req)
    assert r.returncode == 0, r.stderr
    st, n_alias, n = struct.unpack_from("<IIQ", r.stdout, 0)
    assert st == 0 and n_alias == 1
    assert struct.unpack_from("<II", r.stdout, 16 + n) == (0, 0)


def test_lower_service_server_frames():
    req = b""
    for text in (H.matmul(64, 32, 48), "not mlir at all"):
        code = text.encode()
        req += struct.pack("<IIIIQ", 4, 256, 64, 0, len(code)) + code
    req += struct.pack("<IIIIQ", 0, 0, 0, 0, 0xFFFFFFFFFFFFFFFF)
    r = _service(["--serve"], req)
    assert r.returncode == 0, r.stderr
    out = r.stdout
    st, _, n = struct.unpack_from("<IIQ", out, 0)
    from pjrt_amd import vmprogram as V
    assert st == 0 and V.parse(out[16:16 + n]).schedule.n_lanes == 4
    st2, _, n2 = struct.unpack_from("<IIQ", out, 16 + n)
    assert st2 == 2 and "LoweringError" in out[32 + n:32 + n + n2].decode()


# --- GPU: the drop-in path ------------------------------------------------------------------

@pytest.mark.gpu
def test_client_compile_execute_mlp():
    """Config 1 as a JAX-shaped StableHLO module, through Client_Create ->
    BufferFromHostBuffer -> Compile -> Execute -> ToHostBuffer."""
    p = plugin()
    print("[gpu] pjrt: client", file=sys.stderr, flush=True)
    client = p.create_client(sys.executable, P.LOWER_SERVICE)
    try:
        name = p.call("PJRT_Client_PlatformName", P.ClientName(client=client))
        assert C.string_at(name.name, name.name_size) == b"mi355x"
        devs = p.call("PJRT_Client_AddressableDevices", P.ClientDevices(client=client))
        assert devs.num_devices == 1
        attrs = p.call("PJRT_Device_GetAttributes", P.DeviceAttrs(device=devs.devices[0]))
        assert attrs.num_attributes >= 1
        from pjrt_amd import configs as CF
        args = CF.mlp_c1_inputs()
        print("[gpu] pjrt: compile", file=sys.stderr, flush=True)
        exe = p.compile(client, H.mlp())
        bufs = [p.to_device(client, a) for a in args]
        print("[gpu] pjrt: execute", file=sys.stderr, flush=True)
        for _ in range(2):
            (out,) = p.execute(exe, bufs)
            y, t = p.to_host(out)
            p.destroy_buffer(out)
            assert t == 11 and y.shape == (256, 64)
            x, w1, b1, w2, b2 = (a.astype(np.float64) for a in args)
            want = np.maximum(x @ w1 + b1, 0) @ w2 + b2
            assert np.abs(y - want).max() <= 1e-3 * np.abs(want).max()
        with pytest.raises(P.PjrtError) as e:
            p.execute(exe, bufs[:4])
        assert e.value.code == 3
        for b in bufs:
            p.destroy_buffer(b)
        p.destroy_executable(exe)
    finally:
        p.destroy_client(client)


@pytest.mark.gpu
def test_client_compile_execute_fused_programs():
    """Config 2's layernorm + GELU + bf16 and a causal bf16 attention, lowered
    and fused by the service, executed through the plugin, against the CPU
    oracle's execution of the same lowering."""
    from oracle import vmref
    from pjrt_amd import lowering as L
    from pjrt_amd import scheduler as S
    from pjrt_amd import vmprogram as V
    p = plugin()
    client = p.create_client(sys.executable, P.LOWER_SERVICE)
    try:
        rng = np.random.default_rng(1002)
        x = rng.standard_normal((256, 4096)).astype(np.float32)
        g = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
        b = (rng.standard_normal(4096) * 0.1).astype(np.float32)
        text = H.ln_gelu(256, 4096)
        exe = p.compile(client, text)
        bufs = [p.to_device(client, a) for a in (x, g, b)]
        (out,) = p.execute(exe, bufs)
        got, t = p.to_host(out)
        assert t == P.BF16
        prog = L.lower_text(text)
        cfg = S.DeviceConfig(nlanes=8, ew_ts=4096, mma_t=128)
        (want,) = vmref.execute(V.serialize(prog, S.schedule_program(prog, cfg)), [x, g, b])
        gf, wf = vmref.bf16_to_f32(got).astype(np.float64), vmref.bf16_to_f32(want).astype(np.float64)
        assert np.all(np.abs(gf - wf) <= 2.0 ** -7 * np.abs(wf) + 1e-6)
        for bb in bufs + [out]:
            p.destroy_buffer(bb)
        p.destroy_executable(exe)

        B, Hh, T, D = 1, 4, 256, 128
        q, k, v = (vmref.f32_to_bf16(rng.standard_normal((B, Hh, T, D)).astype(np.float32)) for _ in range(3))
        exe = p.compile(client, H.attention(B, Hh, T, D))
        bufs = [p.to_device(client, a, bf16=True) for a in (q, k, v)]
        (out,) = p.execute(exe, bufs)
        got, _ = p.to_host(out)
        qf, kf, vf = (vmref.bf16_to_f32(a).astype(np.float64) for a in (q, k, v))
        s = np.einsum("bhqd,bhkd->bhqk", qf, kf) * D ** -0.5
        s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
        pr = np.exp(s - s.max(-1, keepdims=True))
        pr /= pr.sum(-1, keepdims=True)
        want = pr @ vf
        gf = vmref.bf16_to_f32(got).astype(np.float64)
        assert np.abs(gf - want).max() <= 1e-2 * np.abs(want).max()
        for bb in bufs + [out]:
            p.destroy_buffer(bb)
        p.destroy_executable(exe)
        with pytest.raises(P.PjrtError) as e:
            p.compile(client, H.mlp().replace("stablehlo.maximum", "stablehlo.cholesky"))
        assert e.value.code == 12 and "cholesky" in e.value.message
    finally:
        p.destroy_client(client)


@pytest.mark.gpu
def test_execute_is_asynchronous_with_real_events():
    """Execute returns once the program is launched: its completion event and its
    outputs' ready events complete with the launch (IsReady, Await, OnReady on
    the client's waiter thread), later launches and copies are ordered after it
    on the one stream, and results read back after two back-to-back Executes
    are both right."""
    import threading
    p = plugin()
    client = p.create_client(sys.executable, P.LOWER_SERVICE)
    try:
        rng = np.random.default_rng(2024)
        a = rng.standard_normal((1024, 1024)).astype(np.float32)
        b = rng.standard_normal((1024, 1024)).astype(np.float32)
        exe = p.compile(client, H.matmul(1024, 1024, 1024, "f32", "f32"))
        bufs = [p.to_device(client, x) for x in (a, b)]
        print("[gpu] pjrt: async executes", file=sys.stderr, flush=True)
        (o1,), e1 = p.execute(exe, bufs, keep_event=True)
        (o2,), e2 = p.execute(exe, [o1, bufs[1]], keep_event=True)     # consumes o1 on the same stream
        seen, done = [], threading.Event()

        def cb(err):
            seen.append(err)
            done.set()
        keep = p.on_ready(e2, cb)
        p.await_event(e1)
        assert p.is_ready(e1)
        r2 = p.ready_event(o2)
        p.await_event(r2)
        assert p.is_ready(r2) and p.is_ready(e2)
        assert done.wait(30) and seen == [None]
        got1, _ = p.to_host(o1)
        got2, _ = p.to_host(o2)
        w1 = a.astype(np.float64) @ b
        w2 = got1.astype(np.float64) @ b
        assert np.abs(got1 - w1).max() <= 1e-3 * np.abs(w1).max()
        assert np.abs(got2 - w2).max() <= 1e-3 * np.abs(w2).max()
        for ev in (e1, e2, r2):
            p.destroy_event(ev)
        del keep
        for bb in bufs + [o1, o2]:
            p.destroy_buffer(bb)
        p.destroy_executable(exe)
    finally:
        p.destroy_client(client)


@pytest.mark.gpu
def test_execute_donates_an_aliased_argument():
    """(x @ w) @ w with x donated: the output takes x's device memory and x is
    deleted; with x listed as non-donatable, or with no execute options, the
    output gets memory of its own and x stays alive.  Results equal numpy."""
    p = plugin()
    client = p.create_client(sys.executable, P.LOWER_SERVICE)
    try:
        rng = np.random.default_rng(2025)
        x = rng.standard_normal((256, 256)).astype(np.float32)
        w = (rng.standard_normal((256, 256)) * 0.1).astype(np.float32)
        want = (x.astype(np.float64) @ w) @ w
        exe = p.compile(client, H.donated_chain(256))
        for nd in (None, [0], []):
            print(f"[gpu] pjrt: donation, non-donatable {nd}", file=sys.stderr, flush=True)
            xb, wb = p.to_device(client, x), p.to_device(client, w)
            xptr = p.pointer(xb)
            (out,) = p.execute(exe, [xb, wb], non_donatable=nd)
            got, _ = p.to_host(out)
            assert np.abs(got - want).max() <= 1e-3 * np.abs(want).max()
            donated = nd == []
            assert p.is_deleted(xb) == donated
            assert (p.pointer(out) == xptr) == donated
            for bb in (xb, wb, out):
                p.destroy_buffer(bb)
        p.destroy_executable(exe)
    finally:
        p.destroy_client(client)
