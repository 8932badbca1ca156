"""ctypes binding of libvmrt.so, the MI355X VM runtime.

Mirrors the reference runtime's host interface (pjrt_plugin/src/runtime.h):

    OclRuntime        -> Runtime        (device, pool, stream, scheduling params)
    LoadedProgram     -> LoadedProgram  (arena, tables, execute)
    cl_mem buffers    -> DeviceBuffer   (pool-owned device memory)

Errors carry the PJRT status code the runtime returns (INVALID_ARGUMENT for a
malformed program or bad arguments, UNIMPLEMENTED for tile ops outside this build,
INTERNAL for launch/VM failures), like the reference's `bool + std::string* err`
convention mapped to PJRT codes (plugin.cc:588-592, 944-972).

There is no CPU fallback: if the library is missing or no MI355X is visible,
constructing a Runtime raises.
"""
from __future__ import annotations

import ctypes
import dataclasses
import sys
import threading
import weakref

import numpy as np

from . import find_runtime_library
from . import scheduler as S
from . import vmprogram as V

OK = 0
INVALID_ARGUMENT = 3
NOT_FOUND = 5
RESOURCE_EXHAUSTED = 8
FAILED_PRECONDITION = 9
UNIMPLEMENTED = 12
INTERNAL = 13
UNAVAILABLE = 14
CODE_NAMES = {OK: "OK", INVALID_ARGUMENT: "INVALID_ARGUMENT", NOT_FOUND: "NOT_FOUND",
              RESOURCE_EXHAUSTED: "RESOURCE_EXHAUSTED", FAILED_PRECONDITION: "FAILED_PRECONDITION",
              UNIMPLEMENTED: "UNIMPLEMENTED", INTERNAL: "INTERNAL", UNAVAILABLE: "UNAVAILABLE"}


class VmrtError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{CODE_NAMES.get(code, code)}] {message}")
        self.code = code
        self.message = message


class _Options(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int32), ("n_lanes", ctypes.c_uint32), ("ew_ts", ctypes.c_uint32),
                ("mma_t", ctypes.c_uint32), ("cooperative", ctypes.c_uint32),
                ("barrier_timeout_ms", ctypes.c_uint32)]


class _DeviceInfo(ctypes.Structure):
    _fields_ = [("n_lanes", ctypes.c_uint32), ("max_lanes", ctypes.c_uint32), ("ew_ts", ctypes.c_uint32),
                ("mma_t", ctypes.c_uint32), ("compute_units", ctypes.c_uint32),
                ("lanes_per_cu", ctypes.c_uint32), ("lds_bytes", ctypes.c_uint32),
                ("cooperative", ctypes.c_uint32), ("arch", ctypes.c_char * 64),
                ("name", ctypes.c_char * 128)]


_VP = ctypes.c_void_p
_SZ = ctypes.c_size_t
_CP = ctypes.c_char_p
_U32 = ctypes.c_uint32
_PU32 = ctypes.POINTER(ctypes.c_uint32)
_PU64 = ctypes.POINTER(ctypes.c_uint64)

# name -> (restype, argtypes); every symbol include/vmrt.h declares
SIGNATURES = {
    "vmrt_version": (ctypes.c_char_p, []),
    "vmrt_default_options": (None, [ctypes.POINTER(_Options)]),
    "vmrt_create": (ctypes.c_int, [ctypes.POINTER(_Options), ctypes.POINTER(_VP), _CP, _SZ]),
    "vmrt_destroy": (None, [_VP]),
    "vmrt_device_info_get": (ctypes.c_int, [_VP, ctypes.POINTER(_DeviceInfo)]),
    "vmrt_load": (ctypes.c_int, [_VP, _VP, _SZ, _U32, _U32, ctypes.POINTER(_VP), _CP, _SZ]),
    "vmrt_unload": (None, [_VP]),
    "vmrt_program_counts": (ctypes.c_int, [_VP, _PU32, _PU32, _PU32]),
    "vmrt_program_io": (ctypes.c_int, [_VP, ctypes.c_int, _U32, _PU32, _PU64, _PU32, _PU64]),
    "vmrt_execute": (ctypes.c_int, [_VP, ctypes.POINTER(_VP), _SZ, ctypes.POINTER(_VP), _SZ, _CP, _SZ]),
    "vmrt_enqueue": (ctypes.c_int, [_VP, ctypes.POINTER(_VP), _SZ, ctypes.POINTER(_VP), _SZ, _VP, _CP, _SZ]),
    "vmrt_program_status": (ctypes.c_int, [_VP, _CP, _SZ]),
    "vmrt_submit": (ctypes.c_int, [_VP, ctypes.POINTER(_VP), _SZ, ctypes.POINTER(_VP), _SZ, ctypes.POINTER(_VP), _CP,
                                   _SZ]),
    "vmrt_launch_query": (ctypes.c_int, [_VP]),
    "vmrt_launch_wait": (ctypes.c_int, [_VP, _CP, _SZ]),
    "vmrt_launch_release": (None, [_VP]),
    "vmrt_run_noalloc": (ctypes.c_int, [_VP, _VP, _SZ, _U32, _U32, ctypes.POINTER(_VP), _SZ, ctypes.POINTER(_VP),
                                        _SZ, _CP, _SZ]),
    "vmrt_program_profile": (ctypes.c_int, [_VP, ctypes.POINTER(ctypes.c_uint64), _SZ, ctypes.c_int, _CP, _SZ]),
    "vmrt_alloc": (ctypes.c_int, [_VP, _SZ, ctypes.POINTER(_VP), _CP, _SZ]),
    "vmrt_free": (ctypes.c_int, [_VP, _VP]),
    "vmrt_h2d": (ctypes.c_int, [_VP, _VP, _VP, _SZ, _CP, _SZ]),
    "vmrt_d2h": (ctypes.c_int, [_VP, _VP, _VP, _SZ, _CP, _SZ]),
    "vmrt_d2d": (ctypes.c_int, [_VP, _VP, _VP, _SZ, _CP, _SZ]),
    "vmrt_synchronize": (ctypes.c_int, [_VP, _CP, _SZ]),
    "vmrt_calibrate": (ctypes.c_int, [_VP, _CP, _SZ, _CP, _SZ]),
    "vmrt_stream": (_VP, [_VP]),
    "vmrt_event_create": (ctypes.c_int, [_VP, ctypes.POINTER(_VP)]),
    "vmrt_event_record": (ctypes.c_int, [_VP, _VP, _VP]),
    "vmrt_event_elapsed_ms": (ctypes.c_int, [_VP, _VP, ctypes.POINTER(ctypes.c_float)]),
    "vmrt_event_destroy": (None, [_VP]),
    "vmrt_event_query": (ctypes.c_int, [_VP]),
    "vmrt_event_synchronize": (ctypes.c_int, [_VP]),
}

_lib = None
_lib_lock = threading.Lock()


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load libvmrt.so and bind every exported entry point (raises if a symbol
    include/vmrt.h declares is missing)."""
    global _lib
    with _lib_lock:
        if _lib is not None and path is None:
            return _lib
        lib = ctypes.CDLL(path or find_runtime_library())
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


_ERRLEN = 1024


def _check(rc: int, err) -> None:
    if rc != OK:
        raise VmrtError(rc, err.value.decode(errors="replace") if err is not None else "")


def _ptr_of(x) -> int:
    """Device address of a DeviceBuffer, a torch CUDA tensor or a raw int."""
    if isinstance(x, DeviceBuffer):
        return x.ptr
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        if hasattr(x, "is_cuda") and not x.is_cuda:
            raise ValueError("torch tensor argument must live on the GPU")
        if hasattr(x, "is_contiguous") and not x.is_contiguous():
            raise ValueError("torch tensor argument must be contiguous")
        return int(x.data_ptr())
    raise TypeError(f"not a device buffer: {type(x).__name__}")


class DeviceBuffer:
    """Pool-owned device memory (OclRuntime::PoolAlloc / PoolFree)."""

    def __init__(self, rt: "Runtime", ptr: int, nbytes: int):
        self.rt = rt
        self.ptr = ptr
        self.nbytes = nbytes

    def to_host(self, dtype=np.uint8, shape=None) -> np.ndarray:
        out = np.empty(self.nbytes, np.uint8)
        if self.nbytes:
            self.rt.d2h(out.ctypes.data, self.ptr, self.nbytes)
        out = out.view(dtype)
        return out.reshape(shape) if shape is not None else out

    def write(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"write of {arr.nbytes} bytes into a {self.nbytes}-byte buffer")
        if self.nbytes:
            self.rt.h2d(self.ptr, arr.ctypes.data, self.nbytes)

    def free(self) -> None:
        if self.ptr and self.rt._h:
            self.rt._lib.vmrt_free(self.rt._h, _VP(self.ptr))
        self.ptr = 0          # after Runtime.close the pool has already released it

    def __del__(self):
        # no native call while the interpreter shuts down: the HIP runtime's own
        # exit handlers (and a profiler's) may already have run
        if sys.is_finalizing():
            return
        try:
            self.free()
        except Exception:
            pass


class Runtime:
    """One HIP device with the VM kernel prepared (OclRuntime::Create)."""

    def __init__(self, device: int = 0, n_lanes: int = 0, ew_ts: int = 0, mma_t: int = 0,
                 cooperative: bool | None = None, barrier_timeout_ms: int = 0, library: str | None = None):
        self._lib = load_library(library)
        opts = _Options()
        self._lib.vmrt_default_options(ctypes.byref(opts))
        opts.device, opts.n_lanes, opts.ew_ts, opts.mma_t = device, n_lanes, ew_ts, mma_t
        if cooperative is not None:
            opts.cooperative = 1 if cooperative else 0
        opts.barrier_timeout_ms = barrier_timeout_ms
        h = _VP()
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self._lib.vmrt_create(ctypes.byref(opts), ctypes.byref(h), err, _ERRLEN), err)
        self._h = h
        self._programs = weakref.WeakSet()      # live LoadedPrograms
        info = _DeviceInfo()
        self._lib.vmrt_device_info_get(self._h, ctypes.byref(info))
        self.info = {k: getattr(info, k) for k, _ in _DeviceInfo._fields_}
        self.info["arch"] = info.arch.decode()
        self.info["name"] = info.name.decode()

    # ---- scheduling contract (PJRT_OCL_NLANES / _EW_TS / _MMA_T) ----
    def scheduler_config(self, **overrides) -> S.DeviceConfig:
        """The scheduler's knobs from the environment (DeviceConfig.from_env),
        with the lane count and tile sizes this runtime advertises."""
        cfg = S.DeviceConfig.from_env()
        cfg.nlanes, cfg.ew_ts, cfg.mma_t = self.info["n_lanes"], self.info["ew_ts"], self.info["mma_t"]
        for k, v in overrides.items():
            setattr(cfg, k, v)
        return cfg

    def lowering_env(self) -> dict:
        """The environment the plugin hands the lowering subprocess
        (plugin.cc:770-780)."""
        return {"PJRT_OCL_NLANES": str(self.info["n_lanes"]), "PJRT_OCL_EW_TS": str(self.info["ew_ts"]),
                "PJRT_OCL_MMA_T": str(self.info["mma_t"])}

    @property
    def stream(self) -> int:
        return int(self._lib.vmrt_stream(self._h) or 0)

    def close(self) -> None:
        """Unload every live program, then release the device (vmrt_destroy,
        which also returns the pool's memory).  Programs and buffers of a closed
        runtime are dead: their close/free do nothing, execute raises."""
        if getattr(self, "_h", None):
            for lp in list(self._programs):
                lp.close()
            self._lib.vmrt_destroy(self._h)
            self._h = None

    @property
    def closed(self) -> bool:
        return not getattr(self, "_h", None)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass

    # ---- memory ----
    def alloc(self, nbytes: int) -> DeviceBuffer:
        p = _VP()
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self._lib.vmrt_alloc(self._h, nbytes, ctypes.byref(p), err, _ERRLEN), err)
        return DeviceBuffer(self, int(p.value or 0), nbytes)

    def to_device(self, arr: np.ndarray) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        buf = self.alloc(arr.nbytes)
        buf.write(arr)
        return buf

    def h2d(self, dst: int, src: int, n: int) -> None:
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self._lib.vmrt_h2d(self._h, _VP(dst), _VP(src), n, err, _ERRLEN), err)

    def d2h(self, dst: int, src: int, n: int) -> None:
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self._lib.vmrt_d2h(self._h, _VP(dst), _VP(src), n, err, _ERRLEN), err)

    def d2d(self, dst: int, src: int, n: int) -> None:
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self._lib.vmrt_d2d(self._h, _VP(dst), _VP(src), n, err, _ERRLEN), err)

    def synchronize(self) -> None:
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self._lib.vmrt_synchronize(self._h, err, _ERRLEN), err)

    def calibrate(self) -> dict:
        """The measured cost table (vmrt_calibrate) as a dict; the scheduler
        takes it as DeviceConfig.costs (or as the JSON file PJRT_OCL_COST_TABLE
        names)."""
        import json
        buf = ctypes.create_string_buffer(4096)
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self._lib.vmrt_calibrate(self._h, buf, 4096, err, _ERRLEN), err)
        return json.loads(buf.value.decode())

    def event(self) -> "Event":
        return Event(self)

    # ---- programs ----
    def load(self, blob: bytes, ew_ts: int = 0, mma_t: int = 0) -> "LoadedProgram":
        blob = bytes(blob)
        buf = ctypes.create_string_buffer(blob, len(blob))
        p = _VP()
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self._lib.vmrt_load(self._h, ctypes.cast(buf, _VP), len(blob), ew_ts, mma_t, ctypes.byref(p),
                                   err, _ERRLEN), err)
        lp = LoadedProgram(self, p)
        lp._blob = blob
        self._programs.add(lp)
        return lp

    def run_noalloc(self, blob: bytes, inputs, outputs, ew_ts: int = 0, mma_t: int = 0) -> None:
        """Run a program once on device buffers without allocating device memory
        (vmrt_run_noalloc: the program lives in the library's static 64 MiB
        array; synchronous)."""
        blob = bytes(blob)
        buf = ctypes.create_string_buffer(blob, len(blob))
        ins = (_VP * max(1, len(inputs)))(*[_ptr_of(x) for x in inputs])
        outs = (_VP * max(1, len(outputs)))(*[_ptr_of(x) for x in outputs])
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self._lib.vmrt_run_noalloc(self._h, ctypes.cast(buf, _VP), len(blob), ew_ts, mma_t, ins, len(inputs),
                                          outs, len(outputs), err, _ERRLEN), err)

    def compile(self, prog: V.VMProgram, arena_reuse: bool = True, **cfg_overrides) -> "LoadedProgram":
        """Schedule a tensor program for this device and load it.  With
        `arena_reuse` the buffers of a copy of the program are first packed by
        liveness (passes.reuse_arena, as the lowering does); `prog` itself is
        left as it is."""
        cfg = self.scheduler_config(**cfg_overrides)
        if arena_reuse:
            from . import passes
            prog = dataclasses.replace(prog, buffers=[dataclasses.replace(b) for b in prog.buffers])
            passes.reuse_arena(prog, cfg)
        blob = V.serialize(prog, S.schedule_program(prog, cfg))
        return self.load(blob, ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)


class Event:
    """A HIP event recorded on a stream (default: the runtime's)."""

    def __init__(self, rt: Runtime):
        self.rt = rt
        self._e = _VP()
        rc = rt._lib.vmrt_event_create(rt._h, ctypes.byref(self._e))
        if rc != OK:
            raise VmrtError(rc, "event create")

    def record(self, stream: int | None = None) -> None:
        rc = self.rt._lib.vmrt_event_record(self.rt._h, self._e, _VP(stream or 0))
        if rc != OK:
            raise VmrtError(rc, "event record")

    def query(self) -> bool:
        """Whether the work recorded before the event has completed."""
        rc = self.rt._lib.vmrt_event_query(self._e)
        if rc not in (OK, UNAVAILABLE):
            raise VmrtError(rc, "event query")
        return rc == OK

    def synchronize(self) -> None:
        rc = self.rt._lib.vmrt_event_synchronize(self._e)
        if rc != OK:
            raise VmrtError(rc, "event synchronize")

    def elapsed_ms(self, stop: "Event") -> float:
        ms = ctypes.c_float()
        rc = self.rt._lib.vmrt_event_elapsed_ms(self._e, stop._e, ctypes.byref(ms))
        if rc != OK:
            raise VmrtError(rc, "event elapsed")
        return float(ms.value)

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.rt._lib.vmrt_event_destroy(self._e)
        except Exception:
            pass


class Launch:
    """One submitted launch and its own status (vmrt_submit)."""

    def __init__(self, rt: Runtime, handle):
        self.rt = rt
        self._h = handle

    def done(self) -> bool:
        """Whether the launch has completed (no wait)."""
        rc = self.rt._lib.vmrt_launch_query(self._h)
        if rc not in (OK, UNAVAILABLE):
            raise VmrtError(rc, "launch query")
        return rc == OK

    def wait(self) -> None:
        """Wait for the launch; raise if it aborted."""
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self.rt._lib.vmrt_launch_wait(self._h, err, _ERRLEN), err)

    def release(self) -> None:
        h, self._h = self._h, None
        if h and not self.rt.closed:
            self.rt._lib.vmrt_launch_release(h)

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.release()
        except Exception:
            pass


class IOSpec:
    def __init__(self, dtype: int, nbytes: int, shape: tuple):
        self.dtype, self.nbytes, self.shape = dtype, nbytes, shape

    @property
    def np_dtype(self):
        return V.DT_NUMPY[self.dtype]

    def __repr__(self):
        return f"IOSpec({V.DT_NAMES[self.dtype]}, {self.shape})"


class LoadedProgram:
    """A loaded VMProgram (LoadedProgram::Load / ExecuteDevice)."""

    def __init__(self, rt: Runtime, handle):
        self.rt = rt
        self._h = handle
        lib = rt._lib
        ni, no, nl = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        lib.vmrt_program_counts(self._h, ctypes.byref(ni), ctypes.byref(no), ctypes.byref(nl))
        self.n_lanes = nl.value
        self.inputs = [self._io(0, i) for i in range(ni.value)]
        self.outputs = [self._io(1, i) for i in range(no.value)]

    def _io(self, is_out: int, i: int) -> IOSpec:
        dt, rank = ctypes.c_uint32(), ctypes.c_uint32()
        nbytes = ctypes.c_uint64()
        dims = (ctypes.c_uint64 * 16)()
        self.rt._lib.vmrt_program_io(self._h, is_out, i, ctypes.byref(dt), ctypes.byref(nbytes), ctypes.byref(rank),
                                     dims)
        return IOSpec(dt.value, nbytes.value, tuple(int(dims[k]) for k in range(rank.value)))

    def close(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        if h and not self.rt.closed:        # a closed runtime has unloaded it already
            self.rt._lib.vmrt_unload(h)

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass

    def _live(self):
        if not getattr(self, "_h", None) or self.rt.closed:
            raise VmrtError(FAILED_PRECONDITION, "program is closed (or its runtime is)")
        return self._h

    def _arrays(self, inputs, outputs):
        if len(inputs) != len(self.inputs):
            raise VmrtError(INVALID_ARGUMENT, f"expected {len(self.inputs)} inputs, got {len(inputs)}")
        if len(outputs) != len(self.outputs):
            raise VmrtError(INVALID_ARGUMENT, f"expected {len(self.outputs)} outputs, got {len(outputs)}")
        ins = (_VP * max(1, len(inputs)))(*[_ptr_of(x) for x in inputs])
        outs = (_VP * max(1, len(outputs)))(*[_ptr_of(x) for x in outputs])
        return ins, outs

    def alloc_outputs(self) -> list:
        return [self.rt.alloc(o.nbytes) for o in self.outputs]

    def execute(self, inputs, outputs=None) -> list:
        """Run on device buffers and wait; returns the output buffers."""
        if outputs is None:
            outputs = self.alloc_outputs()
        ins, outs = self._arrays(inputs, outputs)
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self.rt._lib.vmrt_execute(self._live(), ins, len(inputs), outs, len(outputs), err, _ERRLEN), err)
        return outputs

    def enqueue(self, inputs, outputs, stream: int | None = None) -> None:
        """Launch without waiting (on `stream`, default the runtime's)."""
        ins, outs = self._arrays(inputs, outputs)
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self.rt._lib.vmrt_enqueue(self._live(), ins, len(inputs), outs, len(outputs), _VP(stream or 0), err,
                                         _ERRLEN), err)

    def submit(self, inputs, outputs) -> "Launch":
        """Launch on the runtime's stream with a status of its own (vmrt_submit)."""
        ins, outs = self._arrays(inputs, outputs)
        err = ctypes.create_string_buffer(_ERRLEN)
        h = _VP()
        _check(self.rt._lib.vmrt_submit(self._live(), ins, len(inputs), outs, len(outputs), ctypes.byref(h), err,
                                        _ERRLEN), err)
        return Launch(self.rt, h)

    def status(self) -> None:
        """Synchronize and raise if the VM aborted (barrier time-out etc.)."""
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self.rt._lib.vmrt_program_status(self._live(), err, _ERRLEN), err)

    def profile(self, reset: bool = True) -> dict:
        """Per-task device time since the last reset (the program must have been
        loaded with PJRT_AMD_PROFILE=1): {"barrier_us", "barriers", "lane_us"
        (launch start to each lane's end, summed over lanes), "flag_us"
        (completion-flag waits), "tasks": [(task, lane_us_sum, max_entry_us,
        entries)]}, microseconds."""
        n_tasks = len(V.parse(self._blob).schedule.tasks)
        words = 4 + 4 * n_tasks
        buf = (ctypes.c_uint64 * words)()
        err = ctypes.create_string_buffer(_ERRLEN)
        _check(self.rt._lib.vmrt_program_profile(self._live(), buf, words, int(reset), err, _ERRLEN), err)
        v = np.frombuffer(buf, np.uint64).astype(np.float64)
        return {"barrier_us": v[0] / 100.0, "barriers": int(v[1]), "lane_us": v[2] / 100.0, "flag_us": v[3] / 100.0,
                "tasks": [(i, v[4 + 4 * i] / 100.0, v[5 + 4 * i] / 100.0, int(v[6 + 4 * i])) for i in range(n_tasks)]}

    def __call__(self, *args):
        """Host convenience: numpy arrays in, numpy arrays out."""
        self._live()
        if len(args) != len(self.inputs):
            raise VmrtError(INVALID_ARGUMENT, f"expected {len(self.inputs)} inputs, got {len(args)}")
        dev_in = []
        for a, spec in zip(args, self.inputs):
            a = np.ascontiguousarray(a)
            if spec.dtype == V.DT_BF16 and a.dtype != np.uint16:
                a = V.f32_to_bf16(a.astype(np.float32))
            elif spec.dtype == V.DT_BOOL:
                a = a.astype(np.uint8)
            else:
                a = a.astype(spec.np_dtype, copy=False)
            if a.nbytes != spec.nbytes:
                raise VmrtError(INVALID_ARGUMENT, f"input of {a.nbytes} bytes, program expects {spec.nbytes}")
            dev_in.append(self.rt.to_device(a))
        outs = self.execute(dev_in)
        res = [o.to_host(spec.np_dtype, spec.shape) for o, spec in zip(outs, self.outputs)]
        for b in dev_in + outs:
            b.free()
        return res
