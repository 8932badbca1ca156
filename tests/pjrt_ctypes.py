"""A ctypes driver of the PJRT C API table (libpjrt_amd.so), for the tests: it
makes the calls jaxlib makes -- GetPjrtApi, Client_Create, BufferFromHostBuffer,
Compile, Execute, ToHostBuffer -- without jax (absent from this image).  The
argument structs mirror pjrt-ocl_amd/csrc/pjrt_abi.h field for field."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ABI_HEADER = os.path.join(ROOT, "pjrt-ocl_amd", "csrc", "pjrt_abi.h")
PKG = os.path.join(ROOT, "pjrt-ocl_amd", "python", "pjrt_amd")
PLUGIN = os.path.join(PKG, "libpjrt_amd.so")
LOWER_SERVICE = os.path.join(PKG, "lower_service.py")

VP, SZ = C.c_void_p, C.c_size_t
CODE_NAMES = {0: "OK", 3: "INVALID_ARGUMENT", 5: "NOT_FOUND", 8: "RESOURCE_EXHAUSTED", 9: "FAILED_PRECONDITION",
              12: "UNIMPLEMENTED", 13: "INTERNAL"}
# PJRT_Buffer_Type of numpy dtypes (bf16 travels as uint16 bit patterns)
PJRT_TYPE = {np.dtype("float32"): 11, np.dtype("int32"): 4, np.dtype("uint32"): 8, np.dtype("bool"): 1,
             np.dtype("int64"): 5, np.dtype("float64"): 12, np.dtype("float16"): 10}
BF16 = 13
NUMPY_OF = {11: np.float32, 4: np.int32, 8: np.uint32, 1: np.bool_, 5: np.int64, 12: np.float64, 10: np.float16,
            13: np.uint16}


def slot_names() -> list:
    text = open(ABI_HEADER).read()
    block = text[text.index("#define PJRT_AMD_API_SLOTS"):text.index("enum PjrtAmdSlot")]
    return re.findall(r"X\((\w+)\)", block)


SLOTS = slot_names()


class Version(C.Structure):
    _fields_ = [("struct_size", SZ), ("ext", VP), ("major", C.c_int), ("minor", C.c_int)]


class Api(C.Structure):
    _fields_ = [("struct_size", SZ), ("ext", VP), ("version", Version), ("slots", VP * len(SLOTS))]


def _args(name, fields):
    return type(name, (C.Structure,), {"_fields_": [("struct_size", SZ), ("ext", VP)] + fields})


class NamedValue(C.Structure):
    _fields_ = [("struct_size", SZ), ("ext", VP), ("name", C.c_char_p), ("name_size", SZ), ("type", C.c_int),
                ("value", C.c_int64), ("value_size", SZ)]


class Program(C.Structure):
    _fields_ = [("struct_size", SZ), ("ext", VP), ("code", C.c_char_p), ("code_size", SZ), ("format", C.c_char_p),
                ("format_size", SZ)]


ErrMessage = _args("ErrMessage", [("error", VP), ("message", VP), ("message_size", SZ)])
ErrCode = _args("ErrCode", [("error", VP), ("code", C.c_int)])
ErrDestroy = _args("ErrDestroy", [("error", VP)])
PluginAttrs = _args("PluginAttrs", [("attributes", C.POINTER(NamedValue)), ("num_attributes", SZ)])
ClientCreate = _args("ClientCreate", [("options", C.POINTER(NamedValue)), ("num_options", SZ), ("kv_get", VP),
                                      ("kv_get_arg", VP), ("kv_put", VP), ("kv_put_arg", VP), ("client", VP),
                                      ("kv_try_get", VP), ("kv_try_get_arg", VP)])
ClientOne = _args("ClientOne", [("client", VP)])
ClientName = _args("ClientName", [("client", VP), ("name", VP), ("name_size", SZ)])
ClientDevices = _args("ClientDevices", [("client", VP), ("devices", C.POINTER(VP)), ("num_devices", SZ)])
ClientCompile = _args("ClientCompile", [("client", VP), ("program", C.POINTER(Program)), ("options", VP),
                                        ("options_size", SZ), ("executable", VP)])
FromHost = _args("FromHost", [("client", VP), ("data", VP), ("type", C.c_int), ("dims", C.POINTER(C.c_int64)),
                              ("num_dims", SZ), ("byte_strides", VP), ("num_byte_strides", SZ),
                              ("semantics", C.c_int), ("device", VP), ("memory", VP), ("layout", VP),
                              ("done", VP), ("buffer", VP)])
ToHost = _args("ToHost", [("src", VP), ("layout", VP), ("dst", VP), ("dst_size", SZ), ("event", VP)])
BufOne = _args("BufOne", [("buffer", VP)])
BufType = _args("BufType", [("buffer", VP), ("type", C.c_int)])
BufDims = _args("BufDims", [("buffer", VP), ("dims", C.POINTER(C.c_int64)), ("num_dims", SZ)])
ExecOptions = _args("ExecOptions", [("send_callbacks", VP), ("recv_callbacks", VP), ("num_send_ops", SZ),
                                    ("num_recv_ops", SZ), ("launch_id", C.c_int),
                                    ("non_donatable", C.POINTER(C.c_int64)), ("num_non_donatable", SZ),
                                    ("context", VP)])
BufPointer = _args("BufPointer", [("buffer", VP), ("pointer", C.c_size_t)])
BufDeleted = _args("BufDeleted", [("buffer", VP), ("is_deleted", C.c_bool)])
EventOne = _args("EventOne", [("event", VP)])
EventReady = _args("EventReady", [("event", VP), ("is_ready", C.c_bool)])
OnReadyCb = C.CFUNCTYPE(None, VP, VP)
EventOnReady = _args("EventOnReady", [("event", VP), ("callback", OnReadyCb), ("user_arg", VP)])
BufEvent = _args("BufEvent", [("buffer", VP), ("event", VP)])
ExeOne = _args("ExeOne", [("executable", VP)])
ExeCount = _args("ExeCount", [("executable", VP), ("count", SZ)])
GetExe = _args("GetExe", [("loaded", VP), ("executable", VP)])
Execute = _args("Execute", [("executable", VP), ("options", VP), ("argument_lists", VP), ("num_devices", SZ),
                            ("num_args", SZ), ("output_lists", VP), ("events", VP), ("device", VP)])
DeviceAssign = _args("DeviceAssign", [("executable", VP), ("bytes", VP), ("bytes_size", SZ), ("da", VP),
                                      ("deleter", VP)])
LogicalIds = _args("LogicalIds", [("executable", VP), ("ids", C.POINTER(C.c_int * 2)), ("num_ids", SZ)])
DeviceAttrs = _args("DeviceAttrs", [("device", VP), ("attributes", C.POINTER(NamedValue)), ("num_attributes", SZ),
                                    ("device_attributes", VP), ("deleter", VP)])
ErrPayload = _args("ErrPayload", [("error", VP), ("visitor", VP), ("user_arg", VP)])


class PjrtError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{CODE_NAMES.get(code, code)}] {message}")
        self.code = code
        self.message = message


class Plugin:
    """The plugin's API table and typed calls through it."""

    def __init__(self, path: str = PLUGIN):
        self.lib = C.CDLL(path)
        self.lib.GetPjrtApi.restype = C.POINTER(Api)
        self.api = self.lib.GetPjrtApi().contents

    def fn(self, name):
        return self.api.slots[SLOTS.index(name)]

    def raw(self, name, args):
        """Call a slot; return the PJRT_Error* (0 when the call succeeded)."""
        args.struct_size = C.sizeof(args)
        f = C.CFUNCTYPE(VP, C.c_void_p)(self.fn(name))
        return f(C.addressof(args)) or 0

    def error_info(self, err):
        m = ErrMessage(error=err)
        m.struct_size = C.sizeof(m)
        C.CFUNCTYPE(None, C.c_void_p)(self.fn("PJRT_Error_Message"))(C.addressof(m))
        msg = C.string_at(m.message, m.message_size).decode()
        c = ErrCode(error=err)
        self.raw("PJRT_Error_GetCode", c)
        return c.code, msg

    def destroy_error(self, err):
        d = ErrDestroy(error=err)
        d.struct_size = C.sizeof(d)
        C.CFUNCTYPE(None, C.c_void_p)(self.fn("PJRT_Error_Destroy"))(C.addressof(d))

    def call(self, name, args):
        err = self.raw(name, args)
        if err:
            code, msg = self.error_info(err)
            self.destroy_error(err)
            raise PjrtError(code, msg)
        return args

    # ---- the jaxlib call sequence ----
    def create_client(self, python_exe=None, lower_service=None):
        opts = []
        keep = []
        for k, v in (("python_exe", python_exe), ("lower_service", lower_service)):
            if v is None:
                continue
            kb, vb = k.encode(), v.encode()
            buf = C.create_string_buffer(vb)
            keep.append(buf)
            nv = NamedValue(name=kb, name_size=len(kb), type=0, value_size=len(vb))
            nv.struct_size = C.sizeof(nv)
            nv.value = C.cast(buf, VP).value
            opts.append(nv)
        arr = (NamedValue * max(1, len(opts)))(*opts)
        a = ClientCreate(options=arr, num_options=len(opts))
        self.call("PJRT_Client_Create", a)
        return a.client

    def destroy_client(self, client):
        self.call("PJRT_Client_Destroy", ClientOne(client=client))

    def compile(self, client, text: str | bytes):
        code = text.encode() if isinstance(text, str) else bytes(text)
        prog = Program(code=code, code_size=len(code), format=b"mlir", format_size=4)
        prog.struct_size = C.sizeof(prog)
        a = ClientCompile(client=client, program=C.pointer(prog))
        self.call("PJRT_Client_Compile", a)
        return a.executable

    def to_device(self, client, arr: np.ndarray, bf16: bool = False):
        arr = np.ascontiguousarray(arr)
        dims = (C.c_int64 * max(1, arr.ndim))(*arr.shape)
        a = FromHost(client=client, data=arr.ctypes.data, type=BF16 if bf16 else PJRT_TYPE[arr.dtype], dims=dims,
                     num_dims=arr.ndim)
        self.call("PJRT_Client_BufferFromHostBuffer", a)
        if a.done:
            self.call("PJRT_Event_Destroy", EventOne(event=a.done))
        return a.buffer

    def to_host(self, buf):
        t = self.call("PJRT_Buffer_ElementType", BufType(buffer=buf)).type
        d = self.call("PJRT_Buffer_Dimensions", BufDims(buffer=buf))
        shape = tuple(d.dims[k] for k in range(d.num_dims))
        q = self.call("PJRT_Buffer_ToHostBuffer", ToHost(src=buf))          # size query
        out = np.empty(q.dst_size, np.uint8)
        r = self.call("PJRT_Buffer_ToHostBuffer", ToHost(src=buf, dst=out.ctypes.data, dst_size=out.size))
        if r.event:
            self.call("PJRT_Event_Destroy", EventOne(event=r.event))
        return out.view(NUMPY_OF[t]).reshape(shape), t

    def destroy_buffer(self, buf):
        self.call("PJRT_Buffer_Destroy", BufOne(buffer=buf))

    def num_outputs(self, loaded):
        e = self.call("PJRT_LoadedExecutable_GetExecutable", GetExe(loaded=loaded)).executable
        n = self.call("PJRT_Executable_NumOutputs", ExeCount(executable=e)).count
        self.call("PJRT_Executable_Destroy", ExeOne(executable=e))
        return n

    def execute(self, loaded, buffers, keep_event=False, non_donatable=None):
        """Output buffers of one Execute; with keep_event also its device
        completion event (the caller destroys it).  non_donatable: None passes
        no execute options (nothing donated), else the indices not to donate."""
        n_out = self.num_outputs(loaded)
        opts = None
        if non_donatable is not None:
            nd = (C.c_int64 * max(1, len(non_donatable)))(*non_donatable)
            opts = ExecOptions(non_donatable=C.cast(nd, C.POINTER(C.c_int64)), num_non_donatable=len(non_donatable))
            opts.struct_size = C.sizeof(ExecOptions)
        args = (VP * max(1, len(buffers)))(*buffers)
        arg_lists = (VP * 1)(C.cast(args, VP))
        outs = (VP * max(1, n_out))()
        out_lists = (VP * 1)(C.cast(outs, VP))
        events = (VP * 1)()
        a = Execute(executable=loaded, argument_lists=C.cast(arg_lists, VP), num_devices=1, num_args=len(buffers),
                    output_lists=C.cast(out_lists, VP), events=C.cast(events, VP),
                    options=C.cast(C.pointer(opts), VP) if opts is not None else None)
        self.call("PJRT_LoadedExecutable_Execute", a)
        if keep_event:
            return [outs[k] for k in range(n_out)], events[0]
        if events[0]:
            self.call("PJRT_Event_Destroy", EventOne(event=events[0]))
        return [outs[k] for k in range(n_out)]

    def pointer(self, buf) -> int:
        return self.call("PJRT_Buffer_UnsafePointer", BufPointer(buffer=buf)).pointer

    def is_deleted(self, buf) -> bool:
        return bool(self.call("PJRT_Buffer_IsDeleted", BufDeleted(buffer=buf)).is_deleted)

    # events
    def is_ready(self, ev) -> bool:
        return bool(self.call("PJRT_Event_IsReady", EventReady(event=ev)).is_ready)

    def await_event(self, ev) -> None:
        self.call("PJRT_Event_Await", EventOne(event=ev))

    def on_ready(self, ev, fn):
        """Register fn(error_or_None) and return the ctypes callback (keep it alive)."""
        def cb(err, _arg):
            fn(self.error_info(err) if err else None)
            if err:
                self.destroy_error(err)
        c = OnReadyCb(cb)
        self.call("PJRT_Event_OnReady", EventOnReady(event=ev, callback=c, user_arg=None))
        return c

    def destroy_event(self, ev) -> None:
        self.call("PJRT_Event_Destroy", EventOne(event=ev))

    def ready_event(self, buf):
        return self.call("PJRT_Buffer_ReadyEvent", BufEvent(buffer=buf)).event

    def destroy_executable(self, loaded):
        self.call("PJRT_LoadedExecutable_Destroy", ExeOne(executable=loaded))
