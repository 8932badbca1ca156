#!/usr/bin/env python3
"""Lowering service: the compile-time subprocess of the PJRT plugin.

One-shot mode, the reference's contract (python/pjrt_ocl/lower_service.py:1-64):

    <python_exe> lower_service.py  < program bytes  > VMProgram v3 bytes

  stdin   PJRT_Program.code: a VHLO portable artifact (needs jaxlib to read) or
          StableHLO MLIR text
  stdout  VMProgram v3 bytes (tensor + schedule sections), empty on failure
  stderr  on failure one JSON object {"error": <class>, "message": <str>}
  exit    0 ok, 2 unsupported program (valid input beyond this lowering's
          coverage), 3 internal error

The device parameters come from the environment the plugin sets
(PJRT_OCL_NLANES, PJRT_OCL_EW_TS, PJRT_OCL_MMA_T, PJRT_OCL_COST_TABLE;
plugin.cc:770-780).

Server mode (``--serve``), used by libpjrt_amd.so: the plugin starts one
service process when its client is created and sends it one request per
compile on stdin, so no process is forked per compile.  Frames are
little-endian:

    request   u32 n_lanes, u32 ew_ts, u32 mma_t, u32 cost_length, u64 length,
              the cost table (cost_length bytes of JSON, vmrt_calibrate's), program bytes
    response  u32 status (the one-shot exit code), u32 n_aliases, u64 length, payload
              (v3 bytes when status is 0, else the JSON error), then n_aliases x
              {u32 input, u32 output}: the donations the program can take
              (lowering.donation_aliases)

A request with length 0xFFFFFFFFFFFFFFFF ends the server.
"""
from __future__ import annotations

import json
import os
import struct
import sys

EXIT_OK = 0
EXIT_UNSUPPORTED = 2
EXIT_INTERNAL = 3
_REQ = struct.Struct("<IIIIQ")
_RESP = struct.Struct("<IIQ")
_ALIAS = struct.Struct("<II")
_END = 0xFFFFFFFFFFFFFFFF


def _package():
    if __package__:
        from . import lowering, scheduler
        return lowering, scheduler
    # run as a script: put the package's parent directory on sys.path
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    from pjrt_amd import lowering, scheduler
    return lowering, scheduler


def compile_bytes(program: bytes, cfg=None, with_aliases: bool = False) -> tuple:
    """(status, payload) for one program; with ``with_aliases`` also the
    [(input, output)] donation aliases."""
    try:
        if not program:
            raise ValueError("empty program (expected a VHLO artifact or StableHLO text)")
        lowering, scheduler = _package()
        if cfg is None:
            cfg = scheduler.DeviceConfig.from_env()
        blob, aliases = lowering.lower_and_schedule(program, cfg, with_aliases=True)
        return (EXIT_OK, blob, aliases) if with_aliases else (EXIT_OK, blob)
    except Exception as e:  # noqa: BLE001 -- the service boundary
        msg = json.dumps({"error": type(e).__name__, "message": str(e)}).encode()
        status = EXIT_UNSUPPORTED if isinstance(e, NotImplementedError) else EXIT_INTERNAL
        return (status, msg, []) if with_aliases else (status, msg)


def _read_exact(f, n: int) -> bytes:
    out = bytearray()
    while len(out) < n:
        chunk = f.read(n - len(out))
        if not chunk:
            raise EOFError
        out += chunk
    return bytes(out)


def serve(inp=None, out=None) -> int:
    inp = inp or sys.stdin.buffer
    out = out or sys.stdout.buffer
    _, scheduler = _package()
    while True:
        try:
            lanes, ew_ts, mma_t, cost_n, n = _REQ.unpack(_read_exact(inp, _REQ.size))
        except EOFError:
            return EXIT_OK
        if n == _END:
            return EXIT_OK
        costs = _read_exact(inp, cost_n).decode(errors="replace") if cost_n else ""
        program = _read_exact(inp, n)
        cfg = scheduler.DeviceConfig.from_env()
        if costs:
            cfg.costs = scheduler.load_cost_table(costs)
        if lanes:
            cfg.nlanes = lanes
        if ew_ts:
            cfg.ew_ts = ew_ts
        if mma_t:
            cfg.mma_t = mma_t
        status, payload, aliases = compile_bytes(program, cfg, with_aliases=True)
        out.write(_RESP.pack(status, len(aliases), len(payload)))
        out.write(payload)
        out.write(b"".join(_ALIAS.pack(i, o) for i, o in aliases))
        out.flush()


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if argv and argv[0] == "--serve":
        return serve()
    status, payload = compile_bytes(sys.stdin.buffer.read())
    if status == EXIT_OK:
        sys.stdout.buffer.write(payload)
        sys.stdout.buffer.flush()
    else:
        sys.stderr.write(payload.decode() + "\n")
    return status


if __name__ == "__main__":
    sys.exit(main())
