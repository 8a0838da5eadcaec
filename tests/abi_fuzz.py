"""Drive every C-ABI entry point with random, mostly invalid arguments.

Run as a child process by test_host_sanitizers.py, against a build of the
library whose host code carries AddressSanitizer and UndefinedBehaviorSanitizer
checks, on a machine where no GPU is visible: device pointers are fake
addresses that the host side must never dereference, so a call that passes
every argument check ends in a HIP error (no device), never in a launch.

Every call must return a documented status (or a size), leave a readable
dels_last_error(), and trip no sanitizer; the sanitizers abort the process on
the first report.  Graph handles and streams are host objects, passed only as
NULL.

Usage: python tests/abi_fuzz.py [calls_per_entry_point] [seed]
"""

from __future__ import annotations

import ctypes
import math
import os
import random
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)


def main() -> int:
    import torch

    if torch.cuda.device_count() != 0:
        print("abi_fuzz: a GPU is visible; refusing to pass fake device pointers", flush=True)
        return 2
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    L = pkg._lib
    lib = L.load()
    n = int(sys.argv[1]) if len(sys.argv) > 1 else 300
    rng = random.Random(int(sys.argv[2]) if len(sys.argv) > 2 else 1234)

    plausible = [1, 8, 16, 32, 64, 128, 256, 512, 1024, 4096, 151936]
    extreme = [-1, 0, 2**31 - 1, 2**31 + 5, 2**40, 2**62, -(2**62), 2**63 - 1]
    fake_ok = 0x7F0000000000          # 256-byte aligned, never mapped here
    fake_odd = 0x7F0000000002

    def i64():
        return rng.choice(plausible) if rng.random() < 0.7 else rng.choice(extreme)

    def i32():
        return rng.choice([0, 1, 2, 3]) if rng.random() < 0.8 else rng.choice([-1, 7, 2**31 - 1, -(2**31)])

    def ptr():
        r = rng.random()
        return fake_ok if r < 0.8 else (None if r < 0.9 else fake_odd)

    def size():
        return rng.choice([1 << 30, 1 << 40]) if rng.random() < 0.7 else rng.choice([0, 256, 2**64 - 1])

    def f32():
        return rng.choice([0.0, 1.0, 0.5, -1.0, 1e-6, math.nan, math.inf, -math.inf])

    def u64():
        return rng.choice([0, 1, 2**63, 2**64 - 1, 12345])

    def value(t):
        if t is L._ptr:
            return ptr()
        if t is L._i64:
            return i64()
        if t is L._int:
            return i32()
        if t is L._sz:
            return size()
        if t is ctypes.c_float:
            return f32()
        if t is ctypes.c_uint64:
            return u64()
        raise TypeError(t)

    def fill(struct_type):
        p = struct_type()
        for name, t in struct_type._fields_:
            setattr(p, name, value(t))
        return p

    statuses = {0, -1, -2, -3, -4, -5}
    calls = 0
    for name, (res, argtypes) in L.SIGNATURES.items():
        fn = getattr(lib, name)
        for _ in range(n):
            args = []
            keep = []
            for i, t in enumerate(argtypes):
                host_object = name in ("dels_graph_launch", "dels_graph_destroy") or (
                    res is L._int and t is L._ptr and i == len(argtypes) - 1)   # graph handle or stream
                if host_object:
                    args.append(None)
                elif isinstance(t, type) and issubclass(t, ctypes._Pointer):
                    if t._type_ is L._ptr:                      # graph handle out-parameter
                        h = L._ptr()
                        keep.append(h)
                        args.append(ctypes.byref(h) if rng.random() < 0.9 else None)
                    else:                                       # rollout parameter struct
                        s = fill(t._type_)
                        keep.append(s)
                        args.append(ctypes.byref(s) if rng.random() < 0.95 else None)
                else:
                    args.append(value(t))
            out = fn(*args)
            calls += 1
            if res is L._int and name not in ("dels_abi_version", "dels_debug_set_decode_spin_limit",
                                              "dels_debug_set_rollout_resident",
                                              "dels_debug_set_resident_spin_limit"):
                if out not in statuses:
                    print(f"abi_fuzz: {name}{tuple(args)} returned {out}", flush=True)
                    return 1
                lib.dels_last_error()
            for k in keep:
                if isinstance(k, L._ptr) and k.value:
                    print(f"abi_fuzz: {name} returned a graph handle without a device", flush=True)
                    return 1
    lib.dels_debug_set_decode_spin_limit(16384)
    lib.dels_debug_set_rollout_resident(1)
    lib.dels_debug_set_resident_spin_limit(65536)
    print(f"abi_fuzz: {calls} calls over {len(L.SIGNATURES)} entry points, no finding", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
