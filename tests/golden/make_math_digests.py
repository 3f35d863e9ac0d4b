"""Writes tests/golden/math_digests.json: per-block digests of glibc's tanhf and
expf over all 2^32 fp32 inputs (256 blocks of 2^24), from the host's libm via
tests/cpp/lib/libge_math_check.so (impl 0). The GPU test compares the device
build of gemmaedge_amd/csrc/ge_math.h against these.

    python tests/golden/make_math_digests.py
"""
import ctypes
import json
import os
import platform

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "..", "cpp", "lib", "libge_math_check.so")


def digests(lib, fn, impl, nthreads):
    out = (ctypes.c_uint64 * 256)()
    rc = lib.ge_test_digest(fn, impl, out, nthreads)
    if rc != 0:
        raise RuntimeError(f"ge_test_digest returned {rc}")
    return [int(x) for x in out]


def load():
    lib = ctypes.CDLL(LIB)
    lib.ge_test_digest.restype = ctypes.c_int
    lib.ge_test_digest.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_uint64), ctypes.c_int]
    lib.ge_test_host_mismatches.restype = ctypes.c_longlong
    lib.ge_test_host_mismatches.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int]
    return lib


if __name__ == "__main__":
    lib = load()
    n = os.cpu_count() or 4
    data = {
        "libc": platform.libc_ver()[1],
        "blocks": 256,
        "block_inputs": 1 << 24,
        "tanhf": [str(x) for x in digests(lib, 0, 0, n)],
        "expf": [str(x) for x in digests(lib, 1, 0, n)],
    }
    with open(os.path.join(HERE, "math_digests.json"), "w") as f:
        json.dump(data, f, indent=0)
    print("wrote", os.path.join(HERE, "math_digests.json"))
