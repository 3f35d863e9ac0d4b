"""The device math must round exactly as glibc 2.35's tanhf / expf, which the
reference calls for the softcap (src/generation.cpp:434) and the softmax
(src/generation.cpp:97). gemmaedge_amd/csrc/ge_math.h restates fdlibm's tanhf /
expm1f and the ARM optimized-routines expf; these tests compare it with the
host's libm on every fp32 input (host build), and on the GPU through
per-block digests against the committed libm digests."""
import ctypes
import json
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "cpp", "lib", "libge_math_check.so")
GOLDEN = os.path.join(HERE, "golden", "math_digests.json")
NT = min(16, os.cpu_count() or 4)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run __graft_entry__.build() or make -C tests/cpp")
    L = ctypes.CDLL(LIB)
    L.ge_test_digest.restype = ctypes.c_int
    L.ge_test_digest.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_uint64), ctypes.c_int]
    L.ge_test_host_mismatches.restype = ctypes.c_longlong
    L.ge_test_host_mismatches.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int]
    L.ge_test_tanhf_decreases.restype = ctypes.c_longlong
    L.ge_test_tanhf_decreases.argtypes = [ctypes.c_int]
    return L


def golden():
    with open(GOLDEN) as f:
        g = json.load(f)
    return {"tanhf": [int(x) for x in g["tanhf"]], "expf": [int(x) for x in g["expf"]]}


def digests(lib, fn, impl):
    out = (ctypes.c_uint64 * 256)()
    assert lib.ge_test_digest(fn, impl, out, NT) == 0
    return [int(x) for x in out]


@pytest.mark.parametrize("fn,name", [(0, "tanhf"), (1, "expf")])
def test_host_build_matches_libm_on_every_input(lib, fn, name):
    assert lib.ge_test_host_mismatches(fn, 0, 1 << 32, NT) == 0, name


@pytest.mark.parametrize("fn,name", [(0, "tanhf"), (1, "expf")])
def test_libm_matches_committed_digests(lib, fn, name):
    # Pins the fixture to this image's glibc: the GPU comparison below is then
    # a comparison with glibc itself.
    assert digests(lib, fn, 0) == golden()[name]


def test_glibc_tanhf_is_monotone(lib):
    # The streaming pass prunes on raw logits; that is exact only because
    # softcap(x) = c * tanhf(x / c) is monotone non-decreasing.
    assert lib.ge_test_tanhf_decreases(NT) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("fn,name", [(0, "tanhf"), (1, "expf")])
def test_device_build_matches_glibc_digests(lib, fn, name):
    print(f"[math] device digests of {name} over 2^32 inputs", flush=True)
    got = digests(lib, fn, 2)
    want = golden()[name]
    bad = [b for b in range(256) if got[b] != want[b]]
    assert not bad, f"{name}: digest mismatch in blocks {bad[:16]} (inputs block << 24)"


def test_exp2_table_is_computed_from_mathematics():
    """Each entry of the expf table is the double nearest 2^(i/32), with
    (i << 47) subtracted from its bit pattern so that adding k << 47 for
    k = 32*e + i scales it by 2^e (gemmaedge_amd/csrc/ge_math.h)."""
    import re
    import struct
    from decimal import Decimal, getcontext

    text = open(os.path.join(HERE, "..", "gemmaedge_amd", "csrc", "ge_math.h")).read()
    body = text[text.index("#define GE_EXP2_TABLE"):]
    body = body[:body.index("}")]
    entries = [int(x, 16) for x in re.findall(r"0x([0-9a-f]+)ull", body)]
    assert len(entries) == 32
    getcontext().prec = 60
    for i, bits in enumerate(entries):
        nearest = float(Decimal(2) ** (Decimal(i) / Decimal(32)))  # correctly rounded
        want = struct.unpack("<Q", struct.pack("<d", nearest))[0] - (i << 47)
        assert bits == want, i
