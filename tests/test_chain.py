"""The full-order sampling path replays the reference's sequential sums
(softmax denominator in double, top-p cumulative and draw walk in float,
src/generation.cpp:96-97, 105-113, 120-124) in closed form per run of equal
addends (gemmaedge_amd/csrc/chain_math.h). These tests compare that closed
form, compiled for the host, with plain left-to-right loops on random runs
that cross binades in both directions, hit ties to even from odd and even
starting values, and stop on thresholds."""
import ctypes
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "cpp", "lib", "libge_chain_check.so")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run __graft_entry__.build() or make -C tests/cpp")
    L = ctypes.CDLL(LIB)
    L.ge_test_chain_random.restype = ctypes.c_longlong
    L.ge_test_chain_random.argtypes = [ctypes.c_int, ctypes.c_ulonglong, ctypes.c_int]
    return L


@pytest.mark.parametrize("which,name,trials", [
    (0, "float ascending with threshold", 200000),
    (1, "float descending with stop", 200000),
    (2, "double ascending with threshold", 200000),
    (3, "double descending with stop", 200000),
    (4, "float ascending, chained runs", 20000),
    (5, "float descending, chained runs", 20000),
    (6, "double ascending, chained runs", 20000),
    (7, "corrected double quotient", 1000000),
    (8, "float ascending, 32-bit version", 200000),
    (9, "float descending, 32-bit version", 200000),
    (10, "float ascending chained runs, 32-bit version", 20000),
    (11, "float descending chained runs, 32-bit version", 20000),
    (12, "float step and threshold from bit fields", 1000000),
    (13, "double step from bit fields (float addend)", 1000000),
    (14, "block replay model, float ascending with threshold", 3000),
    (15, "block replay model, float descending with stop", 3000),
    (16, "block replay model, double ascending", 3000),
])
def test_closed_form_matches_loop(lib, which, name, trials):
    for seed in (1, 2, 3):
        assert lib.ge_test_chain_random(which, seed, trials) == 0, name
