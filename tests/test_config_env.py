"""The sampling configuration surface from the environment (CPU only):
gemmaedge_amd.SamplingConfig.from_env, the Python twin of the header-only
include/gemmaedge/sampling_env.h (checked under the sanitizers by
tests/cpp/asan_check.cpp with the same cases). The reference reads its one
tuning variable the same way: a malformed value keeps the default
(src/main.cpp:109-115)."""
import pytest

from gemmaedge_amd.sampler import SamplingConfig


def test_defaults_when_unset():
    assert SamplingConfig.from_env(environ={}) == SamplingConfig()


def test_values_taken():
    env = {"GEMMAEDGE_TEMPERATURE": " 0.7 ", "GEMMAEDGE_TOP_K": "40", "GEMMAEDGE_TOP_P": "0.9",
           "GEMMAEDGE_MIN_P": "0.05", "GEMMAEDGE_SEED": "18446744073709551615", "GEMMAEDGE_SOFTCAP": "30",
           "GEMMAEDGE_REPETITION_PENALTY": "1.15"}
    c = SamplingConfig.from_env(environ=env)
    import numpy as np
    assert c.temperature == float(np.float32(0.7)) and c.top_k == 40 and c.top_p == float(np.float32(0.9))
    assert c.min_p == float(np.float32(0.05)) and c.seed == 2**64 - 1
    assert c.softcap == 30.0 and c.repetition_penalty == float(np.float32(1.15))


def test_base_kept_for_unset_fields():
    base = SamplingConfig(temperature=0.0, top_k=1)
    c = SamplingConfig.from_env(base, environ={"GEMMAEDGE_TOP_P": "0.5"})
    assert (c.temperature, c.top_k, c.top_p) == (0.0, 1, 0.5)
    assert base.top_p == 0.95  # base untouched


@pytest.mark.parametrize("v", ["", "  ", "abc", "0.5x", "nan", "inf", "1e99", "0.5 7", "0x1p-1", "1_0"])
def test_malformed_float_ignored(v):
    assert SamplingConfig.from_env(environ={"GEMMAEDGE_TOP_P": v}).top_p == 0.95


@pytest.mark.parametrize("v", ["-1", "+3", "4294967296", "12.5", "0x10", "99999999999999999999", ""])
def test_malformed_integer_ignored(v):
    assert SamplingConfig.from_env(environ={"GEMMAEDGE_TOP_K": v}).top_k == 64


def test_top_k_zero_disables():
    assert SamplingConfig.from_env(environ={"GEMMAEDGE_TOP_K": "0"}).top_k == 0


@pytest.mark.parametrize("v,want", [("1e-40", 1e-40), ("1e-50", 0.0), ("-1e-46", -0.0)])
def test_underflow_takes_the_rounded_value(v, want):
    # Below the float range: the rounded subnormal (or signed zero), the same
    # value the C++ parser stores (asan_check.cpp checks the same cases).
    import numpy as np
    got = SamplingConfig.from_env(environ={"GEMMAEDGE_MIN_P": v}).min_p
    assert np.float32(got).tobytes() == np.float32(want).tobytes()
