"""The drop-in boundary without a GPU: the C-ABI library loads, exports every
entry point include/gemmaedge_sampler.h declares, its ctypes structs match the
C layout, it validates arguments before touching a device, and the C++ drop-in
exports gemmaedge::sample_token with the reference's exact mangled signature
(include/gemmaedge/generation.h:69-71)."""
import ctypes
import os
import re
import subprocess

import pytest

import gemmaedge_amd as G
from gemmaedge_amd import sampler as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gemmaedge_sampler.h")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libge_ref.so")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|void|const char\*)\s+(ge_\w+)\s*\(", text, re.M)))


def test_library_loads_and_exports_every_declared_function():
    lib = S.load_library()
    names = declared_functions()
    assert names, "no declarations parsed"
    assert set(names) == set(S.EXPORTS)
    for n in names:
        assert hasattr(lib, n), f"{n} not exported"


def test_struct_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "gemmaedge_sampler.h"\n'
        "int main(void){\n"
        ' printf("%zu %zu %zu\\n", sizeof(ge_sample_params), sizeof(ge_sample_args), '
        "offsetof(ge_sample_args, params));\n"
        ' printf("%zu %zu %zu %zu\\n", offsetof(ge_sample_args, row_params), '
        "offsetof(ge_sample_args, ring_capacity), offsetof(ge_sample_args, uniforms), "
        "offsetof(ge_sample_args, flags_out));\n return 0; }\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    got = [int(x) for x in out]
    want = [ctypes.sizeof(S.SampleParams), ctypes.sizeof(S.SampleArgs), S.SampleArgs.params.offset,
            S.SampleArgs.row_params.offset, S.SampleArgs.ring_capacity.offset,
            S.SampleArgs.uniforms.offset, S.SampleArgs.flags_out.offset]
    assert got == want


def test_oracle_params_layout_matches_abi():
    import ge_oracle as O

    assert ctypes.sizeof(O.Params) == ctypes.sizeof(S.SampleParams)
    for (n1, _), (n2, _) in zip(O.Params._fields_, S.SampleParams._fields_):
        assert n1 == n2


def test_constants():
    assert G.max_top_k() == 1024
    assert S.GE_DTYPE_F32 == 0 and S.GE_DTYPE_BF16 == 1


def test_argument_validation_without_device():
    lib = S.load_library()
    h = ctypes.c_void_p()
    assert lib.ge_sampler_create(0, 0, 10, 0, ctypes.byref(h)) == S.GE_ERR_INVALID_ARG
    assert "max_rows" in S.last_error()
    assert lib.ge_sampler_create(0, 1, 10, 0, None) == S.GE_ERR_INVALID_ARG
    assert lib.ge_sampler_create(0, 1, 1 << 30, 0, ctypes.byref(h)) == S.GE_ERR_CAPACITY
    assert lib.ge_sample(None, None, None) == S.GE_ERR_INVALID_ARG


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks the no-device path")
def test_no_device_is_reported_not_hidden():
    lib = S.load_library()
    assert lib.ge_sampler_available() == 0
    h = ctypes.c_void_p()
    assert lib.ge_sampler_create(0, 1, 16, 0, ctypes.byref(h)) == S.GE_ERR_NO_DEVICE
    with pytest.raises(S.SamplerError):
        S.Sampler(1, 16)


def _exported(path, pattern):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return sorted(line.split()[-1] for line in out.splitlines() if pattern in line)


def test_cpp_drop_in_symbol():
    syms = _exported(G.LIB_PATH, "sample_token")
    # gemmaedge::sample_token(std::vector<float> const&, SamplingConfig const&, std::mt19937_64&)
    ref_sig = [s for s in syms if s.endswith("EE") and "mersenne" in s and "PKi" not in s]
    assert len(ref_sig) == 1, syms
    assert ref_sig[0].startswith("_ZN9gemmaedge12sample_tokenERKSt6vectorIfSaIfEERKNS_14SamplingConfigE")


@pytest.mark.skipif(not os.path.exists(REF_SO), reason="oracle/_ref not built (needs /root/reference)")
def test_cpp_drop_in_symbol_is_the_reference_symbol():
    ours = [s for s in _exported(G.LIB_PATH, "sample_token") if "PKi" not in s]
    ref = _exported(REF_SO, "sample_token")
    assert ours == ref
