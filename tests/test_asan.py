"""Host code paths under the address and undefined-behaviour sanitizers:
tests/cpp/bin/asan_check (built by `make -C tests/cpp`, g++ -fsanitize=
address,undefined without recovery) runs the C ABI's argument checks and
routing, the host build of the glibc-exact math, the closed-form chain
replay against plain loops, and the CPU oracle on random and edge-case
batches. Any sanitizer finding aborts the program."""
import os
import subprocess

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "asan_check")


def test_host_paths_under_asan_and_ubsan():
    assert os.path.exists(BIN), "build tests/cpp first (make -C tests/cpp)"
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "asan checks passed" in r.stdout
