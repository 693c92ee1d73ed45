"""The C-ABI's host code under AddressSanitizer and UBSan
(tests/host_asan/abi_host_check.cpp, built by tests/host_asan/build.py from
__graft_entry__.build()): argument validation without a GPU, and on the GPU
create / outliers / forward / destroy of linears (block 16, 24, 64), the MoE,
the KV cache and the kernel-timing report, checked against fp64 restatements.
Any sanitizer report makes the executable exit non-zero, leaks included
(the ROCm runtime's own allocations kept until exit are suppressed by
tests/host_asan/lsan.supp; none of their stacks holds a frame of this
library)."""
import os
import subprocess

import pytest

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "host_asan", "_build",
                   "abi_host_check")


def _run():
    if not os.path.exists(EXE):                     # built by __graft_entry__.build(); else here
        import importlib.util
        spec = importlib.util.spec_from_file_location(
            "_host_asan_build",
            os.path.join(os.path.dirname(os.path.abspath(__file__)), "host_asan", "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build(verbose=False)
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:abort_on_error=0:halt_on_error=1"
    env["LSAN_OPTIONS"] = "suppressions=" + os.path.join(os.path.dirname(EXE), "..", "lsan.supp")
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=300, env=env)
    print(r.stdout[-2000:], r.stderr[-4000:])
    return r


def test_host_check_argument_validation():
    """Runs everywhere: with no device visible only the validation checks run."""
    r = _run()
    assert r.returncode == 0 and "HOST_CHECK_OK" in r.stdout


@pytest.mark.gpu
def test_host_check_on_gpu():
    r = _run()
    assert r.returncode == 0 and "HOST_CHECK_OK" in r.stdout
    assert "devices 0" not in r.stdout
    assert r.stdout.count("linear K=") >= 6 and "moe rel" in r.stdout and "kv rel" in r.stdout
