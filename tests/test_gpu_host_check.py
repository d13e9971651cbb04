"""tests/host/dm_host_check: a C++ caller that binds only include/dashmi.h and libdashmi.so (no HIP
headers or HIP calls of its own; device buffers through dm_device_alloc and the dm_copy_*
helpers), run as a child process. Its checks are closed forms computed in double precision on
the host (see the program's header): attention forward and backward with q = 0, decode with
q = 0, and the recurrent step from a zero state."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "host", "dm_host_check")


def _run():
    if not os.path.exists(BIN):
        pytest.skip("tests/host/dm_host_check is not built (dashmag_amd.build.build_host_check)")
    return subprocess.run([BIN], capture_output=True, text=True, timeout=120)


@pytest.mark.gpu
def test_host_caller_through_the_c_abi():
    r = _run()
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout


def test_host_caller_without_a_gpu_is_refused():
    """Without a HIP device the program stops at dm_describe's refusal (exit status 2)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    r = _run()
    assert r.returncode == 2, r.stdout + r.stderr
    assert "no usable device" in r.stdout
