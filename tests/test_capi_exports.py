"""CPU-side checks of the C ABI: the library loads, exports every function
include/ttlab_hip.h declares, and fails loudly (no CPU fallback) without a GPU."""
import ctypes as C

import pytest

import ttlab_amd


def test_library_exports_every_declared_symbol():
    lib = ttlab_amd.load_library()
    declared = ttlab_amd.header_symbols()
    assert len(declared) >= 20
    missing = [name for name in declared if getattr(lib, name, None) is None]
    assert missing == []


def test_create_without_gpu_fails_with_error_code():
    lib = ttlab_amd.load_library()
    try:
        import subprocess
        has_gpu = subprocess.run(["sh", "-c", "ls /dev/kfd"], capture_output=True).returncode == 0
    except OSError:
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is present; the failure path is for GPU-less hosts")
    p = C.c_void_p()
    rc = lib.ttl_create(0, C.byref(p))
    assert rc == -4  # TTL_ERR_NO_DEVICE
    assert b"no HIP device" in lib.ttl_last_error()
    with pytest.raises(ttlab_amd.TtlError):
        ttlab_amd.Device(0)


def test_null_arguments_are_rejected_before_any_launch():
    lib = ttlab_amd.load_library()
    assert lib.ttl_matvec_mxfp4(None, None, None, None, None, 0) == -1
    assert lib.ttl_mxfp4_upload(None, None, 16, 2880, 1, None) == -1
    assert lib.ttl_sync(None) == -1
