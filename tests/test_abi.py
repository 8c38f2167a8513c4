"""C-ABI surface checks that need no GPU: the library loads, exports every symbol the header
declares, and rejects invalid arguments with the reference's status convention (status 1 and
a heap error string) before touching the device."""
import ctypes
import subprocess

import pytest

from castforge_amd import ffi


def test_library_exports_every_header_symbol():
    declared = ffi.header_symbols()
    assert len(declared) >= 15
    out = subprocess.run(["nm", "-D", "--defined-only", str(ffi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    assert set(ffi.SIGNATURES) == set(declared)
    for s in declared:
        assert hasattr(ffi.lib(), s)


def test_version_string():
    assert ffi.version().startswith("castforge-hip ")


def test_free_string_accepts_null():
    ffi.lib().castforge_hip_free_string(None)


def _status(name, *args):
    err = ctypes.c_char_p()
    rc = getattr(ffi.lib(), name)(*args, ctypes.byref(err))
    msg = err.value.decode() if err.value else None
    if err.value is not None:
        ffi.lib().castforge_hip_free_string(ctypes.cast(err, ctypes.c_void_p))
    return rc, msg


@pytest.mark.parametrize("call,needle", [
    (("castforge_hip_quantize_int4g", 1, 4, 128, 3, 1, 1, 1, None), "group"),
    (("castforge_hip_quantize_int4g", 1, 4, 12, 128, 1, 1, 1, None), "multiple of 8"),
    (("castforge_hip_quantize_int4g", None, 4, 128, 128, None, None, None, None), "NULL"),
    (("castforge_hip_quantize_int4g", 1, -1, 128, 128, 1, 1, 1, None), "non-negative"),
    (("castforge_hip_quantize_nf4", 1, 4, 128, 48, 1, 1, None), "block"),
    (("castforge_hip_quantize_int8", 1, 4, 128, 8, 7, 0, 1, 1, None), "granularity"),
    (("castforge_hip_quantize_int8", 1, 4, 128, 8, 1, 9, 1, 1, None), "round_mode"),
    (("castforge_hip_quantize_fp8", 1, 5, 4, 128, 1, 1, None), "src_dtype"),
    (("castforge_hip_gemv_w4a16", 1, 1, 16, 100, 128, 1, 1, 1, 1, 0, None), "multiple of 8"),
    (("castforge_hip_gemv_w4a16", 1, 1, 16, 128, 128, 1, 1, 1, 1, 5, None), "y_dtype"),
    (("castforge_hip_gemv_w8a16", 1, 1, 16, 128, 1, 1, 3, 1, 0, None), "granularity"),
    (("castforge_hip_gemv_nf4", 1, 1, 16, 128, 5, 1, 1, 1, 0, None), "block"),
])
def test_invalid_arguments_report_status_1(call, needle):
    rc, msg = _status(*call)
    assert rc == 1 and msg and needle in msg, (rc, msg)


def test_batched_rejects_bad_count_and_m():
    arr = (ffi.W4A16Problem * 1)()
    rc, msg = _status("castforge_hip_gemv_w4a16_batched", arr, 9, 1, 0, None)
    assert rc == 1 and "count" in msg
    rc, msg = _status("castforge_hip_gemv_w4a16_batched", arr, 1, 65, 0, None)
    assert rc == 1 and "m <= 64" in msg


def test_error_pointer_optional():
    # NULL out_error: status only, nothing written
    f = ffi.lib().castforge_hip_quantize_int4g
    assert f(1, 4, 128, 3, 1, 1, 1, None, None) == 1


def test_empty_shapes_are_noops():
    # zero rows / zero m: validated and returns 0 without a launch
    assert _status("castforge_hip_quantize_int4g", None, 0, 128, 128, None, None, None, None)[0] == 0
    assert _status("castforge_hip_quantize_nf4", None, 4, 0, 64, None, None, None)[0] == 0
    assert _status("castforge_hip_gemv_w4a16", None, 0, 16, 128, 128, None, None, None, None, 0, None)[0] == 0
    assert _status("castforge_hip_gemv_w4a16_batched", None, 0, 1, 0, None)[0] == 0
