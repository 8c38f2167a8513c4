"""castforge_hip_quantize_groupwise_noalloc (static per-device scratch, no allocation) against
castforge_hip_quantize_groupwise (caller workspace), bit for bit, through the C ABI: two calls
in a row on one device, the second with a smaller tensor, so the second call runs on the
scratch contents the first one left."""
import ctypes

import numpy as np
import pytest
import torch

from castforge_amd import ffi, synth

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _run(w, bits, gs, awq, ratio, noalloc):
    n = w.numel()
    deq = torch.empty_like(w)
    scales = torch.empty((n + gs - 1) // gs, dtype=torch.float32, device=w.device)
    cnt = ctypes.c_int64(-1)
    stream = ctypes.c_void_p(torch.cuda.current_stream(w.device).cuda_stream)
    if noalloc:
        ffi.call("castforge_hip_quantize_groupwise_noalloc", _ptr(w), n, bits, gs, int(awq), float(ratio), 0,
                 _ptr(deq), _ptr(scales), ctypes.byref(cnt), stream)
    else:
        ws = torch.empty(ffi.GROUPWISE_WORKSPACE_BYTES // 4, dtype=torch.int32, device=w.device)
        ffi.call("castforge_hip_quantize_groupwise", _ptr(w), n, bits, gs, int(awq), float(ratio), 0,
                 _ptr(deq), _ptr(scales), _ptr(ws), ctypes.byref(cnt), stream)
    torch.cuda.synchronize()
    return deq.cpu().numpy().view(np.uint32), scales.cpu().numpy().view(np.uint32), cnt.value


@pytest.mark.parametrize("awq", [True, False])
def test_noalloc_matches_workspace_entry_two_calls(cuda, awq):
    big = torch.from_numpy(synth.weight(91, 0, 512, 1000)).to(cuda)
    small = torch.from_numpy(synth.weight(91, 1, 37, 129)).to(cuda)
    for w, bits, gs, ratio in ((big, 4, 32, 0.01), (small, 8, 7, 0.2)):
        got = _run(w, bits, gs, awq, ratio, noalloc=True)
        ref = _run(w, bits, gs, awq, ratio, noalloc=False)
        assert got[2] == ref[2], f"salient count {got[2]} != {ref[2]}"
        assert np.array_equal(got[0], ref[0]), "dequantized values differ"
        assert np.array_equal(got[1], ref[1]), "group scales differ"


def test_noalloc_rejects_oversized_tensor(cuda):
    w = torch.zeros(8, device=cuda)
    cnt = ctypes.c_int64(0)
    with pytest.raises(ffi.CastForgeHipError, match="2\\^32"):
        ffi.call("castforge_hip_quantize_groupwise_noalloc", _ptr(w), 1 << 32, 4, 32, 1, 0.01, 0, _ptr(w), _ptr(w),
                 ctypes.byref(cnt), None)
