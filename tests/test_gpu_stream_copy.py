"""GPU: emel_stream_copy, the measurement reference bench divides by.

Every shape must be an exact bit copy (NaN payloads included) at sizes that
end inside a wave's span, a workgroup's span and the resident walk's
stride, and must leave the bytes after the copied range untouched.
Misaligned pointers, a byte count that is not a multiple of 16 and unknown
shapes are refused before any launch.
"""
import numpy as np
import pytest
import torch

import emel_hip as eh

pytestmark = pytest.mark.gpu

SIZES = [16, 1024, 16 * 63, 16 * 64 * 8 + 16, 16 * 256 * 8 - 16, 16 * 1000003, 16 * 2097152 * 2 + 48]


@pytest.mark.parametrize("shape", list(eh.CopyShape))
def test_every_shape_copies_exactly(gpu, shape):
    g = np.random.Generator(np.random.PCG64(41 + int(shape)))
    for nbytes in SIZES:
        words = nbytes // 4
        src_h = g.integers(0, 2**32, words + 64, dtype=np.uint64).astype(np.uint32)
        src_h[::97] = 0x7FC00123  # NaN payloads travel as bits
        src = torch.from_numpy(src_h.view(np.int32)).to(gpu)
        dst = torch.full((words + 64,), -1, dtype=torch.int32, device=gpu)
        st = eh.stream_copy(src.data_ptr(), dst.data_ptr(), nbytes, shape, torch.cuda.current_stream().cuda_stream)
        assert st == eh.Status.OK, eh.last_error()
        got = dst.cpu().numpy().view(np.uint32)
        assert (got[:words] == src_h[:words]).all(), (shape, nbytes)
        assert (got[words:] == 0xFFFFFFFF).all(), (shape, nbytes, "wrote past the end")


def test_refusals(gpu):
    src = torch.zeros(1024, dtype=torch.float32, device=gpu)
    dst = torch.zeros(1024, dtype=torch.float32, device=gpu)
    s = torch.cuda.current_stream().cuda_stream
    assert eh.stream_copy(src.data_ptr(), dst.data_ptr(), 24, eh.CopyShape.FLAT, s) == eh.Status.INVALID_ARGUMENT
    assert eh.stream_copy(src.data_ptr() + 4, dst.data_ptr(), 32, eh.CopyShape.FLAT, s) == eh.Status.INVALID_ARGUMENT
    assert eh.stream_copy(src.data_ptr(), dst.data_ptr() + 8, 32, eh.CopyShape.WAVE8, s) == eh.Status.INVALID_ARGUMENT
    assert eh.stream_copy(src.data_ptr(), dst.data_ptr(), 32, 7, s) == eh.Status.INVALID_ARGUMENT
    assert eh.stream_copy(src.data_ptr(), dst.data_ptr(), 0, eh.CopyShape.WALK, s) == eh.Status.OK
