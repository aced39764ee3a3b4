"""GPU: the streaming copies that bench.py times as HBM ceilings copy exactly.

Flat: sizes that leave a tail past the last full four-vector sweep of the
grid and one vector alone. Rows: row lengths for each register form (16, 20 and
24 vectors a lane), a partial last vector, fewer rows than CUs and more.
Mix: every destination stream is the XOR of the sources plus its index, for
the stream counts bench.py uses and the bounds, one vector and a grid tail.
"""
import pytest
import torch

from _util import gpu
from kernels import _lib

pytestmark = pytest.mark.gpu


def _copy(src, rows, row_bytes, mode):
    dst = torch.zeros_like(src)
    rc = _lib.load().hk_stream_copy(dst.data_ptr(), src.data_ptr(), rows, row_bytes, mode, _lib.stream_of(src.device))
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return dst


@pytest.mark.parametrize("nbytes", [16, 16 * 1000, 16 * (256 * 256 * 4 * 3 + 17), 64 << 20])
def test_flat_copy(nbytes):
    src = torch.randint(-128, 127, (nbytes,), dtype=torch.int8, device=gpu())
    assert torch.equal(_copy(src, 1, nbytes, _lib.COPY_FLAT), src)


@pytest.mark.parametrize("rows,row_bytes", [(3, 16), (7, 256512), (300, 256512), (513, 303872), (40, 24 * 1024 * 16),
                                            (260, 16 * 1024 * 16 + 16)])
def test_rows_copy(rows, row_bytes):
    src = torch.randint(-128, 127, (rows * row_bytes,), dtype=torch.int8, device=gpu())
    assert torch.equal(_copy(src, rows, row_bytes, _lib.COPY_ROWS), src)


def _mix_ref(src, n_read, n_write, nbytes, stride):
    words = src.view(n_read, stride // 4)[:, :nbytes // 4]
    acc = words[0].clone()
    for k in range(1, n_read):
        acc ^= words[k]
    return torch.stack([acc + w for w in range(n_write)])


@pytest.mark.parametrize("n_read,n_write,nbytes,pad", [(1, 1, 16, 0), (2, 1, 16 * 5003, 0), (3, 1, 1 << 20, 4352),
                                                       (2, 2, 16 * 777, 16), (3, 2, 16 * 4099, 4352),
                                                       (8, 1, 1 << 16, 0), (9, 8, 16 * 1000, 4352)])
def test_mix(n_read, n_write, nbytes, pad):
    stride = nbytes + pad
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (n_read * stride // 4,), dtype=torch.int32, device=gpu())
    dst = torch.full((n_write * stride // 4,), 7, dtype=torch.int32, device=gpu())
    rc = _lib.load().hk_stream_mix(dst.data_ptr(), src.data_ptr(), nbytes, stride, n_read, n_write,
                                   _lib.stream_of(src.device))
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    out = dst.view(n_write, stride // 4)
    assert torch.equal(out[:, :nbytes // 4], _mix_ref(src, n_read, n_write, nbytes, stride))
    assert bool((out[:, nbytes // 4:] == 7).all()), "the gaps between streams are not written"
