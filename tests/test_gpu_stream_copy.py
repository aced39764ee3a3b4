"""GPU: the streaming copies that bench.py times as HBM ceilings copy exactly.

Flat: sizes that leave a tail past the last full four-vector sweep of the
grid and one vector alone. Rows: row lengths for each register form (16, 20 and
24 vectors a lane), a partial last vector, fewer rows than CUs and more.
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
