"""The benchmark's measurement floors (include/nspeech_rocm.h, nsr_calib_*):
every copy form reproduces its source bit for bit, including sizes that
leave a partial tile and a grid smaller than the work, and the empty kernel
runs. These kernels time the floors the fused kernels are judged against, so
they must move exactly the bytes they claim."""
import numpy as np
import pytest
import torch

from nspeech_amd import abi

from ._util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096, 16 * 1000 + 16, 8519680 // 2, (1 << 22) + 48])
@pytest.mark.parametrize("form,per_cu", [(0, 0), (1, 0), (2, 0), (1, 1), (2, 3)])
def test_copy_forms_are_exact(dev, nbytes, form, per_cu):
    say("calib copy", nbytes, form, per_cu)
    g = np.random.default_rng(nbytes + form)
    src = torch.from_numpy(g.integers(0, 2**31, nbytes // 4, dtype=np.int64).astype(np.int32)).cuda()
    dst = torch.full_like(src, -1)
    abi.check(abi.lib().nsr_calib_copy(src.data_ptr(), dst.data_ptr(), nbytes, form, per_cu,
                                       torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(dst, src)


@pytest.mark.parametrize("rows,row_bytes", [(1, 16), (3, 8192 + 16), (300, 115200 * 4), (5, 16 * 512 * 9)])
def test_row_copy_is_exact(dev, rows, row_bytes):
    say("calib row copy", rows, row_bytes)
    g = np.random.default_rng(rows)
    src = torch.from_numpy(g.integers(0, 2**31, rows * row_bytes // 4, dtype=np.int64).astype(np.int32)).cuda()
    dst = torch.full_like(src, -1)
    abi.check(abi.lib().nsr_calib_copy_rows(src.data_ptr(), dst.data_ptr(), rows, row_bytes,
                                            torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(dst, src)


def test_empty_kernel_runs(dev):
    abi.check(abi.lib().nsr_calib_empty(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
