"""The benchmark's measurement floors (include/nspeech_rocm.h, nsr_calib_*):
every copy form reproduces its source bit for bit, including sizes that
leave a partial tile and a grid smaller than the work, and the empty kernel
runs. These kernels time the floors the fused kernels are judged against, so
they must move exactly the bytes they claim. The c4b timeline entry point
must give the row kernel's output exactly, with stamps for every workgroup."""
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


@pytest.mark.parametrize("C,T", [(300, 115200), (40, 4 * (512 * 56 + 1)), (7, 4 * 512 * 57)])
def test_adain_timeline_matches_the_row_kernel(dev, C, T):
    """nsr_calib_adain_timeline is the c4b row kernel plus stamps: the same output bit for bit as
    nsr_adain_snake_f32, and stamps that describe every workgroup (its XCD, start, each wave's end after
    each of its rows landed)."""
    say("calib adain timeline", C, T)
    L = abi.lib()
    st = torch.cuda.current_stream().cuda_stream
    g = np.random.default_rng(C)
    x = torch.from_numpy(g.standard_normal((1, C, T), dtype=np.float32)).cuda()
    gam = torch.from_numpy((0.1 * g.standard_normal((1, C))).astype(np.float32)).cuda()
    bet = torch.from_numpy((0.1 * g.standard_normal((1, C))).astype(np.float32)).cuda()
    alp = torch.from_numpy(g.uniform(0.5, 1.5, C).astype(np.float32)).cuda()
    ref, out = torch.empty_like(x), torch.full_like(x, float("nan"))
    abi.check(L.nsr_adain_snake_f32(x.data_ptr(), gam.data_ptr(), bet.data_ptr(), alp.data_ptr(), 0, C, C,
                                    ref.data_ptr(), 1, C, T, 1e-5, st))
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    stamps = torch.zeros(n_cu * 80, dtype=torch.int64, device="cuda")
    abi.check(L.nsr_calib_adain_timeline(x.data_ptr(), gam.data_ptr(), bet.data_ptr(), alp.data_ptr(),
                                         out.data_ptr(), 1, C, T, stamps.data_ptr(), stamps.numel(), st))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    s = stamps.view(n_cu, 80).cpu().numpy()
    wg = min(C, n_cu)
    assert (s[:wg, 1] > 0).all() and (s[wg:] == 0).all()
    assert ((s[:wg, 0] >= 0) & (s[:wg, 0] < 64)).all()
    for i in range(wg):
        n_rows_i = len(range(i, C, wg))
        land = s[i, 10:10 + 8 * min(n_rows_i, 8)].reshape(-1, 8)
        assert (land >= s[i, 1]).all() and (np.diff(land, axis=0) >= 0).all()
        assert (s[i, 2:10] >= land[-1]).all()


def test_adain_timeline_rejects_other_shapes(dev):
    L = abi.lib()
    st = torch.cuda.current_stream().cuda_stream
    x = torch.zeros(4 * 115200, dtype=torch.float32, device="cuda")
    p = torch.zeros(8, dtype=torch.float32, device="cuda")
    stamps = torch.zeros(80, dtype=torch.int64, device="cuda")
    # a row length outside the kernel's bucket, then too few stamp words for 4 workgroups
    assert L.nsr_calib_adain_timeline(x.data_ptr(), p.data_ptr(), p.data_ptr(), p.data_ptr(), x.data_ptr(), 1, 4,
                                      4 * 512 * 56, stamps.data_ptr(), stamps.numel(), st) != 0
    assert L.nsr_calib_adain_timeline(x.data_ptr(), p.data_ptr(), p.data_ptr(), p.data_ptr(), x.data_ptr(), 1, 4,
                                      115200, stamps.data_ptr(), stamps.numel(), st) != 0
    torch.cuda.synchronize()
