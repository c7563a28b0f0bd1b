"""GPU runs of the calibration kernels.  The MFMA ceiling
(jules_hip_mfma_ceiling) launches, its output is finite and deterministic
(the operands are a fixed hash), and an odd workgroup count covers the output
indexing; the HBM read floor (jules_hip_hbm_read_floor) reads every chunk of
its buffer exactly once."""
import numpy as np
import pytest
import torch

from jules_amd import _lib, ops
from tests.helpers import case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("workgroups,iters", [(1, 1), (7, 16), (256, 64)])
def test_mfma_ceiling_runs(dev, workgroups, iters):
    case(f"mfma_ceiling wg={workgroups} iters={iters}")
    L = _lib.lib()
    out = torch.full((workgroups * 256,), float("nan"), dtype=torch.float32, device=dev)
    st = L.jules_hip_mfma_ceiling(out.data_ptr(), workgroups, iters, None)
    assert st == 0, L.jules_hip_last_error()
    torch.cuda.synchronize()
    a = out.cpu().numpy().copy()
    assert np.isfinite(a).all()
    st = L.jules_hip_mfma_ceiling(out.data_ptr(), workgroups, iters, None)
    assert st == 0
    torch.cuda.synchronize()
    assert np.array_equal(a, out.cpu().numpy())


@pytest.mark.parametrize("n", [(1 << 20) + 16 * 37, (9 << 20) + 16 * 37, (20 << 20) + 16 * 5])
def test_hbm_read_floor_reads_every_chunk_once(dev, n):
    """XOR over all lanes' results equals the XOR of every 4-byte word of the
    buffer: each 16-byte chunk is read exactly once.  256 workgroups x 256
    lanes read 1 MiB per round; the sizes give 1, 9 and 20 whole rounds (the
    8-deep load ring not used, used without its steady-state loop, and with
    it) plus a partial last round."""
    case(f"hbm read floor: every chunk read once, {n} bytes")
    host = np.random.default_rng(3).integers(-2**31, 2**31 - 1, n // 4, dtype=np.int64).astype(np.int32)
    buf = torch.from_numpy(host).to(dev)
    out = torch.empty(256 * 256, dtype=torch.int32, device=dev)
    assert ops.hbm_read_floor(buf, out, 256) == n
    got = np.bitwise_xor.reduce(out.cpu().numpy())
    assert got == np.bitwise_xor.reduce(host)
