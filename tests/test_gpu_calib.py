"""GPU run of the MFMA calibration kernel (jules_hip_mfma_ceiling): it
launches, its output is finite and deterministic (the operands are a fixed
hash), and an odd workgroup count covers the output indexing."""
import numpy as np
import pytest
import torch

from jules_amd import _lib
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
