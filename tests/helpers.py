"""Shared helpers for the GPU parity tests."""
import numpy as np
import torch


def to_dev(a, dtype, dev):
    """numpy -> device tensor.  For bf16 the array must already hold bf16
    values (widened to fp32), so the conversion is exact."""
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(device=dev, dtype=dtype).contiguous()


def to_np(t):
    return t.detach().float().cpu().numpy() if t.dtype == torch.bfloat16 else t.detach().cpu().numpy()


def case(msg):
    """Print and flush the case name before a GPU step, so that a run that
    ends the process still names what it was doing."""
    print(f"[case] {msg}", flush=True)
