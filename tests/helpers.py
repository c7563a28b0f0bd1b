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


_DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.int8: 2, torch.int32: 3}


def registry_call(name, inputs, outputs, config=None):
    """Call an extern_kernel name through jules_hip_lookup with contiguous
    descriptors built from device tensors; returns the status."""
    from jules_amd import _lib

    def fill(d, t):
        d.data = t.data_ptr()
        d.offset = 0
        d.rank = t.dim()
        d.dtype = _DTYPE_CODE[t.dtype]
        for i, (n, s) in enumerate(zip(t.shape, t.stride())):
            d.sizes[i] = n
            d.strides[i] = s

    ins = (_lib.JhTensor * len(inputs))()
    outs = (_lib.JhTensor * len(outputs))()
    for d, t in zip(ins, inputs):
        fill(d, t)
    for d, t in zip(outs, outputs):
        fill(d, t)
    fn = _lib.lookup(name)
    assert fn is not None, name
    return fn(len(inputs), ins, len(outputs), outs, config,
              torch.cuda.current_stream().cuda_stream)
