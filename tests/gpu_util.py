"""Small helpers for GPU tests: numpy <-> device buffers through torch."""
import numpy as np

from market_sim_amd import abi, ops


def dev(a: np.ndarray):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype.kind in "ui":
        a = a.view({1: np.int8, 2: np.int16, 4: np.int32, 8: np.int64}[a.dtype.itemsize])
    return torch.from_numpy(a).cuda()


def empty(n: int, dtype):
    import torch
    t = {np.uint32: torch.int32, np.float32: torch.float32, np.uint16: torch.int16}[dtype]
    return torch.empty(n, dtype=t, device="cuda")


def host(t, dtype) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(dtype).copy()


def B(t) -> ops.DeviceBuffer:
    return ops.DeviceBuffer.of(t)


_STREAM = None


def stream() -> int:
    """A dedicated non-default stream (the reference API rejects the null
    stream).  Synchronizes the device first so that inputs uploaded by torch
    on its own stream are complete."""
    global _STREAM
    import torch
    if _STREAM is None:
        _STREAM = torch.cuda.Stream()
    torch.cuda.synchronize()
    return _STREAM.cuda_stream


def ok(status) -> None:
    abi.check("op", status)
