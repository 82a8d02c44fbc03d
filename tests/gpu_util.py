"""Device-memory plumbing for the GPU tests (torch is only the allocator)."""
import sys

import numpy as np
import torch


def dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    t = torch.from_numpy(a.view(np.uint8).reshape(-1).copy())
    return t.to("cuda:0")


def empty(nbytes: int) -> torch.Tensor:
    return torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")


def host(t: torch.Tensor, dtype) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy().view(dtype)


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def rel(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()
