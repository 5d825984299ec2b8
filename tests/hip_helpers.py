"""Helpers shared by the GPU parity tests (test infrastructure)."""
import numpy as np
import pytest
import torch

DEV = "cuda"


def need_gpu():
    """GPU tests fail (never skip) when no ROCm device is present: a silent skip would hide a missing backend."""
    assert torch.cuda.is_available(), "GPU tests need an MI355X (run with -m 'not gpu' on CPU-only machines)"


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def unpermute_layout1(q: np.ndarray, K: int) -> np.ndarray:
    """Undo the layout-1 order of activation codes: byte 4s+j of each 16-group holds code 4j+s."""
    M, ldq = q.shape
    g = q.reshape(M, ldq // 16, 4, 4)          # [m, group, s, j]
    return np.ascontiguousarray(g.transpose(0, 1, 3, 2)).reshape(M, ldq)[:, :K]


def normwise(a, b) -> float:
    """max |a - b| / max |b| (the tolerance metric for outputs with heavy cancellation)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = max(np.max(np.abs(b)), 1e-30)
    return float(np.max(np.abs(a - b)) / den)


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.numpy()


TOL = {torch.float32: 1e-3, torch.bfloat16: 2e-2}


gpu = pytest.mark.gpu
