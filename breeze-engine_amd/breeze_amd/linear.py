"""Dense linear backend, same API as breeze/linear.py:25-46.

``backend()`` names the GEMM in use, ``prepare_weight`` stores a dequantized
``[K, N]`` fp32 weight in that backend's form, ``linear`` computes ``a @ w``
and returns fp32 NumPy.  With a GPU the weight lives in device memory as
fp16 and the product runs through PyTorch-ROCm (fp32 accumulate); without
one, NumPy fp32 is used, as the reference does when torch is absent.  This is
the dense fallback API only; the quantized path is ``hip_backend``.
"""
import numpy as np

try:
    import torch

    _GPU = bool(torch.cuda.is_available())
except Exception:  # noqa: BLE001 - torch is optional
    torch = None
    _GPU = False


def backend():
    return "torch-hip-fp16" if _GPU else "numpy-fp32"


def prepare_weight(w_fp32):
    """Return the weight ``w_fp32`` (dequantized, ``[K, N]``) as the backend
    keeps it: an fp16 device tensor with a GPU, else contiguous fp32 NumPy."""
    w = np.ascontiguousarray(w_fp32, dtype=np.float32)
    if _GPU:
        return torch.from_numpy(w).to(device="cuda", dtype=torch.float16)
    return w


def linear(a_fp32, w):
    """Product of an activation of shape ``[.., K]`` with a weight from
    ``prepare_weight``; the result is an fp32 NumPy array of shape ``[.., N]``."""
    a = np.asarray(a_fp32)
    m = a.reshape(-1, a.shape[-1])
    n = int(w.shape[1])
    if _GPU:
        t = torch.from_numpy(np.ascontiguousarray(m, dtype=np.float32)).to("cuda", torch.float16)
        out = torch.matmul(t, w).to(torch.float32).cpu().numpy()
    else:
        out = np.asarray(m, np.float32) @ w
    return out.reshape(*a.shape[:-1], n)
