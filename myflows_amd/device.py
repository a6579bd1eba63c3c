"""The active device for new parameters and inputs (the reference's CPU / CUDA switch,
``core/device.py:146-170``). Arrays are torch tensors; ``"cuda"`` is the current HIP GPU. The
hip_native operators run only on the GPU and reject CPU tensors with a ValueError.
"""

from __future__ import annotations

import torch

_active = "cuda" if torch.cuda.is_available() else "cpu"
_GPU_NAMES = ("cuda", "gpu", "hip", "cuda:0")


def cuda_available() -> bool:
    return torch.cuda.is_available()


def get_device() -> str:
    return _active


def set_device(device: str) -> str:
    global _active
    name = str(device).strip().lower()
    if name == "cpu":
        _active = "cpu"
    elif name in _GPU_NAMES:
        if not torch.cuda.is_available():
            raise RuntimeError("a GPU was requested but none is visible")
        _active = "cuda"
    else:
        raise ValueError(f"unsupported device {device!r}; use 'cpu' or 'cuda'")
    return _active


def torch_device():
    return torch.device("cuda", torch.cuda.current_device()) if _active == "cuda" else torch.device("cpu")


def asarray(value, dtype=torch.float32):
    """A tensor of ``dtype`` on the active device (NumPy arrays and Python values are copied)."""
    if isinstance(value, torch.Tensor):
        return value.to(device=torch_device(), dtype=dtype)
    return torch.as_tensor(value, dtype=dtype, device=torch_device())
