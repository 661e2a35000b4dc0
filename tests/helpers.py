"""Conversions between the oracle's NumPy storage (bf16 as uint16 bits) and torch tensors."""

from __future__ import annotations

import numpy as np
import torch

TORCH_DTYPE = {"bf16": torch.bfloat16, "f16": torch.float16}


def act_to_torch(arr: np.ndarray, dtype: str, device="cuda") -> torch.Tensor:
    """Oracle activation storage -> torch tensor of the activation dtype on ``device``."""
    if dtype == "bf16":
        t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.uint16).view(np.int16))
        t = t.view(torch.bfloat16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float16))
    return t.to(device)


def torch_to_act(t: torch.Tensor, dtype: str) -> np.ndarray:
    """torch 16-bit tensor -> oracle storage (uint16 bits for bf16, float16 for f16)."""
    c = t.detach().cpu().contiguous()
    if dtype == "bf16":
        return c.view(torch.int16).numpy().view(np.uint16)
    return c.numpy()


def words_to_torch(w: np.ndarray, device="cuda") -> torch.Tensor:
    """uint32 packed weights -> int32 torch tensor holding the same bits."""
    return torch.from_numpy(np.ascontiguousarray(w, dtype=np.uint32).view(np.int32)).to(device)


def affine_to_torch(triple, dtype: str, device="cuda"):
    w, s, b = triple
    return (words_to_torch(w, device), act_to_torch(s, dtype, device),
            act_to_torch(b, dtype, device))
