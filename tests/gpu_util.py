"""Helpers shared by the GPU parity tests (inputs are generated on the host
from seeded numpy generators, uploaded, and the same arrays go to the oracle)."""
import numpy as np
import torch

from oracle import tallax_oracle as O


def to_dev(x_f32: np.ndarray, dtype: str, device) -> torch.Tensor:
    if dtype == "bf16":
        bits = O.f32_to_bf16_bits(x_f32)
        return torch.from_numpy(bits.view(np.int16).copy()).to(device).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(x_f32, dtype=np.float32)).to(device)


def host_values(x_f32: np.ndarray, dtype: str) -> np.ndarray:
    """The exact f32 values the device tensor holds."""
    return O.round_to_dtype(x_f32, dtype)


def from_dev_vals(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return O.bf16_bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return t.cpu().numpy()


def bits(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).view(np.uint32)
