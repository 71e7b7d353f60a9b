"""Host<->device helpers for the GPU parity tests (bit patterns stay exact)."""
import numpy as np


def dev_bits16(torch, bits: np.ndarray, dtype=None):
    """uint16 bit patterns -> device tensor of dtype (bfloat16 by default)."""
    dtype = dtype or torch.bfloat16
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to("cuda")
    return t.view(dtype)


def host_bits16(t) -> np.ndarray:
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def dev_f32(torch, a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda")


def dev_u8(torch, a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to("cuda")


def rel_max_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got-ref| / max|ref| — the BASELINE.json tolerance measure."""
    scale = float(np.abs(ref).max())
    return float(np.abs(got.astype(np.float64) - ref.astype(np.float64)).max()) / max(scale, 1e-30)
