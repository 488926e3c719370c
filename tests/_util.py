"""Conversions between numpy bf16 bit patterns and torch tensors for the tests."""
import numpy as np
import torch


def bf16_bits(x_f32):
    """bf16-valued float32 -> uint16 bit patterns (exact: the low 16 bits are zero)."""
    return (np.ascontiguousarray(x_f32, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def to_dev(u16, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).view(torch.bfloat16).to(device)


def to_host(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def rand_bf16(rng, shape, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)
