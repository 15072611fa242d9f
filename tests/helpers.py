"""Small helpers shared by the GPU tests (bf16 bit patterns <-> torch)."""
import numpy as np
import torch


def dev_bf16(bits: np.ndarray) -> torch.Tensor:
    """uint16 bf16 bit patterns -> a bf16 tensor on the GPU."""
    t = torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16))
    return t.view(torch.bfloat16).cuda()


def host_bits(t: torch.Tensor) -> np.ndarray:
    """A bf16 tensor -> uint16 bit patterns on the host."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def rand_bf16_bits(rng: np.random.Generator, shape, std=1.0) -> np.ndarray:
    """Seeded N(0, std) values rounded to bf16 by torch (RNE)."""
    a = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * std)
    return a.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = float(np.sum(b * b))
    num = float(np.sum((a - b) ** 2))
    return (num / den) ** 0.5 if den > 0 else num ** 0.5


def max_rel(a, b) -> float:
    """max |a - b| / max |b| (the 1e-2 bar's definition)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    mb = float(np.max(np.abs(b))) if b.size else 0.0
    md = float(np.max(np.abs(a - b))) if a.size else 0.0
    return md / mb if mb > 0 else md
