"""Helpers shared by the GPU parity tests (device <-> numpy, seeded inputs)."""
import numpy as np
import torch


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def randn(r: np.random.Generator, *shape, scale: float = 1.0) -> np.ndarray:
    return (r.standard_normal(shape) * scale).astype(np.float32)


def empty(*shape) -> torch.Tensor:
    # NaN-filled so an unwritten output never passes by accident.
    return torch.full(shape, float("nan"), dtype=torch.float32, device="cuda")
