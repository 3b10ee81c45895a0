"""Helpers shared by the GPU parity tests."""
from __future__ import annotations

import sys

import numpy as np
import torch

DEV = "cuda:0"


def announce(msg: str) -> None:
    """Name the case before a GPU step, so a fault can be traced to it."""
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def bf16_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV).to(torch.bfloat16)


def f32_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV)


def rand_bf16(rng: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    """Random values already representable in bf16 (so host and device see the same inputs)."""
    from oracle.moe_oracle import bf16_round

    return bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def zipf_counts(M: int, E: int, s: float, nonempty: int, rng: np.random.Generator) -> np.ndarray:
    """Zipf(s) counts over `nonempty` ranks (remainder to rank 1), placed on a
    seeded permutation of the E experts; the other experts get zero rows."""
    r = np.arange(1, nonempty + 1, dtype=np.float64)
    w = r ** (-s)
    c = np.floor(M * w / w.sum()).astype(np.int64)
    c[0] += M - c.sum()
    counts = np.zeros(E, np.int64)
    counts[rng.permutation(E)[:nonempty]] = c
    return counts


def labels_from_counts(counts: np.ndarray, rng: np.random.Generator) -> np.ndarray:
    """Flat labels with the given histogram, in random order (non-trivial permute)."""
    lab = np.repeat(np.arange(counts.size), counts)
    return rng.permutation(lab)


def topk_labels(T: int, K: int, E: int, rng: np.random.Generator) -> np.ndarray:
    """[T, K] distinct experts per token."""
    return np.argsort(rng.random((T, E)), axis=1)[:, :K].astype(np.int64)
