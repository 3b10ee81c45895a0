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


def rel_err_rows(got: np.ndarray, ref: np.ndarray) -> float:
    """Largest per-row error: max over rows r of max|got_r - ref_r| / max|ref_r|
    (rows of a 2-D array, or the leading index of any array).  A row whose
    reference is all zero must be all zero too (its error is then max|got_r|)."""
    g = np.asarray(got, np.float64).reshape(len(got), -1)
    r = np.asarray(ref, np.float64).reshape(len(ref), -1)
    num = np.abs(g - r).max(axis=1)
    den = np.abs(r).max(axis=1)
    zero = den == 0
    err = np.where(zero, num, num / np.where(zero, 1.0, den))
    return float(err.max()) if err.size else 0.0


def assert_close(got: np.ndarray, ref: np.ndarray, tol: float, what: str = "") -> None:
    """The parity bar of the path, stated twice: norm-wise over the whole
    tensor (max|d| / max|ref|) and for every row on its own (leading index:
    a token row of an output, an expert slice of a weight gradient), so an
    error confined to one small row or one lightly loaded expert is not
    hidden by the largest ones."""
    from oracle.moe_oracle import max_rel_err

    e_all = max_rel_err(got, ref)
    e_row = rel_err_rows(got, ref)
    assert e_all < tol, f"{what}: norm-wise relative error {e_all:.3e} >= {tol}"
    assert e_row < tol, f"{what}: worst row/slice relative error {e_row:.3e} >= {tol}"


def assert_dot_close(got: np.ndarray, ref: np.ndarray, abs_scale: np.ndarray, tol: float, what: str = "") -> None:
    """Per-element check of dot products (routing-score gradients): the
    error of <a, b> is bounded relative to sum |a_i b_i| (the classic
    dot-product error bound), not to |<a, b>|, which can cancel to ~0."""
    g = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    s = np.asarray(abs_scale, np.float64).ravel()
    err = np.abs(g - r) / np.maximum(s, 1e-30)
    assert float(err.max()) < tol, f"{what}: worst |d| / sum|a b| = {float(err.max()):.3e} >= {tol}"


def edge_rows(offs_incl: np.ndarray, tile_rows=(32, 256, 320), experts=None) -> np.ndarray:
    """Rows at the edges of every expert segment (or of the given experts'
    segments) and of every 32/256/320-row tile inside it (first and last row
    of each), for sampled full-size checks."""
    offs_incl = np.asarray(offs_incl, np.int64)
    starts = np.concatenate([[0], offs_incl[:-1]])
    rows = []
    for x, (s, e) in enumerate(zip(starts.tolist(), offs_incl.tolist())):
        if e <= s or (experts is not None and x not in experts):
            continue
        rows += [s, e - 1]
        for h in tile_rows:
            for b in range(s + h, e, h):
                rows += [b - 1, b]
    return np.unique(np.asarray(rows, np.int64))
