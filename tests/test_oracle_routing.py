"""Pins the oracle's integer routing functions (CPU only).

Checks: torch.argsort(stable=True) / bincount golden vectors, a brute-force
Python counting sort on small random inputs, invariants, and planted
mistakes that the checks must catch.
"""
from __future__ import annotations

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from conftest import golden_names, load_golden
from oracle import moe_oracle as O


def brute_stable_order(labels, E):
    lab = [int(v) for v in np.asarray(labels).reshape(-1)]
    out = []
    for e in range(E):
        out += [s for s, v in enumerate(lab) if v == e]
    out += [s for s, v in enumerate(lab) if not 0 <= v < E]
    return np.array(out, dtype=np.int32)


@pytest.mark.parametrize("name", golden_names("routing_"))
def test_stable_order_matches_torch_golden(name):
    g = load_golden(name)
    E = int(g["num_experts"])
    np.testing.assert_array_equal(O.stable_order(g["labels"], E), g["sorted_indices"])
    np.testing.assert_array_equal(O.histogram(g["labels"], E), g["counts"])


@settings(max_examples=200, deadline=None)
@given(
    E=st.integers(1, 40),
    labels=st.lists(st.integers(-2, 42), min_size=0, max_size=300),
)
def test_stable_order_brute_force(E, labels):
    lab = np.array(labels, dtype=np.int64)
    np.testing.assert_array_equal(O.stable_order(lab, E), brute_stable_order(lab, E))
    counts = O.histogram(lab, E)
    assert counts.sum() == int(((lab >= 0) & (lab < E)).sum())
    for e in range(E):
        assert counts[e] == int((lab == e).sum())


@settings(max_examples=100, deadline=None)
@given(T=st.integers(1, 60), K=st.integers(1, 8), E=st.integers(8, 64), seed=st.integers(0, 2**31 - 1))
def test_routing_invariants(T, K, E, seed):
    rng = np.random.default_rng(seed)
    lab = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    s = O.stable_order(lab, E)
    flat = lab.reshape(-1)
    assert sorted(s.tolist()) == list(range(T * K))  # a permutation
    assert np.all(np.diff(flat[s]) >= 0)  # labels non-decreasing
    for e in range(E):  # within one expert, ascending flat slot
        grp = s[flat[s] == e]
        assert np.all(np.diff(grp) > 0)
    off = O.offsets_from_counts(O.histogram(lab, E))
    assert off[-1] == T * K
    inv = O.inverse_order(s)
    np.testing.assert_array_equal(s[inv], np.arange(T * K))


def test_permute_unpermute_golden():
    g = load_golden("permute_basic")
    K, E = int(g["top_k"]), int(g["num_experts"])
    permuted, sidx = O.permute(g["tokens"], g["labels"], K, E)
    np.testing.assert_array_equal(sidx, g["sorted_indices"])
    np.testing.assert_array_equal(permuted, g["permuted"])
    out = O.unpermute(permuted, sidx, g["probs"], K)
    np.testing.assert_allclose(out, g["unpermuted"], rtol=0, atol=1e-2 * np.abs(g["unpermuted"]).max())
    out1 = O.unpermute(permuted, sidx, None, K)
    np.testing.assert_array_equal(out1, g["unpermuted_noprob"])


def test_unpermute_inverts_permute():
    rng = np.random.default_rng(7)
    T, E, D = 37, 5, 8
    tok = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    lab = rng.integers(0, E, T)
    permuted, sidx = O.permute(tok, lab, 1, E)
    np.testing.assert_array_equal(O.unpermute(permuted, sidx, None, 1), tok)


def test_unpermute_grad_is_adjoint():
    """<unpermute(p), g> == <p, unpermute_grad(g)> for top_k > 1 with probs."""
    rng = np.random.default_rng(8)
    T, K, E, D = 12, 3, 6, 4
    lab = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    probs = rng.random((T, K)).astype(np.float32)
    sidx = O.stable_order(lab, E)
    p = rng.standard_normal((T * K, D)).astype(np.float32)
    gout = rng.standard_normal((T, D)).astype(np.float32)
    un = O._unpermute_f32(p, sidx, probs.reshape(-1), K)
    s = sidx
    gp = gout[s // K] * probs.reshape(-1)[s][:, None]
    assert np.isclose((un * gout).sum(), (p * gp).sum(), rtol=1e-5)
    gperm, gprobs = O.unpermute_grad(gout, sidx, probs, K, permuted=p)
    # d/dprobs of <unpermute(p, probs), gout> = <p[pos(s)], gout[s//K]>
    ref = np.zeros(T * K)
    for j, sl in enumerate(sidx):
        ref[sl] = p[j] @ gout[sl // K]
    np.testing.assert_allclose(gprobs, ref, rtol=1e-5, atol=1e-6)


def test_group_labels_golden():
    g = load_golden("regroup_labels")
    E_loc = int(g["num_local_experts"])
    lab = O.group_labels(g["counts_group"], E_loc, g["labels"].size)
    np.testing.assert_array_equal(lab, g["labels"])
    # rows past the total get the out-of-range label
    lab2 = O.group_labels(g["counts_group"], E_loc, g["labels"].size + 3)
    assert np.all(lab2[-3:] == E_loc)


def test_regroup_identity_at_ep1():
    rng = np.random.default_rng(3)
    E_loc = 6
    counts = rng.integers(0, 5, E_loc)
    x = rng.standard_normal((int(counts.sum()), 4)).astype(np.float32)
    permuted, sidx, ntpe = O.regroup_permute(x, counts, 1, E_loc)
    np.testing.assert_array_equal(sidx, np.arange(x.shape[0]))
    np.testing.assert_array_equal(permuted, x)
    np.testing.assert_array_equal(ntpe, counts)


def test_regroup_rank_major_to_expert_major():
    # 2 ranks x 2 experts, rows tagged with (rank, expert, i)
    counts = np.array([2, 1, 1, 3])  # (r0,e0)=2 (r0,e1)=1 (r1,e0)=1 (r1,e1)=3
    tags = np.array([0, 1, 10, 100, 110, 111, 112], dtype=np.float32)[:, None]
    permuted, sidx, ntpe = O.regroup_permute(tags, counts, 2, 2)
    np.testing.assert_array_equal(permuted[:, 0], [0, 1, 100, 10, 110, 111, 112])
    np.testing.assert_array_equal(ntpe, [3, 4])


def test_planted_unstable_sort_is_caught():
    """A plausible mistake -- an unstable sort -- fails the brute-force check."""
    lab = np.array([3, 1, 3, 3, 0, 1, 3, 0, 3, 1, 3, 3, 1, 0, 3] * 20)
    wrong = np.argsort(lab, kind="quicksort").astype(np.int32)[::-1]
    wrong = wrong[np.argsort(lab[wrong], kind="stable")]  # grouped right, order within groups reversed
    assert not np.array_equal(wrong, brute_stable_order(lab, 4))
    np.testing.assert_array_equal(O.stable_order(lab, 4), brute_stable_order(lab, 4))
