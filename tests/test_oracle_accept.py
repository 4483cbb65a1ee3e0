"""Pins the acceptance oracle (oracle/accept.py) by exhaustive enumeration and hand cases."""

import itertools

import numpy as np
import pytest

from oracle import accept as A


def _first_mismatch(draft, pred):
    # independent formulation: index of the first disagreement, K if none
    diffs = [i for i in range(len(draft)) if draft[i] != pred[i]]
    return diffs[0] if diffs else len(draft)


@pytest.mark.parametrize("k", [0, 1, 2, 3, 4])
def test_accept_exhaustive(k):
    alphabet = range(3)
    for draft in itertools.product(alphabet, repeat=k):
        for pred in itertools.product(alphabet, repeat=k + 1):
            n, bonus, keep = A.accept(list(draft), list(pred))
            m = _first_mismatch(draft, pred)
            assert n == m and bonus == pred[m] and keep == m + 1
            emitted = list(draft[:n]) + [bonus]
            assert emitted == list(pred[:n + 1])  # greedy-exact: emitted tokens are the target's own argmaxes


def test_argmax_first_index_on_ties():
    rng = np.random.default_rng(0)
    for _ in range(200):
        row = rng.integers(0, 4, size=rng.integers(1, 40)).astype(np.float32)
        i = A.argmax_first(row)
        assert row[i] == row.max() and all(row[j] < row.max() for j in range(i))
    assert A.argmax_first(np.array([1.0, 3.0, 3.0, 2.0])) == 1


def test_prompt_lookup_hand_cases():
    # trailing 3-gram (1, 2, 3) seen earlier, followed by 4, 5
    assert A.prompt_lookup([1, 2, 3, 4, 5, 9, 1, 2, 3], 3, 2) == [4, 5]
    # the latest earlier occurrence wins
    assert A.prompt_lookup([7, 8, 1, 7, 8, 2, 7, 8], 2, 1) == [2]
    # falls back to shorter n-grams, then to nothing
    assert A.prompt_lookup([5, 6, 9, 6], 3, 3) == [9, 6]
    assert A.prompt_lookup([1, 2, 3], 3, 2) == []
    # the match may run into the tail, and is cut at k
    assert A.prompt_lookup([4, 4, 4, 4], 2, 5) == [4]


def _deepest_matched(tokens, parents, pred):
    # independent formulation: a node is reached when every edge on its ancestor chain carries the
    # prediction of the edge's parent; the deepest reached node (siblings carry distinct tokens)
    reached = [True] + [False] * (len(tokens) - 1)
    depth = [0] * len(tokens)
    for v in range(1, len(tokens)):
        p = parents[v]
        depth[v] = depth[p] + 1
        reached[v] = reached[p] and tokens[v] == pred[p]
    best = max((v for v in range(len(tokens)) if reached[v]), key=lambda v: depth[v])
    chain = [best]
    while chain[-1] != 0:
        chain.append(parents[chain[-1]])
    return chain[::-1]


def test_tree_accept_against_deepest_matched_node():
    import random

    rng = random.Random(0)
    for trial in range(2000):
        M = rng.randrange(1, 17)
        parents = [-1] + [rng.randrange(0, i) for i in range(1, M)]
        tokens, used = [rng.randrange(50)], {}
        for v in range(1, M):  # distinct tokens among siblings, as top-k drafting gives
            taken = used.setdefault(parents[v], set())
            t = rng.choice([x for x in range(6) if x not in taken] or [99 + v])
            taken.add(t)
            tokens.append(t)
        pred = [rng.randrange(6) for _ in range(M)]
        n, bonus, path = A.tree_accept(tokens, parents, pred)
        assert path == _deepest_matched(tokens, parents, pred)
        assert n == len(path) - 1 and bonus == pred[path[-1]]


@pytest.mark.parametrize("k", [0, 1, 2, 3])
def test_tree_accept_on_chains_is_linear_acceptance(k):
    alphabet = range(3)
    for draft in itertools.product(alphabet, repeat=k):
        for pred in itertools.product(alphabet, repeat=k + 1):
            tokens = [7] + list(draft)
            parents = [-1] + list(range(k))
            n, bonus, path = A.tree_accept(tokens, parents, list(pred))
            assert (n, bonus, n + 1) == A.accept(list(draft), list(pred)) and path == list(range(n + 1))
