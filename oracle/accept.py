"""Greedy acceptance and prompt-lookup drafting restated (oracle; tests only).

Reference:
  * pred = mx.argmax over each verify row; mx.argmax returns the first maximal index
    (skinny_mlx/spec.py:137);
  * n = longest prefix with draft[i] == pred[i]; emitted draft[:n] + [pred[n]]; the cache
    keeps n + 1 of the K + 1 fed tokens (spec.py:142-147);
  * prompt lookup: propose what followed the latest earlier occurrence of the trailing
    n-gram, trying n = ngram .. 1 (spec.py:41-48).

  * draft trees (no counterpart in the reference, which verifies chains; its stated next step,
    README.md:84): from the root, step to the first child (node order) whose token equals the
    prediction at the current node; the path, n = its length - 1 and the bonus pred[last].

Pins (tests/test_oracle_accept.py): exhaustive enumeration of every draft/prediction
pattern over a small alphabet for K <= 4 against an independent formulation (the first
mismatch index), argmax ties against the smallest index among maxima, and hand-worked
prompt-lookup cases; the tree walk against an independent formulation (the deepest node whose
whole ancestor chain matches the predictions) on random trees, and against `accept` on chains.
"""

from __future__ import annotations

import numpy as np


def argmax_first(row) -> int:
    """Index of the maximum, the first one on ties."""
    row = np.asarray(row)
    return int(np.flatnonzero(row == row.max())[0])


def accept(draft, pred):
    """(n accepted drafts, bonus token pred[n], keep = n + 1)."""
    n = 0
    while n < len(draft) and draft[n] == pred[n]:
        n += 1
    return n, int(pred[n]), n + 1


def prompt_lookup(ctx, ngram: int, k: int):
    for n in range(ngram, 0, -1):
        tail = ctx[-n:]
        for start in range(len(ctx) - n - 1, -1, -1):
            if ctx[start:start + n] == tail:
                return ctx[start + n:start + n + k]
    return []


def tree_accept(tokens, parents, pred):
    """(n, bonus, path) for a draft tree: node 0 is the root, parents[i] < i for i > 0."""
    path = [0]
    cur = 0
    while True:
        nxt = next((c for c in range(cur + 1, len(tokens)) if parents[c] == cur and tokens[c] == pred[cur]), None)
        if nxt is None:
            break
        path.append(nxt)
        cur = nxt
    return len(path) - 1, int(pred[cur]), path
