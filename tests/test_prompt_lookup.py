"""The product's incremental prompt-lookup drafter proposes exactly what the oracle's
restatement of the reference's scan proposes (oracle/accept.py, reference spec.py:41-48), at
every step of a growing context. CPU only: the drafter is host code."""

import random

import pytest

from oracle import accept as A
from skinny_mlx.spec import PromptLookupDrafter


@pytest.mark.parametrize("ngram", [1, 2, 3, 4])
@pytest.mark.parametrize("alphabet", [2, 3, 7])
def test_incremental_index_matches_scan(ngram, alphabet):
    rng = random.Random(ngram * 100 + alphabet)
    for trial in range(30):
        prompt = [rng.randrange(alphabet) for _ in range(rng.randrange(0, 12))]
        first = rng.randrange(alphabet)
        d = PromptLookupDrafter(ngram)
        d.begin(prompt, None, first)
        ctx = list(prompt) + [first]
        for step in range(12):
            k = rng.randrange(0, 6)
            assert d.draft(k) == A.prompt_lookup(ctx, ngram, k), (prompt, first, ctx, k)
            new = [rng.randrange(alphabet) for _ in range(rng.randrange(1, 5))]
            d.update(None, new)
            ctx += new


def test_hand_cases_through_the_drafter():
    d = PromptLookupDrafter(3)
    d.begin([1, 2, 3, 4, 5, 9, 1, 2], None, 3)
    assert d.draft(2) == [4, 5]
    d.update(None, [4])
    assert d.draft(3) == [5, 9, 1]  # (2, 3, 4) seen at the start, followed by 5 9 1
    with pytest.raises(ValueError):
        PromptLookupDrafter(0)
