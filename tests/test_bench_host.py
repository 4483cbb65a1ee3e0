"""Host logic of bench.py that needs no GPU."""
import bench


def test_stack_batch_balances_bytes_over_streams():
    """The batch form of the stack deals its launches to the streams largest first, each to the
    stream with the fewest bytes so far: every stream is used, and no stream's bytes exceed the
    mean by more than the largest launch (the greedy bound)."""
    st = bench.Stack.__new__(bench.Stack)  # the lane rule needs only the launch shapes
    st.weights = [(t, None, None, None) for t in bench.LAYER_SHAPES * bench.LAYERS + [bench.HEAD_SHAPE]]
    sizes = [bench.qmm_bytes(8, *t) for t, *_ in st.weights]
    for streams in (2, 3, 4, 8):
        lanes = st.lanes(streams)
        assert len(lanes) == len(st.weights) and set(lanes) == set(range(streams))
        per = [sum(s for s, x in zip(sizes, lanes) if x == lane) for lane in range(streams)]
        assert max(per) - sum(sizes) / streams <= max(sizes)
        assert lanes == st.lanes(streams)  # deterministic


def test_calibrated_drafts_keep_the_reference_acceptance():
    """Drafts of the calibrated drafter: each position its greedy token with probability p, else a
    token greedy verification rejects; the expected tokens per step at p match the reference's
    measured 2.51 / 3.05 / 3.47 at K = 2 / 3 / 4 within 0.08."""
    ref = list(range(1000, 21000))
    d = bench.calibrated_drafts(ref, bench.REFERENCE_DRAFT_P, 151936, seed=3).tolist()
    right = [a == b for a, b in zip(d, ref)]
    assert abs(sum(right) / len(ref) - bench.REFERENCE_DRAFT_P) < 0.01
    assert all(a != b for a, b, ok in zip(d, ref, right) if not ok)
    assert d == bench.calibrated_drafts(ref, bench.REFERENCE_DRAFT_P, 151936, seed=3).tolist()
    p = bench.REFERENCE_DRAFT_P
    for k, measured in ((2, 2.51), (3, 3.05), (4, 3.47)):
        assert abs(sum(p ** i for i in range(k + 1)) - measured) < 0.08
