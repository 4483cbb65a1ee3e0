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
