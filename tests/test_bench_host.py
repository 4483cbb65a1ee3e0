"""Host logic of bench.py that needs no GPU."""
import bench


def test_stack_batch_puts_one_shape_per_stream():
    """The batch form of the stack spreads its launches over the streams one (K, N) shape per
    stream in turn, using every stream (split-K calls keep a workspace per stream, so the
    split-K shape needs no stream of its own)."""
    st = bench.Stack.__new__(bench.Stack)  # the lane rule needs only the launch order
    st.weights = [(t, None, None, None) for t in bench.LAYER_SHAPES * bench.LAYERS + [bench.HEAD_SHAPE]]
    for streams in (2, 3, 4, 8):
        lanes = st.lanes(streams)
        assert len(lanes) == len(st.weights) and all(0 <= x < streams for x in lanes)
        lane_of = {}
        for (t, *_), x in zip(st.weights, lanes):
            assert lane_of.setdefault(t, x) == x  # one stream per shape
        assert len(set(lanes)) == min(streams, len(bench.LAYER_SHAPES) + 1)
