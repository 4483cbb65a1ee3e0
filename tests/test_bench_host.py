"""Host logic of bench.py that needs no GPU."""
import bench
from skinny_mlx import qmm as Q


def test_stack_batch_keeps_split_k_shapes_on_one_stream():
    """The batch form of the stack spreads its launches over the streams one (K, N) shape per
    stream, with every split-K shape on one stream: split-K calls share the device's workspace."""
    st = bench.Stack.__new__(bench.Stack)  # the lane rule needs only the launch order
    shapes = bench.LAYER_SHAPES + [bench.HEAD_SHAPE]
    st.weights = [(t, None, None, None) for t in bench.LAYER_SHAPES * bench.LAYERS + [bench.HEAD_SHAPE]]
    split = {t for t in shapes if Q._plain_config(*t)[0] > 1}
    assert split  # the down projection
    for streams in (2, 3, 4, 8):
        lanes = st.lanes(streams)
        assert len(lanes) == len(st.weights) and all(0 <= x < streams for x in lanes)
        lane_of = {}
        for (t, *_), x in zip(st.weights, lanes):
            assert lane_of.setdefault(t, x) == x  # one stream per shape
        assert len({lane_of[t] for t in split}) == 1
    assert len(set(st.lanes(4))) == 4
