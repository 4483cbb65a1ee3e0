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


def test_single_leg_flags_and_the_one_gpu_rule(capsys):
    """The flags behind the committed kernel summaries parse, and --gpus above 1 exits with a
    message before anything touches a device (this path runs on exactly one GPU)."""
    a = bench.parse_args(["--spec-only", "3", "--spec-tokens", "256"])
    assert (a.spec_only, a.spec_tokens) == (3, 256)
    a = bench.parse_args(["--verify-only", "8", "--verify-preset", "qwen35-4b"])
    assert (a.verify_only, a.verify_preset) == (8, "qwen35-4b")
    assert bench.parse_args([]).spec_only == 0
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_qwen35_step_table_matches_its_m_list():
    """The reference's step-cost table that rides along with the Qwen3.5-4B-shaped verify curve
    covers exactly the token counts the curve measures."""
    assert set(bench.REFERENCE_QWEN35_STEP["ms"]) == set(bench.QWEN35_MS)
    assert bench.REFERENCE_QWEN35_STEP["ms"][8] / bench.REFERENCE_QWEN35_STEP["ms"][1] < 1.71
