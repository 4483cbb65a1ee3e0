"""The decoders on the GPU: patched forward vs the numpy oracle decoder, patched vs unpatched,
bitwise M-invariance of the verify forward, and patch_model's counts."""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import w4
from skinny_mlx import patch as P
from skinny_mlx import qmm as Q
from skinny_mlx.cache import make_prompt_cache
from skinny_mlx.model import build_model
from skinny_mlx.spec import forward
from tests.helpers import bits16, model_cfg, near_tie_ok, state_numpy

pytestmark = pytest.mark.gpu


def _f(t):
    return w4.bf16_to_f32(bits16(t)).astype(np.float64)


@pytest.mark.parametrize("preset", ["tiny-dense", "tiny-hybrid", "tiny-qwen35"])
def test_patched_forward_matches_oracle(preset):
    model = build_model(preset)
    oracle = OM.Decoder(state_numpy(model), model_cfg(model))
    P.patch_model(model)
    g = torch.Generator().manual_seed(1)
    toks = torch.randint(0, model.args.vocab_size, (21,), generator=g).tolist()
    cache = make_prompt_cache(model)
    h1, l1 = forward(model, toks[:13], cache)   # a prompt (pieces of 16)
    h2, l2 = forward(model, toks[13:], cache)   # then a verify-sized step of 8
    got = np.concatenate([_f(l1), _f(l2)])
    hid = np.concatenate([_f(h1), _f(h2)])
    ref_h, ref_l = oracle.forward(toks)
    assert w4.rel_err(got, ref_l) <= 2e-2
    assert w4.rel_err(hid, ref_h) <= 2e-2
    assert near_tie_ok(ref_l, got)


@pytest.mark.parametrize("preset", ["tiny-dense", "tiny-hybrid", "tiny-qwen35"])
def test_patched_matches_unpatched(preset):
    ref_model = build_model(preset)
    model = build_model(preset)
    P.patch_model(model)
    toks = list(range(3, 30, 2))
    _, a = forward(ref_model, toks, make_prompt_cache(ref_model))
    _, b = forward(model, toks, make_prompt_cache(model))
    assert w4.rel_err(_f(b), _f(a)) <= 2e-2
    assert near_tie_ok(_f(a), _f(b))


@pytest.mark.parametrize("preset", ["tiny-dense", "tiny-hybrid", "tiny-qwen35"])
def test_verify_forward_bitwise_equals_single_steps(preset):
    model = build_model(preset)
    P.patch_model(model)
    prompt = list(range(40, 77))
    steps = [5, 99, 7, 12, 500, 3, 8, 1000]
    c1 = make_prompt_cache(model)
    forward(model, prompt, c1)
    h_batch, l_batch = forward(model, steps, c1)           # one pass of M = 8
    c2 = make_prompt_cache(model)
    forward(model, prompt, c2)
    singles = [forward(model, [t], c2) for t in steps]     # eight passes of M = 1
    assert torch.equal(l_batch, torch.cat([l for _, l in singles]))
    assert torch.equal(h_batch, torch.cat([h for h, _ in singles]))


@pytest.mark.parametrize("preset", ["tiny-dense", "tiny-hybrid", "tiny-qwen35"])
def test_long_input_pieces_replayed_from_a_graph(preset):
    """An input of four or more 16-token pieces replays one captured pass per piece: bitwise what
    the pieces give run one by one, and the graph is reused by the cache's next prompt."""
    model = build_model(preset)
    P.patch_model(model)
    ids = torch.randint(0, model.args.vocab_size, (75,), generator=torch.Generator().manual_seed(3))
    c1 = make_prompt_cache(model)
    h1, l1 = forward(model, ids.tolist(), c1)
    assert getattr(c1, "_piece_step", None) is not None
    c2 = make_prompt_cache(model)
    dev_ids = ids.to(device=model.device, dtype=torch.int32)
    h2 = torch.cat([model.hidden(dev_ids[i:i + 16], c2) for i in range(0, 75, 16)])
    assert torch.equal(h1, h2) and torch.equal(l1, model.logits(h2))
    graph = c1._piece_step
    h3, _ = forward(model, ids[:64].tolist(), c1)   # a second prompt on the same cache
    h4 = torch.cat([model.hidden(dev_ids[i:i + 16], c2) for i in range(0, 64, 16)])
    assert c1._piece_step is graph and torch.equal(h3, h4)


@pytest.mark.parametrize("conv", [0, 1])
@pytest.mark.parametrize("preset", ["tiny-dense", "tiny-hybrid", "tiny-qwen35"])
def test_folded_norms_bitwise_equal_separate_norms(preset, conv, monkeypatch):
    """Model.fold_norms (on by default): in one-token forwards each RMSNorm before a fused q|k|v or
    gate|up projection runs inside that projection's launch, and with conv = 1 the one before the
    Gated-DeltaNet input projection too (off by default). Hidden states and logits of a prompt
    (separate norms: pieces of up to 16 tokens) followed by single-token steps are bitwise those
    with every norm as its own launch, and a verify forward over the same tokens is bitwise the
    folded single steps."""
    monkeypatch.setitem(P.NORMIN_TOKENS, Q.NORMIN_CONV, conv)
    model = build_model(preset)
    P.patch_model(model)
    assert model.fold_norms
    toks = list(range(5, 40, 3))
    steps = [5, 99, 7, 12, 500, 3, 8, 1000]
    got = []
    for fold in (True, False):
        model.fold_norms = fold
        c = make_prompt_cache(model)
        forward(model, toks, c)
        got.append([forward(model, [t], c) for t in steps])
    model.fold_norms = True
    for (ha, la), (hb, lb) in zip(*got):
        assert torch.equal(ha, hb) and torch.equal(la, lb)
    c = make_prompt_cache(model)
    forward(model, toks, c)
    _, l_batch = forward(model, steps, c)
    assert torch.equal(l_batch, torch.cat([l for _, l in got[0]]))


@pytest.mark.parametrize("preset,expect", [("dense-36", (72, 73, 0)), ("hybrid-36", (72, 73, 0))])
def test_patch_counts_full_size(preset, expect):
    model = build_model(preset)
    st = P.patch_model(model)
    assert (st["fused_groups"], st["single"], st["heads"]) == expect
    # the fused GDN projection is qkv + z + b + a = 6144 + 2048 + 16 + 16 rows
    if preset.startswith("hybrid"):
        proj = model.layers[0].linear_attn.in_proj_qkv.projection
        assert proj.packed.shape[0] == 8224
        assert [(c.start, c.stop) for c in proj.columns] == [(0, 6144), (6144, 8192), (8192, 8208), (8208, 8224)]
    mlp = model.layers[0].mlp
    assert mlp.gate_proj.projection is mlp.up_proj.projection and mlp.gate_proj.projection.gate_up
    del model
    torch.cuda.empty_cache()


@pytest.mark.parametrize("preset", ["tiny-dense", "tiny-hybrid"])
def test_mtp_head_matches_oracle(preset):
    """The patched MTP head (skinny kernels, split-K o_proj/down, fused attention) against the
    numpy restatement of mtp.py:51-67, over a prompt and a 4-token chain step."""
    from skinny_mlx import kernels as K
    from skinny_mlx.mtp import load_mtp_head, make_mtp_cache

    model = build_model(preset)
    head = load_mtp_head(model, patch=False)
    oracle = OM.MTPHead(state_numpy(head), model_cfg(model))
    P.patch_model(head)
    g = torch.Generator().manual_seed(3)
    T = 15
    toks = torch.randint(0, model.args.vocab_size, (T,), generator=g).to(torch.int32).to(model.device)
    hid = (torch.randn((T, model.args.hidden_size), generator=g) * 2).to(torch.bfloat16).to(model.device)
    cache = make_mtp_cache(head)
    emb = K.embed(toks, model.embed_tokens)
    out = torch.cat([head(emb[:11], hid[:11], cache), head(emb[11:], hid[11:], cache)])
    got = _f(out)
    embs, hids = _f(emb), _f(hid)
    ref = np.stack([oracle.step(embs[t], hids[t]) for t in range(T)])
    assert w4.rel_err(got, ref) <= 2e-2
    # the drafters' entry (embedding, input norms and concat in one launch) is bitwise forward()
    cache2 = make_mtp_cache(head)
    fused = torch.cat([head.forward_tokens(toks[:11], model.embed_tokens, hid[:11], cache2),
                       head.forward_tokens(toks[11:], model.embed_tokens, hid[11:], cache2)])
    assert torch.equal(fused, out)


def test_skinny_range_routes_token_counts(monkeypatch):
    """The routing rule (reference patch.py:22, 30-35; toggled at bench/step_cost_curve.py:53-56):
    with SKINNY_RANGE = (6, 16), the reference's range, calls of M = 1..5 tokens take the unpatched
    dequantise + fp32 GEMM and M = 6..16 the skinny kernel, for single and fused linears; with
    (99, 99) every M takes the unpatched path, longer inputs included. Outputs agree with the oracle
    either way."""
    from skinny_mlx import kernels as K

    model = build_model("tiny-dense")
    P.patch_model(model)
    down = model.layers[0].mlp.down_proj      # a SkinnyQuantizedLinear
    qproj = model.layers[0].self_attn.q_proj  # a slice of the fused q|k|v projection
    seen = []
    real_sk, real_dq = P.skinny_qmm, K.quantized_matmul
    monkeypatch.setattr(P, "skinny_qmm", lambda *a, **k: (seen.append("skinny"), real_sk(*a, **k))[1])
    monkeypatch.setattr(K, "quantized_matmul", lambda *a, **k: (seen.append("dequant"), real_dq(*a, **k))[1])
    g = torch.Generator().manual_seed(4)
    ref_w = {m: (m.weight, m.scales, m.biases) for m in (down,)}
    w, s, b = ref_w[down]
    proj = qproj.projection
    for rng_, expect in (((6, 16), lambda m: "skinny" if 6 <= m <= 16 else "dequant"),
                         ((99, 99), lambda m: "dequant")):
        monkeypatch.setattr(P, "SKINNY_RANGE", rng_)
        for m in list(range(1, 17)) + [40]:
            x = torch.randn((m, down.in_features), generator=g).to(torch.bfloat16).to(model.device)
            seen.clear()
            y = down(x)
            want = expect(m) if m <= 16 else ("skinny" if rng_[0] <= 16 <= rng_[1] else "dequant")
            assert seen == [want], (rng_, m, seen)
            ref = w4.qmm(bits16(x), w.cpu().numpy().view(np.uint32), bits16(s), bits16(b))
            assert w4.rel_err(_f(y), ref) <= 4e-3, (rng_, m)
            xq = torch.randn((m, proj.w.shape[1] * 8), generator=g).to(torch.bfloat16).to(model.device)
            seen.clear()
            yq = qproj(xq)
            assert seen == [want], ("fused", rng_, m, seen)
            refq = w4.qmm(bits16(xq), proj.w.cpu().numpy().view(np.uint32), bits16(proj.s), bits16(proj.b))
            assert w4.rel_err(_f(yq), refq[:, qproj.columns]) <= 4e-3, ("fused", rng_, m)
