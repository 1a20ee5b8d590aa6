"""GPU parity of the C++ host layer (run on the MI355X).

* HipAccelerationManager: every hot-path IAccelerationManager method against
  the CPU oracle on the reference parity suite's closed-form inputs
  (AccelerationManagerParityTests.cs:313-500, 755-768, 1087-1218), plus the
  resident-weight shadow compare and the decode capability.
* LanguageModel (the reference's call sequence on the manager) and
  DeviceLanguageModel (device-resident engine): logits against the float64
  golden fixtures and the oracle, and greedy token ids identical to the
  oracle's, for the tiny test model and the config-1 text model.
* The config-5 time-series regression transformer (continuous inputs) against
  a composition of oracle functions.

Bar: |got - want| <= 1e-4 + 1e-3 |want| per element; token ids exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_parity, load_lm_golden
from oracle import oracle as O
from cdml import host, synth

pytestmark = pytest.mark.gpu

M, Vec = synth.matrix, synth.vector


def parity(a, e, what="", atol=1e-4, rtol=1e-3):
    assert_parity(a, e, atol=atol, rtol=rtol, what=what)


@pytest.fixture(scope="module")
def H():
    return host.module()


@pytest.fixture(scope="module")
def mgr(H):
    m = H.HipAccelerationManager(0)
    yield m
    m.Dispose()


# ------------------------------------------------------------ the manager
def test_manager_project_qkv(mgr):
    x = M(6, 5, 124)
    args = (M(8, 5, 125), Vec(8, 128), M(8, 5, 126), Vec(8, 129), M(8, 5, 127), Vec(8, 130))
    for got, want, n in zip(mgr.ProjectQKV(x, *args), O.project_qkv(x, *args), "QKV"):
        parity(got, want, f"ProjectQKV {n}")
    xg = M(192, 128, 142)
    args = (M(128, 128, 143), Vec(128, 146), M(128, 128, 144), Vec(128, 147), M(128, 128, 145), Vec(128, 148))
    for got, want, n in zip(mgr.ProjectQKV(xg, *args), O.project_qkv(xg, *args), "QKV"):
        parity(got, want, f"ProjectQKV 192x128 {n}")


def test_manager_attention(mgr, ops_golden):
    g = ops_golden
    qs, ks, vs = M(4, 8, 118), M(4, 8, 119), M(4, 8, 120)
    qc, kc, vc = M(4, 8, 121), M(5, 8, 122), M(5, 8, 123)
    parity(mgr.ScaledDotProductAttention(qs, ks, vs, 2), O.sdpa(qs, ks, vs, 2), "SDPA self")
    parity(mgr.ScaledDotProductAttention(qs, ks, vs, 2, g["self_mask"].astype(bool)),
           O.sdpa(qs, ks, vs, 2, mask=g["self_mask"]), "SDPA self mask")
    causal = mgr.ScaledDotProductAttention(qs, ks, vs, 2, None, True)
    parity(causal, O.sdpa(qs, ks, vs, 2, causal=True), "SDPA causal")
    parity(mgr.ScaledDotProductAttention(qs, ks, vs, 2, mgr.CreateCausalMask(4)), causal, "flag == mask")
    parity(mgr.ScaledDotProductAttention(qc, kc, vc, 2, g["cross_mask"].astype(bool)),
           O.sdpa(qc, kc, vc, 2, mask=g["cross_mask"]), "SDPA cross mask")
    am = mgr.ScaledDotProductAttention(qc, kc, vc, 2, g["all_masked_mask"].astype(bool))
    assert np.all(am[0] == 0)
    q6, k6, v6 = M(4, 6, 31), M(4, 6, 32), M(4, 6, 33)
    sc = float(g["mha_causal_scale"])
    parity(mgr.MultiHeadAttentionForward(q6, k6, v6, 2, sc, O.causal_mask(4).astype(bool)),
           O.mha_forward(q6, k6, v6, 2, sc, mask=O.causal_mask(4)), "MHA d_h=3")
    qg, kg, vg = M(128, 64, 110), M(128, 64, 111), M(128, 64, 112)
    parity(mgr.MultiHeadAttentionForward(qg, kg, vg, 4, 0.25), O.mha_forward(qg, kg, vg, 4, 0.25), "MHA 128")
    parity(mgr.ScaledDotProductAttention(qg, kg, vg, 4, None, True), O.sdpa(qg, kg, vg, 4, causal=True),
           "SDPA 128 causal")


def test_manager_projection_rope_layernorm_embed(mgr):
    parity(mgr.ProjectOutputBatch(M(4, 6, 56), M(3, 6, 57), Vec(3, 58), 4, 3),
           O.project_output_batch(M(4, 6, 56), M(3, 6, 57), Vec(3, 58)), "ProjectOutputBatch")
    x = M(10, 8, 3)
    parity(mgr.BatchDotProductAddBias(M(5, 8, 4), x, 2, 6, Vec(5, 5)),
           O.batch_dot_add_bias(M(5, 8, 4), x[2:8], Vec(5, 5)), "BatchDotProductAddBias slice")
    m = M(4, 8, 97)
    got = m.copy()
    mgr.ApplyRotaryPositionEmbeddingInPlace(got, 2, 10000.0, False)
    parity(got, O.rope(m, 2), "RoPE in place")
    mgr.ApplyRotaryPositionEmbeddingInPlace(got, 2, 10000.0, True)
    assert np.allclose(got, m, atol=5e-4)  # AccelerationManagerParityTests.cs:1107-1111
    h = m.copy()
    mgr.ApplyRotaryPositionEmbeddingHeadInPlace(h, 2, 4, 10000.0, False)
    parity(h, O.rope_head(m, 2, 4), "RoPE one head")
    a, b = M(5, 6, 27), M(5, 6, 28)
    g, be = synth.positive_vector(6, 28), Vec(6, 29)
    parity(mgr.ResidualLayerNorm(a, b, g, be), O.residual_layernorm(a, b, g, be), "ResidualLayerNorm")
    table = M(6, 5, 64)
    assert np.array_equal(mgr.EmbedTokenIds(np.array([0, 2, 4], np.int32), table, 5),
                          O.embed_tokens([0, 2, 4], table))
    assert np.array_equal(mgr.EmbedTokenIds(np.array([9, 1, 3, 9], np.int32), 1, 2, table, 5),
                          O.embed_tokens([1, 3], table))


def test_manager_ffn(mgr):
    x = synth.normal(1, (40, 32))
    w1, b1 = synth.xavier_uniform(2, 64, 32), synth.normal(3, (64,)) * np.float32(0.1)
    w2, b2 = synth.xavier_uniform(4, 32, 64), synth.normal(5, (32,)) * np.float32(0.1)
    want = O.batch_dot_add_bias(w2, O.activation(O.batch_dot_add_bias(w1, x, b1), 3), b2)
    parity(mgr.FFNForwardBatch(x, 40, 32, [w1, w2], [b1, b2], [3, 0]), want, "FFNForwardBatch")


def test_manager_resident_weights_follow_host_changes(mgr):
    """A weight array changed in place after its first upload must be seen
    (the shadow compare of DeviceResidentCache.cs:65-69)."""
    x, w, b = M(7, 16, 1), M(9, 16, 2), Vec(9, 3)
    first = mgr.ProjectOutputBatch(x, w, b, 7, 9)
    parity(first, O.project_output_batch(x, w, b), "first")
    w[3, 5] += np.float32(1.0)
    b[0] -= np.float32(0.5)
    parity(mgr.ProjectOutputBatch(x, w, b, 7, 9), O.project_output_batch(x, w, b), "after in-place change")


def test_manager_attention_backward(mgr):
    """MultiHeadAttentionBackward, both overloads, on the parity suite's
    closed-form case (AccelerationManagerParityTests.cs:355-382: 4x6, 2 heads,
    scale 1/sqrt 3, decoder flag and explicit causal mask), the consistency
    suite's 6x8 no-mask / decoder and 5x8 cross cases
    (AccelerationConsistencyTests.cs:962-1020), and causal cases on the MFMA
    kernels: 300x128 (head dim 64) by flag and by mask, 237x128 and 700x128
    (head dim 32, either side of the short stored-dS kernel's 512 rows)."""
    q, k, v, d = M(4, 6, 31), M(4, 6, 32), M(4, 6, 33), M(4, 6, 34)
    scale = float(np.float32(1) / np.sqrt(np.float32(3)))
    causal = np.tril(np.ones((4, 4), bool))
    want = O.mha_backward(q, k, v, d, 2, scale, use_decoder_mask=True)
    for got, w, n in zip(mgr.MultiHeadAttentionBackward(q, k, v, d, 2, scale, True), want, ("dQ", "dK", "dV")):
        parity(got, w, f"MHA backward (bool) {n}")
    for got, w, n in zip(mgr.MultiHeadAttentionBackward(q, k, v, d, 2, scale, causal), want, ("dQ", "dK", "dV")):
        parity(got, w, f"MHA backward (mask) {n}")
    for lq, lk, dec in ((6, 6, False), (6, 6, True), (5, 8, False)):
        q, k, v, d = M(lq, 8, 51), M(lk, 8, 52), M(lk, 8, 53), M(lq, 8, 54)
        s = float(np.float32(1) / np.sqrt(np.float32(4)))
        want = O.mha_backward(q, k, v, d, 2, s, use_decoder_mask=dec)
        for got, w, n in zip(mgr.MultiHeadAttentionBackward(q, k, v, d, 2, s, dec), want, ("dQ", "dK", "dV")):
            parity(got, w, f"MHA backward {lq}x{lk} decoder={dec} {n}")
    L, D, Hh = 300, 128, 2
    q, k, v, d = (synth.normal(60 + i, (L, D)) for i in range(4))
    s = 0.125
    want = O.mha_backward(q, k, v, d, Hh, s, use_decoder_mask=True)
    for got, w, n in zip(mgr.MultiHeadAttentionBackward(q, k, v, d, Hh, s, True), want, ("dQ", "dK", "dV")):
        parity(got, w, f"MHA backward 300x128 causal {n}")
    # the same case through the bool[,] overload (no stored dS with a mask),
    # and head dim 32 with a ragged last block (stored dS, the short dQ kernel)
    tri = np.tril(np.ones((L, L), bool))
    for got, w, n in zip(mgr.MultiHeadAttentionBackward(q, k, v, d, Hh, s, tri), want, ("dQ", "dK", "dV")):
        parity(got, w, f"MHA backward 300x128 mask {n}")
    L, Hh = 237, 4
    q, k, v, d = (synth.normal(70 + i, (L, D)) for i in range(4))
    s = float(np.float32(1) / np.sqrt(np.float32(32)))
    want = O.mha_backward(q, k, v, d, Hh, s, use_decoder_mask=True)
    for got, w, n in zip(mgr.MultiHeadAttentionBackward(q, k, v, d, Hh, s, True), want, ("dQ", "dK", "dV")):
        parity(got, w, f"MHA backward 237x128 head dim 32 causal {n}")
    # head dim 32 past 512 rows: the stored-dS dQ of the long-sequence kernel
    L = 700
    q, k, v, d = (synth.normal(90 + i, (L, D)) for i in range(4))
    want = O.mha_backward(q, k, v, d, Hh, s, use_decoder_mask=True)
    for got, w, n in zip(mgr.MultiHeadAttentionBackward(q, k, v, d, Hh, s, True), want, ("dQ", "dK", "dV")):
        parity(got, w, f"MHA backward 700x128 head dim 32 causal {n}")


def test_manager_projection_backward(mgr):
    """BackpropQKV, BackpropLinearProjection and BackpropOutputProjection with
    nonzero gradient accumulators on entry (they must accumulate), on the
    consistency suite's shapes (AccelerationConsistencyTests.cs:633-700) and a
    projection-sized case."""
    for rows, ind, out in ((4, 8, 8), (300, 256, 256)):
        x, dq, dk, dv = M(rows, ind, 71), M(rows, out, 72), M(rows, out, 73), M(rows, out, 74)
        w = [M(out, ind, 75 + i) for i in range(3)]
        g0 = [M(out, ind, 80), Vec(out, 81), M(out, ind, 82), Vec(out, 83), M(out, ind, 84), Vec(out, 85)]
        want = O.backprop_qkv(x, dq, dk, dv, *w, *g0)
        g = [a.copy() for a in g0]
        dx = mgr.BackpropQKV(x, dq, dk, dv, *w, *g)
        for got, e, n in zip((dx, *g), want, ("dInput", "WQGrad", "biasQGrad", "WKGrad", "biasKGrad",
                                               "WVGrad", "biasVGrad")):
            parity(got, e, f"BackpropQKV {rows}x{ind} {n}")
        wg0, bg0, dx0 = M(out, ind, 90), Vec(out, 91), M(rows, ind, 92)
        want = O.backprop_linear_projection(x, dq, w[0], wg0, bg0, dx0)
        wg, bg, dxi = wg0.copy(), bg0.copy(), dx0.copy()
        mgr.BackpropLinearProjection(x, dq, w[0], wg, bg, dxi)
        for got, e, n in zip((wg, bg, dxi), want, ("weightGrad", "biasGrad", "dInput")):
            parity(got, e, f"BackpropLinearProjection {rows}x{ind} {n}")
    seq, outd, emb = 4, 8, 6
    dl, x, w = M(seq, outd, 93), M(seq, emb, 94), M(outd, emb, 95)
    wg0, bg0 = M(outd, emb, 96), Vec(outd, 97)
    want = O.backprop_output_projection(dl, x, w, wg0, bg0)
    wg, bg = wg0.copy(), bg0.copy()
    dX = mgr.BackpropOutputProjection(dl, x, w, wg, bg, seq, outd, emb)
    for got, e, n in zip((dX, wg, bg), want, ("dX", "weightGrad", "biasGrad")):
        parity(got, e, f"BackpropOutputProjection {n}")
    # the LM-head shape of config 1: vocab 200, D 64, 64 rows
    dl, x, w = synth.normal(98, (64, 200)), synth.normal(99, (64, 64)), M(200, 64, 100)
    wg0, bg0 = np.zeros((200, 64), np.float32), np.zeros(200, np.float32)
    want = O.backprop_output_projection(dl, x, w, wg0, bg0)
    wg, bg = wg0.copy(), bg0.copy()
    dX = mgr.BackpropOutputProjection(dl, x, w, wg, bg, 64, 200, 64)
    for got, e, n in zip((dX, wg, bg), want, ("dX", "weightGrad", "biasGrad")):
        parity(got, e, f"BackpropOutputProjection LM head {n}")


def test_manager_training_methods(mgr):
    """MatrixMultiply / MatrixMultiplyTranspose, ResidualLayerNormForward,
    LayerNormBackward, CrossEntropyLossAndGradient, MSELossAndGradient and
    AccumulateTokenEmbeddingGrad against the oracle (MatrixMultiply against
    float64 matrix algebra, the reference's textbook product)."""
    A, B = synth.normal(1, (130, 257)), synth.normal(2, (257, 66))
    ref = A.astype(np.float64) @ B.astype(np.float64)
    parity(mgr.MatrixMultiply(A, B), ref, "MatrixMultiply")
    parity(mgr.MatrixMultiplyTranspose(A, np.ascontiguousarray(B.T)), ref, "MatrixMultiplyTranspose")
    x, sl = synth.normal(3, (40, 96)), synth.normal(4, (40, 96))
    g, be = synth.positive_vector(96, 5), synth.normal(6, (96,))
    got = mgr.ResidualLayerNormForward(x, sl, g, be)
    want = O.residual_layernorm_forward(x, sl, g, be)
    for a, e, n in zip(got, want, ("output", "means", "variances", "normalized", "residual")):
        parity(a, e, f"ResidualLayerNormForward {n}")
    d = synth.normal(7, (40, 96))
    got = mgr.LayerNormBackward(d, want[3], g, want[4], want[1], want[2])
    for a, e, n in zip(got, O.layernorm_backward(d, want[3], g, want[4], want[1], want[2]),
                       ("dInput", "dGamma", "dBeta")):
        parity(a, e, f"LayerNormBackward {n}")
    logits = synth.normal(8, (12, 200)) * np.float32(2)
    t = (np.arange(20) * 37 % 200).astype(np.int32)
    loss, dl = mgr.CrossEntropyLossAndGradient(logits, t, 3, 10)
    wl, wd = O.cross_entropy(logits, t, 10, target_start=3)
    assert abs(loss - wl) <= 1e-5 + 1e-5 * abs(wl)
    parity(dl, wd, "CrossEntropyLossAndGradient")
    pred, tgt = synth.normal(11, (12, 3)), synth.normal(12, (20, 3))
    loss, dp = mgr.MSELossAndGradient(pred, tgt, 4, 9)
    wl, wd = O.mse_loss(pred, tgt, 9, target_start=4)
    assert abs(loss - wl) <= 1e-5 + 1e-5 * abs(wl)
    parity(dp, wd, "MSELossAndGradient")
    assert not dp[9:].any()
    eg = synth.normal(9, (50, 16))
    dx = synth.normal(10, (30, 16))
    ids = (np.arange(40) * 7 % 50).astype(np.int32)
    ids[5:15] = 4
    want = O.accumulate_token_embedding_grad(eg, dx, ids[5:35])
    got = eg.copy()
    mgr.AccumulateTokenEmbeddingGrad(got, dx, ids, 5, 30, 16)
    assert np.array_equal(got, want)


def test_manager_decode_step_matches_prefill(mgr):
    """The decode capability over T steps reproduces causal prefill row by row
    (RoPE at the absolute position, append, attend)."""
    T, D, Hh = 40, 64, 4
    q, k, v = (synth.normal(60 + i, (T, D)) for i in range(3))
    qr, kr = O.rope(q, Hh), O.rope(k, Hh)
    pre = O.sdpa(qr, kr, v, Hh, causal=True)
    keys = np.zeros((T, D), np.float32)
    vals = np.zeros((T, D), np.float32)
    for t in range(T):
        qt, kt = q[t:t + 1].copy(), k[t:t + 1].copy()
        out = mgr.DecodeSelfAttention(qt, kt, v[t:t + 1], keys, vals, t, Hh)
        parity(out[0], pre[t], f"decode step {t}")
        parity(qt[0], qr[t], f"rotated q {t}")
    parity(keys, kr, "host key cache")
    assert np.array_equal(vals, v)


# ------------------------------------------------------ language models
@pytest.mark.parametrize("name", ["lm_tiny", "lm_c1"])
def test_language_model_forward_and_generate(mgr, name):
    g = load_lm_golden(name)
    lm, _ = host.language_model(g["cfg"], g["weights"], mgr)
    logits = lm.Forward(g["ids"])
    parity(logits, g["logits"], f"{name} LanguageModel.Forward vs float64 golden")
    parity(logits, O.LanguageModel(g["cfg"], g["weights"]).forward(g["ids"]), f"{name} vs oracle")
    out = lm.Generate(g["ids"][: int(g["prompt_len"])], int(g["n_new"]))
    assert np.array_equal(out, g["greedy"]), f"{name}: greedy tokens differ"


@pytest.mark.parametrize("name", ["lm_tiny", "lm_c1"])
def test_device_language_model(H, mgr, name):
    g = load_lm_golden(name)
    lm, _ = host.language_model(g["cfg"], g["weights"], mgr)
    dev = H.DeviceLanguageModel(lm, 4)
    ids = g["ids"]
    got = dev.Forward(ids[None, :])
    parity(got, g["logits"], f"{name} device forward vs golden")
    P = int(g["prompt_len"])
    out = dev.GenerateGreedy(ids[None, :P], int(g["n_new"]))
    assert np.array_equal(out[0], g["greedy"]), f"{name}: device greedy tokens differ"


def test_checkpoint_load_then_forward(H, mgr, tmp_path):
    """LanguageModel.Load of the golden checkpoint directory (written by
    tests/golden/make_checkpoint_fixture.py in the reference's format), then
    Forward against the oracle on the stored arrays; Save -> Load keeps Forward
    within the reference's own 1e-5 (MultiTypeTransformerTests.cs:858-874), here
    exactly, and the device engine built from the loaded model agrees."""
    import os
    gold = os.path.join(os.path.dirname(__file__), "golden")
    e = np.load(os.path.join(gold, "checkpoint_tiny_expected.npz"))
    cfg = {"vocab": 5, "dim": 4, "heads": 2, "layers": 2, "ff": 6, "max_seq": 8, "activation": 3}
    w = {"token_embedding": e["token_embedding"], "out_proj": e["out_proj"], "out_bias": e["out_bias"],
         "layers": [{k[3:]: e[k] for k in e.files if k.startswith(f"l{i}_")} for i in range(2)]}
    lm = H.LanguageModel.Load(os.path.join(gold, "checkpoint_tiny"), mgr)
    ids = np.array([1, 4, 0, 3, 2, 2, 1], np.int32)
    got = lm.Forward(ids)
    parity(got, O.LanguageModel(cfg, w).forward(ids), "loaded checkpoint Forward vs oracle")
    lm.Save(str(tmp_path))
    again = H.LanguageModel.Load(str(tmp_path), mgr).Forward(ids)
    assert np.array_equal(got, again), "Save -> Load changed Forward"
    dev = H.DeviceLanguageModel(lm, 2)
    parity(dev.Forward(np.stack([ids, ids[::-1].copy()])),
           np.vstack([got, lm.Forward(ids[::-1].copy())]), "device engine from the loaded model")


def test_device_language_model_c1_batch():
    """Config 1: batch 4 of 64 uniform token ids, full forward, then greedy
    generation of 20 tokens from 32-token prompts, per sequence against the
    oracle's LanguageModel (which feeds the prompt token by token)."""
    Hm = host.module()
    cfg = {"vocab": 200, "dim": 64, "heads": 4, "layers": 2, "ff": 128, "max_seq": 64}
    w = synth.lm_weights(cfg, 7)
    lm, _ = host.language_model(cfg, w)
    dev = Hm.DeviceLanguageModel(lm, 4)
    ids = synth.token_ids(11, 4 * 64, 200).reshape(4, 64)
    logits = dev.Forward(ids)
    ref = O.LanguageModel(cfg, w)
    for b in range(4):
        parity(logits[b * 64:(b + 1) * 64], ref.forward(ids[b]), f"c1 seq {b}")
    gen = dev.GenerateGreedy(ids[:, :32], 20)
    assert gen.shape == (4, 52)
    for b in range(4):
        assert np.array_equal(gen[b], ref.generate_greedy(ids[b, :32], 20)), f"c1 seq {b} tokens"
    # the length cap: a 60-token prompt yields only 4 new tokens (MaxSequenceLength 64)
    cap = dev.GenerateGreedy(ids[:, :60], 20)
    assert cap.shape == (4, 64)
    for b in range(2):
        assert np.array_equal(cap[b], ref.generate_greedy(ids[b, :60], 20))
    full = dev.GenerateGreedy(ids, 5)
    assert np.array_equal(full, ids)


def test_generate_graph_replays_match_eager():
    """GenerateGreedy's recorded graph (one per batch x prompt length x new
    tokens) against the same model launching every kernel from the host:
    replays with new prompt ids of the recorded shape, a second recorded
    shape beside the first, and eager work and synchronisations between the
    replays, every result compared."""
    Hm = host.module()
    cfg = {"vocab": 200, "dim": 64, "heads": 4, "layers": 2, "ff": 128, "max_seq": 64}
    lm, _ = host.language_model(cfg, synth.lm_weights(cfg, 8))
    dev, eager = Hm.DeviceLanguageModel(lm, 4), Hm.DeviceLanguageModel(lm, 4)
    eager.use_graphs = False
    assert dev.use_graphs
    for rep in range(4):
        ids = synth.token_ids(50 + rep, 4 * 64, 200).reshape(4, 64)
        for plen, n in ((32, 20), (40, 9)):
            got = dev.GenerateGreedy(ids[:, :plen], n)
            want = eager.GenerateGreedy(ids[:, :plen], n)
            assert np.array_equal(got, want), f"replay {rep}, prompt {plen}, {n} tokens"
        # eager work on the same model between replays
        dev.use_graphs = False
        assert np.array_equal(dev.GenerateGreedy(ids[:2, :10], 3), eager.GenerateGreedy(ids[:2, :10], 3))
        dev.Forward(ids)
        dev.use_graphs = True


@pytest.mark.parametrize("name", ["c1", "deep_ffn", "odd_width", "widest"])
def test_generate_fused_decode_matches_per_kernel_path(name):
    """The fused decode launch (every step after the prefill in one kernel)
    against the per-kernel decode steps of the same model: identical greedy
    tokens for several prompt lengths, up to the MaxSequenceLength cap, and
    the same KV caches' effect on later tokens."""
    Hm = host.module()
    if name == "c1":
        cfg = {"vocab": 200, "dim": 64, "heads": 4, "layers": 2, "ff": 128, "max_seq": 64}
    elif name == "deep_ffn":
        cfg = {"vocab": 97, "dim": 32, "heads": 2, "layers": 3, "ff": 48, "max_seq": 40}
    elif name == "odd_width":  # 256 / D leaves threads without a key group
        cfg = {"vocab": 301, "dim": 96, "heads": 3, "layers": 1, "ff": 200, "max_seq": 40}
    else:  # the fused path's largest model width and FFN width
        cfg = {"vocab": 500, "dim": 256, "heads": 4, "layers": 2, "ff": 1024, "max_seq": 64}
    lm, _ = host.language_model(cfg, synth.lm_weights(cfg, 12, biased=True))
    fused, plain = Hm.DeviceLanguageModel(lm, 4), Hm.DeviceLanguageModel(lm, 4)
    assert fused.fused_decode_available
    plain.use_fused_decode = False
    S = cfg["max_seq"]
    ids = synth.token_ids(13, 4 * S, cfg["vocab"]).reshape(4, S)
    for plen, n in ((1, 10), (5, 20), (S // 2, 30), (S - 3, 20)):
        got = fused.GenerateGreedy(ids[:, :plen], n)
        want = plain.GenerateGreedy(ids[:, :plen], n)
        assert got.shape == want.shape == (4, min(S, plen + n))
        assert np.array_equal(got, want), f"prompt {plen}, {n} tokens"


def _oracle_continuous(cfg, w, x):
    """LanguageModel.Forward(float[,]) from oracle functions: input projection,
    post-LN blocks, output projection."""
    H = cfg["heads"]
    h = O.batch_dot_add_bias(w["input_proj"], x, w["input_bias"])
    for L in w["layers"]:
        q, k, v = O.project_qkv(h, L["wq"], L["bq"], L["wk"], L["bk"], L["wv"], L["bv"])
        a = O.sdpa(O.rope(q, H), O.rope(k, H), v, H, causal=True)
        n1 = O.residual_layernorm(h, O.project_output_batch(a, L["wo"], L["bo"]), L["ln1_g"], L["ln1_b"])
        f = O.batch_dot_add_bias(L["ffn_w2"], O.activation(O.batch_dot_add_bias(L["ffn_w1"], n1, L["ffn_b1"]), 3),
                                 L["ffn_b2"])
        h = O.residual_layernorm(n1, f, L["ln2_g"], L["ln2_b"])
    return O.project_output_batch(h, w["out_proj"], w["out_bias"])


def test_time_series_transformer_c5_sampled():
    """Config 5 (F 5 -> D 256, 8 x 32, 6 layers, FF 1024, out 1; B 256 x 512,
    random-walk features): the whole batch on the device engine, three windows
    against the oracle composition, and the drop-in LanguageModel on one."""
    Hm = host.module()
    cfg = {"dim": 256, "heads": 8, "layers": 6, "ff": 1024, "max_seq": 512, "discrete": False,
           "input_dim": 5, "output_dim": 1}
    w = synth.continuous_lm_weights(cfg, 21)
    lm, _ = host.language_model(cfg, w)
    B, L = 256, 512
    x = synth.random_walk_windows(31, B, L, 5)
    dev = Hm.DeviceLanguageModel(lm, B)
    out = dev.ForwardContinuous(x.reshape(B * L, 5), B, L)
    assert out.shape == (B * L, 1) and np.all(np.isfinite(out))
    for b in (0, 100, 255):
        want = _oracle_continuous(cfg, w, x[b])
        parity(out[b * L:(b + 1) * L], want, f"c5 window {b}")
    parity(lm.ForwardContinuous(x[100]), _oracle_continuous(cfg, w, x[100]), "c5 drop-in LanguageModel")
