"""The reference's TransformerTrainer call sequence on HipAccelerationManager.

host/transformer_trainer.cpp restates TransformerTrainer.TrainBatchDiscrete
(TransformerTrainer.cs:217-327) call for call on the manager: the forward
with cache (:540-622, :723-848, :1123-1141), the backward (:874-987,
:989-1120), ScaleGradients / ComputeGradientNorm / ClipGradients /
UpdateParameters (:1269-1394).  One step must equal oracle.train_batch (the
finite-difference-pinned restatement) and the device-resident DeviceTrainer
on identical weights.  The manager methods it adds (the elementwise
training methods, the segmented attention and RoPE that the reference runs
inline, the FFN's ComputeInputGradientBatch) are checked one by one first.

Bar: |got - want| <= 1e-4 + 1e-3 |want| per element; gradient sums over
many rows also against float64 (conftest.assert_parity_with_exact).
"""
from __future__ import annotations

import numpy as np
import pytest

from cdml import host, synth
from conftest import assert_parity, assert_parity_with_exact
from oracle import oracle as O

pytestmark = pytest.mark.gpu
F64 = np.float64
C1 = {"vocab": 200, "dim": 64, "heads": 4, "layers": 2, "ff": 128, "max_seq": 64}


def parity(a, e, what=""):
    assert_parity(a, e, 1e-4, 1e-3, what)


@pytest.fixture(scope="module")
def mgr():
    m = host.module().HipAccelerationManager(0)
    yield m
    m.Dispose()


def test_elementwise_training_methods(mgr):
    """ZeroMatrix/Vector, MatrixAddInPlace, VectorAccumulate, Matrix/Vector
    ScaleInPlace, Matrix/VectorUpdate (AccelerationCPU.cs:507-568,
    2514-2597) are exact in fp32; the squared norms meet the bar against
    float64."""
    a, b = synth.normal(1, (300, 257)), synth.normal(2, (300, 257))
    t = a.copy()
    mgr.MatrixAddInPlace(t, b)
    assert np.array_equal(t, a + b)
    mgr.MatrixScaleInPlace(t, 0.37)
    assert np.array_equal(t, (a + b) * np.float32(0.37))
    w = a.copy()
    mgr.MatrixUpdate(w, b, 0.01)
    assert np.array_equal(w, a - np.float32(0.01) * b)
    # the update of an array the manager holds as a resident weight
    x = synth.normal(3, (8, 257))
    bias = np.zeros(300, np.float32)
    y0 = mgr.ProjectOutputBatch(x, w, bias, 8, 300)
    mgr.MatrixUpdate(w, b, 0.5)
    parity(mgr.ProjectOutputBatch(x, w, bias, 8, 300), O.project_output_batch(x, w, bias), "after MatrixUpdate")
    assert not np.array_equal(y0, mgr.ProjectOutputBatch(x, w, bias, 8, 300))
    v, u = synth.normal(4, (1000,)), synth.normal(5, (1000,))
    tv = v.copy()
    mgr.VectorAccumulate(tv, u)
    assert np.array_equal(tv, v + u)
    mgr.VectorScaleInPlace(tv, -2.0)
    assert np.array_equal(tv, (v + u) * np.float32(-2.0))
    wv = v.copy()
    mgr.VectorUpdate(wv, u, 0.1)
    assert np.array_equal(wv, v - np.float32(0.1) * u)
    big = synth.normal(6, (2048, 1024))
    assert mgr.MatrixSquaredNorm(big) == pytest.approx(float((big.astype(F64) ** 2).sum()), rel=1e-5)
    assert mgr.VectorSquaredNorm(v) == pytest.approx(float((v.astype(F64) ** 2).sum()), rel=1e-5)
    assert mgr.MatrixSquaredNorm(np.zeros((0, 5), np.float32)) == 0.0
    mgr.ZeroMatrix(t)
    mgr.ZeroVector(tv)
    assert not t.any() and not tv.any()
    # a zeroed array the manager held: the next read sees the zeros
    assert mgr.MatrixSquaredNorm(t) == 0.0


@pytest.mark.parametrize("seg_len,segs,dim,heads,causal", [(33, 4, 64, 4, True), (128, 3, 128, 2, True),
                                                         (17, 8, 64, 4, True), (40, 2, 96, 3, False)])
def test_segmented_attention_capabilities(mgr, seg_len, segs, dim, heads, causal):
    """The segmented trainer's inline attention forward (TransformerTrainer.cs:
    747-796), its backward (:989-1120) and ApplySegmentedRotaryInPlace
    (:811-848) against the oracle's single-sequence functions per segment."""
    rows = seg_len * segs
    q, k, v, d = (synth.normal(10 + i, (rows, dim)) for i in range(4))
    qr, kr = q.copy(), k.copy()
    mgr.ApplySegmentedRotaryInPlace(qr, kr, heads, seg_len, False)
    for s in range(segs):
        sl = slice(s * seg_len, (s + 1) * seg_len)
        parity(qr[sl], O.rope(q[sl], heads), f"segmented RoPE Q segment {s}")
        parity(kr[sl], O.rope(k[sl], heads), f"segmented RoPE K segment {s}")
    back = qr.copy(), kr.copy()
    mgr.ApplySegmentedRotaryInPlace(back[0], back[1], heads, seg_len, True)
    parity(back[0], q, "segmented RoPE round trip")
    out = mgr.SegmentedAttentionForward(qr, kr, v, heads, seg_len, segs, causal)
    scale = float(np.float32(1) / np.sqrt(np.float32(dim // heads)))
    dq, dk, dv = mgr.SegmentedMultiHeadAttentionBackward(qr, kr, v, d, heads, scale, seg_len, segs, causal)
    for s in range(segs):
        sl = slice(s * seg_len, (s + 1) * seg_len)
        parity(out[sl], O.sdpa(qr[sl], kr[sl], v[sl], heads, causal=causal), f"segmented attention segment {s}")
        want = O.mha_backward(qr[sl], kr[sl], v[sl], d[sl], heads, scale, use_decoder_mask=causal)
        for got, w, n in zip((dq, dk, dv), want, "QKV"):
            parity(got[sl], w, f"segmented backward d{n} segment {s}")
    with pytest.raises(host.module().ArgumentException, match="segmented"):
        mgr.SegmentedAttentionForward(qr, kr, v, heads, seg_len + 1, segs, causal)


@pytest.mark.parametrize("rows,d,ff,act", [(64, 64, 128, 3), (300, 256, 1024, 3), (77, 96, 200, 5),
                                           (40, 32, 64, 1)])
def test_ffn_input_gradient_batch(mgr, rows, d, ff, act):
    """NeuralNetwork.ComputeInputGradientBatch with gradient storage
    (NeuralNetwork.cs:773-985) for the transformer FFN [d, ff, d] with
    activations [act, None], accumulating into nonzero gradient arrays."""
    x, dout = synth.normal(20, (rows, d)), synth.normal(21, (rows, d))
    w = [synth.xavier_uniform(22, ff, d), synth.xavier_uniform(23, d, ff)]
    b = [synth.normal(24, (ff,)) * np.float32(0.1), synth.normal(25, (d,)) * np.float32(0.1)]
    wg = [synth.normal(26, (ff, d)), synth.normal(27, (d, ff))]
    bg = [synth.normal(28, (ff,)), synth.normal(29, (d,))]
    wg0, bg0 = [a.astype(F64) for a in wg], [a.astype(F64) for a in bg]
    wg_o, bg_o = [a.copy() for a in wg], [a.copy() for a in bg]
    want = O.ffn_input_gradient(x, dout, w, b, [act, 0], wg_o, bg_o)
    got = mgr.FFNInputGradientBatch(x, dout, w, b, [act, 0], wg, bg)
    X, D = x.astype(F64), dout.astype(F64)
    Z = X @ w[0].T.astype(F64) + b[0]
    sig = 1 / (1 + np.exp(-Z))
    deriv = {3: (Z >= 0).astype(F64), 1: sig * (1 - sig), 5: sig + Z * sig * (1 - sig)}[act]
    Hh = {3: np.maximum(Z, 0), 1: sig, 5: Z * sig}[act]
    DH = (D @ w[1].astype(F64)) * deriv
    assert_parity_with_exact(got, want, DH @ w[0].astype(F64), what="dInput")
    assert_parity_with_exact(wg[1], wg_o[1], wg0[1] + D.T @ Hh, what="W2 grad")
    assert_parity_with_exact(bg[1], bg_o[1], bg0[1] + D.sum(0), what="b2 grad")
    assert_parity_with_exact(wg[0], wg_o[0], wg0[0] + DH.T @ X, what="W1 grad")
    assert_parity_with_exact(bg[0], bg_o[0], bg0[0] + DH.sum(0), what="b1 grad")


def _named(w):
    """lm_weights / oracle dict -> flat names (DeviceTrainer's)."""
    out = {"token_embedding": w["token_embedding"], "out_proj": w["out_proj"], "out_bias": w["out_bias"]}
    for i, L in enumerate(w["layers"]):
        for k, v in L.items():
            if k in ("ffn_weights", "ffn_biases", "ffn_activations"):
                continue
            out[f"layers.{i}.{k}"] = v
    return out


def _replay(cfg, w, use_clip=True):
    H = host.module()
    lm, m = host.language_model(cfg, w)
    tc = H.TrainingConfig()
    tc.UseGradientClipping = use_clip
    return H.TransformerTrainer(lm, tc), lm, m


@pytest.mark.parametrize("batch,seq,use_clip", [(4, 33, True), (1, 64, False), (8, 17, True)])
def test_trainer_replay_step_matches_oracle_and_device_trainer(batch, seq, use_clip):
    """One TrainBatchDiscrete step of the config-1 text model through the
    reference's call sequence on the manager (segmented attention for
    batch > 1, the single-sequence path for batch 1): loss, norm, every
    gradient and every updated weight against oracle.train_batch, and the
    weights against DeviceTrainer's on the same weights."""
    H = host.module()
    w = synth.lm_weights(C1, 12, biased=True)
    seqs = list(synth.token_ids(40 + batch, batch * seq, C1["vocab"]).reshape(batch, seq))
    t, lm, m = _replay(C1, w, use_clip)
    print(f"[replay] batch {batch} x {seq}", flush=True)
    loss = t.TrainBatch(seqs, 0.01)
    want_loss, want_g, want_w = O.train_batch(C1, w, seqs, 0.01, use_clipping=use_clip)
    assert abs(loss - want_loss) <= 1e-5 + 1e-5 * abs(want_loss)
    assert t.last_norm == pytest.approx(want_g["norm"], rel=1e-4)
    got_g, want_gn = t.gradients(), _named(want_g)
    assert set(got_g) == set(want_gn), set(got_g) ^ set(want_gn)
    for k, v in got_g.items():
        parity(v, np.asarray(want_gn[k]), f"replay gradient {k}")
    got_w = _named(lm.weights())
    for k, v in _named(want_w).items():
        parity(got_w[k], v, f"replay weight {k}")
    # the device-resident trainer on the same weights and batch
    lm2, _ = host.language_model(C1, w)
    tc = H.TrainingConfig()
    tc.UseGradientClipping = use_clip
    dt = H.DeviceTrainer(lm2, tc, batch, seq - 1)
    dt.TrainBatch(seqs, 0.01)
    dev_w = dt.weights()
    for k, v in dev_w.items():
        parity(np.asarray(got_w[k]).reshape(-1), v, f"replay vs DeviceTrainer {k}")
    # the single-sequence path's backward started from the forward's statistics
    if batch == 1:
        assert m.transfer_stats()["backward_from_saved"] >= C1["layers"]


def test_trainer_replay_mixed_batch_and_steps():
    """Two length buckets, a single-sequence bucket and skipped sequences in
    one batch, then two more steps: the weights track the oracle's."""
    w = synth.lm_weights(C1, 13, biased=True)
    rng = np.random.default_rng(5)
    batch = [rng.integers(0, 200, 20).astype(np.int32) for _ in range(3)]
    batch += [rng.integers(0, 200, 12).astype(np.int32) for _ in range(2)]
    batch += [rng.integers(0, 200, 30).astype(np.int32), np.array([7], np.int32),
              np.array([1, 200, 3], np.int32)]
    t, lm, m = _replay(C1, w)
    loss = t.TrainBatch(batch, 0.02)
    want_loss, _, ww = O.train_batch(C1, w, batch, 0.02)
    assert abs(loss - want_loss) <= 1e-5 + 1e-5 * abs(want_loss)
    for step in range(2):
        seqs = list(synth.token_ids(60 + step, 4 * 25, 200).reshape(4, 25))
        t.TrainBatch(seqs, 0.02)
        _, _, ww = O.train_batch(C1, ww, seqs, 0.02)
    got = _named(lm.weights())
    for k, v in _named(ww).items():
        parity(got[k], v, f"after 3 steps {k}")


# ---- continuous-input models (TrainContinuous / TrainBatchContinuous) and
# validation (Validate / ValidateContinuous) --------------------------------

C5R = {"dim": 64, "heads": 2, "layers": 2, "ff": 128, "max_seq": 64, "discrete": False, "input_dim": 5,
       "output_dim": 3}


def _named_any(w):
    """Weight / gradient dict (oracle or LanguageModel.weights layout) ->
    flat names, for token and continuous models alike."""
    heads = ("token_embedding",) if "token_embedding" in w and "input_proj" not in w else ("input_proj", "input_bias")
    out = {k: w[k] for k in heads + ("out_proj", "out_bias")}
    for i, L in enumerate(w["layers"]):
        for k, v in L.items():
            if k in ("ffn_weights", "ffn_biases", "ffn_activations"):
                continue
            out[f"layers.{i}.{k}"] = v
    return out


def _windows(rng, kind, lens, features=5, outputs=3):
    wins = [rng.uniform(0, 1, (n, features)).astype(np.float32) for n in lens]
    if kind == "regression":
        tg = [rng.standard_normal((n, outputs)).astype(np.float32) for n in lens]
    else:
        tg = [rng.integers(0, outputs, n).astype(np.int32) for n in lens]
    return wins, tg


def _target_kw(kind, tg):
    return ({"regressionTargets": tg}, {"reg_targets": tg}) if kind == "regression" else \
        ({"classTargets": tg}, {"class_targets": tg})


def _splitmix_orders(n, seed, epochs):
    """The epoch orders of Train / TrainContinuous: a Fisher-Yates shuffle per
    epoch (from the last element, j in [0, i]) driven by SplitMix64 from
    `seed`."""
    m = (1 << 64) - 1
    state = seed
    orders = []
    for _ in range(epochs):
        order = list(range(n))
        for i in range(n, 1, -1):
            state = (state + 0x9E3779B97F4A7C15) & m
            z = state
            z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
            z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
            z ^= z >> 31
            j = z % i
            order[i - 1], order[j] = order[j], order[i - 1]
        orders.append(order)
    return orders


@pytest.mark.parametrize("kind", ["regression", "classification"])
def test_trainer_replay_continuous_step_matches_oracle_and_device_trainer(kind):
    """One TrainBatchContinuous step (TransformerTrainer.cs:329-512) of a
    config-5-shaped time-series model (F 5 -> D 64, head dim 32, 2 layers,
    OutputDim 3) through the reference's call sequence on the manager: a
    bucket of three 40-step windows (segmented attention, flattened targets,
    dOutput scaled by 3), a lone 25-step window (the single-sequence path with
    target offset 1), and skipped windows (1 step, a NaN feature, no
    targets).  Loss, norm, every gradient and every updated weight against
    oracle.train_batch_continuous, then the weights against DeviceTrainer's
    on the same weights and batch."""
    H = host.module()
    cfg = dict(C5R, data_type=1 if kind == "regression" else 2)
    w = synth.continuous_lm_weights(cfg, 17)
    rng = np.random.default_rng(31)
    wins, tg = _windows(rng, kind, [41, 26, 41, 41, 1, 41, 41])
    wins[5][7, 2] = np.nan
    tg[6] = None
    kw, okw = _target_kw(kind, tg)
    t, lm, m = _replay(cfg, w)
    print(f"[replay continuous] {kind}", flush=True)
    loss = t.TrainBatchContinuous(wins, learningRate=0.01, **kw)
    want_loss, want_g, want_w = O.train_batch_continuous(cfg, w, wins, 0.01, **okw)
    assert abs(loss - want_loss) <= 1e-5 + 1e-5 * abs(want_loss)
    assert t.last_norm == pytest.approx(want_g["norm"], rel=1e-4)
    got_g, want_gn = t.gradients(), _named_any(want_g)
    assert set(got_g) == set(want_gn), set(got_g) ^ set(want_gn)
    assert "input_proj" in got_g and "token_embedding" not in got_g
    for k, v in got_g.items():
        parity(v, np.asarray(want_gn[k]), f"continuous {kind} gradient {k}")
    got_w = _named_any(lm.weights())
    for k, v in _named_any(want_w).items():
        parity(got_w[k], v, f"continuous {kind} weight {k}")
    lm2, _ = host.language_model(cfg, w)
    dt = H.DeviceTrainer(lm2, H.TrainingConfig(), 4, 40)
    dt.TrainBatchContinuous(wins, learningRate=0.01, **kw)
    for k, v in dt.weights().items():
        parity(np.asarray(got_w[k]).reshape(-1), v, f"continuous {kind} replay vs DeviceTrainer {k}")
    # a batch in which no window can train: loss 0 and no update
    before = _named_any(lm.weights())
    assert t.TrainBatchContinuous([wins[4], wins[5]], learningRate=0.01,
                                  **_target_kw(kind, [tg[4], tg[5]])[0]) == 0.0
    after = _named_any(lm.weights())
    assert all(np.array_equal(before[k], after[k]) for k in before)


def test_backprop_input_projection_against_float64():
    """BackpropInputProjection (AccelerationCPU.cs:2280-2330): a row slice of
    a wider input (the reference reads inputFeatureDim of its columns),
    accumulation into nonzero gradients, and the argument rules."""
    mgr = host.module().HipAccelerationManager(0)
    E, F, cols, rows, start, n = 96, 5, 7, 300, 40, 211
    dx, x = synth.normal(70, (n, E)), synth.normal(71, (rows, cols))
    wg, bg = synth.normal(72, (E, F)), synth.normal(73, (E,))
    wg0, bg0 = wg.copy(), bg.copy()
    mgr.BackpropInputProjection(dx, x, start, wg, bg, n, E, F)
    want_w = wg0.astype(F64) + dx.astype(F64).T @ x[start:start + n, :F].astype(F64)
    want_b = bg0.astype(F64) + dx.astype(F64).sum(0)
    wo, bo = O.backprop_input_projection(dx, np.ascontiguousarray(x[:, :F]), wg0, bg0, row_start=start)
    assert_parity_with_exact(wg, wo, want_w, what="input projection weight gradient")
    assert_parity_with_exact(bg, bo, want_b, what="input projection bias gradient")
    Hm = host.module()
    with pytest.raises(Hm.ArgumentOutOfRangeException):
        mgr.BackpropInputProjection(dx, x, rows - n + 1, wg, bg, n, E, F)
    with pytest.raises(Hm.ArgumentException):
        mgr.BackpropInputProjection(dx, x, 0, wg, bg, n, E, cols + 1)
    mgr.Dispose()


def _oracle_continuous_forward(cfg, w, x):
    """LanguageModel.Forward(float[,]) / ForwardContinuousSlice from oracle
    functions: input projection, post-LN blocks, output projection."""
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


def test_trainer_validate_matches_oracle():
    """Validate (TransformerTrainer.cs:1142-1182): the per-token mean
    cross-entropy of ForwardTokenSlice(seq, 0, len - 1) against seq[1:],
    weighted by each sequence's predicted rows, skipping short sequences and
    sequences with out-of-vocabulary ids; the oracle's LanguageModel forward
    and cross-entropy give the expected value."""
    w = synth.lm_weights(C1, 14, biased=True)
    rng = np.random.default_rng(8)
    seqs = [rng.integers(0, 200, n).astype(np.int32) for n in (33, 9, 64, 2)]
    seqs += [np.array([5], np.int32), np.array([1, 250, 3], np.int32)]
    t, lm, m = _replay(C1, w)
    got = t.Validate(seqs)
    ref = O.LanguageModel(C1, w)
    total, tokens = np.float32(0), 0
    for s in seqs:
        if s.size < 2 or s.max() >= 200:
            continue
        n = s.size - 1
        loss, _ = O.cross_entropy(ref.forward(s[:n]), s, n, target_start=1)
        total = np.float32(total + np.float32(loss) * np.float32(n))
        tokens += n
    want = float(total / np.float32(tokens))
    assert abs(got - want) <= 1e-5 + 1e-5 * abs(want), (got, want)
    assert t.Validate([np.array([3], np.int32)]) == 0.0
    # a 66-token sequence predicts 65 rows: past MaxSequenceLength 64, the
    # slice forward throws (ValidateTokenSlice, LanguageModel.cs:602-619)
    with pytest.raises(host.module().ArgumentException, match="MaxSequenceLength"):
        t.Validate([rng.integers(0, 200, 66).astype(np.int32)])


@pytest.mark.parametrize("kind", ["regression", "classification"])
def test_trainer_validate_continuous_matches_oracle(kind):
    """ValidateContinuous (TransformerTrainer.cs:1183-1267): MSE or
    cross-entropy of ForwardContinuousSlice(x, 0, T - 1) against targets from
    offset 1, weighted by predicted rows; windows without targets or shorter
    than 2 steps are skipped."""
    cfg = dict(C5R, data_type=1 if kind == "regression" else 2)
    w = synth.continuous_lm_weights(cfg, 19)
    rng = np.random.default_rng(12)
    wins, tg = _windows(rng, kind, [40, 17, 1, 64, 30])
    tg[4] = None
    kw, _ = _target_kw(kind, tg)
    t, lm, m = _replay(cfg, w)
    got = t.ValidateContinuous(wins, **kw)
    total, items = np.float32(0), 0
    for x, y in zip(wins, tg):
        if x.shape[0] < 2 or y is None:
            continue
        n = x.shape[0] - 1
        out = _oracle_continuous_forward(cfg, w, x[:n])
        if kind == "regression":
            loss, _ = O.mse_loss(out, y, n, target_start=1)
        else:
            loss, _ = O.cross_entropy(out, y, n, target_start=1)
        total = np.float32(total + np.float32(loss) * np.float32(n))
        items += n
    want = float(total / np.float32(items))
    assert abs(got - want) <= 1e-5 + 1e-5 * abs(want), (got, want)
    # no targets at all: nothing to score
    assert t.ValidateContinuous(wins) == 0.0


def test_trainer_train_validates_at_the_interval():
    """Train with validation sequences (TransformerTrainer.cs:43-128): after
    every ValidationInterval-th batch of an epoch the trainer runs Validate;
    replaying TrainBatch in the SplitMix64 epoch order with Validate at the
    same points gives the same losses and weights."""
    H = host.module()
    w = synth.lm_weights(C1, 15, biased=True)
    rng = np.random.default_rng(9)
    data = [rng.integers(0, 200, n).astype(np.int32) for n in (17, 17, 9, 17, 12)]
    val = [rng.integers(0, 200, n).astype(np.int32) for n in (20, 11)]
    trainers = []
    for _ in range(2):
        lm, _ = host.language_model(C1, w)
        tc = H.TrainingConfig()
        tc.BatchSize, tc.Epochs, tc.ValidationInterval = 2, 2, 2
        trainers.append((H.TransformerTrainer(lm, tc), lm))
    (a, lma), (b, lmb) = trainers
    a.Train(data, seed=4, validationSequences=val)
    want_val = []
    for order in _splitmix_orders(len(data), 4, 2):
        nb = 0
        for i in range(0, len(order), 2):
            b.TrainBatch([data[j] for j in order[i:i + 2]], float(np.float32(0.0001)))
            nb += 1
            if nb % 2 == 0:
                want_val.append(b.Validate(val))
    assert len(a.validation_losses) == len(want_val) == 2
    assert np.array_equal(np.float32(a.validation_losses), np.float32(want_val))
    ga, gb = _named(lma.weights()), _named(lmb.weights())
    for k in ga:
        assert np.array_equal(ga[k], gb[k]), k


def test_trainer_train_continuous_equals_batch_steps():
    """TrainContinuous (TransformerTrainer.cs:130-207): the windows with at
    least 2 steps, shuffled per epoch, in batches of BatchSize with the
    learning-rate decay, give the same bits as TrainBatchContinuous called in
    that order; a window of the wrong width is rejected up front."""
    H = host.module()
    cfg = dict(C5R, data_type=1)
    w = synth.continuous_lm_weights(cfg, 23)
    rng = np.random.default_rng(10)
    wins, tg = _windows(rng, "regression", [21, 21, 13, 1, 21, 8, 13])
    valid = [i for i, x in enumerate(wins) if x.shape[0] >= 2]
    trainers = []
    for _ in range(2):
        lm, _ = host.language_model(cfg, w)
        tc = H.TrainingConfig()
        tc.BatchSize, tc.Epochs, tc.LearningRate = 3, 2, 0.02
        tc.UseLearningRateDecay, tc.LearningRateDecay = True, 0.8
        trainers.append((H.TransformerTrainer(lm, tc), lm))
    (a, lma), (b, lmb) = trainers
    got = a.TrainContinuous(wins, regressionTargets=tg, seed=11)
    lr = np.float32(0.02)
    for order in _splitmix_orders(len(valid), 11, 2):
        losses = []
        for i in range(0, len(order), 3):
            idx = [valid[j] for j in order[i:i + 3]]
            losses.append(b.TrainBatchContinuous([wins[j] for j in idx], regressionTargets=[tg[j] for j in idx],
                                                 learningRate=float(lr)))
        lr = np.float32(lr * np.float32(0.8))
    assert got == pytest.approx(float(np.float32(sum(np.float32(x) for x in losses) / np.float32(len(losses)))),
                                rel=1e-6)
    ga, gb = _named_any(lma.weights()), _named_any(lmb.weights())
    for k in ga:
        assert np.array_equal(ga[k], gb[k]), k
    bad = [np.zeros((5, 4), np.float32)]
    with pytest.raises(H.ArgumentException, match="feature dimension"):
        a.TrainContinuous(bad, regressionTargets=[np.zeros((5, 3), np.float32)])
    with pytest.raises(H.ArgumentException, match="regressionTargets"):
        a.TrainContinuous(wins)
