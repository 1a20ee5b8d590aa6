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
