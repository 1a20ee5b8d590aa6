"""GPU parity of the training-step kernels against the CPU oracle
(oracle/refcpu_train.c), through the C ABI.

Bar: |got - want| <= 1e-4 + 1e-3 |want| per element (gradients summed over
many rows also against float64, see conftest.assert_parity_with_exact);
the SGD update is bit-exact given the same gradient.
"""
from __future__ import annotations

import numpy as np
import pytest

import abi_ops as G
from cdml import synth
from conftest import assert_parity, assert_parity_with_exact
from oracle import oracle as O

pytestmark = pytest.mark.gpu
F64 = np.float64


def parity(a, e, what=""):
    assert_parity(a, e, 1e-4, 1e-3, what)


@pytest.mark.parametrize("rows,ind,out,act", [(64, 64, 128, 3), (300, 256, 1024, 3), (77, 130, 33, 1),
                                              (1024, 512, 2048, 5), (40, 32, 64, 2),
                                              (16384, 64, 1024, 3),   # 256x128 tiles, full wave blocks
                                              (16484, 64, 1000, 1),  # 256x128 tiles, ragged row and column tiles
                                              (5000, 64, 3, 1),      # few columns: 16 lanes per row
                                              (5000, 5, 256, 5)])    # short K
def test_linear_preact(rows, ind, out, act):
    """The FFN hidden layer with its cache: z = x W^T + b, y = act(z)."""
    x, w, b = synth.normal(1, (rows, ind)), synth.xavier_uniform(2, out, ind), synth.normal(3, (out,))
    z, y = G.linear_preact(x, w, b, act)
    zw = O.batch_dot_add_bias(w, x, b, mt=rows > 4096)
    parity(z, zw, "pre-activation")
    parity(y, O.activation(zw, act), "activation")
    assert np.array_equal(y, O.activation(z, act)) if act == 3 else True  # ReLU of the stored z, exactly


@pytest.mark.parametrize("rows,ind,out,act", [(600, 256, 512, 3), (16384, 64, 1024, 3), (77, 130, 33, 3),
                                              (600, 256, 512, 4), (40, 32, 64, 4)])
def test_ffn_backward_from_output(rows, ind, out, act):
    """The hidden layer without its pre-activation (z = NULL, then
    CDML_ACT_FROM_OUTPUT): y equals act(z) as numbers, ReLU's zero carries
    the sign of z < 0, and every gradient has the bits of the z form --
    including rows whose z is exactly 0, where the reference's ReLU
    derivative is 1 (NeuralNetwork.cs:885-944)."""
    x = synth.normal(4, (rows, ind))
    x[::7] = 0.0                                  # z = b on these rows ...
    b1 = synth.normal(6, (out,)) * np.float32(0.1)
    b1[::3] = 0.0                                 # ... and exactly 0 in every third column
    w1 = synth.xavier_uniform(5, out, ind)
    w2 = synth.xavier_uniform(7, ind, out)
    dout, resid = synth.normal(9, (rows, ind)), synth.normal(10, (rows, ind))
    wg = [synth.normal(11, (out, ind)), synth.normal(12, (ind, out))]
    bg = [synth.normal(13, (out,)), synth.normal(14, (ind,))]
    z, h = G.linear_preact(x, w1, b1, act)
    y = G.linear_preact_output_only(x, w1, b1, act)
    assert (z == 0).any() and (z < 0).any()
    assert np.array_equal(y, h)                   # as numbers (-0 == 0)
    if act == 3:
        assert np.array_equal(np.signbit(y), z < 0)
    else:
        assert np.array_equal(y.view(np.uint32), h.view(np.uint32))
    want = G.linear_backward_act(h, dout, w2, wg[1], bg[1], dz=z, act=act)
    got = G.linear_backward_act(y, dout, w2, wg[1], bg[1], dz=y, act=act | 0x100)
    for a, e, n in zip(got, want, ("dh", "W2 grad", "b2 grad")):
        assert np.array_equal(a.view(np.uint32), e.view(np.uint32)), n
    d1 = G.linear_backward_act(x, got[0], w1, wg[0], bg[0], add=resid)
    d0 = G.linear_backward_act(x, want[0], w1, wg[0], bg[0], add=resid)
    for a, e in zip(d1, d0):
        assert np.array_equal(a.view(np.uint32), e.view(np.uint32))


@pytest.mark.parametrize("rows,ind,out,act", [(64, 64, 128, 3), (600, 256, 512, 3), (77, 130, 33, 1),
                                              (2048, 128, 512, 5), (40, 32, 64, 4),
                                              (3000, 64, 3, 3)])  # 3-wide hidden layer: short-K input gradient
def test_ffn_backward_layers(rows, ind, out, act):
    """NeuralNetwork.ComputeInputGradientBatch of a [ind, out, ind] FFN as two
    cdml_linear_backward_act calls (hidden deltas through act'(z), the input
    gradient plus a residual gradient), against the oracle's FFN backward
    followed by MatrixAddInPlace."""
    x = synth.normal(4, (rows, ind))
    w1, b1 = synth.xavier_uniform(5, out, ind), synth.normal(6, (out,)) * np.float32(0.1)
    w2, b2 = synth.xavier_uniform(7, ind, out), synth.normal(8, (ind,)) * np.float32(0.1)
    dout, resid = synth.normal(9, (rows, ind)), synth.normal(10, (rows, ind))
    wg = [synth.normal(11, (out, ind)), synth.normal(12, (ind, out))]
    bg = [synth.normal(13, (out,)), synth.normal(14, (ind,))]
    wg_o, bg_o = [a.copy() for a in wg], [a.copy() for a in bg]
    want = O.ffn_input_gradient(x, dout, [w1, w2], [b1, b2], [act, 0], wg_o, bg_o) + resid
    z, h = G.linear_preact(x, w1, b1, act)
    dh, gw2, gb2 = G.linear_backward_act(h, dout, w2, wg[1], bg[1], dz=z, act=act)
    dx, gw1, gb1 = G.linear_backward_act(x, dh, w1, wg[0], bg[0], add=resid)
    # float64 of the same chain for the long reductions
    X, D = x.astype(F64), dout.astype(F64)
    Z = X @ w1.T.astype(F64) + b1
    deriv = {3: (Z >= 0).astype(F64), 1: (lambda s: s * (1 - s))(1 / (1 + np.exp(-Z))),
             5: (lambda s: s + Z * s * (1 - s))(1 / (1 + np.exp(-Z))), 4: np.where(Z <= 0, 0.1, 1.0)}[act]
    Hh = {3: np.maximum(Z, 0), 1: 1 / (1 + np.exp(-Z)), 5: Z / (1 + np.exp(-Z)), 4: np.where(Z > 0, Z, 0.01 * Z)}[act]
    DH = (D @ w2.astype(F64)) * deriv
    assert_parity_with_exact(gw2, wg_o[1], wg[1] + D.T @ Hh, what="W2 grad")
    assert_parity_with_exact(gb2, bg_o[1], bg[1] + D.sum(0), what="b2 grad")
    assert_parity_with_exact(gw1, wg_o[0], wg[0] + DH.T @ X, what="W1 grad")
    assert_parity_with_exact(gb1, bg_o[0], bg[0] + DH.sum(0), what="b1 grad")
    assert_parity_with_exact(dx, want, DH @ w1.astype(F64) + resid, what="dInput + residual")


@pytest.mark.parametrize("rows,f", [(5, 7), (64, 64), (300, 256), (1000, 1024), (33, 2048), (4, 1)])
def test_residual_layernorm_forward_cache(rows, f):
    a, b = synth.normal(15, (rows, f)), synth.normal(16, (rows, f))
    g, be = synth.positive_vector(f, 17), synth.normal(18, (f,))
    got = G.residual_layernorm_fwd(a, b, g, be)
    want = O.residual_layernorm_forward(a, b, g, be)
    for x, e, n in zip(got, want, ("out", "mean", "variance", "normalized", "residual")):
        parity(x, e, f"ResidualLayerNormForward {n}")
    assert np.array_equal(got[4], want[4])  # a + b exactly


@pytest.mark.parametrize("rows,f,with_norm", [(5, 7, True), (64, 64, False), (300, 256, False),
                                              (1000, 1024, False), (130, 2048, True), (200, 300, False),
                                              (77, 516, True), (70, 258, False),
                                              (20000, 256, False),  # 313 row blocks: sums in two passes
                                              (33000, 300, True),  # the same with ragged rows
                                              (1000, 130, True),  # 32-row blocks, scalar loads
                                              (33001, 200, False)])  # 32-row blocks, ragged, float4
def test_layernorm_backward(rows, f, with_norm):
    a, b = synth.normal(19, (rows, f)), synth.normal(20, (rows, f))
    g, be = synth.positive_vector(f, 21), synth.normal(22, (f,))
    _, mean, var, norm, res = O.residual_layernorm_forward(a, b, g, be)
    d1, d2 = synth.normal(23, (rows, f)), synth.normal(24, (rows, f))
    want = O.layernorm_backward(d1 + d2, norm, g, res, mean, var)
    got = G.layernorm_backward(d1, norm if with_norm else None, g, res, mean, var, dout2=d2)
    G64 = (d1 + d2).astype(F64)
    N64 = norm.astype(F64)
    assert_parity_with_exact(got[0], want[0], want[0], what="dInput")
    assert_parity_with_exact(got[1], want[1], (G64 * N64).sum(0), what="dGamma")
    assert_parity_with_exact(got[2], want[2], G64.sum(0), what="dBeta")
    acc = G.layernorm_backward(d1, None, g, res, mean, var, dout2=d2, dgamma0=np.ones(f, np.float32),
                               dbeta0=np.full(f, 2, np.float32))
    parity(acc[1], want[1] + 1, "dGamma accumulated")
    parity(acc[2], want[2] + 2, "dBeta accumulated")


@pytest.mark.parametrize("rows,v,eff,scale", [(6, 11, 4, 1.0), (64, 200, 64, 4.0), (300, 1000, 257, 1.0),
                                              (16, 50000, 16, 2.0), (3, 7, 0, 1.0)])
def test_cross_entropy(rows, v, eff, scale):
    logits = synth.normal(25, (rows, v)) * np.float32(3)
    t = (np.arange(rows) * 7919 % v).astype(np.int32)
    loss, dl = G.cross_entropy(logits, t, eff, grad_scale=scale)
    if eff == 0:
        assert loss == 0 and not dl.any()
        return
    want_loss, want_dl = O.cross_entropy(logits, t, eff)
    assert abs(loss - want_loss) <= 1e-5 + 1e-5 * abs(want_loss)
    parity(dl, want_dl * np.float32(scale), "dLogits")
    assert not dl[eff:].any()


def test_cross_entropy_bad_target_gives_nan_loss():
    logits = synth.normal(26, (4, 9))
    loss, _ = G.cross_entropy(logits, np.array([1, 2, 9, 0], np.int32), 4)
    assert np.isnan(loss)


@pytest.mark.parametrize("rows,vocab,dim", [(12, 5, 3), (256, 200, 64), (16384, 50000, 64), (300, 7, 1024)])
def test_embedding_grad(rows, vocab, dim):
    ids = (np.arange(rows) * 31 % vocab).astype(np.int32)
    if rows > 12:
        ids[::5] = 3  # a token repeated many times
    dx, dx2 = synth.normal(27, (rows, dim)), synth.normal(28, (rows, dim))
    eg = synth.normal(29, (vocab, dim))
    got = G.embedding_grad(eg, dx, ids, dx2)
    want = O.accumulate_token_embedding_grad(eg, dx + dx2, ids)
    assert np.array_equal(got, want)  # same rows, same order, same sums


def test_grad_norm_clip_and_update():
    """Global norm with the trainer's grouping, clipping and the SGD update;
    the update is bit-exact against w - lr * g' with g' the oracle's scaled
    gradients."""
    shapes = [(200, 64), (64,), (64, 64), (64, 64), (64, 64), (64, 64), (64,), (64,), (128, 64), (7,)]
    groups = [0, 1, 2, 2, 2, 2, 3, 3, 4, 5]
    ws = [synth.normal(30 + i, s) for i, s in enumerate(shapes)]
    gs = [synth.normal(50 + i, s) for i, s in enumerate(shapes)]
    prescale = float(np.float32(1) / np.float32(3))
    scaled = [g.copy() for g in gs]
    for g in scaled:
        O.scale_inplace(g, prescale)
    total = np.float32(0)
    i = 0
    while i < len(shapes):  # groups of consecutive equal ids
        j = i
        s = np.float32(0)
        while j < len(shapes) and groups[j] == groups[i]:
            s = np.float32(s + np.float32(O.squared_norm(scaled[j])))
            j += 1
        total = np.float32(total + s)
        i = j
    norm_want = float(np.sqrt(total, dtype=np.float32))
    for clip_on, thr in ((False, 1.0), (True, 1.0), (True, 1e6)):
        lr = 0.05
        norm, clip, finite, neww, after = G.norm_and_update(ws, gs, groups, lr, prescale, clip_on, thr)
        assert finite == 1.0
        assert norm == pytest.approx(norm_want, rel=1e-5)
        want_clip = thr / norm if (clip_on and norm > thr) else 1.0
        assert clip == pytest.approx(want_clip, rel=1e-6)
        for w, g, nw, ga in zip(ws, scaled, neww, after):
            gp = g.copy()
            if clip != 1.0:
                O.scale_inplace(gp, clip)
            assert np.array_equal(ga, gp)  # the gradient left as the in-place scaling leaves it
            wp = w.copy()
            O.sgd_update(wp, gp, lr)
            assert np.array_equal(nw, wp)
    # zero_grads clears every gradient; a non-finite norm skips the update
    bad = [g.copy() for g in gs]
    bad[3][1, 2] = np.inf
    _, _, finite, neww, after = G.norm_and_update(ws, bad, groups, 0.05, prescale, True, 1.0, zero_grads=True)
    assert finite == 0.0
    assert all(np.array_equal(a, b) for a, b in zip(neww, ws)) and not any(a.any() for a in after)


# ------------------------------------------------------------- the trainer
def _trainer(cfg, weights, batch_cap, seq_cap, clip=1.0, use_clip=True):
    from cdml import host
    H = host.module()
    lm, _ = host.language_model(cfg, weights)
    tc = H.TrainingConfig()
    tc.UseGradientClipping = use_clip
    tc.GradientClipThreshold = clip
    return H.DeviceTrainer(lm, tc, batch_cap, seq_cap), lm


def _oracle_named(d):
    """oracle train_batch dicts -> the trainer's flat names."""
    out = {"token_embedding": d["token_embedding"], "out_proj": d["out_proj"], "out_bias": d["out_bias"]}
    for i, L in enumerate(d["layers"]):
        for k, v in L.items():
            k2 = {"ffn_w1": "ffn_w1", "ffn_w2": "ffn_w2", "ffn_b1": "ffn_b1", "ffn_b2": "ffn_b2"}.get(k, k)
            out[f"layers.{i}.{k2}"] = v
    return out


def _compare(got: dict, want: dict, what: str):
    w = _oracle_named(want)
    assert set(got) == set(w), set(got) ^ set(w)
    for k, v in got.items():
        parity(v, np.asarray(w[k]).reshape(-1), f"{what} {k}")


C1 = {"vocab": 200, "dim": 64, "heads": 4, "layers": 2, "ff": 128, "max_seq": 64}


@pytest.mark.parametrize("batch,seq,use_clip", [(4, 33, True), (1, 64, False), (8, 17, True)])
def test_device_trainer_step_matches_oracle(batch, seq, use_clip):
    """One TrainBatchDiscrete step of the config-1 text model (segmented
    attention for batch > 1, the single-sequence path for batch 1): loss,
    every gradient after the 1/B and clipping scales, and every updated
    weight against the oracle."""
    w = synth.lm_weights(C1, 12, biased=True)
    seqs = synth.token_ids(40 + batch, batch * seq, C1["vocab"]).reshape(batch, seq)
    t, _ = _trainer(C1, w, batch, seq - 1, use_clip=use_clip)
    loss = t.TrainBatch(list(seqs), 0.01)
    want_loss, want_g, want_w = O.train_batch(C1, w, list(seqs), 0.01, use_clipping=use_clip)
    assert abs(loss - want_loss) <= 1e-5 + 1e-5 * abs(want_loss)
    assert t.last_norm == pytest.approx(want_g["norm"], rel=1e-4)
    _compare(t.gradients(), want_g, "gradient")
    _compare(t.weights(), want_w, "weight")


def test_device_trainer_mixed_batch_and_several_steps():
    """Buckets of two lengths, a single-sequence bucket and skipped sequences
    in one batch, then three more steps: weights track the oracle's."""
    w = synth.lm_weights(C1, 13, biased=True)
    rng = np.random.default_rng(5)
    batch = [rng.integers(0, 200, 20).astype(np.int32) for _ in range(3)]
    batch += [rng.integers(0, 200, 12).astype(np.int32) for _ in range(2)]
    batch += [rng.integers(0, 200, 30).astype(np.int32), np.array([7], np.int32),
              np.array([1, 200, 3], np.int32)]
    t, lm = _trainer(C1, w, 4, 32)
    loss = t.TrainBatch(batch, 0.02)
    want_loss, want_g, want_w = O.train_batch(C1, w, batch, 0.02)
    assert abs(loss - want_loss) <= 1e-5 + 1e-5 * abs(want_loss)
    _compare(t.gradients(), want_g, "mixed gradient")
    _compare(t.weights(), want_w, "mixed weight")
    ww = want_w
    for step in range(3):
        seqs = list(synth.token_ids(60 + step, 4 * 25, 200).reshape(4, 25))
        t.TrainBatch(seqs, 0.02)
        _, _, ww = O.train_batch(C1, ww, seqs, 0.02)
    _compare(t.weights(), ww, "after 4 steps")
    # CopyWeightsTo writes the trained weights back into the host model
    t.CopyWeightsTo(lm)
    got = lm.weights()
    parity(got["out_proj"], ww["out_proj"], "CopyWeightsTo out_proj")
    parity(got["layers"][1]["ffn_w1"], ww["layers"][1]["ffn_w1"], "CopyWeightsTo ffn_w1")


def test_device_trainer_loss_decreases():
    """Training on a fixed batch drives its loss down (the reference's own
    convergence tests, MultiTypeTransformerTests, check the same)."""
    w = synth.lm_weights(C1, 14)
    seqs = list(synth.token_ids(70, 8 * 33, 200).reshape(8, 33))
    t, _ = _trainer(C1, w, 8, 32)
    losses = [t.TrainBatch(seqs, 0.05) for _ in range(40)]
    assert all(b < a for a, b in zip(losses[:10], losses[1:11])), losses
    assert losses[-1] < 0.8 * losses[0], losses


# (1, 700, 64, 2) and (2, 1000, 256, 8): head dim 32 past 512 rows, where the
# stored-dS dQ takes flash_bwd_dq_ds_kernel<32, 64> instead of the short
# kernel; (1, 256, 128, 2) / (1, 257, 128, 2): head dim 64 at the short
# kernel's last length and one past it.
@pytest.mark.parametrize("batch,L,dim,heads", [(2, 300, 128, 2), (1, 257, 256, 2), (3, 130, 96, 3), (2, 64, 512, 4),
                                               (4, 63, 64, 4), (2, 100, 96, 2), (2, 200, 128, 2), (1, 512, 256, 8),
                                               (3, 33, 64, 2), (1, 700, 64, 2), (2, 1000, 256, 8),
                                               (1, 256, 128, 2), (1, 257, 128, 2)])
def test_sdpa_bwd_from_saved_statistics(batch, L, dim, heads):
    """The trainer's attention backward from the forward's saved output and
    row statistics (cdml_sdpa_fwd_lse + cdml_sdpa_bwd_saved) gives the same
    bits as cdml_sdpa_bwd, which recomputes them, and the forward's output is
    the same as cdml_sdpa_fwd's."""
    import ctypes as C
    from cdml import native as N
    rows = batch * L
    q, k, v, g = (synth.normal(80 + i, (rows, dim)) for i in range(4))
    scale = float(np.float32(1) / np.sqrt(np.float32(dim // heads)))
    bq, bk, bv, bg = (G.up(a) for a in (q, k, v, g))
    o1, o2 = N.DeviceBuffer(rows * dim * 4), N.DeviceBuffer(rows * dim * 4)
    lse = N.DeviceBuffer(batch * heads * L * 4)
    s = G.stream().handle
    lib = N.lib()
    N.check(lib.cdml_sdpa_fwd(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, o1.ptr, dim, batch, L, L, dim, heads, scale,
                              1, None, s))
    N.check(lib.cdml_sdpa_fwd_lse(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, o2.ptr, dim, lse.ptr, batch, L, L, dim,
                                  heads, scale, 1, None, s))
    assert np.array_equal(G.down(o1, (rows, dim)), G.down(o2, (rows, dim)))
    ws = C.c_size_t(0)
    N.check(lib.cdml_sdpa_bwd_workspace_size(batch, L, L, dim, heads, C.byref(ws)))
    bws = N.DeviceBuffer(ws.value)
    outs = [[N.DeviceBuffer(rows * dim * 4) for _ in range(3)] for _ in range(2)]
    N.check(lib.cdml_sdpa_bwd(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, bg.ptr, dim, outs[0][0].ptr, dim,
                              outs[0][1].ptr, dim, outs[0][2].ptr, dim, batch, L, L, dim, heads, scale, 1, None,
                              bws.ptr, ws.value, s))
    small = batch * heads * L * 4
    N.check(lib.cdml_sdpa_bwd_saved(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, o2.ptr, dim, lse.ptr, bg.ptr, dim,
                                    outs[1][0].ptr, dim, outs[1][1].ptr, dim, outs[1][2].ptr, dim, batch, L, L,
                                    dim, heads, scale, 1, None, bws.ptr, small, s))
    for a, b, n in zip(outs[0], outs[1], "QKV"):
        assert np.array_equal(G.down(a, (rows, dim)), G.down(b, (rows, dim))), f"d{n}"
    want = O.mha_backward(q[:L], k[:L], v[:L], g[:L], heads, scale, use_decoder_mask=True)
    for a, e, n in zip(outs[1], want, "QKV"):
        parity(G.down(a, (rows, dim))[:L], e, f"saved-statistics d{n} vs oracle")
    rc = lib.cdml_sdpa_bwd_saved(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, o2.ptr, dim, lse.ptr, bg.ptr, dim,
                                 outs[1][0].ptr, dim, outs[1][1].ptr, dim, outs[1][2].ptr, dim, batch, L, L, dim,
                                 heads, scale, 1, None, bws.ptr, small - 4, s)
    assert rc == -1
    # with room for the stored dS blocks (head dims 32 and 64): dK and dV are
    # the same bits, dQ is one product over the stored blocks
    big = C.c_size_t(0)
    N.check(lib.cdml_sdpa_bwd_saved_workspace_size(batch, L, L, dim, heads, 1, C.byref(big)))
    hd = dim // heads
    assert (big.value > small) == (hd in (32, 64))
    bbig = N.DeviceBuffer(big.value)
    out3 = [N.DeviceBuffer(rows * dim * 4) for _ in range(3)]
    N.check(lib.cdml_sdpa_bwd_saved(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, o2.ptr, dim, lse.ptr, bg.ptr, dim,
                                    out3[0].ptr, dim, out3[1].ptr, dim, out3[2].ptr, dim, batch, L, L,
                                    dim, heads, scale, 1, None, bbig.ptr, big.value, s))
    for a, b, n in zip(outs[1][1:], out3[1:], "KV"):
        assert np.array_equal(G.down(a, (rows, dim)), G.down(b, (rows, dim))), f"stored-dS d{n}"
    # the drop-in form with its own larger workspace takes the same path: the
    # recomputed forward gives the saved output's bits, so all three agree
    bigd = C.c_size_t(0)
    N.check(lib.cdml_sdpa_bwd_stored_ds_workspace_size(batch, L, L, dim, heads, 1, C.byref(bigd)))
    assert (bigd.value > ws.value) == (hd in (32, 64))
    bbigd = N.DeviceBuffer(bigd.value)
    out4 = [N.DeviceBuffer(rows * dim * 4) for _ in range(3)]
    N.check(lib.cdml_sdpa_bwd(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, bg.ptr, dim, out4[0].ptr, dim,
                              out4[1].ptr, dim, out4[2].ptr, dim, batch, L, L, dim, heads, scale, 1, None,
                              bbigd.ptr, bigd.value, s))
    for a, b, n in zip(out3, out4, "QKV"):
        assert np.array_equal(G.down(a, (rows, dim)), G.down(b, (rows, dim))), f"drop-in stored-dS d{n}"
    dq3 = G.down(out3[0], (rows, dim))
    for sq in range(batch):
        r = slice(sq * L, (sq + 1) * L)
        want = O.mha_backward(q[r], k[r], v[r], g[r], heads, scale, use_decoder_mask=True)
        parity(dq3[r], want[0], f"stored-dS dQ, sequence {sq}")


# head dim 32: the short stored-dS dQ kernel (300, 512 rows), the long one
# (700); head dim 64: short (256) and long (257); head dims 16 and 48: scalar
# loads and the recomputing dQ kernel; each with the minimum workspace
# (recomputing dQ) and with room for the stored dS blocks.
@pytest.mark.parametrize("batch,L,dim,heads", [(2, 300, 256, 8), (1, 512, 256, 8), (1, 700, 64, 2),
                                               (1, 256, 128, 2), (1, 257, 128, 2), (2, 100, 64, 4),
                                               (3, 130, 96, 2)])
@pytest.mark.parametrize("stored", [False, True])
def test_sdpa_bwd_saved_rope_equals_saved_then_table_rope(batch, L, dim, heads, stored):
    """cdml_sdpa_bwd_saved_rope rotates dQ and dK as its kernels store them:
    the same bits as cdml_sdpa_bwd_saved followed by cdml_rope_qk_table
    (inverse, each row at its index in its sequence), dV untouched; the
    rotation itself is pinned by the table RoPE's own tests."""
    import ctypes as C
    from cdml import native as N
    rows, hd = batch * L, dim // heads
    q, k, v, g = (synth.normal(90 + i, (rows, dim)) for i in range(4))
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    bq, bk, bv, bg = (G.up(a) for a in (q, k, v, g))
    o, lse = N.DeviceBuffer(rows * dim * 4), N.DeviceBuffer(batch * heads * L * 4)
    s = G.stream().handle
    lib = N.lib()
    N.check(lib.cdml_sdpa_fwd_lse(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, o.ptr, dim, lse.ptr, batch, L, L, dim,
                                  heads, scale, 1, None, s))
    ws = C.c_size_t(batch * heads * L * 4)
    if stored:
        N.check(lib.cdml_sdpa_bwd_saved_workspace_size(batch, L, L, dim, heads, 1, C.byref(ws)))
    bws = N.DeviceBuffer(ws.value)
    cs = N.DeviceBuffer(L * hd * 4)
    N.check(lib.cdml_rope_table(cs.ptr, L, hd, 10000.0, s))
    outs = [[N.DeviceBuffer(rows * dim * 4) for _ in range(3)] for _ in range(2)]
    N.check(lib.cdml_sdpa_bwd_saved(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, o.ptr, dim, lse.ptr, bg.ptr, dim,
                                    outs[0][0].ptr, dim, outs[0][1].ptr, dim, outs[0][2].ptr, dim, batch, L, L, dim,
                                    heads, scale, 1, None, bws.ptr, ws.value, s))
    N.check(lib.cdml_rope_qk_table(outs[0][0].ptr, outs[0][1].ptr, rows, dim, hd, heads, cs.ptr, L, 0, L, 1, s))
    N.check(lib.cdml_sdpa_bwd_saved_rope(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, o.ptr, dim, lse.ptr, bg.ptr, dim,
                                         outs[1][0].ptr, dim, outs[1][1].ptr, dim, outs[1][2].ptr, dim, batch, L,
                                         L, dim, heads, scale, 1, None, cs.ptr, L, bws.ptr, ws.value, s))
    for a, b, n in zip(outs[0], outs[1], "QKV"):
        assert np.array_equal(G.down(a, (rows, dim)).view(np.uint32), G.down(b, (rows, dim)).view(np.uint32)), \
            f"d{n}: fused inverse RoPE != saved + cdml_rope_qk_table"
    # a table one position short, and an odd head dim, are refused
    assert lib.cdml_sdpa_bwd_saved_rope(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, o.ptr, dim, lse.ptr, bg.ptr, dim,
                                        outs[1][0].ptr, dim, outs[1][1].ptr, dim, outs[1][2].ptr, dim, batch, L,
                                        L, dim, heads, scale, 1, None, cs.ptr, L - 1, bws.ptr, ws.value, s) == -1


def test_sdpa_bwd_stored_scores_c3_shape():
    """The c3 shape (4 x 4096, 16 heads of 64, causal) through
    cdml_sdpa_fwd_lse + cdml_sdpa_bwd_saved with the stored-dS workspace
    (2.1 GB of dS blocks); two (sequence, head) pairs against float64."""
    import ctypes as C
    from cdml import native as N
    from test_gpu_parity import _attention_bwd64
    B, L, D, H = 4, 4096, 1024, 16
    hd = D // H
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    q, k, v, g = (synth.normal(20 + i, (B * L, D)) for i in range(4))
    bq, bk, bv, bg = (G.up(a) for a in (q, k, v, g))
    o, lse = N.DeviceBuffer(B * L * D * 4), N.DeviceBuffer(B * H * L * 4)
    s = G.stream().handle
    lib = N.lib()
    N.check(lib.cdml_sdpa_fwd_lse(bq.ptr, D, bk.ptr, D, bv.ptr, D, o.ptr, D, lse.ptr, B, L, L, D, H, scale, 1,
                                  None, s))
    ws = C.c_size_t(0)
    N.check(lib.cdml_sdpa_bwd_saved_workspace_size(B, L, L, D, H, 1, C.byref(ws)))
    assert ws.value > 2 * L * L * B * H
    bws = N.DeviceBuffer(ws.value)
    outs = [N.DeviceBuffer(B * L * D * 4) for _ in range(3)]
    N.check(lib.cdml_sdpa_bwd_saved(bq.ptr, D, bk.ptr, D, bv.ptr, D, o.ptr, D, lse.ptr, bg.ptr, D, outs[0].ptr, D,
                                    outs[1].ptr, D, outs[2].ptr, D, B, L, L, D, H, scale, 1, None, bws.ptr,
                                    ws.value, s))
    dq, dk, dv = (G.down(x, (B * L, D)) for x in outs)
    for b, h in [(0, 0), (3, 13)]:
        rows, cols = slice(b * L, (b + 1) * L), slice(h * hd, (h + 1) * hd)
        want = _attention_bwd64(*(t[rows, cols].astype(np.float64) for t in (q, k, v, g)), scale)
        for a, e, n in zip((dq, dk, dv), want, "QKV"):
            parity(a[rows, cols], e, f"c3 stored-dS (b {b}, h {h}) d{n}")


C5S = {"dim": 64, "heads": 2, "layers": 2, "ff": 128, "max_seq": 64, "discrete": False, "input_dim": 5,
       "output_dim": 3}


def test_device_trainer_continuous_c5_width_matches_oracle():
    """One TrainBatchContinuous step at the config-5 layer width (F 5 -> D 256,
    8 heads of 32, FF 1024 ReLU, a 1-wide regression head) on four 300-step
    windows, 1196 rows: the Q/K/V input gradient as one K-segmented product,
    the ReLU layer cached by its output alone, the short-K input projection and
    its gradient, the 16-lanes-per-row head and its K = 1 input gradient all
    run at their real widths; loss, norm, gradients and weights against the
    oracle."""
    cfg = {"dim": 256, "heads": 8, "layers": 2, "ff": 1024, "max_seq": 512, "discrete": False,
           "input_dim": 5, "output_dim": 1, "data_type": 1}
    w = synth.continuous_lm_weights(cfg, 16)
    rng = np.random.default_rng(22)
    wins = [rng.uniform(0, 1, (300, 5)).astype(np.float32) for _ in range(4)]
    tg = [rng.standard_normal((300, 1)).astype(np.float32) for _ in range(4)]
    t, _ = _trainer(cfg, w, 4, 300)
    loss = t.TrainBatchContinuous(wins, regressionTargets=tg, learningRate=0.01)
    want_loss, want_g, want_w = O.train_batch_continuous(cfg, w, wins, 0.01, reg_targets=tg)
    assert abs(loss - want_loss) <= 1e-5 + 1e-5 * abs(want_loss)
    assert t.last_norm == pytest.approx(want_g["norm"], rel=1e-4)

    def named(d):
        out = {k: d[k] for k in ("input_proj", "input_bias", "out_proj", "out_bias")}
        for i, L in enumerate(d["layers"]):
            for k, v in L.items():
                out[f"layers.{i}.{k}"] = v
        return out

    for got, want, what in ((t.gradients(), want_g, "gradient"), (t.weights(), want_w, "weight")):
        ww = named(want)
        for k, v in got.items():
            parity(v, np.asarray(ww[k]).reshape(-1), f"c5-width {what} {k}")


@pytest.mark.parametrize("kind", ["regression", "classification"])
def test_device_trainer_continuous_matches_oracle(kind):
    """TrainBatchContinuous of a time-series model (input projection F 5 ->
    D 64, head dim 32 on the saved-statistics attention backward): a bucket
    of four 33-step windows, a lone 20-step window and skipped windows, then
    two more steps; loss, gradients and weights against the oracle."""
    cfg = dict(C5S, data_type=1 if kind == "regression" else 2)
    w = synth.continuous_lm_weights(cfg, 15)
    rng = np.random.default_rng(21)
    wins = [rng.uniform(0, 1, (33, 5)).astype(np.float32) for _ in range(4)] + \
           [rng.uniform(0, 1, (20, 5)).astype(np.float32)]
    if kind == "regression":
        tg = [rng.standard_normal((x.shape[0], 3)).astype(np.float32) for x in wins]
        kw, okw = {"regressionTargets": tg + [None]}, {"reg_targets": tg + [None]}
    else:
        tg = [rng.integers(0, 3, x.shape[0]).astype(np.int32) for x in wins]
        kw, okw = {"classTargets": tg + [None]}, {"class_targets": tg + [None]}
    inputs = wins + [rng.uniform(0, 1, (33, 5)).astype(np.float32)]  # no targets: skipped
    t, lm = _trainer(cfg, w, 4, 32)
    loss = t.TrainBatchContinuous(inputs, learningRate=0.01, **kw)
    want_loss, want_g, want_w = O.train_batch_continuous(cfg, w, inputs, 0.01, **okw)
    assert abs(loss - want_loss) <= 1e-5 + 1e-5 * abs(want_loss)
    assert t.last_norm == pytest.approx(want_g["norm"], rel=1e-4)
    names = set(t.gradients())
    assert "input_proj" in names and "token_embedding" not in names

    def named(d):
        out = {k: d[k] for k in ("input_proj", "input_bias", "out_proj", "out_bias")}
        for i, L in enumerate(d["layers"]):
            for k, v in L.items():
                out[f"layers.{i}.{k}"] = v
        return out

    for got, want, what in ((t.gradients(), want_g, "gradient"), (t.weights(), want_w, "weight")):
        ww = named(want)
        for k, v in got.items():
            parity(v, np.asarray(ww[k]).reshape(-1), f"continuous {kind} {what} {k}")
    ww = want_w
    for step in range(2):
        more = [rng.uniform(0, 1, (25, 5)).astype(np.float32) for _ in range(3)]
        if kind == "regression":
            mt = [rng.standard_normal((25, 3)).astype(np.float32) for _ in range(3)]
            t.TrainBatchContinuous(more, regressionTargets=mt, learningRate=0.01)
            _, _, ww = O.train_batch_continuous(cfg, ww, more, 0.01, reg_targets=mt)
        else:
            mt = [rng.integers(0, 3, 25).astype(np.int32) for _ in range(3)]
            t.TrainBatchContinuous(more, classTargets=mt, learningRate=0.01)
            _, _, ww = O.train_batch_continuous(cfg, ww, more, 0.01, class_targets=mt)
    got = t.weights()
    named_w = named(ww)
    for k in ("input_proj", "layers.1.wq", "layers.0.ffn_w2", "out_proj"):
        parity(got[k], np.asarray(named_w[k]).reshape(-1), f"after 3 steps {k}")


def _splitmix_order(n, seed, epochs):
    """The epoch orders of DeviceTrainer.Train / TrainContinuous: a
    Fisher-Yates shuffle per epoch driven by SplitMix64 from `seed`."""
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


@pytest.mark.parametrize("kind", ["tokens", "regression"])
def test_device_trainer_epochs_equal_batch_steps(kind):
    """Train / TrainContinuous (TransformerTrainer.cs:43-215): epochs of
    shuffled batches of BatchSize with learning-rate decay give the same bits
    as TrainBatch / TrainBatchContinuous called in that order; sequences
    shorter than 2 are dropped first, and the result is the last epoch's mean
    batch loss."""
    from cdml import host
    H = host.module()
    epochs, bs, lr0, decay = 3, 3, 0.02, 0.8
    if kind == "tokens":
        cfg, w = C1, synth.lm_weights(C1, 31)
        rng = np.random.default_rng(5)
        data = [rng.integers(0, 200, int(n)).astype(np.int32) for n in (17, 17, 9, 1, 17, 12, 9, 17)]
        valid = [d for d in data if d.shape[0] >= 2]
    else:
        cfg = dict(C5S, data_type=1)
        w = synth.continuous_lm_weights(cfg, 33)
        rng = np.random.default_rng(6)
        data = [rng.uniform(0, 1, (int(n), 5)).astype(np.float32) for n in (21, 21, 13, 1, 21, 8, 13)]
        targets = [rng.standard_normal((x.shape[0], 3)).astype(np.float32) for x in data]
        keep = [i for i, d in enumerate(data) if d.shape[0] >= 2]
        valid, vt = [data[i] for i in keep], [targets[i] for i in keep]
    trainers = []
    for _ in range(2):
        lm, _ = host.language_model(cfg, w)
        tc = H.TrainingConfig()
        tc.BatchSize, tc.Epochs, tc.LearningRate = bs, epochs, lr0
        tc.UseLearningRateDecay, tc.LearningRateDecay = True, decay
        trainers.append(H.DeviceTrainer(lm, tc, 4, 32))
    a, b = trainers
    got = a.Train(data, seed=9) if kind == "tokens" else a.TrainContinuous(data, regressionTargets=targets, seed=9)
    lr = np.float32(lr0)
    for order in _splitmix_order(len(valid), 9, epochs):
        losses = []
        for i in range(0, len(order), bs):
            idx = order[i:i + bs]
            if kind == "tokens":
                losses.append(b.TrainBatch([valid[j] for j in idx], float(lr)))
            else:
                losses.append(b.TrainBatchContinuous([valid[j] for j in idx], regressionTargets=[vt[j] for j in idx],
                                                     learningRate=float(lr)))
        lr = np.float32(lr * np.float32(decay))
    want = float(np.float32(sum(np.float32(x) for x in losses)) / np.float32(len(losses)))
    assert got == pytest.approx(want, rel=1e-6)
    wa, wb = a.weights(), b.weights()
    for k in wa:
        assert np.array_equal(wa[k], wb[k]), k


def test_device_trainer_steps_are_deterministic():
    """Every reduction in the training step runs in a fixed order and no
    kernel uses atomics, so two trainers from the same weights on the same
    batches end with the same bits.  The shape takes split-K weight gradients
    with a ragged tail (2 x 1023 rows), the stored-dS attention backward
    (head dim 64) and vectorised LayerNorm (D 256)."""
    cfg = {"vocab": 300, "dim": 256, "heads": 4, "layers": 2, "ff": 512, "max_seq": 1024}
    w = synth.lm_weights(cfg, 77)
    seqs = list(synth.token_ids(78, 2 * 1024, 300).reshape(2, 1024))
    short = list(synth.token_ids(79, 3 * 300, 300).reshape(3, 300))
    runs = []
    for _ in range(2):
        t, _ = _trainer(cfg, w, 3, 1023)
        losses = [t.TrainBatch(seqs, 0.01), t.TrainBatch(short, 0.01), t.TrainBatch(seqs, 0.01)]
        runs.append((losses, t.weights(), t.last_norm))
    (la, wa, na), (lb, wb, nb) = runs
    assert la == lb and na == nb
    for k in wa:
        assert np.array_equal(wa[k], wb[k]), k
