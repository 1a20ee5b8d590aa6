"""Pins the training-step oracle (oracle/refcpu_train.c and oracle.train_step)
without the reference, which cannot run here.

* Each new operation against what the mathematics fixes: LayerNormBackward
  and the FFN backward (ComputeInputGradientBatch) against float64 central
  finite differences of their forward passes; CrossEntropyLossAndGradient
  against scipy's log-softmax and the closed form (softmax - onehot) / N.
* The whole TrainBatchDiscrete step: every gradient of a two-layer model
  against float64 central finite differences of the mean next-token
  cross-entropy, computed by an independent float64 numpy forward of the
  model; the SGD update bit-exactly against w - lr * g in float32; clipping
  against the global-norm rule.
* A planted mistake (a dropped residual gradient) must fail the
  finite-difference check.
"""
from __future__ import annotations

import numpy as np
import pytest
from scipy.special import log_softmax

from cdml import synth
from oracle import oracle as O

F64 = np.float64


# ---------------------------------------------------------------- float64 model
def _ln(r, g, b, eps=1e-5):
    m = r.mean(1, keepdims=True)
    v = ((r - m) ** 2).mean(1, keepdims=True)
    return (r - m) / np.sqrt(v + eps) * g + b


def _rope(x, H, S, inverse=False):
    rows, D = x.shape
    hd = D // H
    pos = (np.arange(rows) % S).astype(F64)[:, None]
    p = np.arange(hd // 2)
    th = pos / (10000.0 ** (2.0 * p / hd))[None, :]
    c, s = np.cos(th), np.sin(th) * (-1 if inverse else 1)
    out = x.copy()
    for h in range(H):
        e, o = h * hd + 2 * p, h * hd + 2 * p + 1
        out[:, e] = x[:, e] * c - x[:, o] * s
        out[:, o] = x[:, e] * s + x[:, o] * c
    return out


def loss64(cfg, w, seqs, drop_ffn_residual=False):
    """Mean next-token cross-entropy of the decoder-only LanguageModel in
    float64 (post-LN blocks, interleaved RoPE at positions row % S, causal
    attention per sequence, ReLU FFN)."""
    B, S = seqs.shape[0], seqs.shape[1] - 1
    D, H = cfg["dim"], cfg["heads"]
    hd = D // H
    ids, tg = seqs[:, :S].reshape(-1), seqs[:, 1:].reshape(-1)
    x = w["token_embedding"][ids]
    for L in w["layers"]:
        q = _rope(x @ L["wq"].T + L["bq"], H, S)
        k = _rope(x @ L["wk"].T + L["bk"], H, S)
        v = x @ L["wv"].T + L["bv"]
        att = np.zeros_like(q)
        mask = np.tril(np.ones((S, S), bool))
        for b in range(B):
            sl = slice(b * S, (b + 1) * S)
            for h in range(H):
                cs = slice(h * hd, (h + 1) * hd)
                sc = q[sl, cs] @ k[sl, cs].T / np.sqrt(hd)
                sc = np.where(mask, sc, -np.inf)
                p = np.exp(sc - sc.max(1, keepdims=True))
                p /= p.sum(1, keepdims=True)
                att[sl, cs] = p @ v[sl, cs]
        n1 = _ln(x + att @ L["wo"].T + L["bo"], L["ln1_g"], L["ln1_b"])
        ff = np.maximum(n1 @ L["ffn_w1"].T + L["ffn_b1"], 0) @ L["ffn_w2"].T + L["ffn_b2"]
        x = _ln((0 if drop_ffn_residual else n1) + ff, L["ln2_g"], L["ln2_b"])
    logits = x @ w["out_proj"].T + w["out_bias"]
    p = np.exp(log_softmax(logits, axis=1))
    return float(np.mean(-np.log(p[np.arange(len(tg)), tg] + 1e-10)))


def cont_loss64(cfg, w, inputs, reg=None, cls=None):
    """TrainBatchContinuous's objective for one bucket in float64: the
    input-projection model of loss64, MSE over rows x outputs against step
    t + 1 (regression) or mean cross-entropy (classification)."""
    B, S = inputs.shape[0], inputs.shape[1] - 1
    D, H = cfg["dim"], cfg["heads"]
    hd = D // H
    x = inputs[:, :S].reshape(B * S, -1) @ w["input_proj"].T + w["input_bias"]
    for L in w["layers"]:
        q = _rope(x @ L["wq"].T + L["bq"], H, S)
        k = _rope(x @ L["wk"].T + L["bk"], H, S)
        v = x @ L["wv"].T + L["bv"]
        att = np.zeros_like(q)
        mask = np.tril(np.ones((S, S), bool))
        for b in range(B):
            sl = slice(b * S, (b + 1) * S)
            for h in range(H):
                cs = slice(h * hd, (h + 1) * hd)
                sc = np.where(mask, q[sl, cs] @ k[sl, cs].T / np.sqrt(hd), -np.inf)
                p = np.exp(sc - sc.max(1, keepdims=True))
                att[sl, cs] = (p / p.sum(1, keepdims=True)) @ v[sl, cs]
        n1 = _ln(x + att @ L["wo"].T + L["bo"], L["ln1_g"], L["ln1_b"])
        ff = np.maximum(n1 @ L["ffn_w1"].T + L["ffn_b1"], 0) @ L["ffn_w2"].T + L["ffn_b2"]
        x = _ln(n1 + ff, L["ln2_g"], L["ln2_b"])
    out = x @ w["out_proj"].T + w["out_bias"]
    if reg is not None:
        return float(np.mean((out - reg[:, 1:S + 1].reshape(B * S, -1)) ** 2))
    tg = cls[:, 1:S + 1].reshape(-1)
    p = np.exp(log_softmax(out, axis=1))
    return float(np.mean(-np.log(p[np.arange(len(tg)), tg] + 1e-10)))


def _to64(w):
    return {k: ([{kk: vv.astype(F64) for kk, vv in L.items()} for L in v] if k == "layers" else v.astype(F64))
            for k, v in w.items()}


def _entries(w):
    for k in ("token_embedding", "out_proj", "out_bias"):
        yield (k,), w[k]
    for i, L in enumerate(w["layers"]):
        for k, v in L.items():
            yield ("layers", i, k), v


def _get(d, key):
    for k in key:
        d = d[k]
    return d


CFG = {"vocab": 12, "dim": 8, "heads": 2, "layers": 2, "ff": 16, "max_seq": 8}


def batch_loss64(cfg, w, buckets, drop_ffn_residual=False):
    """TrainBatchDiscrete's objective over several length buckets: the
    bucket means weighted by their sequence counts, over the valid count."""
    n = [b.shape[0] for b in buckets]
    return sum(k * loss64(cfg, w, b, drop_ffn_residual) for k, b in zip(n, buckets)) / sum(n)


def _fd_check(seqs, per_tensor=6, seed=0, drop_ffn_residual=False):
    buckets = seqs if isinstance(seqs, list) else [seqs]
    w = synth.lm_weights(CFG, 3, biased=True)
    flat = [s for b in buckets for s in b]
    loss, g, _ = O.train_batch(CFG, w, flat, 0.1, use_clipping=False)
    w64 = _to64(w)
    lossf = lambda ww: batch_loss64(CFG, ww, buckets, drop_ffn_residual)
    assert abs(loss - lossf(w64)) < 1e-5 or drop_ffn_residual
    used_ids = np.unique(np.concatenate([b[:, :-1].reshape(-1) for b in buckets]))
    rng = np.random.default_rng(seed)
    eps = 1e-6
    worst = 0.0
    for key, arr in _entries(w64):
        flat = arr.reshape(-1)
        gr = _get(g, key).reshape(-1)
        if key == ("token_embedding",):  # rows of used tokens carry the gradient
            cand = (used_ids[:, None] * CFG["dim"] + np.arange(CFG["dim"])[None, :]).reshape(-1)
        else:
            cand = np.arange(flat.size)
        for e in rng.choice(cand, size=min(per_tensor, cand.size), replace=False):
            keep = flat[e]
            flat[e] = keep + eps
            lp = lossf(w64)
            flat[e] = keep - eps
            lm = lossf(w64)
            flat[e] = keep
            fd = (lp - lm) / (2 * eps)
            err = abs(gr[e] - fd) - (3e-5 + 1e-3 * abs(fd))
            worst = max(worst, err)
            if err > 0:
                return False, f"{key}[{e}]: oracle {gr[e]:.7g}, finite difference {fd:.7g}"
    return True, worst


@pytest.mark.parametrize("batch", [3, 1])
def test_train_step_gradients_against_finite_differences(batch):
    seqs = synth.token_ids(5 + batch, batch * 6, CFG["vocab"]).reshape(batch, 6)
    ok, info = _fd_check(seqs)
    assert ok, info


def test_mixed_length_batch_gradients_against_finite_differences():
    """Two buckets (three sequences of 6 tokens, one of 4) plus sequences the
    trainer skips (too short, an id outside the vocabulary): the gradients
    accumulate over the buckets before the 1/validCount scale."""
    a = synth.token_ids(31, 3 * 6, CFG["vocab"]).reshape(3, 6)
    b = synth.token_ids(32, 4, CFG["vocab"]).reshape(1, 4)
    w = synth.lm_weights(CFG, 3, biased=True)
    skipped = [np.array([5], np.int32), np.array([1, CFG["vocab"], 2], np.int32)]
    full = O.train_batch(CFG, w, [a[0], skipped[0], b[0], a[1], skipped[1], a[2]], 0.1, use_clipping=False)
    ref = O.train_batch(CFG, w, [a[0], b[0], a[1], a[2]], 0.1, use_clipping=False)
    assert full[0] == ref[0] and np.array_equal(full[1]["out_proj"], ref[1]["out_proj"])
    ok, info = _fd_check([a, b])
    assert ok, info


CCFG = {"dim": 8, "heads": 2, "layers": 2, "ff": 16, "max_seq": 8, "discrete": False, "input_dim": 5,
        "output_dim": 3}


@pytest.mark.parametrize("kind", ["regression", "classification"])
def test_continuous_train_batch_against_finite_differences(kind):
    """TrainBatchContinuous: a bucket of three 6-step windows and a lone
    4-step window (plus windows the trainer skips), every gradient against
    float64 finite differences of the bucket-weighted loss."""
    rng = np.random.default_rng(11)
    w = synth.continuous_lm_weights(CCFG, 7)
    wins = [rng.uniform(0, 1, (6, 5)).astype(np.float32) for _ in range(3)] + \
           [rng.uniform(0, 1, (4, 5)).astype(np.float32)]
    if kind == "regression":
        tg = [rng.standard_normal((t.shape[0] + 1, 3)).astype(np.float32) for t in wins]  # longer is allowed
        bad_t = rng.standard_normal((6, 3)).astype(np.float32)
        bad_t[2, 1] = np.nan
        kw = {"reg_targets": tg + [bad_t, None]}
    else:
        tg = [rng.integers(0, 3, t.shape[0]).astype(np.int32) for t in wins]
        kw = {"class_targets": tg + [np.array([0, 1, 7, 0, 1, 2], np.int32), None]}
    inputs = wins + [rng.uniform(0, 1, (6, 5)).astype(np.float32), np.zeros((1, 5), np.float32)]
    loss, g, _ = O.train_batch_continuous(CCFG, w, inputs, 0.1, use_clipping=False, **kw)
    w64 = _to64(w)
    a_in, b_in = np.stack(wins[:3]).astype(F64), wins[3][None].astype(F64)
    if kind == "regression":
        A, Bt = np.stack([t[:6] for t in tg[:3]]).astype(F64), tg[3][None, :4].astype(F64)
        lossf = lambda ww: (3 * cont_loss64(CCFG, ww, a_in, reg=A) + cont_loss64(CCFG, ww, b_in, reg=Bt)) / 4
    else:
        A, Bt = np.stack(tg[:3]), tg[3][None]
        lossf = lambda ww: (3 * cont_loss64(CCFG, ww, a_in, cls=A) + cont_loss64(CCFG, ww, b_in, cls=Bt)) / 4
    assert abs(loss - lossf(w64)) < 1e-5
    rng2 = np.random.default_rng(0)
    eps = 1e-6
    for key, arr in [(("input_proj",), w64["input_proj"]), (("input_bias",), w64["input_bias"])] + \
            [e for e in _entries(w64) if e[0] != ("token_embedding",)]:
        flat = arr.reshape(-1)
        gr = _get(g, key).reshape(-1)
        for e in rng2.choice(flat.size, size=min(5, flat.size), replace=False):
            keep = flat[e]
            flat[e] = keep + eps
            lp = lossf(w64)
            flat[e] = keep - eps
            lm = lossf(w64)
            flat[e] = keep
            fd = (lp - lm) / (2 * eps)
            assert abs(gr[e] - fd) < 3e-5 + 1e-3 * abs(fd), (key, e, gr[e], fd)


def test_mse_loss_closed_form():
    rng = np.random.default_rng(4)
    p, t = rng.standard_normal((5, 3)).astype(np.float32), rng.standard_normal((7, 3)).astype(np.float32)
    loss, d = O.mse_loss(p, t, 4, target_start=2)
    diff = p[:4].astype(F64) - t[2:6]
    assert loss == pytest.approx(np.mean(diff ** 2), rel=1e-6)
    assert np.allclose(d[:4], 2 * diff / 12, atol=1e-7) and not d[4].any()


def test_planted_mistake_fails_the_gradient_check():
    """The float64 loss without the FFN residual is a different function: the
    oracle's gradients must not match its finite differences."""
    seqs = synth.token_ids(8, 3 * 6, CFG["vocab"]).reshape(3, 6)
    ok, _ = _fd_check(seqs, drop_ffn_residual=True)
    assert not ok


def test_train_step_update_and_clipping():
    w = synth.lm_weights(CFG, 4, biased=True)
    seqs = synth.token_ids(9, 2 * 7, CFG["vocab"]).reshape(2, 7)
    lr = 0.05
    loss, g, nw = O.train_step(CFG, w, seqs, lr, use_clipping=False)
    for key, arr in _entries(w):
        want = arr - np.float32(lr) * _get(g, key)
        assert np.array_equal(_get(nw, key), want), key
    # clipping: with a threshold below the norm every gradient is scaled by threshold / norm
    _, gc, _ = O.train_step(CFG, w, seqs, lr, clip=0.25, use_clipping=True)
    assert gc["norm"] == pytest.approx(g["norm"], rel=1e-6) and g["norm"] > 0.25
    tot = sum(float(np.sum(_get(gc, k).astype(F64) ** 2)) for k, _ in _entries(w))
    assert np.sqrt(tot) == pytest.approx(0.25, rel=1e-5)
    assert loss == pytest.approx(loss64(CFG, _to64(w), seqs), abs=1e-5)


def test_layernorm_backward_against_finite_differences():
    rng = np.random.default_rng(1)
    a, b = rng.standard_normal((5, 7)).astype(np.float32), rng.standard_normal((5, 7)).astype(np.float32)
    gam, bet = (1 + 0.1 * rng.standard_normal(7)).astype(np.float32), rng.standard_normal(7).astype(np.float32)
    dout = rng.standard_normal((5, 7)).astype(np.float32)
    out, mean, var, norm, res = O.residual_layernorm_forward(a, b, gam, bet)
    assert np.allclose(out, _ln(a.astype(F64) + b, gam.astype(F64), bet), atol=2e-6)
    assert np.array_equal(out, O.residual_layernorm(a, b, gam, bet))  # same as the inference form
    dx, dg, db = O.layernorm_backward(dout, norm, gam, res, mean, var)
    f = lambda r, g_, b_: float(np.sum(dout.astype(F64) * _ln(r, g_, b_)))
    r64, g64, b64 = res.astype(F64), gam.astype(F64), bet.astype(F64)
    eps = 1e-6
    for arr, got in ((r64, dx), (g64, dg), (b64, db)):
        flat = arr.reshape(-1)
        for e in range(flat.size):
            k = flat[e]
            flat[e] = k + eps
            fp = f(r64, g64, b64)
            flat[e] = k - eps
            fm = f(r64, g64, b64)
            flat[e] = k
            assert abs(got.reshape(-1)[e] - (fp - fm) / (2 * eps)) < 2e-5


def test_cross_entropy_against_log_softmax():
    rng = np.random.default_rng(2)
    logits = (3 * rng.standard_normal((6, 11))).astype(np.float32)
    t = rng.integers(0, 11, 9).astype(np.int32)
    loss, dl = O.cross_entropy(logits, t, 4, target_start=2)
    ls = log_softmax(logits.astype(F64), axis=1)
    want = -np.mean([np.log(np.exp(ls[i, t[2 + i]]) + 1e-10) for i in range(4)])
    assert loss == pytest.approx(want, abs=2e-6)
    p = np.exp(ls[:4])
    p[np.arange(4), t[2:6]] -= 1
    assert np.allclose(dl[:4], p / 4, atol=1e-7) and not dl[4:].any()
    with pytest.raises(O.OracleError):
        O.cross_entropy(logits, t, 8, target_start=2)


def test_ffn_input_gradient_against_finite_differences():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 6)).astype(np.float32)
    w1, b1 = rng.standard_normal((9, 6)).astype(np.float32), rng.standard_normal(9).astype(np.float32)
    w2, b2 = rng.standard_normal((6, 9)).astype(np.float32), rng.standard_normal(6).astype(np.float32)
    dout = rng.standard_normal((4, 6)).astype(np.float32)
    for act in (3, 1, 2, 5):
        wg = [np.zeros_like(w1), np.zeros_like(w2)]
        bg = [np.zeros_like(b1), np.zeros_like(b2)]
        dx = O.ffn_input_gradient(x, dout, [w1, w2], [b1, b2], [act, 0], wg, bg)
        fns = {3: lambda z: np.maximum(z, 0), 1: lambda z: 1 / (1 + np.exp(-z)), 2: np.tanh,
               5: lambda z: z / (1 + np.exp(-z))}
        ps = [x.astype(F64), w1.astype(F64), b1.astype(F64), w2.astype(F64), b2.astype(F64)]

        def f():
            h = fns[act](ps[0] @ ps[1].T + ps[2])
            return float(np.sum(dout * (h @ ps[3].T + ps[4])))

        eps = 1e-6
        for arr, got in zip(ps, (dx, wg[0], bg[0], wg[1], bg[1])):
            flat = arr.reshape(-1)
            for e in range(flat.size):
                k = flat[e]
                flat[e] = k + eps
                fp = f()
                flat[e] = k - eps
                fm = f()
                flat[e] = k
                fd = (fp - fm) / (2 * eps)
                assert abs(got.reshape(-1)[e] - fd) < 2e-5 + 1e-4 * abs(fd), (act, e)


def test_token_embedding_grad_accumulates_in_row_order():
    eg = np.zeros((5, 3), np.float32)
    dx = np.arange(12, dtype=np.float32).reshape(4, 3)
    got = O.accumulate_token_embedding_grad(eg, dx, [2, 0, 2, 4])
    assert np.array_equal(got[2], dx[0] + dx[2]) and np.array_equal(got[0], dx[1])
    assert not got[1].any() and not got[3].any()
    with pytest.raises(O.OracleError):
        O.accumulate_token_embedding_grad(eg, dx, [2, 0, 5, 4])
