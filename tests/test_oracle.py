"""Pins the CPU oracle (oracle/refcpu.c) before it is trusted as the checker.

Three kinds of evidence, none of them a retyping of the oracle's loops:
* the reference test suite's own known answers (RoPE cos/sin values,
  MatrixMultiplyTranspose 17/23/67, masked-softmax sums, LayerNorm stats,
  the all-masked-row and causal-cross-attention rules);
* float64 textbook results on the reference tests' closed-form inputs
  (tests/golden/ops.npz, lm_*.npz, written by tests/golden/gen_golden.py);
* invariants the mathematics fixes (causal flag == explicit lower-triangular
  mask, decode of the last position == last row of causal prefill, causal
  invariance to future tokens, greedy decode with a KV cache == greedy with
  full-prefix recompute).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import assert_parity, load_lm_golden
from oracle import oracle as O
from cdml import synth

M, Vec = synth.matrix, synth.vector


def close(a, e, atol=2e-6, rtol=1e-5, what=""):
    assert_parity(a, e, atol=atol, rtol=rtol, what=what)


# ----------------------------------------------------------- known answers
def test_rope_known_values():
    # RotaryPositionEmbeddingTests.cs:138-177
    x = O.rope(np.array([[1, 2, 3, 4], [5, 6, 7, 8]], np.float32), 1)
    assert np.allclose(x[0], [1, 2, 3, 4], atol=1e-5)
    y = O.rope(np.array([[1, 0], [1, 0], [0, 1]], np.float32), 1)
    assert np.allclose(y[0], [1, 0], atol=1e-5)
    assert np.allclose(y[1], [math.cos(1), math.sin(1)], atol=1e-5)
    assert np.allclose(y[2], [-math.sin(2), math.cos(2)], atol=1e-5)


def test_rope_heads_independent_and_round_trip():
    # RotaryPositionEmbeddingTests.cs:179-196, 223-266; parity tests :1107-1111
    x = O.rope(np.array([[1, 2, 3, 4], [1, 0, 0, 1]], np.float32), 2)
    assert np.allclose(x[1], [math.cos(1), math.sin(1), -math.sin(1), math.cos(1)], atol=1e-5)
    m = M(4, 8, 97)
    back = O.rope(O.rope(m, 2), 2, inverse=True)
    assert np.allclose(back, m, atol=5e-4)


def test_rope_rejects_odd_head_dim():
    with pytest.raises(O.OracleError):
        O.rope(np.zeros((2, 6), np.float32), 2)


def test_matrix_multiply_transpose_known_values():
    # MultiTypeTransformerTests.cs:664-674 via y = h W^T + 0
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8], [9, 10]], np.float32)
    c = O.project_output_batch(a, b, np.zeros(3, np.float32))
    assert c.shape == (2, 3)
    assert c[0, 0] == 17 and c[0, 1] == 23 and c[1, 2] == 67


def test_softmax_masked_rows():
    # MultiTypeTransformerTests.cs:634-662
    s = O.softmax(np.array([[1, 2, 3], [-1, 0, 1]], np.float32),
                  np.array([[1, 0, 1], [0, 1, 1]], np.uint8))
    assert abs(s[0, 1]) < 1e-7 and abs(s[1, 0]) < 1e-7
    assert abs(s[0, 0] + s[0, 2] - 1) < 1e-6 and abs(s[1, 1] + s[1, 2] - 1) < 1e-6
    z = O.softmax(np.array([[1, 2, 3]], np.float32), np.zeros((1, 3), np.uint8))
    assert np.all(z == 0)


def test_layernorm_row_stats():
    # MultiTypeTransformerTests.cs:676-700
    x = np.array([[1, 2, 3, 4], [-1, 0, 1, 2]], np.float32)
    y = O.residual_layernorm(x, np.zeros_like(x), np.ones(4, np.float32), np.zeros(4, np.float32))
    assert np.all(np.abs(y.mean(axis=1)) < 1e-5)
    assert np.all(np.abs(y.var(axis=1) - 1) < 1e-3)


def test_sdpa_rules():
    # AccelerationManagerParityTests.cs:438-458
    q, k, v = M(4, 8, 121), M(5, 8, 122), M(5, 8, 123)
    with pytest.raises(O.OracleError):
        O.sdpa(q, k, v, 2, causal=True)
    m = np.ones((4, 5), np.uint8)
    m[0] = 0
    out = O.sdpa(q, k, v, 2, mask=m)
    assert np.all(out[0] == 0)
    # one key: softmax weight is exactly 1, so the output is V itself
    one = O.sdpa(q[:1], k[:1], v[:1], 2)
    assert np.array_equal(one, v[:1])


# ------------------------------------------------------- float64 goldens
def test_sdpa_golden(ops_golden):
    g = ops_golden
    qs, ks, vs = M(4, 8, 118), M(4, 8, 119), M(4, 8, 120)
    qc, kc, vc = M(4, 8, 121), M(5, 8, 122), M(5, 8, 123)
    close(O.sdpa(qs, ks, vs, 2), g["sdpa_self_nomask"], what="self/no mask")
    close(O.sdpa(qs, ks, vs, 2, mask=g["self_mask"]), g["sdpa_self_mask"], what="self/mask")
    close(O.sdpa(qs, ks, vs, 2, causal=True), g["sdpa_self_causal"], what="self/causal")
    close(O.sdpa(qc, kc, vc, 2), g["sdpa_cross_nomask"], what="cross/no mask")
    close(O.sdpa(qc, kc, vc, 2, mask=g["cross_mask"]), g["sdpa_cross_mask"], what="cross/mask")
    close(O.sdpa(qc, kc, vc, 2, mask=g["all_masked_mask"]), g["sdpa_cross_allmasked"], what="all masked")


def test_mha_golden(ops_golden):
    g = ops_golden
    q6, k6, v6 = M(4, 6, 31), M(4, 6, 32), M(4, 6, 33)
    close(O.mha_forward(q6, k6, v6, 2, float(g["mha_causal_scale"]), mask=O.causal_mask(4)),
          g["mha_causal"], what="mha causal d_h=3")
    qg, kg, vg = M(128, 64, 110), M(128, 64, 111), M(128, 64, 112)
    close(O.mha_forward(qg, kg, vg, 4, 0.25), g["mha128_nomask"], what="mha128")
    close(O.sdpa(qg, kg, vg, 4, causal=True), g["mha128_causal"], what="sdpa128 causal")
    qh, kh, vh = (synth.normal(900 + i, (1024, 64)) for i in range(3))
    close(O.sdpa(qh, kh, vh, 1, causal=True), g["c2_head_causal"], what="c2 head slice, causal")


def test_causal_flag_equals_explicit_mask():
    # AccelerationManagerParityTests.cs:410-421 (bit-identical in the reference CPU manager)
    q, k, v = M(37, 16, 1), M(37, 16, 2), M(37, 16, 3)
    a = O.sdpa(q, k, v, 2, causal=True)
    b = O.sdpa(q, k, v, 2, mask=O.causal_mask(37))
    assert np.array_equal(a, b)


def test_projections_golden(ops_golden):
    g = ops_golden
    x = M(6, 5, 124)
    q, k, v = O.project_qkv(x, M(8, 5, 125), Vec(8, 128), M(8, 5, 126), Vec(8, 129), M(8, 5, 127), Vec(8, 130))
    close(q, g["qkv_small_q"], what="Q")
    close(k, g["qkv_small_k"], what="K")
    close(v, g["qkv_small_v"], what="V")
    xg = M(192, 128, 142)
    q, k, v = O.project_qkv(xg, M(128, 128, 143), Vec(128, 146), M(128, 128, 144), Vec(128, 147),
                            M(128, 128, 145), Vec(128, 148))
    close(q, g["qkv_big_q"], atol=1e-5, what="Q big")
    close(k, g["qkv_big_k"], atol=1e-5, what="K big")
    close(v, g["qkv_big_v"], atol=1e-5, what="V big")
    close(O.project_output_batch(M(4, 6, 56), M(3, 6, 57), Vec(3, 58)), g["project_output"], what="POB")
    assert np.array_equal(O.embed_tokens([0, 2, 4], M(6, 5, 64)), g["embed"])
    with pytest.raises(O.OracleError):
        O.embed_tokens([0, 6], M(6, 5, 64))


def test_rope_golden(ops_golden):
    g = ops_golden
    close(O.rope(M(4, 8, 97), 2), g["rope_all"], what="rope all heads")
    close(O.rope_head(M(4, 8, 97), 2, 4), g["rope_head"], what="rope one head")
    close(O.rope(M(300, 32, 7), 4), g["rope_long"], atol=2e-5, what="rope 300 positions")


def test_softmax_layernorm_golden(ops_golden):
    g = ops_golden
    close(O.softmax(M(4, 4, 26)), g["softmax_nomask"], what="softmax")
    close(O.softmax(M(4, 4, 26), g["softmax_mask_in"]), g["softmax_mask"], what="softmax mask")
    close(O.residual_layernorm(M(5, 6, 27), np.zeros((5, 6), np.float32), synth.positive_vector(6, 28),
                               Vec(6, 29)), g["layernorm"], what="layernorm")


# ---------------------------------------------------- language model flow
def _oracle_lm(g):
    return O.LanguageModel(g["cfg"], g["weights"])


@pytest.mark.parametrize("name", ["lm_tiny", "lm_c1"])
def test_lm_forward_golden(name):
    g = load_lm_golden(name)
    lm = _oracle_lm(g)
    close(lm.forward(g["ids"]), g["logits"], atol=2e-5, rtol=1e-4, what=f"{name} logits")


@pytest.mark.parametrize("name", ["lm_tiny", "lm_c1"])
def test_lm_greedy_matches_full_recompute(name):
    g = load_lm_golden(name)
    assert np.all(g["greedy_margins"] > 1e-3), "fixture margins too small to pin argmax"
    lm = _oracle_lm(g)
    out = lm.generate_greedy(g["ids"][: int(g["prompt_len"])], int(g["n_new"]))
    assert np.array_equal(out, g["greedy"])


def test_lm_causal_invariance():
    # MultiTypeTransformerTests.cs:135-166: a future token never changes earlier logits
    g = load_lm_golden("lm_tiny")
    lm = _oracle_lm(g)
    ids = g["ids"].copy()
    a = lm.forward(ids)
    ids[-1] = (ids[-1] + 1) % g["cfg"]["vocab"]
    b = lm.forward(ids)
    assert np.max(np.abs(a[:-1] - b[:-1])) < 1e-5
    assert np.max(np.abs(a[-1] - b[-1])) > 0


def test_lm_generate_bounds():
    # LanguageModel.cs:487-496
    g = load_lm_golden("lm_tiny")
    lm = _oracle_lm(g)
    full = np.zeros(g["cfg"]["max_seq"], np.int32)
    assert np.array_equal(lm.generate_greedy(full, 5), full)
    assert np.array_equal(lm.generate_greedy(g["ids"][:3], 0), g["ids"][:3])
    with pytest.raises(O.OracleError):
        lm.generate_greedy(np.array([g["cfg"]["vocab"]], np.int32), 2)


def test_decode_equals_last_prefill_row():
    D, H, T = 64, 4, 77
    q, k, v = synth.normal(11, (T, D)), synth.normal(12, (T, D)), synth.normal(13, (T, D))
    pre = O.sdpa(q, k, v, H, causal=True)
    for t in (1, 2, 40, T):
        dec = O.decode_attention(q[t - 1], k, v, t, H, 1.0 / math.sqrt(D // H))
        close(dec, pre[t - 1], atol=1e-5, what=f"decode t={t}")


def test_mt_restatement_matches_single_thread():
    x = synth.normal(1, (33, 48))
    w = [synth.xavier_uniform(2 + i, 48, 48) for i in range(3)]
    b = [synth.normal(9 + i, (48,)) for i in range(3)]
    st = O.project_qkv(x, w[0], b[0], w[1], b[1], w[2], b[2])
    mt = O.project_qkv(x, w[0], b[0], w[1], b[1], w[2], b[2], mt=True)
    for a, e in zip(mt, st):
        close(a, e, atol=1e-5)
    close(O.project_output_batch(x, w[0], b[0], mt=True), O.project_output_batch(x, w[0], b[0]), atol=1e-5)
    close(O.batch_dot_add_bias(w[0], x, b[0], mt=True), O.batch_dot_add_bias(w[0], x, b[0]), atol=1e-5)
    assert np.array_equal(O.rope(x, 4, mt=True), O.rope(x, 4))
    close(O.sdpa(x, x, x, 4, causal=True, mt=True), O.sdpa(x, x, x, 4, causal=True), atol=1e-5)
    close(O.residual_layernorm(x, x, b[0], b[1], mt=True), O.residual_layernorm(x, x, b[0], b[1]))
    kc = synth.normal(5, (3, 20, 48))
    vc = synth.normal(6, (3, 20, 48))
    qd = synth.normal(7, (3, 48))
    lens = np.array([20, 7, 1], np.int32)
    seq = O.decode_attention_batch(qd, kc, vc, lens, 4, 0.25, parallel=False)
    par = O.decode_attention_batch(qd, kc, vc, lens, 4, 0.25, parallel=True)
    assert np.array_equal(seq, par)
    for i in range(3):
        assert np.array_equal(seq[i], O.decode_attention(qd[i], kc[i], vc[i], int(lens[i]), 4, 0.25))


def test_oracle_detects_planted_mistake(ops_golden):
    """A plausible slip (keys and values swapped) must fail the golden check."""
    qs, ks, vs = M(4, 8, 118), M(4, 8, 119), M(4, 8, 120)
    wrong = O.sdpa(qs, vs, ks, 2)
    with pytest.raises(AssertionError):
        close(wrong, ops_golden["sdpa_self_nomask"])


def test_activation_library_values():
    """The FFN activations (NeuralNetwork.cs:670-716) against library routines:
    scipy's logistic function, numpy's tanh, and the piecewise-linear forms."""
    from scipy.special import expit

    x = np.concatenate([np.linspace(-30, 30, 601), [0.0, -0.0, 1e-8, -1e-8]]).astype(np.float32)
    x64 = x.astype(np.float64)
    close(O.activation(x, 0), x, atol=0, rtol=0, what="none")
    close(O.activation(x, 1), expit(x64), atol=1e-7, rtol=1e-6, what="sigmoid")
    close(O.activation(x, 2), np.tanh(x64), atol=1e-7, rtol=1e-6, what="tanh")
    close(O.activation(x, 3), np.maximum(x64, 0), atol=0, rtol=0, what="relu")
    close(O.activation(x, 4), np.where(x64 > 0, x64, 0.01 * x64), atol=1e-9, rtol=1e-6, what="leakyrelu")
    close(O.activation(x, 5), x64 * expit(x64), atol=1e-6, rtol=1e-6, what="swish")


# ------------------------------------------------------------ backward path
def _attention64(q, k, v, heads, scale, visible):
    """float64 attention forward: per head softmax(q k^T * scale) v over the
    visible keys (bool [lq, lk]); a row with no visible key gives zeros."""
    lq, dim = q.shape
    hd = dim // heads
    out = np.zeros((lq, dim))
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        s = (q[:, sl] @ k[:, sl].T) * scale
        s = np.where(visible, s, -np.inf)
        for i in range(lq):
            if not visible[i].any():
                continue
            e = np.exp(s[i] - s[i].max())
            out[i, sl] = (e / e.sum()) @ v[:, sl]
    return out


def _fd_grads(q, k, v, dout, heads, scale, visible, eps=1e-6):
    """Central differences of L = sum(dout * attention(q, k, v)) in float64:
    the gradients by brute force, with no derivation of the backward."""
    args = [np.array(a, np.float64) for a in (q, k, v)]
    g = [np.zeros_like(a) for a in args]
    for t in range(3):
        for idx in np.ndindex(args[t].shape):
            keep = args[t][idx]
            args[t][idx] = keep + eps
            up = np.sum(dout * _attention64(*args, heads, scale, visible))
            args[t][idx] = keep - eps
            dn = np.sum(dout * _attention64(*args, heads, scale, visible))
            args[t][idx] = keep
            g[t][idx] = (up - dn) / (2 * eps)
    return g


@pytest.mark.parametrize("case", ["parity_decoder", "parity_mask", "nomask_6x8", "decoder_6x8", "cross_5x8",
                                  "decoder_lq_gt_lk", "sparse_mask"])
def test_mha_backward_against_finite_differences(case):
    """MultiHeadAttentionBackward (AccelerationCPU.cs:1011-1280) on the shapes
    of AccelerationManagerParityTests.cs:354-383 (closed-form inputs, 4 x 6,
    2 heads, scale 1/sqrt(3)) and AccelerationConsistencyTests.cs:964-1022
    (6 x 8 and cross 5 x 8, 2 heads)."""
    if case.startswith("parity"):
        q, k, v, dout = M(4, 6, 31), M(4, 6, 32), M(4, 6, 33), M(4, 6, 34)
        heads, scale = 2, float(np.float32(1.0) / np.sqrt(np.float32(3.0)))
    else:
        lq, lk = {"cross_5x8": (5, 8), "decoder_lq_gt_lk": (7, 4)}.get(case, (6, 6))
        q, k, v = synth.normal(1, (lq, 8)), synth.normal(2, (lk, 8)), synth.normal(3, (lk, 8))
        dout = synth.normal(4, (lq, 8))
        heads, scale = 2, 0.5
    lq, lk = q.shape[0], k.shape[0]
    tril = np.tril(np.ones((lq, lk), bool))  # key j visible to query i iff j <= i
    mask = None
    if case == "parity_mask":
        mask = O.causal_mask(4).astype(bool)
        got = O.mha_backward(q, k, v, dout, heads, scale, mask=mask)
        visible = mask
    elif case == "sparse_mask":
        mask = synth.normal(9, (lq, lk)) > 0.3
        mask[2] = False  # a row with no visible key contributes nothing
        got = O.mha_backward(q, k, v, dout, heads, scale, mask=mask)
        visible = mask
    elif case in ("parity_decoder", "decoder_6x8", "decoder_lq_gt_lk"):
        got = O.mha_backward(q, k, v, dout, heads, scale, use_decoder_mask=True)
        visible = tril
    else:
        got = O.mha_backward(q, k, v, dout, heads, scale)
        visible = np.ones((lq, lk), bool)
    want = _fd_grads(q, k, v, np.asarray(dout, np.float64), heads, scale, visible)
    for g, w, n in zip(got, want, "QKV"):
        close(g, w, atol=2e-5, rtol=1e-4, what=f"{case} d{n}")
    if case == "sparse_mask":
        assert np.all(got[0][2] == 0)
    # a planted sign error in the oracle's softmax-gradient term must fail the check
    dq_bad = got[0] + 0.01 * np.sign(want[0] + 1e-9)
    with pytest.raises(AssertionError):
        close(dq_bad, want[0], atol=2e-5, rtol=1e-4)


def test_backprop_qkv_closed_form():
    """BackpropQKV (AccelerationCPU.cs:2071-2186) on the closed-form inputs of
    AccelerationManagerParityTests.cs:462-537 (6 rows, 5 -> 8, accumulators
    starting from nonzero values): dInput = dQ WQ + dK WK + dV WV,
    W*Grad += d*^T x, bias*Grad += column sums of d*, in float64."""
    x = M(6, 5, 124)
    wq, wk, wv = M(8, 5, 125), M(8, 5, 126), M(8, 5, 127)
    dq, dk, dv = M(6, 8, 131), M(6, 8, 132), M(6, 8, 133)
    g0 = [M(8, 5, 134), Vec(8, 137), M(8, 5, 135), Vec(8, 138), M(8, 5, 136), Vec(8, 139)]
    dx, wqg, bqg, wkg, bkg, wvg, bvg = O.backprop_qkv(x, dq, dk, dv, wq, wk, wv, *g0)
    X, D = x.astype(np.float64), [a.astype(np.float64) for a in (dq, dk, dv)]
    W = [a.astype(np.float64) for a in (wq, wk, wv)]
    close(dx, D[0] @ W[0] + D[1] @ W[1] + D[2] @ W[2], what="dInput")
    for got, g_init, d, n in [(wqg, g0[0], D[0], "WQ"), (wkg, g0[2], D[1], "WK"), (wvg, g0[4], D[2], "WV")]:
        close(got, g_init + d.T @ X, what=f"{n}Grad")
    for got, b_init, d, n in [(bqg, g0[1], D[0], "bQ"), (bkg, g0[3], D[1], "bK"), (bvg, g0[5], D[2], "bV")]:
        close(got, b_init + d.sum(0), what=f"{n}Grad")


def test_backprop_linear_and_output_projection():
    """BackpropLinearProjection (AccelerationCPU.cs:2188-2229: dInput
    accumulates) and BackpropOutputProjection (:2231-2270: dX overwritten) on
    the shapes of AccelerationConsistencyTests.cs:633-700,1108-1125."""
    x, dy, w = synth.normal(1, (4, 8)), synth.normal(2, (4, 8)), synth.normal(3, (8, 8))
    wg0, bg0, dx0 = synth.normal(4, (8, 8)), synth.normal(5, (8,)), synth.normal(6, (4, 8))
    wg, bg, dx = O.backprop_linear_projection(x, dy, w, wg0, bg0, dx0)
    X, DY, W = (a.astype(np.float64) for a in (x, dy, w))
    close(wg, wg0 + DY.T @ X, what="linear weightGrad")
    close(bg, bg0 + DY.sum(0), what="linear biasGrad")
    close(dx, dx0 + DY @ W, what="linear dInput (accumulated)")
    for seq, out, emb in [(4, 8, 6), (16, 32, 16)]:
        dl, xin, wo = synth.normal(7, (seq, out)), synth.normal(8, (seq, emb)), synth.normal(9, (out, emb))
        wg0, bg0 = synth.normal(10, (out, emb)), synth.normal(11, (out,))
        dxo, wgo, bgo = O.backprop_output_projection(dl, xin, wo, wg0, bg0)
        DL, XI, WO = (a.astype(np.float64) for a in (dl, xin, wo))
        close(dxo, DL @ WO, what="output dX")
        close(wgo, wg0 + DL.T @ XI, what="output weightGrad")
        close(bgo, bg0 + DL.sum(0), what="output biasGrad")
