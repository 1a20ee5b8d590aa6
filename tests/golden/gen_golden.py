"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/gen_golden.py).

Every expected output here is computed in float64 by the textbook definition
of the operation, written with numpy matrix algebra (not the reference's
per-row loops), on the reference test suite's closed-form inputs
(AccelerationManagerParityTests.cs:2180-2205) and on seeded SplitMix64 inputs.
The oracle in oracle/ restates the reference's float32 loops; the tests
compare the two, so a dropped term, a transposed operand or a wrong index in
the oracle fails against these files.

Cases follow the reference tests that cover the path:
  ScaledDotProductAttention  AccelerationManagerParityTests.cs:386-459, 1188-1201
  MultiHeadAttentionForward  :354-355, 1196-1198
  ProjectQKV                 :461-500, 1203-1218
  ProjectOutputBatch         :755
  EmbedTokenIds              :768
  RoPE                       :1087-1112
  Softmax / LayerNorm        :313-324
and a tiny decoder-only LanguageModel (vocab 12, D 8, 2 heads, 1 layer,
FF 16, MultiTypeTransformerTests.cs:730-741) plus a config-1-shaped model
(vocab 200, D 64, 4 heads, 2 layers, FF 128), whose logits come from a float64
restatement of LanguageModel.Forward and whose greedy continuation comes from
recomputing the full prefix each step (no KV cache).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "callaghandev.ml_amd"))

from cdml import synth  # noqa: E402

M, Vec, PV = synth.matrix, synth.vector, synth.positive_vector


# ---------------------------------------------------------------- textbook ops
def t_linear(x, w, b):
    return x.astype(np.float64) @ w.astype(np.float64).T + b.astype(np.float64)


def t_softmax(s, allowed):
    s = np.where(allowed, s, -np.inf)
    mx = s.max(axis=-1, keepdims=True)
    ok = np.isfinite(mx)
    e = np.where(allowed, np.exp(s - np.where(ok, mx, 0.0)), 0.0)
    z = e.sum(axis=-1, keepdims=True)
    return np.where(z > 0, e / np.where(z > 0, z, 1.0), 0.0)


def t_attention(q, k, v, heads, scale, mask=None, causal=False):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    lq, d = q.shape
    lk = k.shape[0]
    hd = d // heads
    allowed = np.ones((lq, lk), bool)
    if mask is not None:
        allowed &= mask.astype(bool)
    if causal:
        allowed &= np.tril(np.ones((lq, lk), bool))
    out = np.zeros((lq, d))
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        p = t_softmax(q[:, sl] @ k[:, sl].T * scale, allowed)
        out[:, sl] = p @ v[:, sl]
    return out


def t_rope(x, heads, base=10000.0, inverse=False, pos=None):
    x = x.astype(np.float64)
    rows, d = x.shape
    hd = d // heads
    p = np.arange(hd // 2)
    pos = np.arange(rows, dtype=np.float64) if pos is None else np.asarray(pos, np.float64)
    theta = pos[:, None] / np.power(base, 2.0 * p / hd)[None, :]
    c, s = np.cos(theta), np.sin(theta)
    if inverse:
        s = -s
    y = x.copy()
    for h in range(heads):
        e = h * hd + 2 * p
        x0, x1 = x[:, e], x[:, e + 1]
        y[:, e] = x0 * c - x1 * s
        y[:, e + 1] = x0 * s + x1 * c
    return y


def t_layernorm(x, g, b, eps=1e-5):
    x = x.astype(np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g.astype(np.float64) + b.astype(np.float64)


def t_lm_hidden(cfg, w, emb):
    x = emb.astype(np.float64)
    H = cfg["heads"]
    hd = cfg["dim"] // H
    for L in w["layers"]:
        q = t_rope(t_linear(x, L["wq"], L["bq"]), H)
        k = t_rope(t_linear(x, L["wk"], L["bk"]), H)
        v = t_linear(x, L["wv"], L["bv"])
        a = t_linear(t_attention(q, k, v, H, 1.0 / np.sqrt(hd), causal=True), L["wo"], L["bo"])
        h = t_layernorm(x + a, L["ln1_g"], L["ln1_b"])
        f = t_linear(np.maximum(t_linear(h, L["ffn_w1"], L["ffn_b1"]), 0.0), L["ffn_w2"], L["ffn_b2"])
        x = t_layernorm(h + f, L["ln2_g"], L["ln2_b"])
    return x


def t_lm_forward(cfg, w, ids):
    emb = w["token_embedding"][ids]
    return t_linear(t_lm_hidden(cfg, w, emb), w["out_proj"], w["out_bias"])


def t_lm_greedy(cfg, w, prompt, max_new):
    toks = list(int(t) for t in prompt)
    margins = []
    for _ in range(max_new):
        if len(toks) >= cfg["max_seq"]:
            break
        logits = t_lm_forward(cfg, w, np.array(toks))[-1]
        order = np.argsort(-logits, kind="stable")
        margins.append(float(logits[order[0]] - logits[order[1]]))
        toks.append(int(order[0]))
    return np.array(toks, np.int32), np.array(margins)


# ------------------------------------------------------------------- fixtures
def main():
    f = {}
    # ScaledDotProductAttention cases (AccelerationManagerParityTests.cs:386-459).
    qs, ks, vs = M(4, 8, 118), M(4, 8, 119), M(4, 8, 120)
    self_mask = np.array([[1, 0, 1, 0], [1, 1, 0, 0], [0, 1, 1, 0], [1, 1, 1, 1]], np.uint8)
    qc, kc, vc = M(4, 8, 121), M(5, 8, 122), M(5, 8, 123)
    cross_mask = np.array([[1, 0, 1, 0, 1], [1, 1, 0, 1, 0], [0, 1, 1, 0, 1], [1, 0, 0, 1, 1]], np.uint8)
    all_masked = cross_mask.copy()
    all_masked[0] = 0
    all_masked[1] = [1, 1, 0, 1, 0]
    sc = 1.0 / np.sqrt(np.float32(4))
    f["sdpa_self_nomask"] = t_attention(qs, ks, vs, 2, sc)
    f["sdpa_self_mask"] = t_attention(qs, ks, vs, 2, sc, mask=self_mask)
    f["sdpa_self_causal"] = t_attention(qs, ks, vs, 2, sc, causal=True)
    f["sdpa_cross_nomask"] = t_attention(qc, kc, vc, 2, sc)
    f["sdpa_cross_mask"] = t_attention(qc, kc, vc, 2, sc, mask=cross_mask)
    f["sdpa_cross_allmasked"] = t_attention(qc, kc, vc, 2, sc, mask=all_masked)
    f["self_mask"], f["cross_mask"], f["all_masked_mask"] = self_mask, cross_mask, all_masked

    # MultiHeadAttentionForward with a causal mask (:354-355), 2 heads, d_h = 3.
    q6, k6, v6 = M(4, 6, 31), M(4, 6, 32), M(4, 6, 33)
    f["mha_causal_scale"] = np.float32(1.0 / np.sqrt(np.float32(3.0)))
    f["mha_causal"] = t_attention(q6, k6, v6, 2, float(f["mha_causal_scale"]),
                                  mask=np.tril(np.ones((4, 4), np.uint8)))

    # GPU-size attention paths (:1188-1201): seq 128, D 64, 4 heads.
    qg, kg, vg = M(128, 64, 110), M(128, 64, 111), M(128, 64, 112)
    f["mha128_nomask"] = t_attention(qg, kg, vg, 4, 1.0 / np.sqrt(16.0))
    f["mha128_causal"] = t_attention(qg, kg, vg, 4, 1.0 / np.sqrt(16.0), causal=True)

    # One c2-sized head slice: config 2 (B 16 x L 1024, D 512, 8 heads) is 128
    # independent causal (sequence, head) problems of L 1024 x d_h 64.
    qh, kh, vh = (synth.normal(900 + i, (1024, 64)) for i in range(3))
    f["c2_head_causal"] = t_attention(qh, kh, vh, 1, 1.0 / 8.0, causal=True)

    # ProjectQKV (:461-500) and the GPU-size case (:1203-1218).
    x = M(6, 5, 124)
    f["qkv_small_q"] = t_linear(x, M(8, 5, 125), Vec(8, 128))
    f["qkv_small_k"] = t_linear(x, M(8, 5, 126), Vec(8, 129))
    f["qkv_small_v"] = t_linear(x, M(8, 5, 127), Vec(8, 130))
    xg = M(192, 128, 142)
    f["qkv_big_q"] = t_linear(xg, M(128, 128, 143), Vec(128, 146))
    f["qkv_big_k"] = t_linear(xg, M(128, 128, 144), Vec(128, 147))
    f["qkv_big_v"] = t_linear(xg, M(128, 128, 145), Vec(128, 148))

    # ProjectOutputBatch (:755) and EmbedTokenIds (:768).
    f["project_output"] = t_linear(M(4, 6, 56), M(3, 6, 57), Vec(3, 58))
    f["embed"] = M(6, 5, 64)[[0, 2, 4]].astype(np.float64)

    # RoPE (:1087-1112): all heads, one head (startCol 2, headDim 4).
    r = M(4, 8, 97)
    f["rope_all"] = t_rope(r, 2)
    head = r.astype(np.float64).copy()
    head[:, 2:6] = t_rope(r[:, 2:6], 1)
    f["rope_head"] = head
    f["rope_long"] = t_rope(M(300, 32, 7), 4)

    # Softmax (:313-324) and LayerNorm (:326-329).
    s = M(4, 4, 26)
    sm_mask = np.array([[1, 0, 0, 0], [1, 1, 0, 0], [1, 0, 1, 0], [1, 1, 1, 1]], np.uint8)
    f["softmax_nomask"] = t_softmax(s.astype(np.float64), np.ones((4, 4), bool))
    f["softmax_mask"] = t_softmax(s.astype(np.float64), sm_mask.astype(bool))
    f["softmax_mask_in"] = sm_mask
    f["layernorm"] = t_layernorm(M(5, 6, 27), PV(6, 28), Vec(6, 29))

    # Expected outputs are stored rounded to float32 (half an ulp, far below
    # every tolerance the tests use) to keep the fixture small.
    f = {k: (v.astype(np.float32) if v.dtype == np.float64 else v) for k, v in f.items()}
    np.savez_compressed(os.path.join(HERE, "ops.npz"), **f)

    # Tiny decoder-only LanguageModels.
    for name, cfg, seed, n_ids, prompt_len, n_new in (
        ("lm_tiny", dict(vocab=12, dim=8, heads=2, layers=1, ff=16, max_seq=32), 42, 10, 5, 12),
        ("lm_c1", dict(vocab=200, dim=64, heads=4, layers=2, ff=128, max_seq=64), 7, 64, 32, 20),
    ):
        w = synth.lm_weights(cfg, seed, biased=True)
        ids = synth.token_ids(seed + 1, n_ids, cfg["vocab"])
        logits = t_lm_forward(cfg, w, ids)
        gen, margins = t_lm_greedy(cfg, w, ids[:prompt_len], n_new)
        # Weights are regenerated from (cfg, seed) by cdml.synth.lm_weights(biased=True).
        out = dict(cfg_keys=np.array(list(cfg.keys())), cfg_vals=np.array(list(cfg.values())),
                   seed=seed, ids=ids, logits=logits.astype(np.float32), prompt_len=prompt_len, n_new=n_new,
                   greedy=gen, greedy_margins=margins)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
