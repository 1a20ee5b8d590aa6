"""Parity of the c3 configuration beyond the attention core: the fused QKV +
RoPE projection at its full shape and the whole 12-layer decoder stack the
headline is quoted on (4 sequences x 4096 tokens, D 1024, 16 heads x 64,
FF 4096, post-LN blocks; TransformerBlock.cs:35-44, MultiHeadAttention.cs:108-111).

The oracle cannot run the full stack in test time, so the full-size run is
checked through properties that do not depend on size: the causal prefix
property (rows 0..P-1 of a sequence depend only on its first P inputs, so
they must equal the stack run on those P rows alone), and a 256-token prefix
through all 12 layers against the multi-threaded oracle composition.  One
whole 4096-token sequence is also recomputed through all 12 layers in
float64 numpy (BLAS), so the deep rows, whose attention spans thousands of
keys, meet the bar against exact arithmetic.
"""
from __future__ import annotations

import numpy as np
import pytest

from cdml import host, synth
from oracle import oracle as O

from abi_ops import project_qkv_rope
from conftest import assert_parity as parity

pytestmark = pytest.mark.gpu

C3 = {"dim": 1024, "heads": 16, "layers": 12, "ff": 4096, "max_seq": 4096, "discrete": False,
      "input_dim": 1024, "output_dim": 1}
B, L = 4, 4096


@pytest.fixture(scope="module")
def c3_stack():
    w = synth.continuous_lm_weights(C3, 41, biased=True)
    lm, mgr = host.language_model(C3, w)
    dev = host.module().DeviceLanguageModel(lm, B)
    x = np.random.default_rng(6).standard_normal((B * L, C3["dim"]), dtype=np.float32)
    print("[c3] full stack 4 x 4096, 12 layers", flush=True)
    out = dev.Layers(x, B, L)
    return w, dev, x, out, (lm, mgr)


def _oracle_layers(w, h, heads):
    """The 12 post-LN blocks from the multi-threaded oracle functions
    (TransformerBlock.Forward: MHA, residual LN, FFN [D, FF, D] ReLU, residual LN)."""
    for Lw in w["layers"]:
        q, k, v = O.project_qkv(h, Lw["wq"], Lw["bq"], Lw["wk"], Lw["bk"], Lw["wv"], Lw["bv"], mt=True)
        a = O.sdpa(O.rope(q, heads, mt=True), O.rope(k, heads, mt=True), v, heads, causal=True, mt=True)
        n1 = O.residual_layernorm(h, O.project_output_batch(a, Lw["wo"], Lw["bo"], mt=True),
                                  Lw["ln1_g"], Lw["ln1_b"], mt=True)
        f = O.activation(O.batch_dot_add_bias(Lw["ffn_w1"], n1, Lw["ffn_b1"], mt=True), 3)
        f = O.batch_dot_add_bias(Lw["ffn_w2"], f, Lw["ffn_b2"], mt=True)
        h = O.residual_layernorm(n1, f, Lw["ln2_g"], Lw["ln2_b"], mt=True)
    return h


def test_c3_stack_output_is_finite_and_normalised(c3_stack):
    _, _, _, out, _ = c3_stack
    assert out.shape == (B * L, C3["dim"])
    assert np.all(np.isfinite(out))
    # the last block ends in a LayerNorm with gamma ~ 1, beta ~ 0 per row
    m = out.mean(axis=1)
    assert np.abs(m).max() < 0.5


@pytest.mark.parametrize("b", [0, 1, 2, 3])
def test_c3_stack_causal_prefix_property(c3_stack, b):
    """Rows 0..511 of sequence b of the full 4 x 4096 run equal the stack run on
    those 512 rows alone (every kernel shape differs between the two runs)."""
    _, dev, x, out, _ = c3_stack
    P = 512
    print(f"[c3] prefix property, sequence {b}", flush=True)
    pre = dev.Layers(np.ascontiguousarray(x[b * L:b * L + P]), 1, P)
    parity(out[b * L:b * L + P], pre, what=f"c3 stack rows 0..{P - 1} of sequence {b} vs the prefix alone")


def test_c3_stack_prefix_vs_oracle(c3_stack):
    """A 256-token prefix of sequence 2 through all 12 layers on the device
    engine against the multi-threaded oracle composition."""
    w, dev, x, out, _ = c3_stack
    P, b = 256, 2
    print("[c3] 256-token prefix vs the oracle (12 layers)", flush=True)
    want = _oracle_layers(w, np.ascontiguousarray(x[b * L:b * L + P]), C3["heads"])
    parity(out[b * L:b * L + P], want, what="c3 stack, 256-token prefix of sequence 2 vs oracle")


def _float64_layers(w, x, heads):
    """The post-LN decoder blocks (TransformerBlock.Forward, TransformerBlock.cs:
    35-44; MultiHeadAttention.Forward, MultiHeadAttention.cs:96-159) in float64
    numpy: QKV with biases, interleaved RoPE base 10000, causal softmax
    attention with scale 1/sqrt(d_h), output projection, residual LayerNorm
    (eps 1e-5, biased variance), FFN [D, FF, D] with ReLU, residual LayerNorm.

    The RoPE angle is the reference's own fp32 quantity, theta =
    fp32(pos / fp32(10000^fp32(2p/d_h))) (AccelerationCPU.cs:4947-4962): at
    position 4095 a last-bit change of the denominator moves theta by
    2e-4 rad, so the angle is taken exactly as the reference defines it and
    only its cosine and sine are evaluated in float64."""
    f8 = np.float64
    n, D = x.shape
    hd = D // heads
    e = (np.float32(2) * np.arange(hd // 2, dtype=np.float32)) / np.float32(hd)
    denom = (f8(10000.0) ** e.astype(f8)).astype(np.float32)
    theta = (np.arange(n, dtype=np.float32)[:, None] / denom[None, :]).astype(f8)  # fp32 division
    cs, sn = np.tile(np.cos(theta), heads), np.tile(np.sin(theta), heads)
    neg = np.where(np.triu(np.ones((n, n), bool), 1), -np.inf, 0.0)  # keys j > i masked

    def ln(r, g, b):
        mu = r.mean(axis=1, keepdims=True)
        var = ((r - mu) ** 2).mean(axis=1, keepdims=True)
        return (r - mu) / np.sqrt(var + 1e-5) * g.astype(f8) + b.astype(f8)

    h = x.astype(f8)
    for li, Lw in enumerate(w["layers"]):
        print(f"[c3] float64 layer {li}", flush=True)
        q, k, v = (h @ Lw[wn].astype(f8).T + Lw[bn].astype(f8)
                   for wn, bn in (("wq", "bq"), ("wk", "bk"), ("wv", "bv")))
        for t in (q, k):
            a, b = t[:, 0::2].copy(), t[:, 1::2].copy()
            t[:, 0::2], t[:, 1::2] = a * cs - b * sn, a * sn + b * cs
        att = np.empty_like(q)
        for hh in range(heads):
            c = slice(hh * hd, (hh + 1) * hd)
            sc = q[:, c] @ k[:, c].T
            sc /= np.sqrt(f8(hd))
            sc += neg
            sc -= sc.max(axis=1, keepdims=True)
            np.exp(sc, out=sc)
            att[:, c] = (sc @ v[:, c]) / sc.sum(axis=1, keepdims=True)
            del sc
        n1 = ln(h + att @ Lw["wo"].astype(f8).T + Lw["bo"].astype(f8), Lw["ln1_g"], Lw["ln1_b"])
        f = np.maximum(n1 @ Lw["ffn_w1"].astype(f8).T + Lw["ffn_b1"].astype(f8), 0.0)
        h = ln(n1 + f @ Lw["ffn_w2"].astype(f8).T + Lw["ffn_b2"].astype(f8), Lw["ln2_g"], Lw["ln2_b"])
    return h


def test_c3_stack_full_sequence_vs_float64(c3_stack):
    """Sequence 3 of the 4 x 4096 run, all 4096 rows through all 12 layers,
    against the float64 composition: every row meets the bar, the deep rows
    3840..4095 (attention over up to 4096 keys in every layer) included."""
    w, _, x, out, _ = c3_stack
    b = 3
    print("[c3] full 4096-token sequence vs float64 (12 layers)", flush=True)
    want = _float64_layers(w, x[b * L:(b + 1) * L], C3["heads"])
    got = out[b * L:(b + 1) * L]
    deep = slice(L - 256, L)
    print(f"[c3] max abs err: all rows {np.abs(got - want).max():.3e}, rows 3840..4095 "
          f"{np.abs(got[deep] - want[deep]).max():.3e}", flush=True)
    parity(got[deep], want[deep], what="c3 stack rows 3840..4095 of sequence 3 vs float64")
    parity(got, want, what="c3 stack, all 4096 rows of sequence 3 vs float64")


def test_project_qkv_rope_c3_full_shape_sampled():
    """cdml_project_qkv_rope at c3's 16384 x 1024 -> 3 x 1024 with per-sequence
    positions (seg_len 4096), sampled row blocks against O.project_qkv + O.rope
    (MultiHeadAttention.cs:108-110); the blocks include sequence starts, the
    boundary between sequences and the last positions."""
    D, H = 1024, 16
    hd = D // H
    rng = np.random.default_rng(11)
    x = rng.standard_normal((B * L, D), dtype=np.float32)
    ws = [synth.xavier_uniform(70 + i, D, D) for i in range(3)]
    bs = [np.float32(0.05) * synth.normal(80 + i, (D,)) for i in range(3)]
    print("[c3] fused QKV + RoPE at 16384 x 1024", flush=True)
    q, k, v = project_qkv_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], hd, n_pos=L, seg_len=L)

    def rope_at(m, pos0):
        # RoPE is row-local: rotate rows at positions pos0.. by padding the
        # rows before them (zero rows, discarded)
        return O.rope(np.concatenate([np.zeros((pos0, D), np.float32), m]), H)[pos0:]

    for r0 in (0, L - 48, L, 2 * L + 1000, B * L - 64):
        rows = slice(r0, r0 + 64)
        qo, ko, vo = O.project_qkv(x[rows], ws[0], bs[0], ws[1], bs[1], ws[2], bs[2])
        # rows of the block split where a sequence ends (positions restart at 0)
        cut = min(64, L - r0 % L)
        qr, kr = rope_at(qo[:cut], r0 % L), rope_at(ko[:cut], r0 % L)
        if cut < 64:
            qr = np.concatenate([qr, rope_at(qo[cut:], 0)])
            kr = np.concatenate([kr, rope_at(ko[cut:], 0)])
        parity(q[rows], qr, what=f"Q rows {r0}..{r0 + 63}")
        parity(k[rows], kr, what=f"K rows {r0}..{r0 + 63}")
        parity(v[rows], vo, what=f"V rows {r0}..{r0 + 63}")
