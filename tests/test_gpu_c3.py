"""Parity of the c3 configuration beyond the attention core: the fused QKV +
RoPE projection at its full shape and the whole 12-layer decoder stack the
headline is quoted on (4 sequences x 4096 tokens, D 1024, 16 heads x 64,
FF 4096, post-LN blocks; TransformerBlock.cs:35-44, MultiHeadAttention.cs:108-111).

The oracle cannot run the full stack in test time, so the full-size run is
checked through properties that do not depend on size: the causal prefix
property (rows 0..P-1 of a sequence depend only on its first P inputs, so
they must equal the stack run on those P rows alone), and a 256-token prefix
through all 12 layers against the multi-threaded oracle composition.
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
