"""GPU parity of every C-ABI kernel against the CPU oracle (run on the MI355X).

Bar: per element |gpu - oracle| <= 1e-4 + 1e-3 |oracle| (the north-star
tolerance, fp32), and bit-exact for the gather / copy kernels.  Cases mirror
the reference's own parity suite (AccelerationManagerParityTests.cs) plus the
BASELINE shapes, ragged lengths and the edge rules (all-masked rows, causal
with Lq != Lk, head dims 3 .. 160).
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

import abi_ops as G
from conftest import assert_parity, assert_parity_with_exact
from oracle import oracle as O
from cdml import native as N
from cdml import synth

pytestmark = pytest.mark.gpu

M, Vec = synth.matrix, synth.vector
ATOL, RTOL = 1e-4, 1e-3


def parity(a, e, what=""):
    assert_parity(a, e, atol=ATOL, rtol=RTOL, what=what)


def setup_module(module):
    N.init(0)
    info = N.device_info(0)
    print(f"\n[device] {info['name']} {info['arch']} CUs={info['compute_units']} "
          f"sclk={info['max_clock_mhz']}MHz", flush=True)


# ------------------------------------------------------------- projections
def test_project_qkv_reference_cases():
    x = M(6, 5, 124)
    args = (M(8, 5, 125), Vec(8, 128), M(8, 5, 126), Vec(8, 129), M(8, 5, 127), Vec(8, 130))
    for got, want, n in zip(G.project_qkv(x, *args), O.project_qkv(x, *args), "QKV"):
        parity(got, want, f"ProjectQKV 6x5->8 {n}")
    xg = M(192, 128, 142)
    args = (M(128, 128, 143), Vec(128, 146), M(128, 128, 144), Vec(128, 147), M(128, 128, 145), Vec(128, 148))
    for got, want, n in zip(G.project_qkv(xg, *args), O.project_qkv(xg, *args), "QKV"):
        parity(got, want, f"ProjectQKV 192x128->128 {n}")


@pytest.mark.parametrize("rows,ind,out", [(1, 64, 64), (33, 96, 200), (130, 257, 129), (1024, 512, 512),
                                          (300, 1024, 1024)])
def test_project_qkv_shapes(rows, ind, out):
    x = synth.normal(rows * 7 + ind, (rows, ind))
    w = [synth.xavier_uniform(i + out, out, ind) for i in range(3)]
    b = [synth.normal(9 + i, (out,)) * np.float32(0.1) for i in range(3)]
    args = (w[0], b[0], w[1], b[1], w[2], b[2])
    for got, want, n in zip(G.project_qkv(x, *args), O.project_qkv(x, *args, mt=True), "QKV"):
        parity(got, want, f"ProjectQKV {rows}x{ind}->{out} {n}")


@pytest.mark.parametrize("act", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("rows,ind,out", [(77, 64, 130), (300, 5, 256), (40, 16, 33), (3, 5, 7), (9, 12, 70),
                                          (1024, 64, 256),    # 128x128 tiles (256x128 would not fill a round)
                                          (300, 128, 256),    # 128x128 tiles, full and ragged wave blocks
                                          (16384, 64, 1024),  # 512 tiles of 256x128, every wave block full
                                          (16484, 64, 1000),  # 256x128 tiles, ragged last row and column tiles
                                          (20000, 256, 1),    # regression head: 16 lanes per row
                                          (5003, 132, 3),     # few columns, ragged K / 64
                                          (20000, 5, 256),    # input projection: 4 rows per pass
                                          (3001, 3, 1000),    # short K, one row per pass
                                          (500, 7, 2000)])    # short K, too wide for the register path
def test_linear_with_activation(act, rows, ind, out):
    """BatchDotProductAddBias + activation on both tile configurations, a
    short reduction (the input projection of F 5 features, K 16) and few rows."""
    x = synth.normal(3, (rows, ind))
    w = synth.xavier_uniform(4, out, ind)
    b = synth.normal(5, (out,))
    want = O.activation(O.batch_dot_add_bias(w, x, b, mt=rows > 4096), act)
    parity(G.linear(x, w, b, act), want, f"linear {rows}x{ind}->{out} act={act}")


@pytest.mark.parametrize("rows,ind,out,act", [(1024, 128, 256, 3), (300, 64, 160, 5), (2048, 256, 384, 0),
                                              (16384, 64, 1024, 3),   # 256x128 tiles
                                              (5000, 64, 3, 1),       # few columns
                                              (5000, 5, 256, 3)])     # short K
def test_linear_row_strides(rows, ind, out, act):
    """cdml_linear with row strides above the widths (ldx = in + 8, ldy = out + 12):
    the full wave blocks of the unpredicated epilogue and the ragged ones give
    the oracle's result, and the stride padding of y keeps its sentinel."""
    ldx, ldy = ind + 8, out + 12
    x = synth.normal(31, (rows, ind))
    w = synth.xavier_uniform(32, out, ind)
    b = synth.normal(33, (out,))
    xp = np.zeros((rows, ldx), np.float32)
    xp[:, :ind] = x
    yp = np.full((rows, ldy), 7.5, np.float32)
    bx, bw, bb, by = G.up(xp), G.up(w), G.up(b), G.up(yp)
    N.check(N.lib().cdml_linear(bx.ptr, ldx, bw.ptr, bb.ptr, by.ptr, ldy, rows, ind, out, act, G.stream().handle))
    got = G.down(by, (rows, ldy))
    assert np.all(got[:, out:] == 7.5), "cdml_linear wrote into the row stride padding"
    parity(got[:, :out], O.activation(O.batch_dot_add_bias(w, x, b, mt=rows > 4096), act),
           f"strided linear {rows}x{ind}->{out}")


def test_project_output_batch_reference_case():
    parity(G.linear(M(4, 6, 56), M(3, 6, 57), Vec(3, 58)),
           O.project_output_batch(M(4, 6, 56), M(3, 6, 57), Vec(3, 58)), "ProjectOutputBatch")
    # MatrixMultiplyTranspose known answers 17 / 23 / 67 (MultiTypeTransformerTests.cs:664-674)
    c = G.linear(np.array([[1, 2], [3, 4]], np.float32), np.array([[5, 6], [7, 8], [9, 10]], np.float32), None)
    assert c[0, 0] == 17 and c[0, 1] == 23 and c[1, 2] == 67


# -------------------------------------------------------------------- RoPE
def test_rope_reference_cases():
    m = M(4, 8, 97)
    parity(G.rope(m, 2), O.rope(m, 2), "RoPE all heads")
    parity(G.rope(m, start_col=2, head_dim=4, num_heads=1), O.rope_head(m, 2, 4), "RoPE one head")
    back = G.rope(G.rope(m, 2), 2, inverse=True)
    assert np.allclose(back, m, atol=5e-4)
    y = G.rope(np.array([[1, 0], [1, 0], [0, 1]], np.float32), 1)
    assert np.allclose(y[1], [math.cos(1), math.sin(1)], atol=1e-5)
    assert np.allclose(y[2], [-math.sin(2), math.cos(2)], atol=1e-5)


@pytest.mark.parametrize("rows,dim,heads", [(4096, 1024, 16), (512, 256, 8), (64, 64, 4), (100, 2048, 16)])
def test_rope_long_positions(rows, dim, heads):
    x = synth.normal(rows + dim, (rows, dim))
    parity(G.rope(x, heads), O.rope(x, heads, mt=True), f"RoPE {rows}x{dim}/{heads}")


def test_rope_segmented_and_absolute_positions():
    x = synth.normal(1, (3 * 50, 64))
    want = np.concatenate([O.rope(x[i * 50:(i + 1) * 50], 4) for i in range(3)])
    parity(G.rope(x, 4, seg_len=50), want, "RoPE segmented")
    pos = np.array([0, 7, 4095, 123], np.int32)
    xr = synth.normal(2, (4, 64))
    want = np.stack([O.rope(np.vstack([np.zeros((p, 64), np.float32), xr[i:i + 1]]), 4)[-1]
                     for i, p in enumerate(pos)])
    parity(G.rope(xr, 4, positions=pos), want, "RoPE absolute positions")


@pytest.mark.parametrize("rows,ld,hd,heads,seg,off,inv", [
    (300, 128, 32, 4, 100, 0, 1),    # the trainer's inverse over 100-row segments, two pairs per thread
    (300, 132, 32, 4, 0, 7, 0),      # row longer than the heads, position offset, forward
    (2044, 256, 32, 8, 511, 0, 1),   # eight 511-row windows of the config-5 model
    (77, 36, 6, 6, 0, 0, 1),         # head dim 6: one pair per thread
    (50, 66, 64, 1, 16, 3, 1),       # odd row pitch: one pair per thread
])
def test_rope_qk_table_equals_rope(rows, ld, hd, heads, seg, off, inv):
    """ApplySegmentedRotaryInPlace (TransformerTrainer.cs:811-848) from the
    table: the same bits as cdml_rope on each matrix, columns past the heads
    untouched; the known answers of cdml_rope pin those bits."""
    q, k = synth.normal(rows + ld, (rows, ld)), synth.normal(rows + ld + 1, (rows, ld))
    n_pos = off + (min(seg, rows) if seg else rows)
    gq, gk = G.rope_qk_table(q, k, hd, heads, n_pos, off, seg, inv)
    for got, x, n in ((gq, q, "Q"), (gk, k, "K")):
        want = G.rope(x, heads, head_dim=hd, inverse=bool(inv), pos_offset=off, seg_len=seg)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{n} {rows}x{ld} hd {hd}"
        assert np.array_equal(got[:, heads * hd:], x[:, heads * hd:])
    only_q, none = G.rope_qk_table(q, None, hd, heads, n_pos, off, seg, inv)
    assert none is None and np.array_equal(only_q, gq)


def test_rope_table_values():
    cs = G.rope_table(4096, 64)
    # position 1, pair 0: theta = 1 (the known answer of the reference's RoPE tests)
    assert np.allclose(cs[1, 0], [math.cos(1), math.sin(1)], atol=1e-6)
    assert np.array_equal(cs[0], np.tile([1.0, 0.0], (32, 1)).astype(np.float32))
    # every entry against float64 cos/sin of the float32 angle pos / powf(base, 2p/d)
    denom = np.array([np.float32(10000.0) ** (np.float32(2 * p) / np.float32(64)) for p in range(32)],
                     np.float32)
    theta = (np.arange(4096, dtype=np.float32)[:, None] / denom[None, :]).astype(np.float64)
    assert np.abs(cs[..., 0] - np.cos(theta)).max() < 2e-6
    assert np.abs(cs[..., 1] - np.sin(theta)).max() < 2e-6


@pytest.mark.parametrize("rows,ind,out,hd,seg,off", [
    (1024, 512, 512, 64, 0, 0),    # 128x128 tiles (256x128 would not fill a round)
    (16384, 64, 384, 64, 1024, 0),  # 576 tiles of 256x128 over 1024-row sequences, full wave blocks
    (16484, 64, 384, 32, 0, 3),    # 256x128 tiles, ragged last row tile, position offset
    (16384, 64, 384, 16, 512, 0),  # 256x128 tiles, head dim 16, table staged in LDS
    (16384, 32, 384, 8, 0, 7),     # 256x128 tiles, head dim 8, position offset
    (16384, 64, 384, 64, 640, 0),  # 256x128 tiles inside one segment (LDS table) and across two (per row)
    (300, 1024, 1024, 64, 0, 0),   # 128x128 tiles, ragged rows
    (150, 64, 64, 16, 50, 0),      # segmented positions (row % 50)
    (1024, 256, 256, 32, 256, 0),  # segments of whole 32-row blocks, full tiles (unpredicated epilogue)
    (1000, 128, 384, 64, 96, 5),   # block-aligned segments, ragged last tile, position offset
    (600, 64, 128, 32, 40, 0),     # 128x128 tiles, blocks across segment boundaries
    (40, 96, 192, 32, 0, 17),      # position offset
    (33, 130, 36, 12, 0, 0),       # generic kernel (K not a multiple of 4)
])
def test_project_qkv_rope(rows, ind, out, hd, seg, off):
    x = synth.normal(rows + ind, (rows, ind))
    w = [synth.xavier_uniform(i + out, out, ind) for i in range(3)]
    b = [synth.normal(19 + i, (out,)) * np.float32(0.1) for i in range(3)]
    args = (w[0], b[0], w[1], b[1], w[2], b[2])
    q, k, v = G.project_qkv_rope(x, *args, head_dim=hd, pos_offset=off, seg_len=seg)
    wq, wk, wv = O.project_qkv(x, *args, mt=True)
    heads = out // hd

    def at_offset(t):  # positions off, off + 1, ... (the reference rotates positions 0, 1, ...)
        return O.rope(np.vstack([np.zeros((off, out), np.float32), t]), heads)[off:] if off else O.rope(t, heads)

    def rotated(t):
        if seg:  # positions off + (row % seg)
            return np.concatenate([at_offset(t[i:i + seg]) for i in range(0, rows, seg)])
        return at_offset(t)

    parity(q, rotated(wq), f"QKV+RoPE {rows}x{ind}->{out} Q")
    parity(k, rotated(wk), f"QKV+RoPE {rows}x{ind}->{out} K")
    parity(v, wv, f"QKV+RoPE {rows}x{ind}->{out} V")
    # the epilogue's rotation is the in-place kernel's, bit for bit
    pq, pk, pv = G.project_qkv(x, *args)
    for got, plain, n in ((q, pq, "Q"), (k, pk, "K")):
        want = G.rope(plain, heads, head_dim=hd, pos_offset=off, seg_len=seg)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{n}: epilogue RoPE != cdml_rope"
    assert np.array_equal(v, pv)


# ------------------------------------------------------- projection gradients
def test_backprop_qkv_reference_case():
    """BackpropQKV on the closed-form inputs of AccelerationManagerParityTests.cs:462-537."""
    x = M(6, 5, 124)
    w = (M(8, 5, 125), M(8, 5, 126), M(8, 5, 127))
    d = (M(6, 8, 131), M(6, 8, 132), M(6, 8, 133))
    g0 = (M(8, 5, 134), Vec(8, 137), M(8, 5, 135), Vec(8, 138), M(8, 5, 136), Vec(8, 139))
    got = G.backprop_qkv(x, *d, *w, *g0)
    want = O.backprop_qkv(x, *d, *w, *g0)
    for a, e, n in zip(got, want, ["dInput", "WQGrad", "biasQGrad", "WKGrad", "biasKGrad", "WVGrad", "biasVGrad"]):
        parity(a, e, f"BackpropQKV {n}")


@pytest.mark.parametrize("rows,ind,out", [(1024, 512, 512),   # tiled kernels (128-row tiles)
                                          (2048, 256, 1024),  # 256-row tiles for W_grad
                                          (656, 256, 256),    # split K with a short last chunk
                                          (1000, 256, 512),   # split K plus a ragged 8-row tail
                                          (300, 1024, 96),    # K = 300 rows: generic W_grad kernel
                                          (130, 257, 129),    # ragged everywhere
                                          (1, 64, 64)])
def test_backprop_qkv_shapes(rows, ind, out):
    x = synth.normal(rows + ind, (rows, ind))
    w = [synth.xavier_uniform(i + out, out, ind) for i in range(3)]
    d = [synth.normal(50 + i, (rows, out)) for i in range(3)]
    g0 = [synth.normal(60, (out, ind)), synth.normal(61, (out,)), synth.normal(62, (out, ind)),
          synth.normal(63, (out,)), synth.normal(64, (out, ind)), synth.normal(65, (out,))]
    got = G.backprop_qkv(x, *d, *w, *g0)
    want = O.backprop_qkv(x, *d, *w, *g0)
    X, Dd = x.astype(np.float64), [a.astype(np.float64) for a in d]
    exact = [sum(Di @ Wi.astype(np.float64) for Di, Wi in zip(Dd, w))]
    for i in range(3):
        exact += [g0[2 * i] + Dd[i].T @ X, g0[2 * i + 1] + Dd[i].sum(0)]
    for a, e, e64, n in zip(got, want, exact, ["dInput", "WQGrad", "biasQGrad", "WKGrad", "biasKGrad", "WVGrad",
                                               "biasVGrad"]):
        assert_parity_with_exact(a, e, e64, what=f"BackpropQKV {rows}x{ind}->{out} {n}")


def test_backprop_qkv_c3_shape_float64():
    """One c3 sequence (4096 rows, 1024 -> 1024) against float64 matrix
    algebra: the identities dInput = sum dX W, W_grad += dX^T x and
    b_grad += column sums that the oracle's loops were pinned on."""
    rows, ind, out = 4096, 1024, 1024
    x = synth.normal(1, (rows, ind))
    w = [synth.xavier_uniform(2 + i, out, ind) for i in range(3)]
    d = [synth.normal(5 + i, (rows, out)) * np.float32(0.05) for i in range(3)]
    g0 = [np.zeros((out, ind), np.float32), np.zeros(out, np.float32)] * 3
    dx, wqg, bqg, wkg, bkg, wvg, bvg = G.backprop_qkv(x, *d, *w, *g0)
    X = x.astype(np.float64)
    D = [a.astype(np.float64) for a in d]
    parity(dx, sum(Di @ Wi.astype(np.float64) for Di, Wi in zip(D, w)), "c3 dInput")
    for got_w, got_b, Di, n in [(wqg, bqg, D[0], "Q"), (wkg, bkg, D[1], "K"), (wvg, bvg, D[2], "V")]:
        parity(got_w, Di.T @ X, f"c3 W{n}Grad")
        parity(got_b, Di.sum(0), f"c3 bias{n}Grad")


@pytest.mark.parametrize("rows,ind,out", [(4, 8, 8), (16, 16, 32), (512, 256, 256), (77, 64, 130),
                                          (4112, 128, 1024),   # split K, 257 k-tiles
                                          (4100, 128, 1000),   # split K + 4-row tail; dX with K = 1000
                                          (252, 64, 200),      # the config-1 LM head of one training bucket
                                          (8192, 5, 256),      # input projection: small output, split rows
                                          (8200, 256, 1),      # regression head [1, D]
                                          (5000, 7, 3),        # both small and odd
                                          (6000, 3, 600),      # narrow input side, 600 output rows
                                          (4096, 18, 36)])     # small output, neither side narrow
def test_linear_backward(rows, ind, out):
    """BackpropLinearProjection (dInput accumulates) and BackpropOutputProjection
    (dX overwritten) on the shapes of AccelerationConsistencyTests.cs:633-700,
    1108-1125 and larger tiled ones."""
    x, dy, w = synth.normal(1, (rows, ind)), synth.normal(2, (rows, out)), synth.normal(3, (out, ind))
    wg0, bg0, dx0 = synth.normal(4, (out, ind)), synth.normal(5, (out,)), synth.normal(6, (rows, ind))
    X, DY, W = x.astype(np.float64), dy.astype(np.float64), w.astype(np.float64)
    xwg, xbg, xdx = wg0 + DY.T @ X, bg0 + DY.sum(0), DY @ W
    wg, bg, dx = G.linear_backward(x, dy, w, wg0, bg0, dx=dx0, accumulate=True)
    ewg, ebg, edx = O.backprop_linear_projection(x, dy, w, wg0, bg0, dx0)
    assert_parity_with_exact(wg, ewg, xwg, what="linear weightGrad")
    assert_parity_with_exact(bg, ebg, xbg, what="linear biasGrad")
    assert_parity_with_exact(dx, edx, dx0 + xdx, what="linear dInput")
    wg, bg, dx = G.linear_backward(x, dy, w, wg0, bg0)
    edx, ewg, ebg = O.backprop_output_projection(dy, x, w, wg0, bg0)
    assert_parity_with_exact(dx, edx, xdx, what="output dX")
    assert_parity_with_exact(wg, ewg, xwg, what="output weightGrad")
    assert_parity_with_exact(bg, ebg, xbg, what="output biasGrad")
    wg, bg, none = G.linear_backward(x, dy, w, wg0, bg0, want_dx=False)
    assert none is None
    assert_parity_with_exact(wg, ewg, xwg, what="weightGrad without dX")


def test_weight_gradient_workspace_contract():
    """The split weight-gradient GEMM asks for a workspace and refuses a
    smaller one with CDML_E_INVALID before launching anything; two calls with
    the same inputs give bit-identical gradients (fixed reduction order)."""
    import ctypes as C
    from cdml import native as N
    rows, ind, out = 8192, 256, 256
    need = C.c_size_t(0)
    N.check(N.lib().cdml_linear_backward_workspace_size(rows, ind, out, C.byref(need)))
    assert need.value > 0
    x, dy = synth.normal(7, (rows, ind)), synth.normal(8, (rows, out))
    w = synth.normal(9, (out, ind))
    bx, bdy, bw = (N.DeviceBuffer.from_array(a) for a in (x, dy, w))
    bwg, bbg = N.DeviceBuffer.from_array(np.zeros((out, ind), np.float32)), N.DeviceBuffer.from_array(np.zeros(out, np.float32))
    small = N.DeviceBuffer(need.value // 2)
    rc = N.lib().cdml_linear_backward(bx.ptr, ind, bdy.ptr, out, bw.ptr, None, ind, bwg.ptr, bbg.ptr, rows, ind,
                                      out, 0, small.ptr, need.value // 2, None)
    assert rc == -1 and b"workspace" in N.lib().cdml_last_error()
    g1 = G.linear_backward(x, dy, w, np.zeros((out, ind), np.float32), np.zeros(out, np.float32), want_dx=False)
    g2 = G.linear_backward(x, dy, w, np.zeros((out, ind), np.float32), np.zeros(out, np.float32), want_dx=False)
    assert np.array_equal(g1[0], g2[0]) and np.array_equal(g1[1], g2[1])
    X, DY = x.astype(np.float64), dy.astype(np.float64)
    parity(g1[0], DY.T @ X, "split weightGrad vs float64")
    parity(g1[1], DY.sum(0), "split biasGrad vs float64")


# ------------------------------------------------------- attention backward
@pytest.mark.parametrize("case", ["parity_decoder", "parity_mask", "nomask_6x8", "decoder_6x8", "cross_5x8"])
def test_sdpa_bwd_reference_cases(case):
    """MultiHeadAttentionBackward on the cases of AccelerationManagerParityTests.cs:354-383
    (closed-form 4 x 6, 2 heads, scale 1/sqrt(3), decoder mask and explicit causal mask)
    and AccelerationConsistencyTests.cs:964-1022 (6 x 8 and cross 5 x 8, 2 heads)."""
    if case.startswith("parity"):
        q, k, v, g = M(4, 6, 31), M(4, 6, 32), M(4, 6, 33), M(4, 6, 34)
        heads, scale = 2, float(np.float32(1.0) / np.sqrt(np.float32(3.0)))
    else:
        lq, lk = (5, 8) if case == "cross_5x8" else (6, 6)
        q, k, v = synth.normal(1, (lq, 8)), synth.normal(2, (lk, 8)), synth.normal(3, (lk, 8))
        g = synth.normal(4, (lq, 8))
        heads, scale = 2, 0.5
    if case == "parity_mask":
        mask = O.causal_mask(4)
        got, want = G.sdpa_bwd(q, k, v, g, heads, scale, mask=mask), O.mha_backward(q, k, v, g, heads, scale, mask=mask)
    else:
        causal = "decoder" in case
        got = G.sdpa_bwd(q, k, v, g, heads, scale, causal=causal)
        want = O.mha_backward(q, k, v, g, heads, scale, use_decoder_mask=causal)
    for a, e, n in zip(got, want, "QKV"):
        parity(a, e, f"{case} d{n}")


@pytest.mark.parametrize("b,lq,lk,dim,heads,causal,masked", [
    (1, 256, 256, 128, 2, True, False),    # head dim 64, causal
    (1, 1000, 1000, 128, 2, True, False),  # ragged causal
    (2, 300, 700, 64, 2, False, False),    # head dim 32, cross attention, two sequences
    (1, 200, 100, 64, 1, True, False),     # decoder mask with lq > lk
    (1, 100, 200, 64, 1, True, False),     # decoder mask with lq < lk
    (1, 257, 257, 128, 2, False, True),    # explicit mask
    (1, 200, 200, 128, 2, True, True),     # mask and decoder rule together
    (1, 300, 300, 256, 2, True, False),    # head dim 128
    (3, 64, 64, 64, 4, True, False),       # segments, head dim 16 (zero-padded to 32)
    (1, 130, 130, 96, 2, True, False),     # head dim 48 (zero-padded to 64)
    (2, 70, 90, 36, 2, False, True),       # head dim 18: rows not 16-byte aligned, scalar loads
    (1, 77, 77, 200, 2, True, False),      # head dim 100 (zero-padded to 128)
    (1, 40, 40, 272, 2, True, False),      # head dim 136: per-row kernel
])
def test_sdpa_bwd_shapes(b, lq, lk, dim, heads, causal, masked):
    hd = dim // heads
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    q, g = synth.normal(lq + dim, (b * lq, dim)), synth.normal(7, (b * lq, dim))
    k, v = synth.normal(lk + 3, (b * lk, dim)), synth.normal(lk + 5, (b * lk, dim))
    mask = (synth.normal(11, (lq, lk)) > -0.5).astype(np.uint8) if masked else None
    if masked:
        mask[lq // 3] = 0  # a row that sees no key
    got = G.sdpa_bwd(q, k, v, g, heads, scale, causal=causal, mask=mask, batch=b)
    # The reference's overloads take the decoder rule or a mask; the ABI
    # composes them, which the oracle sees as the mask of both.
    omask = mask * np.tril(np.ones((lq, lk), np.uint8)) if (masked and causal) else mask
    for s in range(b):
        qs, gs = slice(s * lq, (s + 1) * lq), slice(s * lk, (s + 1) * lk)
        want = O.mha_backward(q[qs], k[gs], v[gs], g[qs], heads, scale, mask=omask,
                              use_decoder_mask=causal and not masked)
        for a, e, n in zip((got[0][qs], got[1][gs], got[2][gs]), want, "QKV"):
            parity(a, e, f"seq {s} d{n} ({lq}x{lk}, hd {hd}, causal {causal}, mask {masked})")


def _attention_bwd64(q, k, v, g, scale):
    """float64 causal attention backward of one head by matrix algebra
    (the identities pinned on the oracle by finite differences)."""
    n = q.shape[0]
    s = (q @ k.T) * scale
    s[np.triu_indices(n, 1)] = -np.inf
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    dp = g @ v.T
    ds = p * (dp - (p * dp).sum(1, keepdims=True))
    return (ds @ k) * scale, (ds.T @ q) * scale, p.T @ g


def test_sdpa_bwd_c3_shape_sampled_heads():
    """The c3 shape (4 x 4096, 16 heads of 64, causal) on the GPU; two
    (sequence, head) pairs checked against float64."""
    B, L, D, H = 4, 4096, 1024, 16
    hd = D // H
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    q, k, v, g = (synth.normal(20 + i, (B * L, D)) for i in range(4))
    dq, dk, dv = G.sdpa_bwd(q, k, v, g, H, scale, causal=True, batch=B)
    for b, h in [(0, 0), (3, 13)]:
        rows, cols = slice(b * L, (b + 1) * L), slice(h * hd, (h + 1) * hd)
        want = _attention_bwd64(*(t[rows, cols].astype(np.float64) for t in (q, k, v, g)), scale)
        for a, e, n in zip((dq, dk, dv), want, "QKV"):
            parity(a[rows, cols], e, f"c3 (b {b}, h {h}) d{n}")


# ------------------------------------------------------------------- SDPA
def test_sdpa_reference_cases(ops_golden):
    g = ops_golden
    qs, ks, vs = M(4, 8, 118), M(4, 8, 119), M(4, 8, 120)
    qc, kc, vc = M(4, 8, 121), M(5, 8, 122), M(5, 8, 123)
    parity(G.sdpa(qs, ks, vs, 2), O.sdpa(qs, ks, vs, 2), "self/no mask")
    parity(G.sdpa(qs, ks, vs, 2, mask=g["self_mask"]), O.sdpa(qs, ks, vs, 2, mask=g["self_mask"]), "self/mask")
    flag = G.sdpa(qs, ks, vs, 2, causal=True)
    parity(flag, O.sdpa(qs, ks, vs, 2, causal=True), "self/causal")
    parity(G.sdpa(qs, ks, vs, 2, mask=O.causal_mask(4)), flag, "causal flag == explicit mask")
    parity(G.sdpa(qc, kc, vc, 2), O.sdpa(qc, kc, vc, 2), "cross/no mask")
    parity(G.sdpa(qc, kc, vc, 2, mask=g["cross_mask"]), O.sdpa(qc, kc, vc, 2, mask=g["cross_mask"]), "cross/mask")
    am = G.sdpa(qc, kc, vc, 2, mask=g["all_masked_mask"])
    assert np.all(am[0] == 0), "all-masked row must be exactly 0"
    parity(am, O.sdpa(qc, kc, vc, 2, mask=g["all_masked_mask"]), "all-masked row")
    with pytest.raises(N.CdmlError) as ei:
        G.sdpa(qc, kc, vc, 2, causal=True)
    assert ei.value.code == N.E_CAUSAL


def test_mha_forward_reference_cases(ops_golden):
    q6, k6, v6 = M(4, 6, 31), M(4, 6, 32), M(4, 6, 33)  # d_h = 3
    sc = float(ops_golden["mha_causal_scale"])
    parity(G.sdpa(q6, k6, v6, 2, mask=O.causal_mask(4), scale=sc),
           O.mha_forward(q6, k6, v6, 2, sc, mask=O.causal_mask(4)), "MHA causal d_h=3")
    qg, kg, vg = M(128, 64, 110), M(128, 64, 111), M(128, 64, 112)
    parity(G.sdpa(qg, kg, vg, 4, scale=0.25), O.mha_forward(qg, kg, vg, 4, 0.25), "MHA 128 no mask")
    pm = synth.periodic_mask(128, 128)
    parity(G.sdpa(qg, kg, vg, 4, scale=0.25, mask=pm), O.mha_forward(qg, kg, vg, 4, 0.25, mask=pm),
           "MHA 128 periodic mask")
    parity(G.sdpa(qg, kg, vg, 4, causal=True), O.sdpa(qg, kg, vg, 4, causal=True), "SDPA 128 causal")


def test_sdpa_c2_batch_head_slice_golden(ops_golden):
    """Config 2 (16 sequences x 1024, D 512, 8 heads, causal) in one launch;
    the golden head slice (float64 textbook attention) sits at sequence 5,
    head 3, among N(0,1) data."""
    B, L, D, H = 16, 1024, 512, 8
    q, k, v = (synth.normal(40 + i, (B * L, D)) for i in range(3))
    rows, cols = slice(5 * L, 6 * L), slice(3 * 64, 4 * 64)
    for i, t in enumerate((q, k, v)):
        t[rows, cols] = synth.normal(900 + i, (L, 64))
    got = G.sdpa(q, k, v, H, causal=True, batch=B)
    parity(got[rows, cols], ops_golden["c2_head_causal"], "c2 head slice vs float64 golden")


@pytest.mark.parametrize("L,D,H", [(64, 64, 4), (1, 64, 4), (33, 96, 3), (130, 512, 8), (257, 256, 8),
                                   (300, 128, 1), (200, 160, 1), (77, 80, 5), (96, 1024, 64)])
def test_sdpa_causal_shapes(L, D, H):
    q, k, v = (synth.normal(L * 3 + D + i, (L, D)) for i in range(3))
    parity(G.sdpa(q, k, v, H, causal=True), O.sdpa(q, k, v, H, causal=True, mt=True), f"causal L={L} D={D} H={H}")


@pytest.mark.parametrize("lq,lk", [(5, 300), (129, 64), (64, 1)])
def test_sdpa_cross_lengths(lq, lk):
    D, H = 128, 2
    q = synth.normal(1, (lq, D))
    k, v = synth.normal(2, (lk, D)), synth.normal(3, (lk, D))
    parity(G.sdpa(q, k, v, H), O.sdpa(q, k, v, H), f"cross {lq}x{lk}")
    mask = synth.periodic_mask(lq, lk)
    parity(G.sdpa(q, k, v, H, mask=mask), O.sdpa(q, k, v, H, mask=mask), f"cross mask {lq}x{lk}")


def test_sdpa_batched_equals_per_sequence():
    B, L, D, H = 3, 200, 128, 4
    q, k, v = (synth.normal(40 + i, (B * L, D)) for i in range(3))
    got = G.sdpa(q, k, v, H, causal=True, batch=B)
    for b in range(B):
        s = slice(b * L, (b + 1) * L)
        parity(got[s], O.sdpa(q[s], k[s], v[s], H, causal=True), f"batch {b}")


@pytest.mark.parametrize("name,B,L,D,H", [("c2", 16, 1024, 512, 8), ("c5", 256, 512, 256, 8)])
def test_sdpa_baseline_configs_sampled(name, B, L, D, H):
    """Whole-batch launch at the BASELINE shape; three sequences checked."""
    q, k, v = (synth.normal(100 + i, (B * L, D)) for i in range(3))
    got = G.sdpa(q, k, v, H, causal=True, batch=B)
    for b in (0, B // 2, B - 1):
        s = slice(b * L, (b + 1) * L)
        parity(got[s], O.sdpa(q[s], k[s], v[s], H, causal=True, mt=True), f"{name} seq {b}")


@pytest.mark.parametrize("B,L,D,H,causal,masked", [
    (64, 300, 256, 8, True, False),   # d_h 32: 3 ragged query tiles, 1536 workgroups
    (64, 200, 256, 8, False, True),   # d_h 32, explicit mask, no causal rule
    (40, 257, 512, 8, True, False),   # d_h 64, 960 tiles: paired (3 tiles: the middle one alone)
    (32, 512, 256, 8, True, False),   # d_h 32, 1024 tiles: paired, two per workgroup
    (600, 64, 96, 3, True, False),    # d_h 32, one tile per sequence
])
def test_sdpa_every_sequence_of_large_launches(B, L, D, H, causal, masked):
    """Launches of many query tiles, every sequence checked against the oracle.
    The paired cases run two causal tiles per workgroup, the second's Q rows
    and first key tile prefetched during the first's last key tile.  The row
    statistics of cdml_sdpa_fwd_lse (log2 of each row's softmax normaliser in
    the exp2(s * scale * log2 e) domain) are checked against float64, and its
    output must equal cdml_sdpa_fwd's bit for bit."""
    hd = D // H
    q, k, v = (synth.normal(B + L + i, (B * L, D)) for i in range(3))
    mask = synth.periodic_mask(L, L) if masked else None
    got = G.sdpa(q, k, v, H, mask=mask, causal=causal, batch=B)
    for b in range(B):
        s = slice(b * L, (b + 1) * L)
        parity(got[s], O.sdpa(q[s], k[s], v[s], H, mask=mask, causal=causal, mt=True), f"sequence {b}")
    # the same launch with row statistics
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    bq, bk, bv = G.up(q), G.up(k), G.up(v)
    bo, bl = N.DeviceBuffer(B * L * D * 4), N.DeviceBuffer(B * H * L * 4)
    bm = G.up(mask, np.uint8) if masked else None
    N.check(N.lib().cdml_sdpa_fwd_lse(bq.ptr, D, bk.ptr, D, bv.ptr, D, bo.ptr, D, bl.ptr, B, L, L, D, H, scale,
                                      int(causal), bm.ptr if bm else None, G.stream().handle))
    assert np.array_equal(G.down(bo, (B * L, D)), got), "cdml_sdpa_fwd_lse output differs from cdml_sdpa_fwd"
    lse = G.down(bl, (B, H, L))
    for b in (0, B // 2, B - 1):
        for h in (0, H - 1):
            cols = slice(h * hd, (h + 1) * hd)
            sc = (q[b * L:(b + 1) * L, cols].astype(np.float64) @ k[b * L:(b + 1) * L, cols].astype(np.float64).T
                  ) * scale * math.log2(math.e)
            vis = np.ones((L, L), bool)
            if causal:
                vis &= np.tril(vis)
            if masked:
                vis &= mask.astype(bool)
            sc = np.where(vis, sc, -np.inf)
            m = sc.max(axis=1, keepdims=True)
            want = (m + np.log2(np.exp2(sc - m).sum(axis=1, keepdims=True)))[:, 0]
            ok = np.isfinite(want)
            assert np.all(np.isinf(lse[b, h][~ok])), "rows with no visible key must have lse +inf"
            parity(lse[b, h][ok], want[ok], f"lse sequence {b} head {h}")


@pytest.mark.parametrize("causal", [True, False])
def test_sdpa_score_jumps_in_large_launches(causal):
    """Launches of at least three workgroups per CU accumulate a sub-block
    without its maximum once every row has its reference, and fall back to the
    full rescaling path when a lane's probabilities sum above 2^32.  Keys from
    position 100 on carry K rows 12 times larger (scores about 50 log2 units
    above the first sub-block's), keys from 200 on 12 times smaller,
    so both the fallback and the plain path run in one launch; sampled
    sequences against the oracle, row statistics against float64."""
    B, L, D, H = 128, 256, 256, 8
    hd = D // H
    q, k, v = (synth.normal(7 + i, (B * L, D)) for i in range(3))
    pos = np.arange(B * L) % L
    k = np.where((pos >= 100)[:, None], k * 12, k).astype(np.float32)
    k = np.where((pos >= 200)[:, None], k / 144, k).astype(np.float32)
    got = G.sdpa(q, k, v, H, causal=causal, batch=B)
    assert np.isfinite(got).all()
    for b in (0, 37, B - 1):
        s = slice(b * L, (b + 1) * L)
        parity(got[s], O.sdpa(q[s], k[s], v[s], H, causal=causal, mt=True), f"sequence {b}")
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    bq, bk, bv = G.up(q), G.up(k), G.up(v)
    bo, bl = N.DeviceBuffer(B * L * D * 4), N.DeviceBuffer(B * H * L * 4)
    N.check(N.lib().cdml_sdpa_fwd_lse(bq.ptr, D, bk.ptr, D, bv.ptr, D, bo.ptr, D, bl.ptr, B, L, L, D, H, scale,
                                      int(causal), None, G.stream().handle))
    assert np.array_equal(G.down(bo, (B * L, D)), got), "cdml_sdpa_fwd_lse output differs from cdml_sdpa_fwd"
    lse = G.down(bl, (B, H, L))
    for b, h in ((0, 0), (B - 1, H - 1)):
        cols = slice(h * hd, (h + 1) * hd)
        sc = (q[b * L:(b + 1) * L, cols].astype(np.float64) @ k[b * L:(b + 1) * L, cols].astype(np.float64).T
              ) * scale * math.log2(math.e)
        if causal:
            sc = np.where(np.tril(np.ones((L, L), bool)), sc, -np.inf)
        m = sc.max(axis=1, keepdims=True)
        want = (m + np.log2(np.exp2(sc - m).sum(axis=1, keepdims=True)))[:, 0]
        parity(lse[b, h], want, f"lse sequence {b} head {h}")


def _mha_layer(x, ws, bs, batch, seq_len, heads, causal=True, mask=None, base=10000.0, table=False):
    """cdml_mha_layer_fwd on host arrays; ws = (wq, wk, wv, wo), bs likewise."""
    rows, dim = x.shape
    lib, st = N.lib(), G.stream()
    size = C.c_size_t(0)
    N.check(lib.cdml_mha_layer_fwd_workspace_size(batch, seq_len, dim, heads, C.byref(size)))
    bx, by = G.up(x), N.DeviceBuffer(rows * dim * 4)
    bw, bb = [G.up(w) for w in ws], [G.up(b) for b in bs]
    ws_buf = N.DeviceBuffer(size.value)
    bm = G.up(mask, np.uint8) if mask is not None else None
    cs = None
    if table:
        cs = N.DeviceBuffer(seq_len * (dim // heads) * 4)
        N.check(lib.cdml_rope_table(cs.ptr, seq_len, dim // heads, base, st.handle))
    N.check(lib.cdml_mha_layer_fwd(bx.ptr, bw[0].ptr, bb[0].ptr, bw[1].ptr, bb[1].ptr, bw[2].ptr, bb[2].ptr,
                                   bw[3].ptr, bb[3].ptr, by.ptr, batch, seq_len, dim, heads, base, int(causal),
                                   bm.ptr if bm else None, cs.ptr if cs else None, ws_buf.ptr, size.value,
                                   st.handle))
    return G.down(by, (rows, dim))


@pytest.mark.parametrize("batch,L,D,H,causal,masked", [
    (1, 64, 64, 4, True, False), (3, 77, 96, 3, True, False), (2, 50, 64, 2, False, True),
    (2, 130, 256, 8, True, False)])
def test_mha_layer_fwd_matches_the_reference_sequence(batch, L, D, H, causal, masked):
    """cdml_mha_layer_fwd = MultiHeadAttention.Forward (MultiHeadAttention.cs:96-155):
    ProjectQKV, RoPE of Q and K per sequence, ScaledDotProductAttention, ProjectOutputBatch,
    each sequence of the batch against the oracle's composition; biases non-zero."""
    x = synth.normal(L + D, (batch * L, D))
    ws = [synth.xavier_uniform(300 + i, D, D) for i in range(4)]
    bs = [np.float32(0.1) * synth.normal(310 + i, (D,)) for i in range(4)]
    mask = synth.periodic_mask(L, L) if masked else None
    got = _mha_layer(x, ws, bs, batch, L, H, causal=causal, mask=mask)
    for b in range(batch):
        s = slice(b * L, (b + 1) * L)
        q, k, v = O.project_qkv(x[s], ws[0], bs[0], ws[1], bs[1], ws[2], bs[2])
        a = O.sdpa(O.rope(q, H), O.rope(k, H), v, H, mask=mask, causal=causal)
        parity(got[s], O.project_output_batch(a, ws[3], bs[3]), f"sequence {b}")


def test_mha_layer_fwd_equals_the_three_entries():
    """The fused entry runs the same kernels as cdml_project_qkv_rope, cdml_sdpa_fwd and
    cdml_linear chained by the host: the same bits, with its own table or a caller's."""
    batch, L, D, H = 2, 300, 256, 8
    hd = D // H
    x = synth.normal(5, (batch * L, D))
    ws = [synth.xavier_uniform(320 + i, D, D) for i in range(4)]
    bs = [np.float32(0.1) * synth.normal(330 + i, (D,)) for i in range(4)]
    q, k, v = G.project_qkv_rope(x, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], hd, n_pos=L, seg_len=L)
    want = G.linear(G.sdpa(q, k, v, H, causal=True, batch=batch), ws[3], bs[3])
    assert np.array_equal(_mha_layer(x, ws, bs, batch, L, H), want)
    assert np.array_equal(_mha_layer(x, ws, bs, batch, L, H, table=True), want)


def test_sdpa_c3_long_context_sampled():
    """c3 shape (B 4, L 4096, D 1024, H 16): one full sequence's sampled heads vs the
    oracle, plus the causal-prefix property on the whole batch."""
    B, L, D, H = 4, 4096, 1024, 16
    q, k, v = (synth.normal(200 + i, (B * L, D)) for i in range(3))
    got = G.sdpa(q, k, v, H, causal=True, batch=B)
    assert np.all(np.isfinite(got))
    b = 1
    s = slice(b * L, (b + 1) * L)
    for h in (0, 9):
        cols = slice(h * 64, (h + 1) * 64)
        want = O.sdpa(q[s, cols], k[s, cols], v[s, cols], 1, causal=True)
        parity(got[s, cols], want, f"c3 seq {b} head {h}")
    # causal prefix: attention of the first 1000 positions alone equals the prefix rows
    pre = G.sdpa(q[:1000], k[:1000], v[:1000], H, causal=True)
    parity(pre, got[:1000], "causal prefix property")


# ----------------------------------------------------------------- decode
@pytest.mark.parametrize("B,T,D,H", [(2, 1000, 2048, 16), (3, 300, 64, 4), (2, 513, 96, 3), (1, 1, 256, 2)])
def test_decode_vs_oracle(B, T, D, H):
    q = synth.normal(1, (B, D))
    kc, vc = synth.normal(2, (B, T, D)), synth.normal(3, (B, T, D))
    lens = np.array([T, max(1, T // 3)] + [1] * (B - 2), np.int32)[:B]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D // H)))
    got = G.decode(q, kc, vc, lens, H, scale)
    want = O.decode_attention_batch(q, kc, vc, lens, H, scale, parallel=True)
    parity(got, want, f"decode B={B} T={T} D={D} H={H}")


def test_decode_wide_grid_ragged_lengths():
    """A launch wide enough for 512-key chunks (64 sequences x 8 heads x 2 chunks),
    with lengths on both sides of the chunk boundaries, against the oracle."""
    B, T, D, H = 64, 1000, 512, 8
    q = synth.normal(61, (B, D))
    kc, vc = synth.normal(62, (B, T, D)), synth.normal(63, (B, T, D))
    base = [1000, 999, 513, 512, 511, 257, 256, 1, 700, 2]
    lens = np.array([base[i % len(base)] for i in range(B)], np.int32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D // H)))
    got = G.decode(q, kc, vc, lens, H, scale)
    want = O.decode_attention_batch(q, kc, vc, lens, H, scale, parallel=True)
    parity(got, want, "decode wide grid, ragged lengths")


def test_decode_equals_last_prefill_row():
    T, D, H = 700, 512, 4
    q, k, v = (synth.normal(50 + i, (T, D)) for i in range(3))
    pre = G.sdpa(q, k, v, H, causal=True)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D // H)))
    dec = G.decode(q[-1:], k[None], v[None], np.array([T], np.int32), H, scale)
    parity(dec[0], pre[-1], "decode == last prefill row")


def test_decode_c4_shape_sampled():
    """c4 shape (B 64, T 8192, H 16, d_h 128), full kernel launch; 4 sequences checked."""
    B, T, D, H = 64, 8192, 2048, 16
    rng = np.random.default_rng(4)  # 2 x 4 GiB of N(0,1): numpy's generator for speed
    q = rng.standard_normal((B, D), dtype=np.float32)
    kc = rng.standard_normal((B, T, D), dtype=np.float32)
    vc = rng.standard_normal((B, T, D), dtype=np.float32)
    lens = np.full(B, T, np.int32)
    lens[5] = 4097
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    got = G.decode(q, kc, vc, lens, H, scale)
    assert np.all(np.isfinite(got))
    idx = [0, 5, 31, 63]
    want = O.decode_attention_batch(q[idx], kc[idx], vc[idx], lens[idx], H, scale, parallel=True)
    parity(got[idx], want, "c4 sampled")


def test_kv_cache_append():
    kc, vc = np.zeros((3, 5, 8), np.float32), np.zeros((3, 5, 8), np.float32)
    kn, vn = synth.normal(1, (3, 8)), synth.normal(2, (3, 8))
    pos = np.array([0, 4, 2], np.int32)
    k2, v2 = G.kv_append(kn, vn, kc, vc, pos)
    for b, p in enumerate(pos):
        assert np.array_equal(k2[b, p], kn[b]) and np.array_equal(v2[b, p], vn[b])
        assert np.count_nonzero(k2[b]) == np.count_nonzero(kn[b])


# ------------------------------------------------------ layernorm, embed
@pytest.mark.parametrize("rows,f", [(5, 6), (64, 64), (100, 1024), (7, 2500)])
def test_residual_layernorm(rows, f):
    a, b = synth.normal(rows, (rows, f)), synth.normal(f, (rows, f))
    g, be = synth.positive_vector(f, 28), synth.vector(f, 29)
    parity(G.residual_layernorm(a, b, g, be), O.residual_layernorm(a, b, g, be), f"LN {rows}x{f}")


def test_embed_tokens_exact():
    table = M(6, 5, 64)
    out, bad = G.embed([0, 2, 4], table)
    assert bad == 0 and np.array_equal(out, O.embed_tokens([0, 2, 4], table))
    t2 = synth.normal(3, (200, 64))
    ids = synth.token_ids(4, 64, 200)
    out, bad = G.embed(ids, t2)
    assert bad == 0 and np.array_equal(out, O.embed_tokens(ids, t2))
    out, bad = G.embed([1, 200, -1], t2)
    assert bad == 2 and np.all(out[1:] == 0) and np.array_equal(out[0], t2[1])


def test_graph_capture_replays_the_recorded_launches():
    """cdml_graph_capture_begin / _end / _launch: a recorded sequence of
    launches (a linear layer with ReLU, a fill, a second linear layer into
    another buffer) replays with the recorded pointers, so new inputs
    uploaded between replays give new results; every replay, with eager
    launches and synchronisations between them, matches the eager result.
    Recording on the default stream is refused, and a graph handle of NULL is
    an argument error."""
    import ctypes as C
    lib = N.lib()
    st = N.Stream()  # a stream of its own: capture must not see the helpers' stream
    s = st.handle
    rows, ind, hid, out = 40, 64, 96, 24
    w1, w2 = synth.xavier_uniform(1, hid, ind), synth.xavier_uniform(2, out, hid)
    b1, b2 = synth.normal(3, (hid,)), synth.normal(4, (out,))
    dw1, dw2, db1, db2 = (N.DeviceBuffer.from_array(a, st) for a in (w1, w2, b1, b2))
    dx, dh, dy = N.DeviceBuffer(rows * ind * 4), N.DeviceBuffer(rows * hid * 4), N.DeviceBuffer(rows * out * 4)
    dcount = N.DeviceBuffer(64 * 4)

    def enqueue():
        N.check(lib.cdml_linear(dx.ptr, ind, dw1.ptr, db1.ptr, dh.ptr, hid, rows, ind, hid, 3, s))
        N.check(lib.cdml_fill_i32_async(dcount.ptr, 64, 7, s))
        N.check(lib.cdml_linear(dh.ptr, hid, dw2.ptr, db2.ptr, dy.ptr, out, rows, hid, out, 0, s))

    def expected(x):
        h = O.activation(O.batch_dot_add_bias(w1, x, b1), 3)
        return O.batch_dot_add_bias(w2, h, b2)

    N.check(lib.cdml_graph_capture_begin(s))
    enqueue()
    g = C.c_void_p()
    N.check(lib.cdml_graph_capture_end(s, C.byref(g)))
    assert g.value
    try:
        for rep in range(4):
            x = synth.normal(10 + rep, (rows, ind))
            dx.upload(x, st)
            N.check(lib.cdml_graph_launch(g, s))
            st.synchronize()
            got = dy.download((rows, out), np.float32, st)
            parity(got, expected(x), f"replay {rep}")
            assert np.all(dcount.download((64,), np.int32, st) == 7)
            # eager work on the same buffers between replays
            enqueue()
            st.synchronize()
            assert np.array_equal(dy.download((rows, out), np.float32, st), got)
    finally:
        N.check(lib.cdml_graph_destroy(g))
    assert lib.cdml_graph_launch(None, s) == N.E_INVALID
    assert lib.cdml_graph_capture_begin(None) == N.E_INVALID
