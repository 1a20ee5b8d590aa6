"""numpy front end of the CPU parity oracle (TEST INFRASTRUCTURE ONLY).

Loads ``oracle/_build/librefcpu.so`` (built from ``refcpu.c`` and
``refcpu_mt.c`` by ``oracle/Makefile``) and exposes its functions on numpy
float32 arrays.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module; the product path
(``libcdml_hip.so`` and the host manager) never does.

Each wrapper names the reference method it restates; the C source cites the
exact reference lines.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# CDML_ORACLE_LIB selects another build of the same sources (the sanitizer
# build, `make asan`, which tests load under libasan).
_LIB_PATH = os.environ.get("CDML_ORACLE_LIB") or os.path.join(_HERE, "_build", "librefcpu.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u8p = C.c_void_p


class OracleError(ValueError):
    """Raised where the reference throws ArgumentException and friends."""


def build(force: bool = False) -> str:
    """Compile the oracle library with make (CPU only, a few seconds)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(_LIB_PATH)
        i, f = C.c_int, C.c_float
        sig = {
            "ref_dot": (f, [_f32p, _f32p, i]),
            "ref_project_qkv": (i, [_f32p] * 7 + [_f32p] * 3 + [i, i, i]),
            "ref_project_output_batch": (i, [_f32p] * 4 + [i, i, i]),
            "ref_batch_dot_add_bias": (i, [_f32p] * 4 + [i, i, i]),
            "ref_activation_inplace": (None, [_f32p, C.c_long, i]),
            "ref_rope_inplace": (i, [_f32p, i, i, i, f, i]),
            "ref_rope_head_inplace": (i, [_f32p, i, i, i, i, f, i]),
            "ref_sdpa": (i, [_f32p] * 4 + [i, i, i, i, _u8p, i]),
            "ref_mha_forward": (i, [_f32p] * 4 + [i, i, i, i, f, _u8p]),
            "ref_softmax": (i, [_f32p, _f32p, i, i, _u8p]),
            "ref_residual_layernorm": (i, [_f32p] * 5 + [i, i, f]),
            "ref_embed_tokens": (i, [_i32p, i, _f32p, i, i, _f32p]),
            "ref_causal_mask": (None, [i, C.c_void_p]),
            "ref_decode_attention": (i, [_f32p, _f32p, _f32p, i, i, i, f, _f32p]),
            "ref_lm_forward": (i, [C.c_void_p, _i32p, i, _f32p]),
            "ref_lm_generate_greedy": (i, [C.c_void_p, _i32p, i, i, _i32p, C.POINTER(i)]),
            "ref_mha_backward": (i, [_f32p] * 7 + [i, i, i, i, f, _u8p, i]),
            "ref_backprop_qkv": (i, [_f32p] * 14 + [i, i, i]),
            "ref_backprop_linear_projection": (i, [_f32p] * 6 + [i, i, i]),
            "ref_backprop_output_projection": (i, [_f32p] * 6 + [i, i, i]),
            "ref_residual_layernorm_forward": (i, [_f32p] * 9 + [i, i, f]),
            "ref_layernorm_backward": (i, [_f32p] * 9 + [i, i, f]),
            "ref_cross_entropy": (i, [_f32p, i, i, _i32p, i, i, i, C.POINTER(f), _f32p]),
            "ref_ffn_input_gradient": (i, [_f32p, _f32p, i, i, _i32p, C.c_void_p, C.c_void_p, _i32p,
                                           C.c_void_p, C.c_void_p, _f32p]),
            "ref_accumulate_token_embedding_grad": (i, [_f32p, _f32p, _i32p, i, i, i]),
            "ref_squared_norm": (f, [_f32p, C.c_long]),
            "ref_scale_inplace": (None, [_f32p, C.c_long, f]),
            "ref_sgd_update": (None, [_f32p, _f32p, C.c_long, f]),
            "ref_mse_loss": (i, [_f32p, i, i, _f32p, i, i, i, C.POINTER(f), _f32p]),
            "ref_backprop_input_projection": (i, [_f32p, _f32p, i, i, i, _f32p, _f32p, i, i, i]),
            "mt_num_threads": (i, []),
            "mt_set_threads": (None, [i]),
            "mt_project_qkv": (i, [_f32p] * 10 + [i, i, i]),
            "mt_project_output_batch": (i, [_f32p] * 4 + [i, i, i]),
            "mt_batch_dot_add_bias": (i, [_f32p] * 4 + [i, i, i]),
            "mt_rope_inplace": (i, [_f32p, i, i, i, f, i]),
            "mt_sdpa": (i, [_f32p] * 4 + [i, i, i, i, _u8p, i]),
            "mt_residual_layernorm": (i, [_f32p] * 5 + [i, i, f]),
            "mt_decode_attention_batch": (i, [_f32p, _f32p, _f32p, _i32p, i, i, i, i, f, _f32p, i]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _mask_ptr(mask):
    if mask is None:
        return None, None
    m = np.ascontiguousarray(mask, dtype=np.uint8)
    return m, m.ctypes.data_as(C.c_void_p)


def _check(rc: int, what: str):
    if rc == -2:
        raise OracleError(f"{what}: causal attention requires queryLen == keyLen")
    if rc != 0:
        raise OracleError(f"{what}: invalid argument (status {rc})")


# ---- AccelerationCPU restatement -----------------------------------------

def dot(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return float(lib().ref_dot(a, b, a.size))


def project_qkv(x, wq, bq, wk, bk, wv, bv, mt: bool = False):
    """AccelerationCPU.ProjectQKV (mt: AccelerationMutliThreadCPU.ProjectQKV)."""
    x = _f32(x)
    rows, in_dim = x.shape
    out_dim = wq.shape[0]
    q = np.empty((rows, out_dim), np.float32)
    k = np.empty_like(q)
    v = np.empty_like(q)
    fn = lib().mt_project_qkv if mt else lib().ref_project_qkv
    _check(fn(x, _f32(wq), _f32(bq), _f32(wk), _f32(bk), _f32(wv), _f32(bv),
              q, k, v, rows, in_dim, out_dim), "ProjectQKV")
    return q, k, v


def project_output_batch(h, w, b, mt: bool = False):
    """AccelerationCPU.ProjectOutputBatch: y = b + h W^T."""
    h = _f32(h)
    rows, in_dim = h.shape
    out_dim = w.shape[0]
    y = np.empty((rows, out_dim), np.float32)
    fn = lib().mt_project_output_batch if mt else lib().ref_project_output_batch
    _check(fn(h, _f32(w), _f32(b), y, rows, in_dim, out_dim), "ProjectOutputBatch")
    return y


def batch_dot_add_bias(w, x, b, mt: bool = False):
    """AccelerationCPU.BatchDotProductAddBias: y = x W^T + b."""
    x = _f32(x)
    rows, in_dim = x.shape
    out_dim = w.shape[0]
    y = np.empty((rows, out_dim), np.float32)
    fn = lib().mt_batch_dot_add_bias if mt else lib().ref_batch_dot_add_bias
    _check(fn(_f32(w), x, _f32(b), y, rows, in_dim, out_dim), "BatchDotProductAddBias")
    return y


def activation(x, act: int):
    """NeuralNetwork.ApplyActivationInPlace on a copy."""
    y = _f32(x).copy()
    lib().ref_activation_inplace(y, y.size, act)
    return y


def rope(x, num_heads: int, base_theta: float = 10000.0, inverse: bool = False, mt: bool = False):
    """AccelerationCPU.ApplyRotaryPositionEmbeddingInPlace on a copy."""
    y = _f32(x).copy()
    rows, dim = y.shape
    fn = lib().mt_rope_inplace if mt else lib().ref_rope_inplace
    _check(fn(y, rows, dim, num_heads, base_theta, int(inverse)), "ApplyRotaryPositionEmbeddingInPlace")
    return y


def rope_head(x, start_col: int, head_dim: int, base_theta: float = 10000.0, inverse: bool = False):
    """AccelerationCPU.ApplyRotaryPositionEmbeddingHeadInPlace on a copy."""
    y = _f32(x).copy()
    rows, dim = y.shape
    _check(lib().ref_rope_head_inplace(y, rows, dim, start_col, head_dim, base_theta, int(inverse)),
           "ApplyRotaryPositionEmbeddingHeadInPlace")
    return y


def sdpa(q, k, v, num_heads: int, mask=None, causal: bool = False, mt: bool = False):
    """AccelerationCPU.ScaledDotProductAttention."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    lq, dim = q.shape
    lk = k.shape[0]
    out = np.empty((lq, dim), np.float32)
    _m, mp = _mask_ptr(mask)
    fn = lib().mt_sdpa if mt else lib().ref_sdpa
    _check(fn(q, k, v, out, lq, lk, dim, num_heads, mp, int(causal)), "ScaledDotProductAttention")
    return out


def mha_forward(q, k, v, num_heads: int, scale: float, mask=None):
    """AccelerationCPU.MultiHeadAttentionForward."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    lq, dim = q.shape
    lk = k.shape[0]
    out = np.empty((lq, dim), np.float32)
    _m, mp = _mask_ptr(mask)
    _check(lib().ref_mha_forward(q, k, v, out, lq, lk, dim, num_heads, scale, mp),
           "MultiHeadAttentionForward")
    return out


def softmax(x, mask=None):
    """AccelerationCPU.Softmax."""
    x = _f32(x)
    out = np.empty_like(x)
    _m, mp = _mask_ptr(mask)
    rc = lib().ref_softmax(x, out, x.shape[0], x.shape[1], mp)
    if rc == -3:
        raise OracleError("Softmax input contains NaN")
    return out


def residual_layernorm(a, b, gamma, beta, eps: float = 1e-5, mt: bool = False):
    """AccelerationCPU.ResidualLayerNorm."""
    a = _f32(a)
    rows, f = a.shape
    out = np.empty_like(a)
    fn = lib().mt_residual_layernorm if mt else lib().ref_residual_layernorm
    _check(fn(a, _f32(b), _f32(gamma), _f32(beta), out, rows, f, eps), "ResidualLayerNorm")
    return out


def embed_tokens(ids, table):
    """AccelerationCPU.EmbedTokenIds."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    table = _f32(table)
    out = np.empty((ids.size, table.shape[1]), np.float32)
    _check(lib().ref_embed_tokens(ids, ids.size, table, table.shape[0], table.shape[1], out),
           "EmbedTokenIds")
    return out


def causal_mask(n: int):
    """AccelerationCPU.CreateCausalMask."""
    m = np.empty((n, n), np.uint8)
    lib().ref_causal_mask(n, m.ctypes.data_as(C.c_void_p))
    return m


def decode_attention(q, kcache, vcache, key_len: int, num_heads: int, scale: float):
    """LanguageModel.DecoderSelfAttentionStep attention core for one query row."""
    q = _f32(q).reshape(-1)
    dim = q.size
    out = np.empty(dim, np.float32)
    lib().ref_decode_attention(q, _f32(kcache), _f32(vcache), key_len, dim, num_heads, scale, out)
    return out


def decode_attention_batch(q, kcache, vcache, kv_len, num_heads: int, scale: float, parallel: bool):
    """Decode attention for B sequences over a [B, Tmax, D] cache."""
    q = _f32(q)
    b, dim = q.shape
    t_max = kcache.shape[1]
    out = np.empty((b, dim), np.float32)
    lib().mt_decode_attention_batch(q, _f32(kcache), _f32(vcache),
                                    np.ascontiguousarray(kv_len, dtype=np.int32),
                                    b, t_max, dim, num_heads, scale, out, int(parallel))
    return out


# ---- backward path (refcpu_bwd.c) ----------------------------------------

def mha_backward(q, k, v, dout, num_heads: int, scale: float, mask=None, use_decoder_mask: bool = False):
    """AccelerationCPU.MultiHeadAttentionBackward (bool and mask overloads) -> (dQ, dK, dV)."""
    q, k, v, dout = _f32(q), _f32(k), _f32(v), _f32(dout)
    lq, dim = q.shape
    lk = k.shape[0]
    dq = np.empty((lq, dim), np.float32)
    dk = np.empty((lk, dim), np.float32)
    dv = np.empty((lk, dim), np.float32)
    m, mp = _mask_ptr(mask)
    _check(lib().ref_mha_backward(q, k, v, dout, dq, dk, dv, lq, lk, dim, num_heads, scale, mp,
                                  int(use_decoder_mask)), "MultiHeadAttentionBackward")
    return dq, dk, dv


def backprop_qkv(x, dq, dk, dv, wq, wk, wv, wq_grad, bq_grad, wk_grad, bk_grad, wv_grad, bv_grad):
    """AccelerationCPU.BackpropQKV on copies of the gradient accumulators ->
    (dInput, WQGrad, biasQGrad, WKGrad, biasKGrad, WVGrad, biasVGrad)."""
    x = _f32(x)
    rows, in_dim = x.shape
    out_dim = wq.shape[0]
    g = [_f32(a).copy() for a in (wq_grad, bq_grad, wk_grad, bk_grad, wv_grad, bv_grad)]
    dx = np.empty((rows, in_dim), np.float32)
    _check(lib().ref_backprop_qkv(x, _f32(dq), _f32(dk), _f32(dv), _f32(wq), _f32(wk), _f32(wv), *g, dx,
                                  rows, in_dim, out_dim), "BackpropQKV")
    return (dx, *g)


def backprop_linear_projection(x, dy, w, w_grad, b_grad, dx):
    """AccelerationCPU.BackpropLinearProjection on copies -> (weightGrad, biasGrad, dInput)."""
    x, dy = _f32(x), _f32(dy)
    rows, in_dim = x.shape
    out_dim = dy.shape[1]
    wg, bg, dxo = _f32(w_grad).copy(), _f32(b_grad).copy(), _f32(dx).copy()
    _check(lib().ref_backprop_linear_projection(x, dy, _f32(w), wg, bg, dxo, rows, in_dim, out_dim),
           "BackpropLinearProjection")
    return wg, bg, dxo


def backprop_output_projection(dl, x, w, w_grad, b_grad):
    """AccelerationCPU.BackpropOutputProjection on copies -> (dX, weightGrad, biasGrad)."""
    dl, x = _f32(dl), _f32(x)
    rows, out_dim = dl.shape
    emb = x.shape[1]
    wg, bg = _f32(w_grad).copy(), _f32(b_grad).copy()
    dx = np.empty((rows, emb), np.float32)
    _check(lib().ref_backprop_output_projection(dl, x, _f32(w), wg, bg, dx, rows, out_dim, emb),
           "BackpropOutputProjection")
    return dx, wg, bg


# ---- training step (refcpu_train.c) ---------------------------------------

def residual_layernorm_forward(a, b, gamma, beta, eps: float = 1e-5):
    """AccelerationCPU.ResidualLayerNormForward -> (out, means, variances, normalized, residual)."""
    a, b = _f32(a), _f32(b)
    rows, f = a.shape
    out, norm, res = (np.empty((rows, f), np.float32) for _ in range(3))
    mean, var = np.empty(rows, np.float32), np.empty(rows, np.float32)
    _check(lib().ref_residual_layernorm_forward(a, b, _f32(gamma), _f32(beta), out, mean, var, norm, res,
                                                rows, f, eps), "ResidualLayerNormForward")
    return out, mean, var, norm, res


def layernorm_backward(dout, normalized, gamma, inp, mean, var, eps: float = 1e-5):
    """AccelerationCPU.LayerNormBackward -> (dInput, dGamma, dBeta)."""
    dout = _f32(dout)
    rows, f = dout.shape
    dx = np.empty((rows, f), np.float32)
    dg, db = np.empty(f, np.float32), np.empty(f, np.float32)
    _check(lib().ref_layernorm_backward(dout, _f32(normalized), _f32(gamma), _f32(inp), _f32(mean), _f32(var),
                                        dx, dg, db, rows, f, eps), "LayerNormBackward")
    return dx, dg, db


def cross_entropy(logits, targets, effective_len: int, target_start: int = 0):
    """AccelerationCPU.CrossEntropyLossAndGradient -> (loss, dLogits)."""
    logits = _f32(logits)
    t = np.ascontiguousarray(targets, dtype=np.int32)
    rows, v = logits.shape
    dl = np.empty((rows, v), np.float32)
    loss = C.c_float(0)
    _check(lib().ref_cross_entropy(logits, rows, v, t, t.size, target_start, effective_len, C.byref(loss), dl),
           "CrossEntropyLossAndGradient")
    return float(np.float32(loss.value)), dl


def ffn_input_gradient(inp, dout, weights, biases, acts, wgrads=None, bgrads=None):
    """NeuralNetwork.ComputeInputGradientBatch: returns dInput; wgrads / bgrads
    (lists of float32 arrays, one per weight layer) accumulate in place."""
    inp, dout = _f32(inp), _f32(dout)
    rows = inp.shape[0]
    n = len(weights)
    ws = [_f32(w) for w in weights]
    bs = [_f32(b) for b in biases]
    widths = np.array([ws[0].shape[1]] + [w.shape[0] for w in ws], np.int32)
    a = np.array(acts, np.int32)
    P = C.c_void_p * n
    wp, bp = P(*[w.ctypes.data for w in ws]), P(*[b.ctypes.data for b in bs])
    if wgrads is not None:
        for g in list(wgrads) + list(bgrads):
            assert g.dtype == np.float32 and g.flags.c_contiguous
        wgp, bgp = P(*[g.ctypes.data for g in wgrads]), P(*[g.ctypes.data for g in bgrads])
    else:
        wgp = bgp = None
    dx = np.empty((rows, widths[0]), np.float32)
    _check(lib().ref_ffn_input_gradient(inp, dout, rows, n, widths, wp, bp, a, wgp, bgp, dx),
           "ComputeInputGradientBatch")
    return dx


def accumulate_token_embedding_grad(eg, dx, ids):
    """AccelerationCPU.AccumulateTokenEmbeddingGrad on a copy of eg."""
    eg = _f32(eg).copy()
    dx = _f32(dx)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    _check(lib().ref_accumulate_token_embedding_grad(eg, dx, ids, ids.size, eg.shape[1], eg.shape[0]),
           "AccumulateTokenEmbeddingGrad")
    return eg


def squared_norm(x) -> float:
    x = _f32(x)
    return float(np.float32(lib().ref_squared_norm(x, x.size)))


def scale_inplace(x, scale: float):
    assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().ref_scale_inplace(x, x.size, scale)


def sgd_update(w, g, lr: float):
    assert w.dtype == np.float32 and w.flags.c_contiguous
    lib().ref_sgd_update(w, _f32(g), w.size, lr)


# Parameter order of the trainer's ZeroAllGradients / ComputeGradientNorm /
# ScaleGradients / UpdateParameters walks (TransformerTrainer.cs:1269-1400).
_ATTN = ("wq", "wk", "wv", "wo")
_ATTN_B = ("bq", "bk", "bv", "bo")


def train_step(cfg: dict, weights: dict, seqs, lr: float, clip: float = 1.0, use_clipping: bool = True):
    """TransformerTrainer.TrainBatchDiscrete for one bucket of equal-length
    token sequences [B, S + 1]; see train_batch."""
    return train_batch(cfg, weights, list(np.ascontiguousarray(seqs, dtype=np.int32)), lr, clip, use_clipping)


def mse_loss(pred, targets, effective_len: int, target_start: int = 0):
    """AccelerationCPU.MSELossAndGradient -> (loss, dOutput)."""
    pred, targets = _f32(pred), _f32(targets)
    rows, o = pred.shape
    d = np.empty((rows, o), np.float32)
    loss = C.c_float(0)
    _check(lib().ref_mse_loss(pred, rows, o, targets, targets.shape[0], target_start, effective_len,
                              C.byref(loss), d), "MSELossAndGradient")
    return float(np.float32(loss.value)), d


def backprop_input_projection(dx, inp, wg, bg, row_start: int = 0):
    """AccelerationCPU.BackpropInputProjection on copies -> (weightGrad, biasGrad)."""
    dx, inp = _f32(dx), _f32(inp)
    wg, bg = _f32(wg).copy(), _f32(bg).copy()
    _check(lib().ref_backprop_input_projection(dx, inp, inp.shape[0], inp.shape[1], row_start, wg, bg,
                                               dx.shape[0], dx.shape[1], wg.shape[1]),
           "BackpropInputProjection")
    return wg, bg


def _bucket_forward_backward(cfg, w, g, seqs=None, inputs=None, reg=None, cls=None):
    """Forward with cache, loss and backward of one bucket
    (TransformerTrainer.cs:255-300, 373-456); gradients accumulate into g.
    Token models take seqs [B, S + 1]; continuous models take inputs
    [B, S + 1, F] with regression targets reg [B, S + 1, O] (MSE) or class
    targets cls [B, S + 1] (cross-entropy); row t's target is step t + 1.
    Returns the bucket's loss, or None when it is not finite (no backward)."""
    discrete = seqs is not None
    if discrete:
        seqs = np.ascontiguousarray(seqs, dtype=np.int32)
        B, S = seqs.shape[0], seqs.shape[1] - 1
        ids, targets = seqs[:, :S].reshape(-1), seqs[:, 1:].reshape(-1)
    else:
        inputs = _f32(inputs)
        B, S = inputs.shape[0], inputs.shape[1] - 1
        flat_in = np.ascontiguousarray(inputs[:, :S].reshape(B * S, -1))
    D, H, nl = cfg["dim"], cfg["heads"], cfg["layers"]
    hd = D // H
    act = cfg.get("ffn_activation", 3)
    rows = B * S
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))

    def seg_rope(m, inverse=False):
        out = m.copy()
        for b in range(B):
            out[b * S:(b + 1) * S] = rope(m[b * S:(b + 1) * S], H, inverse=inverse)
        return out

    # forward with cache
    if discrete:
        x = embed_tokens(ids, w["token_embedding"])
    else:
        x = batch_dot_add_bias(w["input_proj"], flat_in, w["input_bias"])
    cache = []
    for L in w["layers"]:
        c = {"input": x}
        q, k, v = project_qkv(x, L["wq"], L["bq"], L["wk"], L["bk"], L["wv"], L["bv"])
        q, k = seg_rope(q), seg_rope(k)
        att = np.vstack([sdpa(q[b * S:(b + 1) * S], k[b * S:(b + 1) * S], v[b * S:(b + 1) * S], H, causal=True)
                         for b in range(B)])
        c.update(q=q, k=k, v=v, att=att)
        ao = project_output_batch(att, L["wo"], L["bo"])
        n1, c["m1"], c["v1"], c["n1"], c["r1"] = residual_layernorm_forward(x, ao, L["ln1_g"], L["ln1_b"])
        c["normed1"] = n1
        h = batch_dot_add_bias(L["ffn_w1"], n1, L["ffn_b1"])
        h = activation(h, act)
        ff = batch_dot_add_bias(L["ffn_w2"], h, L["ffn_b2"])
        x, c["m2"], c["v2"], c["n2"], c["r2"] = residual_layernorm_forward(n1, ff, L["ln2_g"], L["ln2_b"])
        cache.append(c)
    logits = project_output_batch(x, w["out_proj"], w["out_bias"])
    if discrete:
        loss, dl = cross_entropy(logits, targets, rows)
    elif reg is not None:
        tg = np.ascontiguousarray(_f32(reg)[:, 1:].reshape(B * S, -1))
        loss, dl = mse_loss(logits, tg, rows)
    else:
        loss, dl = cross_entropy(logits, np.ascontiguousarray(np.asarray(cls, np.int32)[:, 1:].reshape(-1)), rows)
    if not (np.isfinite(loss) and np.all(np.isfinite(dl))):
        return None
    if B > 1:
        scale_inplace(dl, float(B))

    dx, g["out_proj"], g["out_bias"] = backprop_output_projection(dl, x, w["out_proj"], g["out_proj"],
                                                                  g["out_bias"])
    for li in reversed(range(nl)):
        L, c, G = w["layers"][li], cache[li], g["layers"][li]
        dr2, dg2, db2 = layernorm_backward(dx, c["n2"], L["ln2_g"], c["r2"], c["m2"], c["v2"])
        G["ln2_g"] += dg2
        G["ln2_b"] += db2
        wg, bg = [G["ffn_w1"], G["ffn_w2"]], [G["ffn_b1"], G["ffn_b2"]]
        dn1 = ffn_input_gradient(c["normed1"], dr2, [L["ffn_w1"], L["ffn_w2"]], [L["ffn_b1"], L["ffn_b2"]],
                                 [act, 0], wg, bg)
        dn1 += dr2
        dr1, dg1, db1 = layernorm_backward(dn1, c["n1"], L["ln1_g"], c["r1"], c["m1"], c["v1"])
        G["ln1_g"] += dg1
        G["ln1_b"] += db1
        G["wo"], G["bo"], dcat = backprop_linear_projection(c["att"], dr1, L["wo"], G["wo"], G["bo"],
                                                            np.zeros((rows, D), np.float32))
        parts = [mha_backward(c["q"][b * S:(b + 1) * S], c["k"][b * S:(b + 1) * S], c["v"][b * S:(b + 1) * S],
                              dcat[b * S:(b + 1) * S], H, scale, use_decoder_mask=True) for b in range(B)]
        dq, dk, dv = (np.vstack([p[i] for p in parts]) for i in range(3))
        dq, dk = seg_rope(dq, inverse=True), seg_rope(dk, inverse=True)
        dxa, G["wq"], G["bq"], G["wk"], G["bk"], G["wv"], G["bv"] = backprop_qkv(
            c["input"], dq, dk, dv, L["wq"], L["wk"], L["wv"], G["wq"], G["bq"], G["wk"], G["bk"], G["wv"], G["bv"])
        dx = dxa + dr1
    if discrete:
        g["token_embedding"] = accumulate_token_embedding_grad(g["token_embedding"], dx, ids)
        g.setdefault("_ids", []).append(ids)
    else:
        g["input_proj"], g["input_bias"] = backprop_input_projection(dx, flat_in, g["input_proj"],
                                                                      g["input_bias"])
    return loss


def train_batch(cfg: dict, weights: dict, batch, lr: float, clip: float = 1.0, use_clipping: bool = True):
    """TransformerTrainer.TrainBatchDiscrete (TransformerTrainer.cs:217-327):
    sequences shorter than 2 tokens or with ids outside the vocabulary are
    skipped, the rest are bucketed by length in order of first appearance;
    per bucket a forward pass with cache (:540-622, segmented attention
    :723-848), cross-entropy over the next-token targets (:660-674) with
    dLogits scaled by the bucket size when it holds several sequences, and
    the backward pass (:874-987, 989-1060) accumulate the gradients; then the
    1/validCount scale, the global norm, clipping and the SGD update
    (:311-327, :1269-1384).  ``weights`` (the lm_weights layout) is not
    modified.  Returns (loss, grads, new_weights); grads are the gradients
    the update applied, keyed like weights, plus ``norm`` (the pre-clipping
    global norm, None when nothing was valid)."""
    buckets = {}
    for seq in batch:
        seq = np.asarray(seq, np.int32)
        if seq.size < 2 or seq.min() < 0 or seq.max() >= cfg["vocab"]:
            continue
        buckets.setdefault(seq.size - 1, []).append(seq)
    work = [(len(m), {"seqs": np.stack(m)}) for m in buckets.values()]
    return _train_core(cfg, weights, work, lr, clip, use_clipping, discrete=True)


def train_batch_continuous(cfg: dict, weights: dict, inputs, lr: float, reg_targets=None, class_targets=None,
                           clip: float = 1.0, use_clipping: bool = True):
    """TransformerTrainer.TrainBatchContinuous (TransformerTrainer.cs:337-485)
    for a continuous-input model (the continuous_lm_weights layout): window i
    is inputs[i] [T_i, F]; with reg_targets (TimeSeriesRegression) its targets
    are reg_targets[i] [>= T_i, O] and the loss is MSE, with class_targets
    (TimeSeriesClassification) they are class ids class_targets[i] (>= T_i of
    them) and the loss is cross-entropy; row t predicts step t + 1.  Windows
    shorter than 2 steps, with non-finite values or invalid targets
    (:1480-1502) are skipped; the rest are bucketed by length like the token
    trainer."""
    F, O = cfg["input_dim"], cfg["output_dim"]
    buckets = {}
    for i, x in enumerate(inputs):
        if x is None:
            continue
        x = _f32(x)
        T = x.shape[0]
        if T < 2 or x.shape[1] != F or not np.all(np.isfinite(x)):
            continue
        if reg_targets is not None:
            t = reg_targets[i] if i < len(reg_targets) else None
            if t is None:
                continue
            t = _f32(t)
            if t.shape[0] < T or t.shape[1] != O or not np.all(np.isfinite(t)):
                continue
            buckets.setdefault(T - 1, []).append((x, t[:T]))
        else:
            t = class_targets[i] if class_targets is not None and i < len(class_targets) else None
            if t is None:
                continue
            t = np.asarray(t, np.int32)
            if t.size < T or np.any((t[1:T] < 0) | (t[1:T] >= O)):
                continue
            buckets.setdefault(T - 1, []).append((x, t[:T]))
    work = []
    for m in buckets.values():
        kw = {"inputs": np.stack([a for a, _ in m])}
        if reg_targets is not None:
            kw["reg"] = np.stack([b for _, b in m])
        else:
            kw["cls"] = np.stack([b for _, b in m])
        work.append((len(m), kw))
    return _train_core(cfg, weights, work, lr, clip, use_clipping, discrete=False)


def _train_core(cfg, weights, work, lr, clip, use_clipping, discrete):
    w = weights
    first = "token_embedding" if discrete else "input_proj"
    z = lambda a: np.zeros_like(_f32(a))
    g = {k: z(w[k]) for k in ((first,) if discrete else ("input_proj", "input_bias"))}
    g.update({"out_proj": z(w["out_proj"]), "out_bias": z(w["out_bias"]),
              "layers": [{k: z(v) for k, v in L.items()} for L in w["layers"]]})
    total_loss = np.float32(0)
    valid = 0
    for n, kw in work:
        loss = _bucket_forward_backward(cfg, w, g, **kw)
        if loss is None:
            continue
        total_loss = np.float32(total_loss + (np.float32(loss) * np.float32(n) if n > 1 else np.float32(loss)))
        valid += n
    neww = {k: _f32(v).copy() for k, v in w.items() if k != "layers"}
    neww["layers"] = [{k: _f32(v).copy() for k, v in L.items()} for L in w["layers"]]
    ids = np.concatenate(g.pop("_ids")) if "_ids" in g else np.zeros(0, np.int32)
    if valid == 0:
        g["norm"] = None
        return 0.0, g, neww
    loss = float(np.float32(total_loss / np.float32(valid)))

    def walk(d):  # every gradient / parameter array once
        if discrete:
            yield d["token_embedding"]
        else:
            yield d["input_proj"]
            yield d["input_bias"]
        yield d["out_proj"]
        yield d["out_bias"]
        for L in d["layers"]:
            for k in _ATTN + _ATTN_B:
                yield L[k]
        for L in d["layers"]:
            yield L["ln1_g"]
            yield L["ln1_b"]
        for L in d["layers"]:
            yield L["ln2_g"]
            yield L["ln2_b"]
        for L in d["layers"]:
            for k in ("ffn_w1", "ffn_w2", "ffn_b1", "ffn_b2"):
                yield L[k]

    inv = float(np.float32(1.0) / np.float32(valid))
    for a in walk(g):
        scale_inplace(a, inv)
    # ComputeGradientNorm (TransformerTrainer.cs:1319-1352): the embedding
    # gradient over its touched rows in first-use order
    # (SparseRowGradientTracker.SquaredNorm) or the input projection and its
    # bias, then the terms in the trainer's grouping
    f32, sn = np.float32, lambda a: np.float32(squared_norm(a))
    if discrete:
        _, firsti = np.unique(ids, return_index=True)
        total = sn(g["token_embedding"][ids[np.sort(firsti)]])
    else:
        total = f32(f32(0) + sn(g["input_proj"]))
        total = f32(total + sn(g["input_bias"]))
    total = f32(total + sn(g["out_proj"]))
    total = f32(total + sn(g["out_bias"]))
    for G in g["layers"]:
        total = f32(total + f32(f32(f32(sn(G["wq"]) + sn(G["wk"])) + sn(G["wv"])) + sn(G["wo"])))
        total = f32(total + f32(f32(f32(sn(G["bq"]) + sn(G["bk"])) + sn(G["bv"])) + sn(G["bo"])))
    for key in ("ln1", "ln2"):
        for G in g["layers"]:
            total = f32(total + f32(sn(G[key + "_g"]) + sn(G[key + "_b"])))
    for G in g["layers"]:
        for k in ("ffn_w1", "ffn_w2", "ffn_b1", "ffn_b2"):
            total = f32(total + sn(G[k]))
    norm = float(np.sqrt(f32(total), dtype=np.float32))
    g["norm"] = norm
    if not np.isfinite(norm):
        return loss, g, neww
    if use_clipping and norm > clip:
        s = float(np.float32(clip) / np.float32(norm))
        for a in walk(g):
            scale_inplace(a, s)
    for a, p in zip(walk(g), walk(neww)):
        sgd_update(p, a, lr)
    return loss, g, neww


def num_threads() -> int:
    return int(lib().mt_num_threads())


def set_threads(n: int):
    lib().mt_set_threads(int(n))


# ---- LanguageModel restatement -------------------------------------------

class _Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "wq", "wk", "wv", "wo", "bq", "bk", "bv", "bo",
        "ln1_g", "ln1_b", "ln2_g", "ln2_b",
        "ffn_w1", "ffn_b1", "ffn_w2", "ffn_b2")]


class _LM(C.Structure):
    _fields_ = [("vocab", C.c_int), ("dim", C.c_int), ("heads", C.c_int),
                ("layers", C.c_int), ("ff", C.c_int), ("max_seq", C.c_int),
                ("ffn_activation", C.c_int),
                ("token_embedding", C.c_void_p), ("out_proj", C.c_void_p),
                ("out_bias", C.c_void_p), ("layer", C.POINTER(_Layer))]


class LanguageModel:
    """Decoder-only LanguageModel over a dict of float32 weights.

    ``weights`` keys: ``token_embedding`` [V, D], ``out_proj`` [V, D],
    ``out_bias`` [V] and ``layers``: a list of dicts with the ``_Layer``
    field names.  The arrays are kept alive by this object.
    """

    def __init__(self, cfg: dict, weights: dict):
        self.cfg = dict(cfg)
        self._keep = []

        def p(a):
            a = _f32(a)
            self._keep.append(a)
            return a.ctypes.data

        nl = cfg["layers"]
        self._layers = (_Layer * nl)()
        for i, lw in enumerate(weights["layers"]):
            for name, _ in _Layer._fields_:
                setattr(self._layers[i], name, p(lw[name]))
        self._lm = _LM(cfg["vocab"], cfg["dim"], cfg["heads"], nl, cfg["ff"],
                       cfg["max_seq"], cfg.get("ffn_activation", 3),
                       p(weights["token_embedding"]), p(weights["out_proj"]),
                       p(weights["out_bias"]),
                       C.cast(self._layers, C.POINTER(_Layer)))

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        logits = np.empty((ids.size, self.cfg["vocab"]), np.float32)
        _check(lib().ref_lm_forward(C.c_void_p(C.addressof(self._lm)), ids, ids.size, logits),
               "LanguageModel.Forward")
        return logits

    def generate_greedy(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(self.cfg["max_seq"] + max(0, max_new) + prompt.size, np.int32)
        n = C.c_int(0)
        _check(lib().ref_lm_generate_greedy(C.c_void_p(C.addressof(self._lm)), prompt, prompt.size,
                                            max_new, out, C.byref(n)), "LanguageModel.Generate")
        return out[: n.value].copy()
