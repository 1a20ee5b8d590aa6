"""numpy-in, numpy-out calls of the C-ABI kernels (test helper).

Each call uploads its operands into caller-owned device buffers, enqueues one
C-ABI entry point on a stream, and downloads the result, which is what a
P/Invoke manager does per IAccelerationManager call.
"""
from __future__ import annotations

import ctypes as C
import numpy as np

from cdml import native as N

_stream = None


def stream() -> N.Stream:
    global _stream
    if _stream is None:
        N.init(0)
        _stream = N.Stream()
    return _stream


def up(a, dtype=np.float32) -> N.DeviceBuffer:
    return N.DeviceBuffer.from_array(np.ascontiguousarray(a, dtype=dtype), stream())


def down(buf, shape, dtype=np.float32):
    return buf.download(shape, dtype, stream())


def project_qkv(x, wq, bq, wk, bk, wv, bv):
    rows, ind = x.shape
    out = wq.shape[0]
    bufs = [up(a) for a in (x, wq, bq, wk, bk, wv, bv)]
    q, k, v = (N.DeviceBuffer(max(4, rows * out * 4)) for _ in range(3))
    N.check(N.lib().cdml_project_qkv(*(b.ptr for b in bufs), q.ptr, k.ptr, v.ptr, rows, ind, out,
                                     stream().handle))
    return tuple(down(t, (rows, out)) for t in (q, k, v))


def rope_table(n_pos, head_dim, base=10000.0):
    cs = N.DeviceBuffer(max(8, n_pos * head_dim * 4))
    N.check(N.lib().cdml_rope_table(cs.ptr, n_pos, head_dim, base, stream().handle))
    return down(cs, (n_pos, head_dim // 2, 2))


def project_qkv_rope(x, wq, bq, wk, bk, wv, bv, head_dim, n_pos=None, pos_offset=0, seg_len=0,
                     base=10000.0):
    rows, ind = x.shape
    out = wq.shape[0]
    if n_pos is None:
        n_pos = pos_offset + (min(rows, seg_len) if seg_len else rows)
    cs = N.DeviceBuffer(max(8, n_pos * head_dim * 4))
    N.check(N.lib().cdml_rope_table(cs.ptr, n_pos, head_dim, base, stream().handle))
    bufs = [up(a) for a in (x, wq, bq, wk, bk, wv, bv)]
    q, k, v = (N.DeviceBuffer(max(4, rows * out * 4)) for _ in range(3))
    N.check(N.lib().cdml_project_qkv_rope(*(b.ptr for b in bufs), q.ptr, k.ptr, v.ptr, rows, ind, out,
                                          head_dim, cs.ptr, n_pos, pos_offset, seg_len,
                                          stream().handle))
    return tuple(down(t, (rows, out)) for t in (q, k, v))


def linear(x, w, b, act=0):
    rows, ind = x.shape
    out = w.shape[0]
    bx, bw = up(x), up(w)
    bb = up(b) if b is not None else None
    y = N.DeviceBuffer(max(4, rows * out * 4))
    N.check(N.lib().cdml_linear(bx.ptr, ind, bw.ptr, bb.ptr if bb else None, y.ptr, out, rows, ind,
                                out, act, stream().handle))
    return down(y, (rows, out))


def sdpa_bwd(q, k, v, dout, num_heads, scale, causal=False, mask=None, batch=1):
    """cdml_sdpa_bwd on q/dout [batch*lq, D], k/v [batch*lk, D] -> (dq, dk, dv)."""
    rows_q, dim = q.shape
    rows_k = k.shape[0]
    lq, lk = rows_q // batch, rows_k // batch
    bq, bk, bv, bg = up(q), up(k), up(v), up(dout)
    dq, dk, dv = (N.DeviceBuffer(max(4, n * dim * 4)) for n in (rows_q, rows_k, rows_k))
    bm = up(mask, np.uint8) if mask is not None else None
    ws = C.c_size_t(0)
    N.check(N.lib().cdml_sdpa_bwd_workspace_size(batch, lq, lk, dim, num_heads, C.byref(ws)))
    bws = N.DeviceBuffer(max(256, ws.value))
    N.check(N.lib().cdml_sdpa_bwd(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, bg.ptr, dim, dq.ptr, dim, dk.ptr, dim,
                                  dv.ptr, dim, batch, lq, lk, dim, num_heads, scale, int(causal),
                                  bm.ptr if bm else None, bws.ptr, ws.value, stream().handle))
    return down(dq, (rows_q, dim)), down(dk, (rows_k, dim)), down(dv, (rows_k, dim))


def linear_backward(x, dy, w, wgrad, bgrad, dx=None, accumulate=False, want_dx=True):
    """cdml_linear_backward -> (wgrad, bgrad, dx) after the call (dx None when skipped)."""
    rows, ind = x.shape
    out = dy.shape[1]
    bx, bdy, bw, bwg, bbg = up(x), up(dy), up(w), up(wgrad), up(bgrad)
    bdx = up(dx) if dx is not None else N.DeviceBuffer(max(4, rows * ind * 4))
    ws = C.c_size_t(0)
    N.check(N.lib().cdml_linear_backward_workspace_size(rows, ind, out, C.byref(ws)))
    bws = N.DeviceBuffer(max(16, ws.value))
    N.check(N.lib().cdml_linear_backward(bx.ptr, ind, bdy.ptr, out, bw.ptr, bdx.ptr if want_dx else None, ind,
                                         bwg.ptr, bbg.ptr, rows, ind, out, int(accumulate), bws.ptr, ws.value,
                                         stream().handle))
    return down(bwg, (out, ind)), down(bbg, (out,)), down(bdx, (rows, ind)) if want_dx else None


def backprop_qkv(x, dq, dk, dv, wq, wk, wv, wq_grad, bq_grad, wk_grad, bk_grad, wv_grad, bv_grad):
    """cdml_backprop_qkv -> (dx, wq_grad, bq_grad, wk_grad, bk_grad, wv_grad, bv_grad)."""
    rows, ind = x.shape
    out = wq.shape[0]
    ins = [up(a) for a in (x, dq, dk, dv, wq, wk, wv)]
    grads = [up(a) for a in (wq_grad, bq_grad, wk_grad, bk_grad, wv_grad, bv_grad)]
    bdx = N.DeviceBuffer(max(4, rows * ind * 4))
    ws = C.c_size_t(0)
    N.check(N.lib().cdml_backprop_qkv_workspace_size(rows, ind, out, C.byref(ws)))
    bws = N.DeviceBuffer(max(16, ws.value))
    N.check(N.lib().cdml_backprop_qkv(*(b.ptr for b in ins), *(g.ptr for g in grads), bdx.ptr, rows, ind, out,
                                      bws.ptr, ws.value, stream().handle))
    shapes = [(out, ind), (out,)] * 3
    return (down(bdx, (rows, ind)), *(down(g, sh) for g, sh in zip(grads, shapes)))


def rope_qk_table(q, k, head_dim, num_heads, n_pos, pos_offset=0, seg_len=0, inverse=True, base=10000.0):
    """cdml_rope_qk_table on copies of q and k (k may be None) -> (q, k)."""
    rows, ld = q.shape
    cs = N.DeviceBuffer(max(8, n_pos * head_dim * 4))
    N.check(N.lib().cdml_rope_table(cs.ptr, n_pos, head_dim, base, stream().handle))
    bq, bk = up(q), (up(k) if k is not None else None)
    N.check(N.lib().cdml_rope_qk_table(bq.ptr, bk.ptr if bk else None, rows, ld, head_dim, num_heads, cs.ptr, n_pos,
                                       pos_offset, seg_len, int(inverse), stream().handle))
    return down(bq, (rows, ld)), (down(bk, (rows, ld)) if bk else None)


def rope(x, num_heads=None, start_col=0, head_dim=None, base=10000.0, inverse=False,
         pos_offset=0, seg_len=0, positions=None):
    rows, dim = x.shape
    if head_dim is None:
        head_dim = dim // num_heads
    if num_heads is None:
        num_heads = 1
    bx = up(x)
    bp = up(positions, np.int32) if positions is not None else None
    N.check(N.lib().cdml_rope(bx.ptr, rows, dim, start_col, head_dim, num_heads, base, int(inverse),
                              pos_offset, seg_len, bp.ptr if bp else None, stream().handle))
    return down(bx, (rows, dim))


def sdpa(q, k, v, num_heads, mask=None, causal=False, scale=None, batch=1):
    """q [batch*lq, D], k/v [batch*lk, D]."""
    rows_q, dim = q.shape
    lq, lk = rows_q // batch, k.shape[0] // batch
    if scale is None:  # ScaledDotProductAttention: 1f / MathF.Sqrt(headDim)
        scale = float(np.float32(1.0) / np.sqrt(np.float32(dim // num_heads)))
    bq, bk, bv = up(q), up(k), up(v)
    bo = N.DeviceBuffer(max(4, rows_q * dim * 4))
    bm = up(mask, np.uint8) if mask is not None else None
    N.check(N.lib().cdml_sdpa_fwd(bq.ptr, dim, bk.ptr, dim, bv.ptr, dim, bo.ptr, dim, batch, lq, lk, dim,
                                  num_heads, scale, int(causal), bm.ptr if bm else None,
                                  stream().handle))
    return down(bo, (rows_q, dim))


def decode(q, kcache, vcache, kv_len, num_heads, scale):
    b, dim = q.shape
    t_max = kcache.shape[1]
    ws = C.c_size_t(0)
    N.check(N.lib().cdml_decode_attn_workspace_size(b, t_max, dim, num_heads, C.byref(ws)))
    bq, bk, bv = up(q), up(kcache), up(vcache)
    bl = up(kv_len, np.int32)
    bo = N.DeviceBuffer(b * dim * 4)
    bw = N.DeviceBuffer(max(4, ws.value))
    N.check(N.lib().cdml_decode_attn(bq.ptr, bk.ptr, bv.ptr, bl.ptr, bo.ptr, b, t_max, dim, num_heads,
                                     scale, bw.ptr, ws.value, stream().handle))
    return down(bo, (b, dim))


def residual_layernorm(a, b, gamma, beta, eps=1e-5):
    rows, f = a.shape
    ba, bb, bg, bt = up(a), up(b), up(gamma), up(beta)
    y = N.DeviceBuffer(max(4, rows * f * 4))
    N.check(N.lib().cdml_residual_layernorm(ba.ptr, bb.ptr, bg.ptr, bt.ptr, y.ptr, rows, f, eps,
                                            stream().handle))
    return down(y, (rows, f))


def embed(ids, table):
    ids = np.ascontiguousarray(ids, np.int32)
    vocab, dim = table.shape
    bi, bt = up(ids, np.int32), up(table)
    bad = up(np.zeros(1, np.int32), np.int32)
    out = N.DeviceBuffer(max(4, ids.size * dim * 4))
    N.check(N.lib().cdml_embed_tokens(bi.ptr, ids.size, bt.ptr, vocab, dim, out.ptr, bad.ptr,
                                      stream().handle))
    return down(out, (ids.size, dim)), int(down(bad, (1,), np.int32)[0])


def kv_append(k_new, v_new, kcache, vcache, positions):
    b, t_max, dim = kcache.shape
    bk, bv, bkc, bvc = up(k_new), up(v_new), up(kcache), up(vcache)
    bp = up(positions, np.int32)
    N.check(N.lib().cdml_kv_cache_append(bk.ptr, bv.ptr, bkc.ptr, bvc.ptr, bp.ptr, b, t_max, dim,
                                         stream().handle))
    return down(bkc, kcache.shape), down(bvc, vcache.shape)


# ---- training step ----------------------------------------------------------

def _ws(fn, *args):
    n = C.c_size_t(0)
    N.check(getattr(N.lib(), fn)(*args, C.byref(n)))
    return N.DeviceBuffer(max(16, n.value)), n.value


def linear_preact(x, w, b, act):
    rows, ind = x.shape
    out = w.shape[0]
    bx, bw, bb = up(x), up(w), up(b)
    z, y = N.DeviceBuffer(max(4, rows * out * 4)), N.DeviceBuffer(max(4, rows * out * 4))
    N.check(N.lib().cdml_linear_preact(bx.ptr, ind, bw.ptr, bb.ptr, z.ptr, y.ptr, out, rows, ind, out, act,
                                       stream().handle))
    return down(z, (rows, out)), down(y, (rows, out))


def linear_preact_output_only(x, w, b, act):
    """cdml_linear_preact with z = NULL (ReLU / leaky ReLU) -> y."""
    rows, ind = x.shape
    out = w.shape[0]
    bx, bw, bb = up(x), up(w), up(b)
    y = N.DeviceBuffer(max(4, rows * out * 4))
    N.check(N.lib().cdml_linear_preact(bx.ptr, ind, bw.ptr, bb.ptr, None, y.ptr, out, rows, ind, out, act,
                                       stream().handle))
    return down(y, (rows, out))


def linear_backward_act(x, dy, w, wgrad, bgrad, dz=None, act=0, add=None):
    """cdml_linear_backward_act -> (dx, wgrad, bgrad)."""
    rows, ind = x.shape
    out = dy.shape[1]
    bx, bdy, bw, bwg, bbg = up(x), up(dy), up(w), up(wgrad), up(bgrad)
    bdz = up(dz) if dz is not None else None
    badd = up(add) if add is not None else None
    bdx = N.DeviceBuffer(max(4, rows * ind * 4))
    ws, nws = _ws("cdml_linear_backward_workspace_size", rows, ind, out)
    N.check(N.lib().cdml_linear_backward_act(bx.ptr, ind, bdy.ptr, out, bw.ptr, bdz.ptr if bdz else None, act,
                                             badd.ptr if badd else None, bdx.ptr, ind, bwg.ptr, bbg.ptr, rows,
                                             ind, out, ws.ptr, nws, stream().handle))
    return down(bdx, (rows, ind)), down(bwg, (out, ind)), down(bbg, (out,))


def residual_layernorm_fwd(a, b, gamma, beta, eps=1e-5):
    """-> (out, mean, var, normalized, residual) like oracle.residual_layernorm_forward."""
    rows, f = a.shape
    ba, bb, bg, bbe = up(a), up(b), up(gamma), up(beta)
    out, res, nrm = (N.DeviceBuffer(max(4, rows * f * 4)) for _ in range(3))
    mean, var = N.DeviceBuffer(max(4, rows * 4)), N.DeviceBuffer(max(4, rows * 4))
    N.check(N.lib().cdml_residual_layernorm_fwd(ba.ptr, bb.ptr, bg.ptr, bbe.ptr, out.ptr, mean.ptr, var.ptr,
                                                res.ptr, nrm.ptr, rows, f, eps, stream().handle))
    return (down(out, (rows, f)), down(mean, (rows,)), down(var, (rows,)), down(nrm, (rows, f)),
            down(res, (rows, f)))


def layernorm_backward(dout, normalized, gamma, inp, mean, var, dout2=None, dgamma0=None, dbeta0=None,
                       eps=1e-5):
    """-> (dinput, dgamma, dbeta); with dgamma0 / dbeta0 the gradients accumulate onto them."""
    rows, f = dout.shape
    acc = dgamma0 is not None
    bd, bg, bx, bm, bv = up(dout), up(gamma), up(inp), up(mean), up(var)
    bn = up(normalized) if normalized is not None else None
    bd2 = up(dout2) if dout2 is not None else None
    bdg = up(dgamma0) if acc else N.DeviceBuffer(max(4, f * 4))
    bdb = up(dbeta0) if acc else N.DeviceBuffer(max(4, f * 4))
    bdx = N.DeviceBuffer(max(4, rows * f * 4))
    ws, nws = _ws("cdml_layernorm_backward_workspace_size", rows, f)
    N.check(N.lib().cdml_layernorm_backward(bd.ptr, bd2.ptr if bd2 else None, bn.ptr if bn else None, bg.ptr,
                                            bx.ptr, bm.ptr, bv.ptr, bdx.ptr, bdg.ptr, bdb.ptr, rows, f, eps,
                                            int(acc), ws.ptr, nws, stream().handle))
    return down(bdx, (rows, f)), down(bdg, (f,)), down(bdb, (f,))


def cross_entropy(logits, targets, effective_len, grad_scale=1.0, loss_scale=1.0):
    rows, v = logits.shape
    bl, bt = up(logits), up(np.asarray(targets, np.int32), np.int32)
    bd, bloss = N.DeviceBuffer(max(4, rows * v * 4)), N.DeviceBuffer(4)
    ws, nws = _ws("cdml_cross_entropy_workspace_size", rows)
    N.check(N.lib().cdml_cross_entropy(bl.ptr, v, bt.ptr, rows, v, effective_len, grad_scale, loss_scale,
                                       bloss.ptr, bd.ptr, v, ws.ptr, nws, stream().handle))
    return float(down(bloss, (1,))[0]), down(bd, (rows, v))


def embedding_groups(ids):
    """Rows grouped by token, each group in increasing row order: (order, start, token)."""
    ids = np.asarray(ids, np.int64)
    order = np.argsort(ids, kind="stable").astype(np.int32)
    tok, start = np.unique(ids[order], return_index=True)
    return order, np.append(start, len(ids)).astype(np.int32), tok.astype(np.int32)


def embedding_grad(eg, dx, ids, dx2=None):
    rows, dim = dx.shape
    order, start, tok = embedding_groups(ids)
    beg, bdx = up(eg), up(dx)
    bdx2 = up(dx2) if dx2 is not None else None
    bo, bs, btk = (up(a, np.int32) for a in (order, start, tok))
    N.check(N.lib().cdml_embedding_grad(beg.ptr, bdx.ptr, bdx2.ptr if bdx2 else None, dim, bo.ptr, bs.ptr,
                                        btk.ptr, len(tok), dim, stream().handle))
    return down(beg, eg.shape)


def norm_and_update(weights, grads, groups, lr, prescale, use_clipping, threshold, zero_grads=False):
    """cdml_grad_norm then cdml_sgd_update -> (norm, clip, finite, new weights, grads after)."""
    bw = [up(w) for w in weights]
    bg = [up(g) for g in grads]
    params = (N.Param * len(weights))(*[N.Param(w.ptr, g.ptr, int(a.size), int(gr), 0)
                                        for w, g, a, gr in zip(bw, bg, weights, groups)])
    bp = N.DeviceBuffer(C.sizeof(params))
    N.check(N.lib().cdml_memcpy_h2d_async(bp.ptr, C.addressof(params), C.sizeof(params), stream().handle))
    res = N.DeviceBuffer(16)
    ws, nws = _ws("cdml_grad_norm_workspace_size", len(weights))
    N.check(N.lib().cdml_grad_norm(bp.ptr, len(weights), prescale, int(use_clipping), threshold, res.ptr, ws.ptr,
                                   nws, stream().handle))
    N.check(N.lib().cdml_sgd_update(bp.ptr, len(weights), lr, prescale, res.ptr, int(zero_grads),
                                    stream().handle))
    r = down(res, (3,))
    return (float(r[0]), float(r[1]), float(r[2]), [down(b, w.shape) for b, w in zip(bw, weights)],
            [down(b, g.shape) for b, g in zip(bg, grads)])
