"""cdml_decode_attn_noalloc: the decode entry point that allocates nothing.

It runs the same kernels as cdml_decode_attn with the split-K partials in
the library's static device scratch instead of a caller workspace, so its
outputs must equal cdml_decode_attn's bit for bit, call after call (the
scratch keeps the previous call's contents), and meet the oracle's bar.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cdml import native as N
from oracle import oracle as O

from conftest import assert_parity

pytestmark = pytest.mark.gpu


def _stream():
    N.init(0)
    return N.Stream()


def _case(seed, B, T, D, H, max_len=None):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, D), dtype=np.float32)
    hi = T if max_len is None else max_len
    lens = rng.integers(1, hi + 1, size=B).astype(np.int32)
    lens[0] = hi
    return q, lens


def _run_both(st, q, kc, vc, lens, B, T, D, H):
    """Both entry points on the same device inputs; returns (noalloc, workspace) outputs."""
    lib = N.lib()
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D // H)))
    dq = N.DeviceBuffer.from_array(q, st)
    dl = N.DeviceBuffer.from_array(lens, st)
    o1, o2 = N.DeviceBuffer(B * D * 4), N.DeviceBuffer(B * D * 4)
    ws = C.c_size_t(0)
    N.check(lib.cdml_decode_attn_workspace_size(B, T, D, H, C.byref(ws)))
    assert ws.value <= 32 << 20
    dws = N.DeviceBuffer(max(4, ws.value))
    N.check(lib.cdml_decode_attn_noalloc(dq.ptr, kc.ptr, vc.ptr, dl.ptr, o1.ptr, B, T, D, H, scale, st.handle))
    N.check(lib.cdml_decode_attn(dq.ptr, kc.ptr, vc.ptr, dl.ptr, o2.ptr, B, T, D, H, scale, dws.ptr, ws.value,
                                 st.handle))
    return o1.download((B, D), stream=st), o2.download((B, D), stream=st), scale


def _full_cache(st, seed, B, T, D):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((B, T, D), dtype=np.float32)
    v = rng.standard_normal((B, T, D), dtype=np.float32)
    return k, v, N.DeviceBuffer.from_array(k, st), N.DeviceBuffer.from_array(v, st)


def test_noalloc_decode_matches_workspace_entry_on_two_calls():
    st = _stream()
    # a larger call first, then a smaller one: the second must not see the
    # first call's partials, which stay in the shared scratch
    for seed, (B, T, D, H) in ((1, (32, 2048, 1024, 16)), (2, (3, 300, 256, 4))):
        print(f"[no_alloc] B={B} T={T} D={D} H={H}", flush=True)
        k, v, dk, dv = _full_cache(st, 100 + seed, B, T, D)
        q, lens = _case(seed, B, T, D, H)
        got, ref, scale = _run_both(st, q, dk, dv, lens, B, T, D, H)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
            f"noalloc differs from cdml_decode_attn at B={B} T={T} D={D} H={H}"
        idx = np.arange(B) if B <= 4 else np.array([0, 7, B - 1])
        want = O.decode_attention_batch(q[idx], k[idx], v[idx], lens[idx], H, scale, parallel=True)
        assert_parity(got[idx], want, what=f"noalloc decode vs oracle B={B} T={T} D={D} H={H}")


def test_noalloc_decode_near_scratch_limit():
    """A shape whose partials fill 97% of the scratch (128 sequences x 32 heads
    x 30 chunks of 66 floats); only the first 256 cache rows of each sequence
    are visible, so only those are uploaded."""
    st = _stream()
    B, T, D, H, vis = 128, 7680, 2048, 32, 256
    lib = N.lib()
    ws = C.c_size_t(0)
    N.check(lib.cdml_decode_attn_workspace_size(B, T, D, H, C.byref(ws)))
    assert 0.9 * (32 << 20) < ws.value <= 32 << 20
    print(f"[no_alloc] near limit: {ws.value} bytes of partials", flush=True)
    rng = np.random.default_rng(5)
    kvis = rng.standard_normal((B, vis, D), dtype=np.float32)
    vvis = rng.standard_normal((B, vis, D), dtype=np.float32)
    dk, dv = N.DeviceBuffer(B * T * D * 4), N.DeviceBuffer(B * T * D * 4)
    row = T * D * 4
    hk = N.DeviceBuffer.from_array(kvis, st)
    hv = N.DeviceBuffer.from_array(vvis, st)
    for b in range(B):
        N.check(lib.cdml_memcpy_d2d_async(dk.ptr + b * row, hk.ptr + b * vis * D * 4, vis * D * 4, st.handle))
        N.check(lib.cdml_memcpy_d2d_async(dv.ptr + b * row, hv.ptr + b * vis * D * 4, vis * D * 4, st.handle))
    st.synchronize()
    q, lens = _case(6, B, T, D, H, max_len=vis)
    got, ref, scale = _run_both(st, q, dk, dv, lens, B, T, D, H)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    idx = np.array([0, 1, 64, B - 1])
    want = O.decode_attention_batch(q[idx], kvis[idx], vvis[idx], lens[idx], H, scale, parallel=True)
    assert_parity(got[idx], want, what="noalloc decode near the scratch limit vs oracle")


def test_noalloc_decode_rejects_shapes_beyond_the_scratch():
    st = _stream()
    lib = N.lib()
    B, T, D, H = 128, 8192, 2048, 32   # 34.6 MB of partials
    ws = C.c_size_t(0)
    N.check(lib.cdml_decode_attn_workspace_size(B, T, D, H, C.byref(ws)))
    assert ws.value > 32 << 20
    small = N.DeviceBuffer(4096)  # never read: the size check comes before any launch
    rc = lib.cdml_decode_attn_noalloc(small.ptr, small.ptr, small.ptr, small.ptr, small.ptr, B, T, D, H, 0.125,
                                      st.handle)
    assert rc == N.E_INVALID
    msg = lib.cdml_last_error().decode()
    assert "static scratch" in msg and "cdml_decode_attn" in msg


def test_noalloc_decode_under_graph_capture():
    """The entry point's stated use: recorded inside cdml_graph_capture_begin /
    _end (it launches kernels only, no allocation and no memset) and replayed.
    Between replays new queries are uploaded and an eager no-allocation call
    of another shape overwrites the shared scratch; every replay must still
    equal cdml_decode_attn on the same inputs bit for bit."""
    st = _stream()
    lib, s = N.lib(), st.handle
    B, T, D, H = 8, 1500, 512, 4
    k, v, dk, dv = _full_cache(st, 300, B, T, D)
    q0, lens = _case(30, B, T, D, H)
    dq, dl = N.DeviceBuffer.from_array(q0, st), N.DeviceBuffer.from_array(lens, st)
    og, oe = N.DeviceBuffer(B * D * 4), N.DeviceBuffer(B * D * 4)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D // H)))
    ws = C.c_size_t(0)
    N.check(lib.cdml_decode_attn_workspace_size(B, T, D, H, C.byref(ws)))
    dws = N.DeviceBuffer(max(4, ws.value))
    # the other shape's eager call, which reuses the scratch between replays
    B2, T2, D2, H2 = 3, 700, 256, 2
    _, _, dk2, dv2 = _full_cache(st, 301, B2, T2, D2)
    q2, lens2 = _case(31, B2, T2, D2, H2)
    dq2, dl2, o2 = N.DeviceBuffer.from_array(q2, st), N.DeviceBuffer.from_array(lens2, st), N.DeviceBuffer(B2 * D2 * 4)
    st.synchronize()
    print(f"[no_alloc] graph capture B={B} T={T} D={D} H={H}", flush=True)
    N.check(lib.cdml_graph_capture_begin(s))
    rc = lib.cdml_decode_attn_noalloc(dq.ptr, dk.ptr, dv.ptr, dl.ptr, og.ptr, B, T, D, H, scale, s)
    g = C.c_void_p()
    N.check(lib.cdml_graph_capture_end(s, C.byref(g)))
    N.check(rc)
    assert g.value
    try:
        for rep in range(4):
            q = np.random.default_rng(40 + rep).standard_normal((B, D), dtype=np.float32)
            dq.upload(q, st)
            N.check(lib.cdml_graph_launch(g, s))
            st.synchronize()
            got = og.download((B, D), stream=st)
            N.check(lib.cdml_decode_attn(dq.ptr, dk.ptr, dv.ptr, dl.ptr, oe.ptr, B, T, D, H, scale, dws.ptr,
                                         ws.value, s))
            want = oe.download((B, D), stream=st)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep}"
            if rep == 0:
                idx = np.array([0, B - 1])
                ref = O.decode_attention_batch(q[idx], k[idx], v[idx], lens[idx], H, scale, parallel=True)
                assert_parity(got[idx], ref, what="graph replay of the noalloc decode vs oracle")
            # eager work on the shared scratch between replays
            N.check(lib.cdml_decode_attn_noalloc(dq2.ptr, dk2.ptr, dv2.ptr, dl2.ptr, o2.ptr, B2, T2, D2, H2, 0.0625,
                                                 s))
            st.synchronize()
    finally:
        N.check(lib.cdml_graph_destroy(g))


def test_init_leaves_the_last_error_alone():
    """cdml_init succeeds without writing the thread's last error (its
    no-allocation scratch lookup reports only through the entry point)."""
    lib = N.lib()
    assert lib.cdml_decode_attn_noalloc(None, None, None, None, None, 1, 1, 4, 1, 1.0, None) == N.E_INVALID
    before = lib.cdml_last_error()
    assert before
    assert lib.cdml_init(0) == N.OK
    assert lib.cdml_last_error() == before
