"""The drop-in manager's boundary contract on the GPU.

* Threads: calls on distinct HipAccelerationManager instances from different
  threads are safe.  RotaryPositionEmbeddingTests.cs:304-322 builds 32
  instances inside Parallel.For, and every FFN builds a manager of its own;
  here 32 managers on 32 threads run the MultiHeadAttention.Forward sequence
  (MultiHeadAttention.cs:108-111) at the same time.
* Resident activations: an array the manager returned stays on the device,
  and the next call that receives it uploads it only when its host contents
  changed (the shadow compare of DeviceResidentCache.cs:44-60 extended from
  weights to activations).  Host edits between calls must be seen, and the
  cache must give the same bits as a manager without it.

Bar: |got - want| <= 1e-4 + 1e-3 |want| per element against the oracle.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

from cdml import host, synth
from conftest import assert_parity
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _mha_inputs(seed, L, D):
    x = synth.normal(seed, (L, D))
    w = [synth.xavier_uniform(seed + 10 + j, D, D) for j in range(4)]
    b = [np.float32(0.1) * synth.normal(seed + 20 + j, (D,)) for j in range(4)]
    return x, w, b


def _mha_manager(m, x, w, b, heads):
    """MultiHeadAttention.Forward's calls on one manager."""
    L, D = x.shape
    q, k, v = m.ProjectQKV(x, w[0], b[0], w[1], b[1], w[2], b[2])
    m.ApplyRotaryPositionEmbeddingInPlace(q, heads, 10000.0, False)
    m.ApplyRotaryPositionEmbeddingInPlace(k, heads, 10000.0, False)
    a = m.ScaledDotProductAttention(q, k, v, heads, None, True)
    return m.ProjectOutputBatch(a, w[3], b[3], L, D)


def _mha_oracle(x, w, b, heads):
    q, k, v = O.project_qkv(x, w[0], b[0], w[1], b[1], w[2], b[2])
    a = O.sdpa(O.rope(q, heads), O.rope(k, heads), v, heads, causal=True)
    return O.project_output_batch(a, w[3], b[3])


def test_32_managers_on_32_threads():
    Hm = host.module()
    n, L, D, heads = 32, 96, 64, 4
    results = [None] * n
    barrier = threading.Barrier(n, timeout=60)

    def work(i):
        try:
            m = Hm.HipAccelerationManager(0)
            x, w, b = _mha_inputs(1000 + 40 * i, L + i, D)
            barrier.wait()  # every manager exists before any computes
            ys = [_mha_manager(m, x, w, b, heads) for _ in range(3)]
            m.Dispose()
            results[i] = (x, w, b, ys)
        except BaseException as e:  # reported by the main thread
            results[i] = e

    print("[boundary] 32 managers on 32 threads", flush=True)
    threads = [threading.Thread(target=work, args=(i,)) for i in range(n)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a manager thread did not finish"
    for i, r in enumerate(results):
        assert not isinstance(r, BaseException), f"thread {i}: {r!r}"
        x, w, b, ys = r
        want = _mha_oracle(x, w, b, heads)
        for rep, y in enumerate(ys):
            assert_parity(y, want, what=f"manager {i} (L {L + i}) call {rep}")
        # repeated calls on one manager: the same bits
        assert all(np.array_equal(ys[0], y) for y in ys[1:])


def test_returned_arrays_stay_resident_and_follow_host_edits():
    Hm = host.module()
    m = Hm.HipAccelerationManager(0)
    L, D, heads = 300, 128, 4
    x, w, b = _mha_inputs(77, L, D)
    nbytes = L * D * 4
    q, k, v = m.ProjectQKV(x, w[0], b[0], w[1], b[1], w[2], b[2])
    s0 = m.transfer_stats()
    m.ApplyRotaryPositionEmbeddingInPlace(q, heads, 10000.0, False)
    m.ApplyRotaryPositionEmbeddingInPlace(k, heads, 10000.0, False)
    s1 = m.transfer_stats()
    # Q and K were on the device already: nothing uploaded, both compared
    assert s1["h2d_bytes"] == s0["h2d_bytes"]
    assert s1["h2d_skipped_bytes"] - s0["h2d_skipped_bytes"] == 2 * nbytes
    qo, ko, vo = O.project_qkv(x, w[0], b[0], w[1], b[1], w[2], b[2])
    assert_parity(q, O.rope(qo, heads), what="RoPE of the resident Q")
    # host edits of returned arrays between calls
    q[5, 3] += np.float32(1.0)
    v[7, :] *= np.float32(-1.0)
    a = m.ScaledDotProductAttention(q, k, v, heads, None, True)
    s2 = m.transfer_stats()
    assert s2["h2d_bytes"] - s1["h2d_bytes"] == 2 * nbytes  # Q and V again, K skipped
    assert_parity(a, O.sdpa(q, k, v, heads, causal=True), what="SDPA after host edits of Q and V")
    # a write that leaves the contents as they were costs no upload
    q[9, :] = q[9, :].copy()
    a2 = m.ScaledDotProductAttention(q, k, v, heads, None, True)
    assert m.transfer_stats()["h2d_bytes"] == s2["h2d_bytes"]
    assert np.array_equal(a, a2)
    # an edit of the result before it goes back in
    a[0, :] = np.float32(2.0)
    y = m.ProjectOutputBatch(a, w[3], b[3], L, D)
    assert_parity(y, O.project_output_batch(a, w[3], b[3]), what="out-proj after an edit of its input")
    # the same sequence with the cache off gives the same bits
    m0 = Hm.HipAccelerationManager(0)
    m0.SetActivationCacheLimit(0)
    assert m0.activation_cache_limit == 0
    y_cached = _mha_manager(m, x, w, b, heads)
    y_plain = _mha_manager(m0, x, w, b, heads)
    assert m0.activation_cache_entries == 0
    assert np.array_equal(y_cached, y_plain)
    m0.Dispose()
    m.Dispose()


def test_small_activation_cache_evicts_and_stays_correct():
    """A limit of three arrays: every call evicts the least recently used
    entries it does not itself use, and the results still match the oracle."""
    Hm = host.module()
    L, D, heads = 257, 64, 2
    m = Hm.HipAccelerationManager(0)
    m.SetActivationCacheLimit(3 * L * D * 4)
    x, w, b = _mha_inputs(91, L, D)
    want = _mha_oracle(x, w, b, heads)
    for rep in range(3):
        assert_parity(_mha_manager(m, x, w, b, heads), want, what=f"limited cache, call {rep}")
    m.SetActivationCacheLimit(1 << 30)
    for rep in range(2):
        assert_parity(_mha_manager(m, x, w, b, heads), want, what=f"cache back on, call {rep}")
    m.Dispose()


def test_cache_allocation_failures_fall_back_to_the_uncached_path():
    """When a cache allocation fails (injected here as an out-of-memory
    cdml_malloc would fail), the manager evicts more and retries, and an array
    it still cannot place takes the uncached scratch path: the call completes
    with the same bits as a manager with the cache off.  A process-wide budget
    smaller than one array sends every array down that path."""
    Hm = host.module()
    M = Hm.HipAccelerationManager
    L, D, heads = 300, 128, 4
    x, w, b = _mha_inputs(93, L, D)
    plain = M(0)
    plain.SetActivationCacheLimit(0)
    want = _mha_manager(plain, x, w, b, heads)
    assert_parity(want, _mha_oracle(x, w, b, heads), what="cache off")
    budget = M.ProcessActivationCacheBudget()
    m = None
    try:
        # a fresh manager allocates a cache entry for each of the sequence's
        # six activations (x, Q, K, V, attention, output)
        for fails in (1, 3, 50):
            m = M(0)
            M.InjectActivationAllocFailures(fails)
            got = _mha_manager(m, x, w, b, heads)
            M.InjectActivationAllocFailures(0)
            assert np.array_equal(got, want), f"{fails} injected failures"
            n = m.transfer_stats()["act_alloc_failures"]
            if fails < 6:
                assert n == fails and m.activation_cache_entries >= 1, (fails, n)
            else:  # every allocation failed: nothing cached, every array went through scratch
                assert n >= 6 and m.activation_cache_entries == 0, n
                # allocations work again: the next call caches and gives the same bits
                assert np.array_equal(_mha_manager(m, x, w, b, heads), want)
                assert m.activation_cache_entries >= 6
            m.Dispose()
        # a budget below one array's 64 KiB-rounded size: nothing is cached
        m = M(0)
        m2 = M(0)
        M.SetProcessActivationCacheBudget(64 << 10)
        before = M.ProcessActivationCacheBytes()
        got = _mha_manager(m2, x.copy(), w, b, heads)
        assert np.array_equal(got, want)
        assert m2.activation_cache_entries == 0
        assert M.ProcessActivationCacheBytes() <= before
        m2.Dispose()
    finally:
        M.InjectActivationAllocFailures(0)
        M.SetProcessActivationCacheBudget(budget)
        if m is not None:
            m.Dispose()
        plain.Dispose()


def test_same_pointer_with_two_shapes_in_one_call():
    """x and x[:n] share a data pointer.  Passed to one call (the attention's
    query and key rows) under a small cache, the second shape replaces the
    first's entry; the buffer already handed out for the first stays valid
    until the call ends (it is parked, not freed or reused), and the result
    matches the oracle."""
    Hm = host.module()
    L, n, D, heads = 256, 200, 64, 2
    q = synth.normal(95, (L, D))
    kv = synth.normal(96, (L, D))
    m = Hm.HipAccelerationManager(0)
    m.SetActivationCacheLimit(2 * L * D * 4)
    try:
        for rep in range(3):
            # Q rows [L, D] and K = V = the first n rows of the same array
            got = m.MultiHeadAttentionForward(q, q[:n], q[:n], heads, 0.125)
            want = O.mha_forward(q, np.ascontiguousarray(q[:n]), np.ascontiguousarray(q[:n]), heads, 0.125)
            assert_parity(got, want, what=f"aliased shapes, call {rep}")
            # an unrelated call in between, which acquires and evicts
            m.ProjectOutputBatch(kv, synth.xavier_uniform(97, D, D), np.zeros(D, np.float32), L, D)
    finally:
        m.Dispose()


def test_inplace_rope_on_resident_arrays_follows_host_edits():
    """In-place RoPE on a returned 4 MiB activation runs on the device copy
    while the host array is compared with its shadow.  An unchanged array is
    not uploaded; an array edited on the host since the manager returned it
    is rotated from the edited contents; and the shadow after either path
    holds the rotated contents (a third rotation starts from them)."""
    Hm = host.module()
    L, D, heads = 1024, 1024, 16
    x = synth.normal(98, (L, D))
    w = [synth.xavier_uniform(99 + j, D, D) for j in range(3)]
    b = [np.zeros(D, np.float32)] * 3
    m = Hm.HipAccelerationManager(0)
    try:
        q, _, _ = m.ProjectQKV(x, w[0], b[0], w[1], b[1], w[2], b[2])
        want = O.rope(q, heads)
        s0 = m.transfer_stats()
        m.ApplyRotaryPositionEmbeddingInPlace(q, heads, 10000.0, False)  # unchanged since returned
        s1 = m.transfer_stats()
        assert_parity(q, want, what="in-place RoPE of an unchanged resident array")
        assert s1["h2d_bytes"] == s0["h2d_bytes"] and s1["h2d_skipped_bytes"] - s0["h2d_skipped_bytes"] >= q.nbytes
        q[5, 7] += 1.0  # a host edit after the last call
        q[L - 1, D - 1] = -3.0
        want = O.rope(q, heads)
        m.ApplyRotaryPositionEmbeddingInPlace(q, heads, 10000.0, False)
        s2 = m.transfer_stats()
        assert_parity(q, want, what="in-place RoPE after a host edit")
        assert s2["h2d_bytes"] - s1["h2d_bytes"] >= q.nbytes
        want = O.rope(q, heads, inverse=True)
        m.ApplyRotaryPositionEmbeddingInPlace(q, heads, 10000.0, True)  # from the shadow of the last result
        assert_parity(q, want, what="inverse RoPE after the edited rotation")
        # the same array through a manager without the cache gives the same bits
        m0 = Hm.HipAccelerationManager(0)
        m0.SetActivationCacheLimit(0)
        q2 = want.copy()
        m0.ApplyRotaryPositionEmbeddingInPlace(q2, heads, 10000.0, False)
        q3 = q.copy()
        m.ApplyRotaryPositionEmbeddingInPlace(q, heads, 10000.0, False)
        m0.ApplyRotaryPositionEmbeddingInPlace(q3, heads, 10000.0, False)
        assert np.array_equal(q, q3)
        m0.Dispose()
    finally:
        m.Dispose()


def test_project_qkv_split_downloads_and_host_edits():
    """ProjectQKV with at least 2048 rows and 16 MiB per output runs in two
    row halves, the first half's downloads overlapping the second half's
    kernel on a copy stream.  Rows on both sides of the split (1280 of 2500)
    meet the bar against the oracle, and a host edit of the resident input
    between two calls reruns both halves from the edited contents."""
    Hm = host.module()
    rows, D = 2500, 2048
    x = synth.normal(110, (rows, D))
    w = [synth.xavier_uniform(111 + j, D, D) for j in range(3)]
    b = [np.float32(0.1) * synth.normal(114 + j, (D,)) for j in range(3)]
    m = Hm.HipAccelerationManager(0)
    try:
        sample = np.array([0, 1, 1279, 1280, 1281, 2047, 2048, rows - 1])
        for step in range(3):
            if step == 2:
                x[1279, 3] += 2.0  # edited on the host after the manager saw it
                x[2400, :] *= 0.5
            q, k, v = m.ProjectQKV(x, w[0], b[0], w[1], b[1], w[2], b[2])
            rws = np.concatenate([sample, [2400]])
            want = O.project_qkv(np.ascontiguousarray(x[rws]), w[0], b[0], w[1], b[1], w[2], b[2])
            for got, wnt, n in zip((q, k, v), want, "QKV"):
                assert_parity(got[rws], wnt, what=f"split ProjectQKV {n}, call {step}")
        assert m.transfer_stats()["h2d_skipped_bytes"] >= x.nbytes  # the unedited second call
    finally:
        m.Dispose()
