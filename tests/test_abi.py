"""CPU-side checks of the C ABI: the library loads, exports exactly what
include/cdml.h declares, and rejects bad arguments before touching a device
(the reference's argument checks, e.g. AccelerationCPU.cs:1859-1862)."""
from __future__ import annotations

import ctypes as C
import subprocess

import pytest

from cdml import native as N


def test_library_exports_every_header_function():
    names = N.header_functions()
    assert len(names) >= 25
    lib = N.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    assert set(names) == set(N.SIGNATURES), "ctypes signatures out of sync with cdml.h"
    out = subprocess.run(["nm", "-D", "--defined-only", N.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T cdml_" in l}
    assert exported == set(names)


def test_version_and_error_text():
    assert b"gfx950" in N.lib().cdml_version()
    rc = N.lib().cdml_sdpa_fwd(None, 8, None, 8, None, 8, None, 8, 1, 4, 5, 8, 2, 0.5, 1, None, None)
    assert rc == N.E_CAUSAL
    assert b"causal" in N.lib().cdml_last_error()


@pytest.mark.parametrize("args,code", [
    ((None, 8, None, 8, None, 8, None, 8, 1, 4, 4, 8, 3, 0.5, 0, None, None), N.E_INVALID),  # 8 % 3
    ((None, 4, None, 8, None, 8, None, 8, 1, 4, 4, 8, 2, 0.5, 0, None, None), N.E_INVALID),  # ldq < dim
    ((None, 8, None, 8, None, 8, None, 8, 1, 4, 4, 8, 2, 0.5, 0, None, None), N.E_INVALID),  # NULL q
])
def test_sdpa_argument_checks(args, code):
    assert N.lib().cdml_sdpa_fwd(*args) == code


def test_other_argument_checks():
    L = N.lib()
    assert L.cdml_rope(None, 4, 6, 0, 3, 2, 10000.0, 0, 0, 0, None, None) == N.E_INVALID  # odd head dim
    assert L.cdml_rope(None, 4, 8, 0, 4, 2, -1.0, 0, 0, 0, None, None) == N.E_INVALID   # bad base
    assert L.cdml_rope(None, 4, 8, 2, 4, 2, 10000.0, 0, 0, 0, None, None) == N.E_INVALID  # heads past row
    assert L.cdml_linear(None, 4, None, None, None, 4, 2, 4, 4, 9, None) == N.E_INVALID   # activation
    assert L.cdml_linear(None, 2, None, None, None, 4, 2, 4, 4, 0, None) == N.E_INVALID   # ldx < in
    assert L.cdml_project_qkv(*([None] * 10), -1, 4, 4, None) == N.E_INVALID
    qkv = [C.c_void_p(16)] * 10  # never dereferenced: every case fails before a launch
    assert L.cdml_project_qkv_rope(*qkv, 8, 4, 8, 3, qkv[0], 8, 0, 0, None) == N.E_INVALID  # odd head_dim
    assert L.cdml_project_qkv_rope(*qkv, 8, 4, 8, 6, qkv[0], 8, 0, 0, None) == N.E_INVALID  # 6 !| 8
    assert L.cdml_project_qkv_rope(*qkv, 8, 4, 8, 4, qkv[0], 7, 0, 0, None) == N.E_INVALID  # row 7 > table
    assert L.cdml_project_qkv_rope(*qkv, 8, 4, 8, 4, qkv[0], 8, 1, 0, None) == N.E_INVALID  # offset past
    assert L.cdml_project_qkv_rope(*qkv, 8, 4, 8, 4, None, 8, 0, 0, None) == N.E_INVALID    # no table
    assert L.cdml_project_qkv_rope(*qkv, 0, 4, 8, 4, None, 0, 0, 0, None) == N.OK           # empty
    assert L.cdml_rope_table(None, 4, 5, 10000.0, None) == N.E_INVALID                     # odd head_dim
    assert L.cdml_rope_table(None, 4, 4, 0.0, None) == N.E_INVALID                         # bad base
    assert L.cdml_rope_table(None, 0, 4, 10000.0, None) == N.OK                            # empty
    fake, fake2 = C.c_void_p(4096), C.c_void_p(8192)  # never dereferenced: every case fails a host check
    assert L.cdml_rope_qk_table(fake, fake2, 4, 8, 3, 2, fake, 4, 0, 0, 1, None) == N.E_INVALID   # odd head dim
    assert L.cdml_rope_qk_table(fake, fake2, 4, 8, 4, 3, fake, 4, 0, 0, 1, None) == N.E_INVALID   # heads past row
    assert L.cdml_rope_qk_table(fake, fake2, 4, 8, 4, 2, fake, 3, 0, 0, 1, None) == N.E_INVALID   # table too short
    assert L.cdml_rope_qk_table(fake, fake2, 8, 8, 4, 2, fake, 5, 2, 4, 1, None) == N.E_INVALID   # offset + segment
    assert L.cdml_rope_qk_table(fake, fake, 4, 8, 4, 2, fake, 4, 0, 0, 1, None) == N.E_INVALID    # q is k
    assert L.cdml_rope_qk_table(None, fake2, 4, 8, 4, 2, fake, 4, 0, 0, 1, None) == N.E_INVALID   # NULL q
    assert L.cdml_rope_qk_table(fake, fake2, 4, 8, 4, 2, C.c_void_p(4100), 4, 0, 0, 1, None) == N.E_INVALID  # cs
    assert L.cdml_rope_qk_table(fake, fake2, -1, 8, 4, 2, fake, 4, 0, 0, 1, None) == N.E_INVALID  # negative rows
    assert L.cdml_rope_qk_table(None, None, 0, 8, 4, 2, None, 0, 0, 0, 1, None) == N.OK           # empty
    # z = NULL only for ReLU / leaky ReLU; CDML_ACT_FROM_OUTPUT only with those
    assert L.cdml_linear_preact(fake, 4, fake, None, None, fake2, 4, 4, 4, 4, 1, None) == N.E_INVALID
    assert L.cdml_linear_preact(None, 4, None, None, None, None, 4, 0, 4, 4, 3, None) == N.OK
    for act in (0x100 | 1, 0x100 | 5, 0x100 | 0, 0x200 | 3):
        assert L.cdml_linear_backward_act(None, 4, None, 4, None, None, act, None, None, 4, None, None, 0, 4, 4,
                                          None, 0, None) == N.E_INVALID, act
    sz = C.c_size_t(0)
    assert L.cdml_decode_attn_workspace_size(64, 8192, 2048, 16, C.byref(sz)) == N.OK
    assert sz.value == 4 * 64 * 16 * 32 * 130
    assert L.cdml_decode_attn_workspace_size(1, 1, 10, 3, C.byref(sz)) == N.E_INVALID
    # empty work is a no-op even without a device
    assert L.cdml_project_qkv(*([None] * 10), 0, 4, 4, None) == N.OK
    assert L.cdml_residual_layernorm(None, None, None, None, None, 0, 8, 1e-5, None) == N.OK


def test_no_device_is_reported_not_faked():
    if N.device_count() > 0:
        pytest.skip("a device is visible")
    assert N.lib().cdml_init(0) == N.E_NODEVICE
    with pytest.raises(N.CdmlError):
        N.DeviceBuffer(1024)


class _TinyLayer(C.Structure):
    """ctypes mirror of cdml_tiny_layer (include/cdml.h)."""
    _fields_ = [(n, C.c_void_p) for n in ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
                                           "ln1g", "ln1b", "ln2g", "ln2b")] + [
        ("ffw", C.c_void_p * 4), ("ffb", C.c_void_p * 4), ("ffrows", C.c_int * 4),
        ("ffcols", C.c_int * 4), ("ffact", C.c_int * 4), ("n_ff", C.c_int),
        ("kcache", C.c_void_p), ("vcache", C.c_void_p)]


class _TinyModel(C.Structure):
    """ctypes mirror of cdml_tiny_model (include/cdml.h)."""
    _fields_ = [("embedding", C.c_void_p), ("out_w", C.c_void_p), ("out_b", C.c_void_p),
                ("rope_cs", C.c_void_p), ("layers", C.c_void_p), ("n_layers", C.c_int),
                ("dim", C.c_int), ("heads", C.c_int), ("vocab", C.c_int), ("max_seq", C.c_int),
                ("eps", C.c_float)]


def _tiny_layer(dim=64, widths=(128, 64), acts=(3, 0)):
    # Addresses are never dereferenced: the checks read only the descriptor.
    L = _TinyLayer()
    for i, n in enumerate(("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
                           "ln1g", "ln1b", "ln2g", "ln2b", "kcache", "vcache")):
        setattr(L, n, 0x10000 + 256 * i)
    cols = dim
    for f, (w, a) in enumerate(zip(widths, acts)):
        L.ffw[f], L.ffb[f] = 0x20000 + 256 * f, 0x30000 + 256 * f
        L.ffrows[f], L.ffcols[f], L.ffact[f] = w, cols, a
        cols = w
    L.n_ff = len(widths)
    return L


def test_tiny_decode_descriptor_checks():
    lib = N.lib()
    check = lambda L, dim=64: lib.cdml_tiny_layer_check(C.byref(L), dim)
    assert check(_tiny_layer()) == N.OK
    assert check(_tiny_layer(), 32) == N.E_INVALID                       # first FFN width != dim
    assert check(_tiny_layer(widths=(128, 32))) == N.E_INVALID           # last width != dim
    assert check(_tiny_layer(widths=(130, 64))) == N.E_INVALID           # width not a multiple of 4
    assert check(_tiny_layer(widths=(2048, 64))) == N.E_INVALID          # width past 1024
    assert check(_tiny_layer(acts=(9, 0))) == N.E_INVALID                # activation code
    assert check(_tiny_layer(widths=(), acts=())) == N.E_INVALID         # no FFN layer
    L = _tiny_layer(); L.wk = 0x10004
    assert check(L) == N.E_INVALID                                       # unaligned weight
    L = _tiny_layer(); L.vcache = None
    assert check(L) == N.E_INVALID                                       # no cache
    L = _tiny_layer(); L.ln2b = None
    assert check(L) == N.E_INVALID                                       # no LayerNorm shift
    L = _tiny_layer(); L.bq = L.ffb[0] = None
    assert check(L) == N.OK                                              # biases may be zero
    L = _tiny_layer(); L.ffw[1] = 0x20108
    assert check(L) == N.E_INVALID                                       # unaligned FFN weight

    tok = (C.c_int * 8)()
    M = _TinyModel(0x40000, 0x50000, 0x60000, 0x70000, 0x80000, 2, 64, 4, 200, 64, 1e-5)
    decode = lambda M, batch=4, pos0=0, n=4: lib.cdml_tiny_decode(C.byref(M), tok, batch, pos0, n, None)
    assert decode(M, n=0) == N.OK                                        # empty work
    assert decode(M, pos0=62, n=3) == N.E_INVALID                        # past max_seq
    assert decode(M, batch=-1) == N.E_INVALID
    for field, value in (("dim", 512), ("heads", 3), ("max_seq", 2048), ("dim", 72)):
        bad = _TinyModel.from_buffer_copy(M); setattr(bad, field, value)
        assert decode(bad) == N.E_INVALID, field                         # outside the limits
    bad = _TinyModel.from_buffer_copy(M); bad.out_w = 0x50008
    assert decode(bad) == N.E_INVALID                                    # unaligned LM head
    bad = _TinyModel.from_buffer_copy(M); bad.layers = None
    assert decode(bad) == N.E_INVALID


def test_sdpa_bwd_workspace_sizes():
    """The drop-in backward's larger workspace is the required one plus the
    stored dS blocks (32 x 32 floats per block of the causal triangle) exactly
    when the shape can use them: causal, lq == lk, head dim 32 or 64."""
    lib = N.lib()

    def size(fn, *args):
        out = C.c_size_t(0)
        assert fn(*args, C.byref(out)) == N.OK
        return out.value

    def align(n):
        return (n + 255) // 256 * 256

    for batch, L, dim, heads, causal in ((4, 4096, 1024, 16, 1), (3, 300, 256, 8, 1), (2, 100, 96, 3, 1),
                                         (2, 100, 256, 4, 0), (2, 100, 48, 1, 1)):
        base = size(lib.cdml_sdpa_bwd_workspace_size, batch, L, L, dim, heads)
        big = size(lib.cdml_sdpa_bwd_stored_ds_workspace_size, batch, L, L, dim, heads, causal)
        hd, nb = dim // heads, (L + 31) // 32
        ds = batch * heads * nb * (nb + 1) // 2 * 1024 * 4 if causal and hd in (32, 64) else 0
        assert big == align(base) + ds, (batch, L, dim, heads, causal)
    # different query and key lengths never store dS
    assert (size(lib.cdml_sdpa_bwd_stored_ds_workspace_size, 2, 64, 128, 256, 4, 1)
            == align(size(lib.cdml_sdpa_bwd_workspace_size, 2, 64, 128, 256, 4)))
    bad = C.c_size_t(0)
    assert lib.cdml_sdpa_bwd_stored_ds_workspace_size(1, 8, 8, 10, 3, 1, C.byref(bad)) == N.E_INVALID
    assert lib.cdml_sdpa_bwd_stored_ds_workspace_size(1, 8, 8, 12, 3, 1, None) == N.E_INVALID


def test_sdpa_bwd_saved_rope_argument_checks():
    """cdml_sdpa_bwd_saved_rope refuses, before any device work, a NULL saved output,
    an odd head dim, a NULL or misaligned (cos, sin) table and a table shorter than
    the sequences."""
    lib = N.lib()
    f = C.c_void_p(0x1000)

    def call(o=f, dim=64, heads=4, cs=f, n_pos=100, lq=100, lk=100):
        return lib.cdml_sdpa_bwd_saved_rope(f, dim, f, dim, f, dim, o, dim, f, f, dim, f, dim, f, dim, f, dim,
                                            2, lq, lk, dim, heads, 0.25, 1, None, cs, n_pos, f, 1 << 20, None)
    assert call(o=None) == N.E_INVALID
    assert call(dim=60, heads=4) == N.E_INVALID          # head dim 15
    assert call(cs=None) == N.E_INVALID
    assert call(cs=C.c_void_p(0x1004)) == N.E_INVALID    # 4-byte aligned table
    assert call(n_pos=99) == N.E_INVALID                 # one position short
    assert call(n_pos=120, lq=100, lk=121) == N.E_INVALID


def test_mha_layer_fwd_argument_checks():
    """cdml_mha_layer_fwd rejects its arguments before any device work: a head dim that
    does not divide D, an odd head dim (RoPE pairs), NULL buffers and a short workspace;
    the workspace size covers Q, K, V, the attention output and the RoPE table."""
    lib = N.lib()
    sz = C.c_size_t(0)
    assert lib.cdml_mha_layer_fwd_workspace_size(2, 100, 64, 4, C.byref(sz)) == N.OK
    act = (2 * 100 * 64 * 4 + 255) // 256 * 256
    assert sz.value == 4 * act + (100 * 16 * 4 + 255) // 256 * 256
    assert lib.cdml_mha_layer_fwd_workspace_size(2, 100, 64, 3, C.byref(sz)) == N.E_INVALID
    fake = C.c_void_p(0x1000)
    w = [fake] * 9

    def call(dim, heads, ws=fake, wsb=1 << 30, x=fake):
        return lib.cdml_mha_layer_fwd(x, *w[:8], fake, 2, 16, dim, heads, 10000.0, 1, None, None, ws, wsb, None)

    assert call(64, 3) == N.E_INVALID                  # 64 % 3
    assert call(66, 2) == N.E_INVALID                  # head dim 33 is odd
    assert call(64, 4, x=None) == N.E_INVALID          # NULL input
    assert call(64, 4, wsb=1024) == N.E_INVALID        # workspace too small
    assert call(64, 4, ws=None) == N.E_INVALID         # no workspace
    assert b"workspace" in lib.cdml_last_error()
    # batch x seq_len beyond int32 rows is rejected in 64-bit arithmetic, in both entries
    assert lib.cdml_mha_layer_fwd_workspace_size(1 << 16, 1 << 16, 64, 4, C.byref(sz)) == N.E_INVALID
    assert b"exceeds" in lib.cdml_last_error()
    assert lib.cdml_mha_layer_fwd(fake, *w[:8], fake, 1 << 16, 1 << 16, 64, 4, 10000.0, 1, None, None, fake,
                                  1 << 30, None) == N.E_INVALID
    assert b"exceeds" in lib.cdml_last_error()


def test_weight_gradient_workspace_never_shrinks_with_rows():
    """A caller sizes the weight-gradient workspace once for its largest row
    count (the trainers do, per capacity): the size asked for must never
    decrease as rows grow, though the split-K chunk count itself can."""
    L = N.lib()
    n = C.c_size_t(0)
    for ind, out in ((64, 64), (64, 200), (256, 256), (1024, 1024), (256, 5), (5, 256), (4096, 1024)):
        for fn in ("cdml_linear_backward_workspace_size", "cdml_backprop_qkv_workspace_size"):
            prev = 0
            for rows in list(range(1, 3000)) + [4095 * 4, 4096 * 4, 511 * 256]:
                assert getattr(L, fn)(rows, ind, out, C.byref(n)) == N.OK
                assert n.value >= prev, f"{fn}({rows}, {ind}, {out}) = {n.value} < {prev}"
                prev = n.value

