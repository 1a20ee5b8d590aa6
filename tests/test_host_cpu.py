"""CPU-side checks of the C++ host layer: the module loads, and every
argument rule the reference enforces raises the reference's exception kind
before any device work (AccelerationCPU.cs validation blocks,
AccelerationManagerParityTests.cs:454-458, TransformerConfig.cs:62-102,
LanguageModel.cs:482-600).  Without a device a compute call must fail loudly
with InvalidOperationException, never fall back to the CPU."""
from __future__ import annotations

import numpy as np
import pytest

from cdml import host, native as N, synth

H = host.module()
M, Vec = synth.matrix, synth.vector


@pytest.fixture(scope="module")
def mgr():
    return H.HipAccelerationManager(0)


def test_exception_hierarchy_mirrors_dotnet():
    assert issubclass(H.ArgumentNullException, H.ArgumentException)
    assert issubclass(H.ArgumentOutOfRangeException, H.ArgumentException)
    assert issubclass(H.ArgumentException, ValueError)
    assert issubclass(H.InvalidOperationException, RuntimeError)


def test_sdpa_argument_rules(mgr):
    q, k, v = M(4, 8, 121), M(5, 8, 122), M(5, 8, 123)
    with pytest.raises(H.ArgumentException, match="causal"):
        mgr.ScaledDotProductAttention(q, k, v, 2, None, True)  # :454-458
    with pytest.raises(H.ArgumentNullException):
        mgr.ScaledDotProductAttention(None, k, v, 2)
    with pytest.raises(H.ArgumentOutOfRangeException):
        mgr.ScaledDotProductAttention(q, k, v, 0)
    with pytest.raises(H.ArgumentException, match="divisible"):
        mgr.ScaledDotProductAttention(q, k, v, 3)
    with pytest.raises(H.ArgumentException, match="Mask shape"):
        mgr.ScaledDotProductAttention(q, k, v, 2, np.ones((4, 4), bool))
    with pytest.raises(H.ArgumentException, match="V row count"):
        mgr.ScaledDotProductAttention(q, k, v[:4], 2)
    with pytest.raises(H.ArgumentException, match="at least one row"):
        mgr.ScaledDotProductAttention(q[:0], k, v, 2)


def test_mha_forward_argument_rules(mgr):
    q, k, v = M(4, 6, 31), M(4, 6, 32), M(4, 6, 33)
    with pytest.raises(H.ArgumentException, match="same sequence length"):
        mgr.MultiHeadAttentionForward(q, k, v[:3], 2, 0.5)
    with pytest.raises(H.ArgumentException, match="Mask shape"):
        mgr.MultiHeadAttentionForward(q, k, v, 2, 0.5, np.ones((3, 4), bool))
    out = mgr.MultiHeadAttentionForward(q[:0], k, v, 2, 0.5)  # empty query: zeros, no device work
    assert out.shape == (0, 6)


def test_project_qkv_argument_rules(mgr):
    x = M(6, 5, 124)
    w, b = M(8, 5, 125), Vec(8, 128)
    with pytest.raises(H.ArgumentNullException):
        mgr.ProjectQKV(x, w, None, w, b, w, b)
    with pytest.raises(H.ArgumentException, match="WK input dimension"):
        mgr.ProjectQKV(x, w, b, M(8, 4, 1), b, w, b)
    with pytest.raises(H.ArgumentException, match="biasV length"):
        mgr.ProjectQKV(x, w, b, w, b, w, Vec(7, 1))
    with pytest.raises(H.ArgumentException, match="output dimensions must match"):
        mgr.ProjectQKV(x, w, b, M(7, 5, 1), Vec(7, 1), w, b)


def test_other_argument_rules(mgr):
    x = M(4, 8, 1)
    with pytest.raises(H.ArgumentOutOfRangeException):
        mgr.BatchDotProductAddBias(M(3, 8, 2), x, 2, 3, Vec(3, 1))
    with pytest.raises(H.ArgumentException, match="Bias length"):
        mgr.BatchDotProductAddBias(M(3, 8, 2), x, Vec(4, 1))
    with pytest.raises(H.ArgumentException, match="even per-head"):
        mgr.ApplyRotaryPositionEmbeddingInPlace(np.zeros((2, 6), np.float32), 2, 10000.0, False)
    with pytest.raises(H.ArgumentOutOfRangeException):
        mgr.ApplyRotaryPositionEmbeddingInPlace(np.zeros((2, 8), np.float32), 2, -1.0, False)
    with pytest.raises(H.ArgumentException, match="Head range"):
        mgr.ApplyRotaryPositionEmbeddingHeadInPlace(np.zeros((2, 8), np.float32), 6, 4, 10000.0, False)
    with pytest.raises(H.ArgumentOutOfRangeException):
        mgr.EmbedTokenIds(np.array([0, 6], np.int32), M(6, 5, 64), 5)
    with pytest.raises(H.ArgumentException, match="Embedding dimension mismatch"):
        mgr.EmbedTokenIds(np.array([0], np.int32), M(6, 5, 64), 4)
    assert mgr.EmbedTokenIds(np.zeros(0, np.int32), M(6, 5, 64), 5).shape == (0, 5)
    with pytest.raises(H.ArgumentException, match="Residual input dimensions"):
        mgr.ResidualLayerNorm(x, M(4, 7, 1), Vec(8, 1), Vec(8, 2))
    with pytest.raises(H.ArgumentOutOfRangeException):
        mgr.CreateCausalMask(-1)


def test_create_causal_mask_is_lower_triangular(mgr):
    # AccelerationCPU.cs:1566-1586 / parity test :410-421
    m = mgr.CreateCausalMask(5)
    assert m.dtype == bool and np.array_equal(m, np.tril(np.ones((5, 5), bool)))


def test_config_and_model_rules():
    with pytest.raises(H.ArgumentException, match="divisible"):
        host.config({"vocab": 12, "dim": 8, "heads": 3, "layers": 1, "ff": 16, "max_seq": 8})
    with pytest.raises(H.ArgumentException, match="even per-head"):
        host.config({"vocab": 12, "dim": 6, "heads": 2, "layers": 1, "ff": 16, "max_seq": 8})
    # ConfigBase.RequirePositive throws ArgumentException itself (ConfigBase.cs:16-22)
    with pytest.raises(H.ArgumentException, match="NumLayers must be positive, got 0") as e:
        host.config({"vocab": 12, "dim": 8, "heads": 2, "layers": 0, "ff": 16, "max_seq": 8})
    assert type(e.value) is H.ArgumentException
    base = {"vocab": 12, "dim": 8, "heads": 2, "layers": 1, "ff": 16, "max_seq": 8}
    for field, value, text in [("DataType", 4, "Invalid DataType: 4"),
                               ("CostFunction", 6, "Invalid CostFunction: 6"),
                               ("ActivationDistribution", 2, "Invalid ActivationDistribution: 2"),
                               ("AccelerationType", 5, "Invalid AccelerationType value: 5"),
                               ("AccelerationDeviceId", -1, "AccelerationDeviceId must be non-negative"),
                               ("L2RegulationLamda", -0.5, "L2RegulationLamda must be non-negative"),
                               ("GradientClippingThreshold", 0.0, "GradientClippingThreshold must be positive")]:
        with pytest.raises(H.ArgumentException, match=text):
            host.config(base, **{field: value})
    with pytest.raises(H.ArgumentException, match="TimeSeriesClassification requires OutputDim >= 2"):
        host.config(dict(base, discrete=False), DataType=2)
    cfg = {"vocab": 12, "dim": 8, "heads": 2, "layers": 1, "ff": 16, "max_seq": 8}
    lm, _ = host.language_model(cfg, synth.lm_weights(cfg, 1))
    with pytest.raises(H.ArgumentOutOfRangeException):
        lm.Generate(np.array([1, 2], np.int32), 3, temperature=0.0)
    with pytest.raises(H.ArgumentOutOfRangeException):
        lm.Generate(np.array([1, 2], np.int32), -1)
    with pytest.raises(H.ArgumentOutOfRangeException):
        lm.Forward(np.array([1, 12], np.int32))
    with pytest.raises(H.ArgumentException, match="exceeds MaxSequenceLength"):
        lm.Forward(np.zeros(9, np.int32))
    with pytest.raises(H.ArgumentException, match="at least one token"):
        lm.Forward(np.zeros(0, np.int32))
    with pytest.raises(H.InvalidOperationException):
        lm.ForwardContinuous(np.zeros((2, 1), np.float32))
    full = np.zeros(8, np.int32)  # a full prompt comes back unchanged (LanguageModel.cs:495-496)
    assert np.array_equal(lm.Generate(full, 5), full)
    assert np.array_equal(lm.Generate(np.array([3, 4], np.int32), 0), [3, 4])
    with pytest.raises(H.ArgumentException, match="shape mismatch"):
        lm.load_weights(synth.lm_weights(dict(cfg, vocab=13), 1))


def test_backward_argument_rules(mgr):
    """MultiHeadAttentionBackwardCore (AccelerationCPU.cs:1037-1063) and
    BackpropQKV (:2071-2133) checks, in the reference's order."""
    q, k, v = M(4, 8, 41), M(5, 8, 42), M(5, 8, 43)
    d = M(4, 8, 44)
    with pytest.raises(H.ArgumentNullException, match="dConcatenated"):
        mgr.MultiHeadAttentionBackward(q, k, v, None, 2, 0.5)
    with pytest.raises(H.ArgumentOutOfRangeException, match="numHeads"):
        mgr.MultiHeadAttentionBackward(q, k, v, d, 0, 0.5)
    with pytest.raises(H.ArgumentException, match="same embedding dimension"):
        mgr.MultiHeadAttentionBackward(q, k[:, :6], v, d, 2, 0.5)
    with pytest.raises(H.ArgumentException, match="same sequence length"):
        mgr.MultiHeadAttentionBackward(q, k, v[:4], d, 2, 0.5)
    with pytest.raises(H.ArgumentException, match="dConcatenated shape"):
        mgr.MultiHeadAttentionBackward(q, k, v, d[:3], 2, 0.5)
    with pytest.raises(H.ArgumentException, match="divisible"):
        mgr.MultiHeadAttentionBackward(q, k, v, d, 3, 0.5)
    with pytest.raises(H.ArgumentException, match="Mask shape"):
        mgr.MultiHeadAttentionBackward(q, k, v, d, 2, 0.5, np.ones((4, 4), bool))
    z = np.zeros
    x, dq = M(3, 6, 45), M(3, 4, 46)
    w = M(4, 6, 47)
    g = lambda: (z((4, 6), np.float32), z(4, np.float32), z((4, 6), np.float32), z(4, np.float32),
                 z((4, 6), np.float32), z(4, np.float32))
    with pytest.raises(H.ArgumentNullException, match="WKGrad"):
        gg = list(g()); gg[2] = None
        mgr.BackpropQKV(x, dq, dq, dq, w, w, w, *gg)
    with pytest.raises(H.ArgumentException, match="dimensions must match"):
        mgr.BackpropQKV(x, dq, dq, dq, w, w[:3], w, *g())
    with pytest.raises(H.ArgumentException, match="row counts"):
        mgr.BackpropQKV(x, dq, dq[:2], dq, w, w, w, *g())
    with pytest.raises(H.ArgumentException, match="WVGrad shape"):
        gg = list(g()); gg[4] = z((4, 5), np.float32)
        mgr.BackpropQKV(x, dq, dq, dq, w, w, w, *gg)
    with pytest.raises(H.ArgumentException, match="bias gradient lengths"):
        gg = list(g()); gg[1] = z(3, np.float32)
        mgr.BackpropQKV(x, dq, dq, dq, w, w, w, *gg)
    with pytest.raises(H.ArgumentException, match="dInput"):
        mgr.BackpropLinearProjection(x, dq, w, z((4, 6), np.float32), z(4, np.float32), z((2, 6), np.float32))
    with pytest.raises(H.ArgumentException, match="outputDim"):
        mgr.BackpropOutputProjection(dq, x, w, z((4, 6), np.float32), z(4, np.float32), 3, 5, 6)
    # empty inputs need no device: zero-row gradients come back
    r = mgr.MultiHeadAttentionBackward(q[:0], k, v, d[:0], 2, 0.5, True)
    assert [a.shape for a in r] == [(0, 8), (5, 8), (5, 8)] and not any(a.any() for a in r)


def test_training_method_argument_rules(mgr):
    z = np.zeros
    with pytest.raises(H.ArgumentException, match="don't match"):
        mgr.MatrixMultiply(M(3, 4, 1), M(5, 2, 2))
    with pytest.raises(H.ArgumentException, match="A\\*B\\^T"):
        mgr.MatrixMultiplyTranspose(M(3, 4, 1), M(5, 2, 2))
    with pytest.raises(H.ArgumentException, match="Residual input dimensions"):
        mgr.ResidualLayerNormForward(M(3, 4, 1), M(3, 5, 2), Vec(4, 3), Vec(4, 4))
    with pytest.raises(H.ArgumentException, match="gamma"):
        mgr.LayerNormBackward(M(3, 4, 1), M(3, 4, 2), Vec(5, 3), M(3, 4, 4), Vec(3, 5), Vec(3, 6))
    with pytest.raises(H.ArgumentOutOfRangeException, match="targetStart"):
        mgr.CrossEntropyLossAndGradient(M(3, 4, 1), np.array([0, 1], np.int32), 1, 2)
    with pytest.raises(H.ArgumentOutOfRangeException, match="Target out of range"):
        mgr.CrossEntropyLossAndGradient(M(3, 4, 1), np.array([0, 4, 1], np.int32), 0, 3)
    loss, dl = mgr.CrossEntropyLossAndGradient(M(3, 4, 1), np.array([0, 1], np.int32), 0, 0)
    assert loss == 0 and dl.shape == (3, 4) and not dl.any()  # no device work
    with pytest.raises(H.ArgumentException, match="Target shape"):
        mgr.MSELossAndGradient(M(3, 2, 1), M(3, 3, 2), 0, 2)
    with pytest.raises(H.ArgumentException, match="Target shape"):
        mgr.MSELossAndGradient(M(3, 2, 1), M(3, 2, 2), 2, 2)
    with pytest.raises(H.ArgumentException, match="effectiveLen exceeds"):
        mgr.MSELossAndGradient(M(3, 2, 1), M(5, 2, 2), 0, 4)
    loss, dp = mgr.MSELossAndGradient(M(3, 2, 1), M(3, 2, 2), 1, 0)
    assert loss == 0 and dp.shape == (3, 2) and not dp.any()  # no device work
    with pytest.raises(H.ArgumentOutOfRangeException, match="tokenStart"):
        mgr.AccumulateTokenEmbeddingGrad(z((5, 2), np.float32), M(3, 2, 1), np.array([0, 1], np.int32), 0, 3, 2)
    with pytest.raises(H.ArgumentOutOfRangeException, match="Token out of range"):
        mgr.AccumulateTokenEmbeddingGrad(z((5, 2), np.float32), M(2, 2, 1), np.array([0, 5], np.int32), 0, 2, 2)


def test_continuous_trainer_argument_rules(mgr):
    """TrainContinuous's checks (TransformerTrainer.cs:130-168), the
    token/continuous entry split, BackpropInputProjection's slice rules
    (AccelerationCPU.cs:2280-2305) and the slice forwards' validation
    (LanguageModel.cs:602-668): all raised before any device work."""
    z = np.zeros
    with pytest.raises(H.ArgumentOutOfRangeException, match="inputRowStart"):
        mgr.BackpropInputProjection(M(3, 4, 1), M(4, 2, 2), 2, z((4, 2), np.float32), z(4, np.float32), 3, 4, 2)
    with pytest.raises(H.ArgumentException, match="smaller than the requested"):
        mgr.BackpropInputProjection(M(3, 4, 1), M(4, 2, 2), 0, z((4, 3), np.float32), z(4, np.float32), 3, 4, 3)
    with pytest.raises(H.ArgumentException, match="weightGrad or biasGrad"):
        mgr.BackpropInputProjection(M(3, 4, 1), M(4, 2, 2), 0, z((3, 2), np.float32), z(4, np.float32), 3, 4, 2)
    cfg = {"dim": 8, "heads": 2, "layers": 1, "ff": 16, "max_seq": 8, "discrete": False, "input_dim": 3,
           "output_dim": 2}
    lm, _ = host.language_model(cfg, synth.continuous_lm_weights(cfg, 2))
    t = H.TransformerTrainer(lm, H.TrainingConfig())
    x = [z((5, 3), np.float32)]
    with pytest.raises(H.ArgumentException, match="regressionTargets is required"):
        t.TrainContinuous(x)
    with pytest.raises(H.ArgumentException, match="length must match"):
        t.TrainContinuous(x, regressionTargets=[])
    with pytest.raises(H.ArgumentException, match="feature dimension 4, expected 3"):
        t.TrainContinuous([z((5, 4), np.float32)], regressionTargets=[z((5, 2), np.float32)])
    with pytest.raises(H.ArgumentException, match="No valid sequences"):
        t.TrainContinuous([z((1, 3), np.float32), None], regressionTargets=[z((1, 2), np.float32), None])
    with pytest.raises(H.InvalidOperationException, match="TrainContinuous"):
        t.Train([np.array([1, 2], np.int32)])
    with pytest.raises(H.InvalidOperationException, match="token model"):
        t.TrainBatch([np.array([1, 2], np.int32)], 0.1)
    with pytest.raises(H.InvalidOperationException, match="ForwardContinuousSlice"):
        t.Validate([np.array([0, 1, 0], np.int32)])  # ids inside the default VocabSize 2
    tok = {"vocab": 12, "dim": 8, "heads": 2, "layers": 1, "ff": 16, "max_seq": 8}
    lm2, _ = host.language_model(tok, synth.lm_weights(tok, 1))
    t2 = H.TransformerTrainer(lm2, H.TrainingConfig())
    with pytest.raises(H.InvalidOperationException, match="Train\\(int"):
        t2.TrainContinuous(x, regressionTargets=[z((5, 2), np.float32)])
    with pytest.raises(H.ArgumentException, match="exceeds MaxSequenceLength"):
        t2.Validate([np.zeros(10, np.int32)])
    assert t2.Validate([np.array([4], np.int32), np.array([1, 12], np.int32)]) == 0.0


def test_no_device_means_loud_failure(mgr):
    if N.device_count() > 0:
        pytest.skip("a device is visible")
    with pytest.raises(H.InvalidOperationException, match="no HIP device"):
        mgr.ScaledDotProductAttention(M(4, 8, 1), M(4, 8, 2), M(4, 8, 3), 2)


def test_attention_backward_workspace_choice():
    """MultiHeadAttentionBackward asks for the stored-dS workspace (the causal
    32 x 32 fp32 dS blocks of every head, about 2 L^2 bytes per head) only
    while its extra bytes stay under the cap; beyond it (long contexts) the
    O(L) base workspace is used."""
    cap = H.STORED_DS_EXTRA_BYTES_CAP
    assert cap == 1 << 30
    # c3 sequence: 16 heads x (128 x 129 / 2) blocks x 4 KiB = 541 MB -> stored dS
    base, stored, pick = H.sdpa_backward_workspace_choice(4096, 4096, 1024, 16, True)
    assert stored - base - 16 * (128 * 129 // 2) * 32 * 32 * 4 in range(0, 256)
    assert pick == stored
    # 16384 keys: 8.6 GB of dS blocks -> the base size
    base, stored, pick = H.sdpa_backward_workspace_choice(16384, 16384, 1024, 16, True)
    assert stored - base > cap and pick == base
    # a smaller cap moves the c3 case to the base size too
    base, stored, pick = H.sdpa_backward_workspace_choice(4096, 4096, 1024, 16, True, extra_cap=1 << 20)
    assert pick == base
    # shapes that cannot use stored dS (no causal flag, head dim 16) never ask for it
    for args in ((512, 512, 512, 8, False), (512, 512, 256, 16, True)):
        base, stored, pick = H.sdpa_backward_workspace_choice(*args)
        assert stored == base and pick == base


def test_parallel_host_copy_and_compare():
    """The manager's host copy engine: copies of sizes around its slice and
    threshold sizes are exact, and a single differing byte anywhere is found."""
    assert H.host_copy_threads() >= 1
    rng = np.random.default_rng(3)
    for n in (0, 1, 1000, (2 << 20) - 4, 2 << 20, (9 << 20) + 12, 40 << 20):
        a = rng.integers(0, 255, size=n, dtype=np.uint8)
        b = H._parallel_copy(a)
        assert b.dtype == np.uint8 and np.array_equal(a, b)
        assert H._parallel_equal(a, b)
        if n:
            for pos in (0, n // 2, n - 1):
                c = b.copy()
                c[pos] ^= 1
                assert not H._parallel_equal(a, c)
