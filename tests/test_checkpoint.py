"""LanguageModel.Save / Load in the reference's checkpoint format (LanguageModel.cs:706-919).

The golden directory tests/golden/checkpoint_tiny/ is written by
tests/golden/make_checkpoint_fixture.py straight from the reference's writer
steps and .NET's documented BinaryWriter encoding, independently of the C++
Save: Load must read it into exactly the stored arrays, and Save of that
model must reproduce its weights.bin byte for byte.  Error cases follow the
reference's checks and messages.  No GPU is needed: Save and Load touch host
arrays only (Forward after Load is covered in test_host_gpu.py).
"""
from __future__ import annotations

import json
import os
import shutil
import struct

import numpy as np
import pytest

from cdml import host, synth

GOLD = os.path.join(os.path.dirname(__file__), "golden")
TINY = os.path.join(GOLD, "checkpoint_tiny")
H = host.module()


@pytest.fixture(scope="module")
def mgr():
    return H.HipAccelerationManager(0)


def expected_tiny():
    e = np.load(os.path.join(GOLD, "checkpoint_tiny_expected.npz"))
    return {k: e[k] for k in e.files}


def test_load_golden_checkpoint(mgr):
    lm = H.LanguageModel.Load(TINY, mgr)
    c = lm.config
    assert (c.VocabSize, c.EmbeddingDim, c.NumHeads, c.NumLayers, c.FeedForwardDim, c.MaxSequenceLength) == \
        (5, 4, 2, 2, 6, 8)
    assert c.UsesDiscreteTokens and c.UseDecoderOnly and c.FFNActivationType == 3
    assert c.AccelerationType == 1 and abs(c.L2RegulationLamda - 0.01) < 1e-9 and c.GradientClippingThreshold == 1.0
    w, e = lm.weights(), expected_tiny()
    for k in ("token_embedding", "out_proj", "out_bias"):
        assert np.array_equal(w[k], e[k]), k
    for i, L in enumerate(w["layers"]):
        for k in ("wq", "wk", "wv", "wo", "bq", "bk", "bv", "bo", "ln1_g", "ln1_b", "ln2_g", "ln2_b",
                  "ffn_w1", "ffn_b1", "ffn_w2", "ffn_b2"):
            assert np.array_equal(L[k], e[f"l{i}_{k}"]), (i, k)
        assert L["ffn_activations"] == [3, 0]
    # the exponent and integral spellings in the FFN file
    assert w["layers"][0]["ffn_w1"][0, 0] == np.float32(1e-5) and w["layers"][0]["ffn_w1"][0, 1] == 1.0


def test_save_reproduces_golden_weights_bin(mgr, tmp_path):
    lm = H.LanguageModel.Load(TINY, mgr)
    lm.Save(str(tmp_path))
    with open(os.path.join(TINY, "weights.bin"), "rb") as a, open(tmp_path / "weights.bin", "rb") as b:
        assert a.read() == b.read()
    cfg = json.loads((tmp_path / "config.json").read_text())
    ref = json.loads(open(os.path.join(TINY, "config.json")).read())
    assert list(cfg) == list(ref)  # the reference's key order (LanguageModel.cs:710-728)
    assert cfg == ref
    for i in range(2):
        raw = (tmp_path / "ffn" / f"ffn_layer_{i}.json").read_bytes()
        assert raw.startswith(b"\xef\xbb\xbf")
        d = json.loads(raw[3:].decode())
        g = json.loads(open(os.path.join(TINY, "ffn", f"ffn_layer_{i}.json"), encoding="utf-8-sig").read())
        assert [L["Size"] for L in d["layers"]] == [4, 6, 4]
        assert d["parameters"]["LayerWidths"] == [4, 6, 4] and d["parameters"]["LayerActivations"] == [0, 3, 0]
        for Ld, Lg in zip(d["layers"], g["layers"]):
            assert Ld["ActivationType"] == Lg["ActivationType"]
            assert np.array_equal(np.float32(Ld["Biases"]), np.float32(Lg["Biases"]))
            assert len(Ld["Weights"]) == len(Lg["Weights"])
            for rd, rg in zip(Ld["Weights"], Lg["Weights"]):
                assert np.array_equal(np.float32(rd), np.float32(rg))


@pytest.mark.parametrize("discrete", [True, False])
def test_round_trip(mgr, tmp_path, discrete):
    cfg = {"vocab": 12, "dim": 8, "heads": 2, "layers": 2, "ff": 16, "max_seq": 8, "discrete": discrete,
           "input_dim": 3, "output_dim": 2}
    w0 = synth.lm_weights(cfg, 5) if discrete else synth.continuous_lm_weights(cfg, 5)
    lm, _ = host.language_model(cfg, w0, mgr)
    lm.Save(str(tmp_path))  # a continuous model saves as TimeSeriesRegression
    back = H.LanguageModel.Load(str(tmp_path), mgr)
    assert back.config.UsesDiscreteTokens == discrete
    assert json.loads((tmp_path / "config.json").read_text())["DataType"] == (0 if discrete else 1)
    a, b = lm.weights(), back.weights()
    keys = ["out_proj", "out_bias"] + (["token_embedding"] if discrete else ["input_proj", "input_bias"])
    for k in keys:
        assert np.array_equal(a[k], b[k]), k
    for La, Lb in zip(a["layers"], b["layers"]):
        for k in La:
            if k.startswith("ffn_") and isinstance(La[k], list):
                if k == "ffn_activations":
                    assert La[k] == Lb[k]
                else:
                    assert all(np.array_equal(x, y) for x, y in zip(La[k], Lb[k])), k
            else:
                assert np.array_equal(La[k], Lb[k]), k


def test_non_finite_and_string_forms_in_ffn_file(mgr, tmp_path):
    """Newtonsoft writes NaN / Infinity as strings; enums may be read by name."""
    shutil.copytree(TINY, tmp_path / "m")
    p = tmp_path / "m" / "ffn" / "ffn_layer_1.json"
    d = json.loads(p.read_bytes()[3:].decode())
    d["layers"][2]["Biases"][0] = "NaN"
    d["layers"][2]["Biases"][1] = "-Infinity"
    d["layers"][1]["ActivationType"] = "Tanh"
    p.write_text(json.dumps(d))  # compact, no byte-order mark: both forms are read
    w = H.LanguageModel.Load(str(tmp_path / "m"), mgr).weights()["layers"][1]
    assert np.isnan(w["ffn_b2"][0]) and w["ffn_b2"][1] == -np.inf
    assert w["ffn_activations"] == [2, 0]


def _broken_copy(tmp_path):
    shutil.copytree(TINY, tmp_path / "m")
    return tmp_path / "m"


def test_load_errors(mgr, tmp_path):
    d = _broken_copy(tmp_path)
    wb = (d / "weights.bin").read_bytes()
    # shape mismatch: the first matrix header says [5, 3] (ReadMatrixInto, :871-889)
    (d / "weights.bin").write_bytes(wb[:1] + struct.pack("<ii", 5, 3) + wb[9:])
    with pytest.raises(H.InvalidOperationException,
                       match=r"Matrix shape mismatch\. File has \[5,3\], target is \[5,4\]\."):
        H.LanguageModel.Load(str(d), mgr)
    # truncated stream (EndOfStreamException's text)
    (d / "weights.bin").write_bytes(wb[:-3])
    with pytest.raises(H.InvalidOperationException, match="Unable to read beyond the end of the stream"):
        H.LanguageModel.Load(str(d), mgr)
    # saved as continuous while the config is discrete: ReadMatrixInto(null) (:811-822)
    (d / "weights.bin").write_bytes(b"\x00" + wb[1:])
    with pytest.raises(H.ArgumentNullException):
        H.LanguageModel.Load(str(d), mgr)
    (d / "weights.bin").write_bytes(wb)
    # a missing FFN file (LoadFeedForwardNetworks, :692-693)
    os.remove(d / "ffn" / "ffn_layer_1.json")
    with pytest.raises(H.FileNotFoundException, match="Missing FFN file"):
        H.LanguageModel.Load(str(d), mgr)
    # config: a missing key, a bad value, an invalid configuration
    cfg = json.loads((d / "config.json").read_text())
    for mutate, exc, text in [(lambda c: c.pop("NumHeads"), H.InvalidOperationException, "NumHeads"),
                              (lambda c: c.update(NumHeads=1.5), H.InvalidOperationException, "NumHeads"),
                              (lambda c: c.update(UseDecoderOnly=1), H.InvalidOperationException, "UseDecoderOnly"),
                              (lambda c: c.update(NumHeads=3), H.ArgumentException, "divisible"),
                              (lambda c: c.update(DataType=9), H.ArgumentException, "Invalid DataType")]:
        bad = dict(cfg)
        mutate(bad)
        (d / "config.json").write_text(json.dumps(bad))
        with pytest.raises(exc, match=text):
            H.LanguageModel.Load(str(d), mgr)
    with pytest.raises(H.FileNotFoundException):
        H.LanguageModel.Load(str(tmp_path / "nowhere"), mgr)
