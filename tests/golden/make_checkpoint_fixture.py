"""Writes tests/golden/checkpoint_tiny/, a LanguageModel checkpoint directory in the
reference's on-disk format (run: python tests/golden/make_checkpoint_fixture.py).

The files are produced here with plain Python (struct, text), step by step from
the reference's writer, independently of the C++ Save they check:

  config.json            the dictionary of LanguageModel.Save (LanguageModel.cs:710-735),
                         System.Text.Json indented (two spaces, keys in insertion order)
  weights.bin            BinaryWriter (LanguageModel.cs:737-765, WriteMatrix/WriteVector
                         :840-864, WriteAttention :865-869): Write(bool) is one byte,
                         Write(int) and Write(float) four little-endian bytes (the
                         documented System.IO.BinaryWriter encoding)
  ffn/ffn_layer_<i>.json  Data.Save (Neural Network/Data.cs:218-236): Newtonsoft.Json,
                         indented, over a StreamWriter with Encoding.UTF8, so the file
                         starts with the UTF-8 byte-order mark; floats in round-trip
                         form with a decimal point, enums as integers

The model is a discrete-token decoder (vocab 5, D 4, 2 heads, 2 layers, FF 6,
ReLU FFN).  Its arrays are also stored in checkpoint_tiny_expected.npz.  The
FFN files use Newtonsoft's number spellings that a reader must accept
(exponent form such as 1E-05, integral values as 1.0).
"""
from __future__ import annotations

import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "checkpoint_tiny")
CFG = dict(vocab=5, dim=4, heads=2, layers=2, ff=6, max_seq=8, activation=3)


def arrays():
    rng = np.random.default_rng(20261201)
    V, D, F = CFG["vocab"], CFG["dim"], CFG["ff"]

    def f(*shape, scale=0.5):
        return (rng.standard_normal(shape) * scale).astype(np.float32)

    w = {"token_embedding": f(V, D), "out_proj": f(V, D), "out_bias": f(V, scale=0.1), "layers": []}
    for _ in range(CFG["layers"]):
        L = {k: f(D, D) for k in ("wq", "wk", "wv", "wo")}
        L.update({k: f(D, scale=0.1) for k in ("bq", "bk", "bv", "bo")})
        L.update(ln1_g=1 + f(D, scale=0.1), ln1_b=f(D, scale=0.1), ln2_g=1 + f(D, scale=0.1),
                 ln2_b=f(D, scale=0.1))
        L.update(ffn_w1=f(F, D), ffn_b1=f(F, scale=0.1), ffn_w2=f(D, F), ffn_b2=f(D, scale=0.1))
        w["layers"].append(L)
    # spellings a reader must handle: a tiny value (exponent form) and an integral one
    w["layers"][0]["ffn_w1"][0, 0] = np.float32(1e-5)
    w["layers"][0]["ffn_w1"][0, 1] = np.float32(1.0)
    return w


def net_float(x: np.float32) -> str:
    """float.ToString("R") with Newtonsoft's EnsureDecimalPlace."""
    x = float(np.float32(x))
    for prec in range(1, 10):
        t = f"{x:.{prec}g}"
        if np.float32(float(t)) == np.float32(x):
            break
    if "e" in t:  # .NET spells the exponent E-05 / E+15
        mant, exp = t.split("e")
        t = f"{mant}E{exp[0]}{int(exp[1:]):02d}"
    if not any(c in t for c in ".E"):
        t += ".0"
    return t


def config_json() -> str:
    items = [("VocabSize", CFG["vocab"]), ("MaxSequenceLength", CFG["max_seq"]), ("EmbeddingDim", CFG["dim"]),
             ("NumHeads", CFG["heads"]), ("NumLayers", CFG["layers"]), ("FeedForwardDim", CFG["ff"]),
             ("UseDecoderOnly", "true"), ("FFNActivationType", CFG["activation"]), ("AccelerationType", 1),
             ("AccelerationDeviceId", 0), ("L2RegulationLamda", "0.01"), ("GradientClippingThreshold", "1"),
             ("DataType", 0), ("InputFeatureDim", 1), ("OutputDim", 1), ("CostFunction", 0),
             ("ActivationDistribution", 0)]
    return "{\n" + ",\n".join(f'  "{k}": {v}' for k, v in items) + "\n}"


def weights_bin(w) -> bytes:
    out = bytearray()

    def mat(m):
        out.extend(struct.pack("<ii", *m.shape))
        out.extend(struct.pack(f"<{m.size}f", *m.ravel()))

    def vec(v):
        out.extend(struct.pack("<i", v.size))
        out.extend(struct.pack(f"<{v.size}f", *v))

    out.extend(struct.pack("<?", True))  # UsesDiscreteTokens
    mat(w["token_embedding"])
    for L in w["layers"]:
        for k in ("wq", "wk", "wv", "wo"):
            mat(L[k])
        for k in ("bq", "bk", "bv", "bo", "ln1_g", "ln1_b", "ln2_g", "ln2_b"):
            vec(L[k])
    mat(w["out_proj"])
    vec(w["out_bias"])
    return bytes(out)


def ffn_json(L) -> str:
    D, F = CFG["dim"], CFG["ff"]
    ind = "  "

    def arr(vals, depth):
        if len(vals) == 0:
            return "[]"
        pad = ind * (depth + 1)
        return "[\n" + ",\n".join(pad + v for v in vals) + "\n" + ind * depth + "]"

    def farr(v, depth):
        return arr([net_float(x) for x in v], depth)

    layers = []
    spec = [(D, 0, np.zeros(D, np.float32), None, 0), (F, D, L["ffn_b1"], L["ffn_w1"], CFG["activation"]),
            (D, F, L["ffn_b2"], L["ffn_w2"], 0)]
    for size, insz, bias, wmat, act in spec:
        zeros = np.zeros(size, np.float32)
        rows = [arr([] if wmat is None else [net_float(x) for x in wmat[r]], 4) for r in range(size)]
        fields = [("Size", str(size)), ("InputSize", str(insz)), ("Activations", farr(zeros, 3)),
                  ("Biases", farr(bias, 3)), ("Derivatives", farr(zeros, 3)), ("Deltas", farr(zeros, 3)),
                  ("Weights", arr(rows, 3)), ("ActivationType", str(act))]
        layers.append(ind * 2 + "{\n" + ",\n".join(f'{ind * 3}"{k}": {v}' for k, v in fields) + "\n" + ind * 2 + "}")
    params = [("HuberLossDelta", "1.0"), ("AccelerationType", "1"), ("AccelerationDeviceId", "0"),
              ("CostFunction", "0"), ("ActivationDistribution", "0"), ("L2RegulationLamda", "0.01"),
              ("GradientClippingThreshold", "1.0"), ("GradientExplosionThreshold", "1000.0"),
              ("GradientVanishingThreshold", "1E-05"), ("LayerWidths", arr(["4", "6", "4"], 2)),
              ("LayerActivations", arr(["0", str(CFG["activation"]), "0"], 2)),
              ("inputActivationMin", farr(np.zeros(D, np.float32), 2)),
              ("inputActivationMax", farr(np.ones(D, np.float32), 2)),
              ("OptimalLearningRate", "null"), ("EpochsTrainedOn", "10")]
    body = ("{\n" + ind + '"layers": [\n' + ",\n".join(layers) + "\n" + ind + "],\n" + ind + '"parameters": {\n' +
            ",\n".join(f'{ind * 2}"{k}": {v}' for k, v in params) + "\n" + ind + "}\n}")
    return "\ufeff" + body  # the byte-order mark of Encoding.UTF8


def main():
    w = arrays()
    os.makedirs(os.path.join(OUT, "ffn"), exist_ok=True)
    with open(os.path.join(OUT, "config.json"), "w", encoding="utf-8", newline="\n") as fh:
        fh.write(config_json())
    with open(os.path.join(OUT, "weights.bin"), "wb") as fh:
        fh.write(weights_bin(w))
    for i, L in enumerate(w["layers"]):
        with open(os.path.join(OUT, "ffn", f"ffn_layer_{i}.json"), "w", encoding="utf-8", newline="\n") as fh:
            fh.write(ffn_json(L))
    flat = {"token_embedding": w["token_embedding"], "out_proj": w["out_proj"], "out_bias": w["out_bias"]}
    for i, L in enumerate(w["layers"]):
        flat.update({f"l{i}_{k}": v for k, v in L.items()})
    np.savez(os.path.join(HERE, "checkpoint_tiny_expected.npz"), **flat)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
