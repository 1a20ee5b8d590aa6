"""Deterministic synthetic inputs for the BASELINE workloads.

One documented generator (SplitMix64, Steele/Lea/Flood 2014) drives every
seeded array so the same bytes can be regenerated anywhere without a
library-version dependency:

* ``uniform(seed, n)``: the top 53 bits of SplitMix64 outputs as doubles in
  [0, 1), rounded to float32 by the caller.
* ``normal(seed, n)``: Box-Muller in double from two uniforms,
  z = sqrt(-2 ln(1 - u1)) cos(2 pi u2).
* ``xavier_uniform(seed, out, in)``: U(-a, a), a = sqrt(6 / (in + out)).

The closed-form ``matrix`` / ``vector`` generators restate the reference test
suite's deterministic inputs
(CallaghanDev.ML.TestConsoleApp/Tests/AccelerationManagerParityTests.cs:2180-2205).
"""
from __future__ import annotations

import math

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n consecutive SplitMix64 outputs starting from state ``seed``."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(seed: int, n: int) -> np.ndarray:
    """Doubles in [0, 1) from the top 53 bits of SplitMix64."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, shape) -> np.ndarray:
    """float32 N(0, 1) by Box-Muller in double."""
    n = int(np.prod(shape))
    u = uniform(seed, 2 * n)
    u1, u2 = u[0::2], u[1::2]
    z = np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * math.pi * u2)
    return z.astype(np.float32).reshape(shape)


def xavier_uniform(seed: int, rows: int, cols: int) -> np.ndarray:
    """float32 [rows, cols] ~ U(-a, a), a = sqrt(6 / (rows + cols))."""
    a = math.sqrt(6.0 / (rows + cols))
    u = uniform(seed, rows * cols)
    return ((2.0 * u - 1.0) * a).astype(np.float32).reshape(rows, cols)


def token_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    """int32 ids uniform on {0 .. vocab-1}."""
    return (splitmix64(seed, n) % np.uint64(vocab)).astype(np.int32)


def matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """Reference test input: 0.25 sin((i+1) 12.9898 + (j+1) 78.233 + seed 0.137)."""
    i = np.arange(1, rows + 1, dtype=np.float64)[:, None]
    j = np.arange(1, cols + 1, dtype=np.float64)[None, :]
    x = np.sin(i * 12.9898 + j * 78.233 + seed * 0.137)
    return (x * 0.25).astype(np.float32)


def vector(n: int, seed: int) -> np.ndarray:
    """Reference test input: 0.25 sin((i+1) 19.19 + seed 0.313)."""
    i = np.arange(1, n + 1, dtype=np.float64)
    return (np.sin(i * 19.19 + seed * 0.313) * 0.25).astype(np.float32)


def positive_vector(n: int, seed: int) -> np.ndarray:
    """Reference test input: |vector| + 0.5."""
    return (np.abs(vector(n, seed)) + np.float32(0.5)).astype(np.float32)


def periodic_mask(rows: int, cols: int) -> np.ndarray:
    """Reference test mask: j == 0 or (31 i + 17 j) % 7 != 0 (1 = attend)."""
    i = np.arange(rows)[:, None]
    j = np.arange(cols)[None, :]
    return ((j == 0) | (((i * 31 + j * 17) % 7) != 0)).astype(np.uint8)


def lm_weights(cfg: dict, seed: int, biased: bool = False) -> dict:
    """Random-init decoder-only LanguageModel weights, Xavier-uniform.

    Layout follows LanguageModel / TransformerBlock / MultiHeadAttention:
    W* [D, D] ([out, in]), attention biases [D], LayerNorm gamma / beta [D],
    FFN [FF, D] and [D, FF] with biases, embedding [V, D] and output head
    [V, D] with bias [V].  With ``biased`` False the biases are 0, gamma 1 and
    beta 0 (the reference's initial state); with ``biased`` True they are
    drawn as 0.1 N(0,1) (gamma 1 + 0.1 N(0,1)) so that parity tests exercise
    every term.
    """
    V, D, FF = cfg["vocab"], cfg["dim"], cfg["ff"]
    s = seed

    def nxt():
        nonlocal s
        s += 1
        return s * 1000003

    def bias(n, centre=0.0):
        if not biased:
            return np.full(n, centre, np.float32)
        return (np.float32(centre) + np.float32(0.1) * normal(nxt(), (n,))).astype(np.float32)

    w = {
        "token_embedding": xavier_uniform(nxt(), V, D),
        "out_proj": xavier_uniform(nxt(), V, D),
        "out_bias": bias(V),
        "layers": [],
    }
    for _ in range(cfg["layers"]):
        w["layers"].append({
            "wq": xavier_uniform(nxt(), D, D), "wk": xavier_uniform(nxt(), D, D),
            "wv": xavier_uniform(nxt(), D, D), "wo": xavier_uniform(nxt(), D, D),
            "bq": bias(D), "bk": bias(D), "bv": bias(D), "bo": bias(D),
            "ln1_g": bias(D, 1.0), "ln1_b": bias(D),
            "ln2_g": bias(D, 1.0), "ln2_b": bias(D),
            "ffn_w1": xavier_uniform(nxt(), FF, D), "ffn_b1": bias(FF),
            "ffn_w2": xavier_uniform(nxt(), D, FF), "ffn_b2": bias(D),
        })
    return w


def random_walk_windows(seed: int, batch: int, length: int, features: int, step: float = 0.02) -> np.ndarray:
    """float32 [batch, length, features] time-series windows: x_0 ~ U[0, 1],
    x_t = x_{t-1} + N(0, step^2) per feature, then min-max rescaled to [0, 1]
    per window and feature (the BASELINE config-5 inputs)."""
    x0 = uniform(seed, batch * features).reshape(batch, 1, features)
    steps = normal(seed + 1, (batch, length - 1, features)).astype(np.float64) * step
    x = np.concatenate([x0, x0 + np.cumsum(steps, axis=1)], axis=1)
    lo = x.min(axis=1, keepdims=True)
    hi = x.max(axis=1, keepdims=True)
    return ((x - lo) / np.where(hi > lo, hi - lo, 1.0)).astype(np.float32)


def continuous_lm_weights(cfg: dict, seed: int, biased: bool = True) -> dict:
    """Weights of a continuous-input model (LanguageModel.Forward(float[,])):
    the lm_weights blocks plus InputProjection [D, F] with bias [D] and the
    output head [OutputDim, D] with bias, Xavier-uniform."""
    w = lm_weights(dict(cfg, vocab=2), seed, biased=biased)
    D, F, O = cfg["dim"], cfg["input_dim"], cfg["output_dim"]
    w["input_proj"] = xavier_uniform(seed + 900, D, F)
    w["out_proj"] = xavier_uniform(seed + 902, O, D)
    if biased:
        w["input_bias"] = np.float32(0.1) * normal(seed + 901, (D,))
        w["out_bias"] = np.float32(0.1) * normal(seed + 903, (O,))
    else:
        w["input_bias"] = np.zeros(D, np.float32)
        w["out_bias"] = np.zeros(O, np.float32)
    return w
