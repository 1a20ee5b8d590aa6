"""Python access to the C++ host side (``_build/_cdml_host*.so``).

``HipAccelerationManager`` mirrors the reference's IAccelerationManager
hot-path methods (host arrays in and out, the reference's exception kinds);
``LanguageModel`` restates Transformers/MultiTypeTransformer/LanguageModel on
it; ``DeviceLanguageModel`` runs the same weights device-resident.  Loading
fails loudly when the module has not been built; there is no Python or CPU
fallback.
"""
from __future__ import annotations

import importlib
import os
import sys

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# CDML_HOST_BUILD selects another build directory of the same module (the
# sanitizer build in _build/asan, which tests load under libasan).
BUILD = os.environ.get("CDML_HOST_BUILD") or os.path.join(PKG, "_build")

_mod = None


def module():
    """The compiled ``_cdml_host`` extension."""
    global _mod
    if _mod is None:
        if BUILD not in sys.path:
            sys.path.insert(0, BUILD)
        try:
            _mod = importlib.import_module("_cdml_host")
        except ImportError as e:  # not built: say so, never fall back
            raise ImportError(f"_cdml_host is not built in {BUILD}; run __graft_entry__.build()") from e
    return _mod


def config(cfg: dict, **overrides):
    """A TransformerConfig from the fixture dict layout (vocab, dim, heads,
    layers, ff, max_seq [, input_dim, output_dim, discrete, decoder_only,
    activation])."""
    m = module()
    c = m.TransformerConfig()
    c.VocabSize = int(cfg.get("vocab", 2))
    c.EmbeddingDim = int(cfg["dim"])
    c.NumHeads = int(cfg["heads"])
    c.NumLayers = int(cfg["layers"])
    c.FeedForwardDim = int(cfg["ff"])
    c.MaxSequenceLength = int(cfg["max_seq"])
    c.UsesDiscreteTokens = bool(cfg.get("discrete", True))
    # TransformerDataType: Text 0 for token models, TimeSeriesRegression 1
    # (or TimeSeriesClassification 2) for continuous ones
    c.DataType = int(cfg.get("data_type", 0 if c.UsesDiscreteTokens else 1))
    c.UseDecoderOnly = bool(cfg.get("decoder_only", True))
    c.InputFeatureDim = int(cfg.get("input_dim", 1))
    c.OutputDim = int(cfg.get("output_dim", 1))
    c.FFNActivationType = int(cfg.get("activation", 3))
    for k, v in overrides.items():
        setattr(c, k, v)
    c.Validate()
    return c


def language_model(cfg: dict, weights: dict, manager=None):
    """A LanguageModel over ``manager`` (a new HipAccelerationManager on
    device 0 when None) holding ``weights`` (cdml.synth.lm_weights layout)."""
    m = module()
    if manager is None:
        manager = m.HipAccelerationManager(0)
    lm = m.LanguageModel(config(cfg), manager)
    lm.load_weights(weights)
    return lm, manager
