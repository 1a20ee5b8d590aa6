"""MI355X (gfx950) implementation of CallaghanDev.ML's causal multi-head
attention forward path: the C-ABI library (libcdml_hip.so), its ctypes
binding (``cdml.native``), the C++ host-side HipAccelerationManager
(``cdml.host``, built as ``_cdml_host``) and the synthetic workload
generators (``cdml.synth``)."""

__all__ = ["native", "synth", "build"]
