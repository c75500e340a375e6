"""bnns_to_c_amd - MI355X (gfx950) engine for the v1 Bi-Real binary UNet.

libbnn_hip.so (built from csrc/ by __graft_entry__.build()) is the product:
a C ABI with the reference's bnn_load / bnn_forward / bnn_free and kernel
entry points (include/bnn_model.h).  This package holds its Python bindings
(engine), the weights.blob v1 format (blob) and seeded synthetic models and
inputs (synth).
"""
from . import blob, synth  # noqa: F401

__all__ = ["blob", "synth", "engine", "build"]
