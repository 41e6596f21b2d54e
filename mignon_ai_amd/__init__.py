"""mignon_ai_amd: batched INT8 inference engine for mignon-ai's Hybrid NCA language model on one AMD
MI355X (gfx950).

The product is the HIP library built from csrc/ (C ABI: include/mignon_hip.h); this package holds its
Python binding (model.py), the model-file writer (mgnn.py), the benchmark configurations and seeded
synthetic weights (synth.py) and the build script (build.py).
"""
from ._lib import LIB_PATH, MignonError, lib  # noqa: F401
from .model import (Model, Session, Sessions, engine_option, gemm_i8, gemm_i8_device, quantize_f32,  # noqa: F401
                    sample_logits)
