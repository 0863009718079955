"""lokal_amd -- MI355X (gfx950) HIP backend for lokal's per-token decode step.

The product is liblokal_hip.so (C ABI: include/lokal_hip.h).  This package is
its Python mirror of lokal's backend seam (Engine / Session / Batcher,
src/engine.rs:13-71) plus kernel-level bindings and synthetic checkpoints.
"""
from ._lib import LokalHipError
from .config import CONFIGS, ModelConfig
from .engine import BatchRow, Batcher, Engine, Session, create, gguf_config

__all__ = ["Engine", "Session", "Batcher", "BatchRow", "create", "ModelConfig", "CONFIGS", "LokalHipError"]
