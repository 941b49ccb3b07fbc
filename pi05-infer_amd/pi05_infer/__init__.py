"""pi0.5 action-expert denoise engine for MI355X (gfx950).

The Python modules mirror the reference package's entry points (``pi05_infer.engine``,
``pi05_infer.builder``); the compute lives in ``libpi05_denoise.so`` (C ABI:
``include/pi05_denoise.h``), loaded by ``pi05_infer._ext``.
"""

from .engine import Engine, EngineConfig, Observation, OpenPi0InferConfig, OpenPi0Inference
from .synthetic import ExpertGeometry

__all__ = ["Engine", "EngineConfig", "ExpertGeometry", "Observation", "OpenPi0InferConfig", "OpenPi0Inference"]
