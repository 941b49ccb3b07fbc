"""pi0.5 inference for MI355X (gfx950): the action-expert denoise engine, the Gemma-2B prefix
prefill (``prefix.PrefixLM``) and the SigLIP vision tower (``vision.VisionTower``).

The Python modules mirror the reference package's entry points (``pi05_infer.engine``,
``pi05_infer.builder``); the compute lives in ``libpi05_denoise.so`` (C ABIs:
``include/pi05_denoise.h``, ``include/pi05_prefill.h``, ``include/pi05_siglip.h``), loaded by
``pi05_infer._ext``.
"""

from .engine import Engine, EngineConfig, Observation, OpenPi0InferConfig, OpenPi0Inference
from .synthetic import ExpertGeometry

__all__ = ["Engine", "EngineConfig", "ExpertGeometry", "Observation", "OpenPi0InferConfig", "OpenPi0Inference"]
