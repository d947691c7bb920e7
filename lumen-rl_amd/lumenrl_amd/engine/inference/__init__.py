"""Inference-engine weight loading (lumenrl/engine/inference mirror)."""

from lumenrl_amd.engine.inference.weight_loader import DynamicWeightLoader

__all__ = ["DynamicWeightLoader"]
