"""Host-side mirror of lumenrl/quantization (no GPU): config, validation, loud failure."""

from __future__ import annotations

import pytest
import torch

from lumenrl_amd import _lib
from lumenrl_amd.quantization import (
    FP8Config,
    QuantizationConfig,
    TrainingQuantConfig,
    WeightQuantizer,
    fp8_e4m3_max,
)


# tests/unit/quantization/test_fp8_config.py:7-29, against the mirror
def test_default_values():
    cfg = FP8Config()
    assert cfg.precision == "bf16"
    assert cfg.recipe == "blockwise"
    assert cfg.use_deep_gemm is True
    assert cfg.use_weight_pow2_scale is False
    assert cfg.is_fp8_enabled() is False


def test_from_config():
    q = QuantizationConfig()
    q.rollout.precision = "bf16"
    q.training = TrainingQuantConfig(fp8="e4m3", fp8_recipe="tensorwise")
    cfg = FP8Config.from_config(q)
    assert cfg.precision == "e4m3"
    assert cfg.recipe == "tensorwise"
    assert cfg.is_fp8_enabled() is True
    assert cfg.use_weight_pow2_scale is False


def test_is_fp8_enabled():
    assert FP8Config(precision="fp8").is_fp8_enabled() is True
    assert FP8Config(precision="hybrid_fp8").is_fp8_enabled() is True
    assert FP8Config(precision="bf16").is_fp8_enabled() is False
    assert FP8Config(precision=" E4M3 ").is_fp8_enabled() is True


def test_from_config_rejects_other_types():
    with pytest.raises(TypeError, match="QuantizationConfig"):
        FP8Config.from_config({"rollout": None})


def test_fp8_max():
    assert fp8_e4m3_max() == 448.0


def test_validation_errors_match_reference_texts():
    wq = WeightQuantizer(FP8Config())
    with pytest.raises(ValueError, match=r"quantize_tensor expects tensor.dim\(\) >= 1"):
        wq.quantize_tensor(torch.tensor(1.0))
    with pytest.raises(ValueError, match=r"Last dim 100 must be divisible by block_size=128"):
        wq.quantize_tensor(torch.zeros(2, 100))
    with pytest.raises(ZeroDivisionError):
        wq.quantize_tensor(torch.zeros(2, 100), block_size=0)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device failure")
def test_no_device_fails_loudly():
    wq = WeightQuantizer(FP8Config())
    with pytest.raises(RuntimeError, match="HIP device"):
        wq.quantize_tensor(torch.zeros(2, 128))
    with pytest.raises(RuntimeError, match="HIP device"):
        wq.quantize_state_dict({"w": torch.zeros(4, 128)})


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/liblrq.so")
    with pytest.raises(_lib.LrqError, match="no non-HIP fallback"):
        _lib.lib()


def test_state_dict_passthrough_rules_without_device():
    """Entries the reference passes through never touch the device (:95-108)."""
    wq = WeightQuantizer(FP8Config())
    sd = {"step": 3, "ids": torch.arange(4), "bias": torch.zeros(128), "odd": torch.zeros(4, 100)}
    out = wq.quantize_state_dict(sd)
    assert list(out) == list(sd)
    for k in sd:
        assert out[k] is sd[k]
