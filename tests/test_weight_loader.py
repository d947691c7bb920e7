"""DynamicWeightLoader drop-in, host side (no GPU): pass-through rules, config
handling and the refusal to cast without a HIP device.

Mirrors the behaviour of lumenrl/engine/inference/weight_loader.py:19-78; the
cast itself is checked on the GPU (test_gpu_cast.py).
"""

from __future__ import annotations

import logging

import pytest
import torch

from lumenrl_amd.engine.inference import DynamicWeightLoader
from lumenrl_amd.engine.inference import weight_loader as wl


class _Engine:
    def __init__(self):
        self.calls = []

    def update_weights(self, sd):
        self.calls.append(sd)


def _sd():
    return {"w": torch.randn(4, 8, dtype=torch.bfloat16), "step": torch.tensor([3]),
            "mask": torch.tensor([True, False])}


@pytest.mark.parametrize("cfg", [None, {}, {"enabled": False}, {"dtype": "fp8"}])
def test_fp8_off_hands_the_same_dict_to_the_engine(cfg):
    sd, eng = _sd(), _Engine()
    DynamicWeightLoader.load_weights(eng, sd, fp8_config=cfg)
    assert len(eng.calls) == 1 and eng.calls[0] is sd


def test_unsupported_fp8_dtype_keeps_every_tensor(caplog):
    sd, eng = _sd(), _Engine()
    with caplog.at_level(logging.INFO, logger=wl.__name__):
        DynamicWeightLoader.load_weights(eng, sd, fp8_config={"enabled": True, "dtype": "E5M2"})
    got = eng.calls[0]
    assert list(got) == list(sd) and all(got[k] is sd[k] for k in sd)
    msgs = [r.getMessage() for r in caplog.records]
    assert any("FP8 dtype e5m2 requested" in m for m in msgs)
    assert any("applied FP8 conversion for 3 tensors" in m for m in msgs)


def test_fp8_cast_without_a_device_raises():
    if torch.cuda.is_available():  # pragma: no cover - GPU box
        pytest.skip("checks the CPU-only refusal")
    with pytest.raises(RuntimeError, match="HIP device"):
        DynamicWeightLoader.load_weights(_Engine(), _sd(), fp8_config={"enabled": True})


def test_only_non_float_tensors_need_no_device():
    sd = {"step": torch.tensor([3]), "ids": torch.arange(5)}
    eng = _Engine()
    DynamicWeightLoader.load_weights(eng, sd, fp8_config={"enabled": True, "dtype": "fp8_e4m3"})
    assert all(eng.calls[0][k] is sd[k] for k in sd)


def test_already_e4m3_tensors_pass_through_without_a_device():
    t = torch.zeros(4, dtype=torch.float8_e4m3fn)
    eng = _Engine()
    DynamicWeightLoader.load_weights(eng, {"q": t}, fp8_config={"enabled": True})
    assert eng.calls[0]["q"] is t
