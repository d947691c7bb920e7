"""End to end on an MI355X: a small causal LM keeps its next-token distribution
through the FP8 round trip.

Mirrors the reference's rollout parity check
(tests/integration/test_fp8_rollout_parity.py:34-54): the state dict of a
TinyLM goes through ``quantize_state_dict`` -> ``dequantize_state_dict``, a
twin model loads the result, and the twin's next-token distribution stays
within KL 0.25 of the original's.  The TinyLM has the reference's layout
(lumenrl/engine/training/fsdp_backend.py:17-32: embedding,
``nn.TransformerEncoderLayer`` blocks, lm_head), built here.

The round trip runs through the drop-in on the device, from a device-resident
and from a host-resident state dict.  Its weights are also compared bit for bit
with the torch restatement of the reference run on the CPU.  Both forwards run
in float32 on the CPU (the bf16 weights widened exactly), so no bf16 attention
runs on the device.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import torch_ref
from lumenrl_amd.quantization import FP8Config, WeightQuantizer

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("needs a HIP device", allow_module_level=True)


class TinyLM(nn.Module):
    def __init__(self, vocab_size: int, dim: int, n_layers: int) -> None:
        super().__init__()
        self.embed = nn.Embedding(vocab_size, dim)
        self.blocks = nn.ModuleList(
            [nn.TransformerEncoderLayer(dim, nhead=4, batch_first=True) for _ in range(n_layers)])
        self.lm_head = nn.Linear(dim, vocab_size)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        x = self.embed(input_ids)
        for block in self.blocks:
            x = block(x)
        return self.lm_head(x)


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.uint8)


@pytest.mark.parametrize("where", ["cuda", "cpu"])
@pytest.mark.parametrize("n_layers", [1, 2])
def test_fp8_bf16_logprob_distribution(where, n_layers):
    print(f"rollout parity: TinyLM n_layers={n_layers}, state dict on {where}", flush=True)
    torch.manual_seed(0)
    model = TinyLM(512, 256, n_layers).to(torch.bfloat16)
    input_ids = torch.randint(0, 512, (2, 24))
    sd = {k: (v.cuda() if where == "cuda" else v) for k, v in model.state_dict().items()}

    wq = WeightQuantizer(FP8Config())
    quantized = wq.quantize_state_dict(sd)
    dq_sd = wq.dequantize_state_dict(quantized)
    assert all(v.device.type == where for v in dq_sd.values())

    # every weight equals the reference's op sequence evaluated on the CPU
    ref = torch_ref.dequantize_state_dict(torch_ref.quantize_state_dict(model.state_dict()))
    assert sorted(ref) == sorted(dq_sd)
    for k, v in ref.items():
        assert v.dtype == dq_sd[k].dtype and torch.equal(_bits(v), _bits(dq_sd[k])), k
    n_q = sum(1 for k in quantized if k.endswith("_fp8_scales"))
    assert n_q == 2 + 4 * n_layers  # embed, lm_head, in_proj/out_proj/linear1/linear2 per block

    twin = TinyLM(512, 256, n_layers).to(torch.bfloat16)
    twin.load_state_dict({k: v.cpu() for k, v in dq_sd.items()}, strict=True)
    model.float().eval()
    twin.float().eval()
    with torch.no_grad():
        log_p = F.log_softmax(model(input_ids)[:, :-1], dim=-1)
        q = F.softmax(twin(input_ids)[:, :-1], dim=-1)
        kl = F.kl_div(log_p, q, reduction="batchmean", log_target=False)
    print(f"  KL = {float(kl):.3e}", flush=True)
    assert kl.isfinite()
    assert float(kl) < 0.25
