"""Weight quantization for trainer -> rollout weight sync (lumenrl/quantization mirror)."""

from lumenrl_amd.quantization.bucket import QuantizedBucketWriter, encode_bucket
from lumenrl_amd.quantization.fp8_config import (
    FP8Config,
    QuantizationConfig,
    RolloutQuantConfig,
    TrainingQuantConfig,
)
from lumenrl_amd.quantization.fp8_kv_cache import FP8KVCacheQuantizer
from lumenrl_amd.quantization.fp8_rollout import FP8RolloutQuantizer
from lumenrl_amd.quantization.ops import (
    CopyPlan,
    DequantPlan,
    QuantPlan,
    TensorScalePlan,
    quantize_fp8_blockwise,
    quantize_mxfp4,
    quantize_mxfp8,
)
from lumenrl_amd.quantization.ops import act_qdq, fp8_block_dequant, fp8_block_quant
from lumenrl_amd.quantization.weight_quantizer import WeightQuantizer, fp8_e4m3_max

__all__ = [
    "CopyPlan",
    "DequantPlan",
    "FP8Config",
    "FP8KVCacheQuantizer",
    "FP8RolloutQuantizer",
    "QuantizationConfig",
    "QuantPlan",
    "QuantizedBucketWriter",
    "encode_bucket",
    "RolloutQuantConfig",
    "TensorScalePlan",
    "TrainingQuantConfig",
    "WeightQuantizer",
    "act_qdq",
    "fp8_block_dequant",
    "fp8_block_quant",
    "fp8_e4m3_max",
    "quantize_fp8_blockwise",
    "quantize_mxfp4",
    "quantize_mxfp8",
]
