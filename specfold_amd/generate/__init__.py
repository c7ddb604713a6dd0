"""Generator and executor classes with the reference's API (specfold/generate/)."""

from specfold_amd.generate.fastdllm_model_executor import ByteTokenizer, FastDLLMModelExecutor
from specfold_amd.generate.fastdllm_v2_folded import (SpecFoldHIPFastDLLMV2Generation,
                                                      SpecFoldTritonFastDLLMV2Generation)
from specfold_amd.generate.fastdllm_v2_generation import FastDLLMV2SpeculativeGeneration
from specfold_amd.generate.nld_folded import (SpecFoldHIPNLDGeneration, SpecFoldNLDGeneration,
                                              SpecFoldTritonNLDGeneration)
from specfold_amd.generate.nld_generation import NLDDiffusionGeneration
from specfold_amd.generate.nld_model_executor import NLDModelExecutor

__all__ = [
    "ByteTokenizer",
    "FastDLLMModelExecutor",
    "FastDLLMV2SpeculativeGeneration",
    "SpecFoldHIPFastDLLMV2Generation",
    "SpecFoldTritonFastDLLMV2Generation",
    "NLDDiffusionGeneration",
    "NLDModelExecutor",
    "SpecFoldHIPNLDGeneration",
    "SpecFoldNLDGeneration",
    "SpecFoldTritonNLDGeneration",
]
