"""Workload configurations of the grouped expert path (BASELINE.json configs C0-C4)."""
from __future__ import annotations

from dataclasses import dataclass, field, replace


@dataclass(frozen=True)
class MoELayerSpec:
    name: str
    hidden: int
    num_experts: int
    intermediate: int
    top_k: int
    rank: int
    renormalize: bool = True          # Mixtral/Qwen renormalise the top-k weights; OLMoE does not by default
    gmap_p: float = 0.15              # Bernoulli density of the split bitmap on non-salient columns
    salient_frac: float = 0.05        # salient columns per expert = ceil(frac * rank)
    group_size: int = 128
    router_std: float = 1.0
    outlier_channels: int = 4
    outlier_scale: float = 20.0
    shared_expert_intermediate: int = 0   # > 0: an always-on fp16 shared expert (A3B-class)
    tokens: tuple = (16,)

    def with_(self, **kw) -> "MoELayerSpec":
        return replace(self, **kw)


C0_OLMOE = MoELayerSpec("olmoe", hidden=2048, num_experts=64, intermediate=1024, top_k=8, rank=256,
                        renormalize=False, tokens=(16,))
C1_MIXTRAL_DECODE = MoELayerSpec("mixtral_decode", hidden=4096, num_experts=8, intermediate=14336, top_k=2, rank=512,
                                 tokens=(1, 4, 16))
C2_MIXTRAL_PREFILL = C1_MIXTRAL_DECODE.with_(name="mixtral_prefill", tokens=(2048,))
C3_A3B = MoELayerSpec("a3b", hidden=2048, num_experts=256, intermediate=512, top_k=8, rank=256, router_std=1.5,
                      shared_expert_intermediate=512, tokens=(1, 32, 1024))
C4_STREAMING = C1_MIXTRAL_DECODE.with_(name="mixtral_streaming", tokens=(8,))
C4_LAYERS = 32
C4_DENSITIES = (0.05, 0.15, 0.30)

CONFIGS = {s.name: s for s in (C0_OLMOE, C1_MIXTRAL_DECODE, C2_MIXTRAL_PREFILL, C3_A3B, C4_STREAMING)}
