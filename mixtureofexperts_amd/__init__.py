"""mixtureofexperts_amd -- MixtureOfExperts.jl's MoE-layer forward path on
MI355X (gfx950).

The API mirrors the reference's exports for this path
(src/MixtureOfExperts.jl:14-40): MoEConfig, MoELayer, Router, TopKGating,
SwitchGating, SharedExpertGating, SoftMoEGating, ExpertChoiceGating,
HashGating, RandomGating, JitterGating, StochasticTopKGating, GatedExpert, StandardExpert,
SwitchTransformerLoss, ZLoss, NoBalancingLoss, AuxiliaryFreeLoss (update_bias!,
get_biased_logits), DeepSeekLoss, compute_gates, compute_loss,
create_moe_config, create_moe_layer, reset_stats (reset_stats!), and the
decode caller moe_ffn_forward (moe_ffn_forward!, src/llama2/inference.jl:58),
convert_layer_to_moe (src/llama2/conversion.jl:191) and the layer's on-disk
format (save_moe_layer / load_moe_layer).  All compute
runs in libmoe_mi355x.so (hand-written HIP kernels); nothing here falls back
to a CPU path.
"""
from ._lib import MoeError, lib
from .activations import gelu, identity, relu, silu, swish
from .balancing import (AuxiliaryFreeLoss, DeepSeekLoss, LoadBalancingLoss, NoBalancingLoss, SwitchTransformerLoss,
                        ZLoss, compute_loss, get_biased_logits, update_bias)
from .experts import Expert, GatedExpert, StandardExpert
from .gating import (ExpertChoiceGating, GatingMechanism, HashGating, JitterGating, RandomGating, SharedExpertGating,
                     SoftMoEGating, StochasticTopKGating, SwitchGating, TopKGating, compute_gates, route_from_logits)
from .layer import MoEConfig, MoELayer, Router, create_moe_config, create_moe_layer, moe_ffn_forward, reset_stats
from .conversion import convert_layer_to_moe, load_moe_layer, save_moe_layer

__all__ = [
    "MoeError", "lib", "gelu", "identity", "relu", "silu", "swish", "LoadBalancingLoss", "NoBalancingLoss",
    "SwitchTransformerLoss", "ZLoss", "AuxiliaryFreeLoss", "DeepSeekLoss", "update_bias", "get_biased_logits",
    "compute_loss", "Expert", "GatedExpert", "StandardExpert",
    "GatingMechanism", "SharedExpertGating", "SwitchGating", "TopKGating", "SoftMoEGating", "ExpertChoiceGating",
    "HashGating", "RandomGating", "JitterGating", "StochasticTopKGating", "compute_gates", "route_from_logits",
    "MoEConfig", "MoELayer", "Router", "create_moe_config", "create_moe_layer", "moe_ffn_forward", "reset_stats",
    "convert_layer_to_moe", "save_moe_layer", "load_moe_layer",
]
