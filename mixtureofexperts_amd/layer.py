"""MoEConfig, Router and MoELayer -- src/core/moe_layer.jl, src/core/router.jl.

The layer keeps the reference's call signature, ``layer(x, training=...,
return_stats=...) -> (output, balance_loss[, stats])`` with ``x`` of Julia
shape (input_dim, T) and ``output`` (output_dim, T) float32.  The whole
forward (router GEMM, gating, permute, grouped expert GEMMs, combine, losses,
statistics) runs in libmoe_mi355x.so on the GPU.
"""
from dataclasses import dataclass, field
from typing import Any, Optional

import numpy as np

from . import _lib
from ._device import DeviceLayer
from .activations import activation_code, gelu
from .balancing import (AuxiliaryFreeLoss, LoadBalancingLoss, NoBalancingLoss, SwitchTransformerLoss, balance_alpha,
                        update_bias)
from .experts import GatedExpert, StandardExpert
from .gating import HOST_ROUTED_GATES, GatingMechanism, TopKGating, gate_spec

_DTYPES = {"f32": _lib.MOE_F32, "fp32": _lib.MOE_F32, "bf16": _lib.MOE_BF16, "fp8": _lib.MOE_FP8_E4M3,
           "fp8_e4m3": _lib.MOE_FP8_E4M3}


@dataclass
class MoEConfig:
    """Base.@kwdef MoEConfig -- src/core/moe_layer.jl:4-29 (same fields and
    defaults), plus ``weight_dtype`` (device GEMM precision: "f32" is the
    reference precision, "bf16" and "fp8" the MI355X paths) and
    ``max_tokens`` (largest batch the device workspace is sized for)."""

    num_experts: int = 8
    expert_type: str = "standard"
    input_dim: int = 768
    hidden_dim: int = 3072
    output_dim: int = 768
    activation: Any = gelu
    expert_dropout: float = 0.0
    gate_type: GatingMechanism = field(default_factory=lambda: TopKGating(2))
    top_k: int = 2
    noise_scale: float = 0.0
    use_noise_network: bool = False
    use_fp32_router: bool = True
    balance_loss: LoadBalancingLoss = field(default_factory=lambda: SwitchTransformerLoss(0.01))
    z_loss_weight: float = 0.001
    capacity_factor: float = 1.25
    drop_tokens: bool = False
    use_cur: bool = False
    cur_rank: Optional[int] = None
    num_shared_experts: int = 0
    weight_dtype: str = "f32"
    max_tokens: int = 4096


def create_moe_config(**kwargs):
    """create_moe_config(; kwargs...) -- src/core/moe_layer.jl:281-283."""
    return MoEConfig(**kwargs)


class Router:
    """Router -- src/core/router.jl:4-46: ``weight`` (E, input_dim) float32 as
    Flux Dense(in, E, bias=false) with its default glorot-uniform init
    (:18); an optional ``bias`` (E,) makes it Dense(W, b).  With
    ``use_noise_network`` a second Dense(in, E, bias=false),
    ``noise_weight`` (:20); ``noise_seed`` seeds the device generator of
    the training noise (router.jl:32-41)."""

    def __init__(self, input_dim, num_experts, gate_type, *, noise_scale=0.0, use_noise_network=False,
                 use_fp32=True, rng=None, weight=None, bias=None, noise_weight=None, noise_seed=None):
        rng = np.random.default_rng() if rng is None else rng
        a = np.sqrt(6.0 / (input_dim + num_experts))
        if weight is None:
            weight = rng.uniform(-a, a, size=(num_experts, input_dim)).astype(np.float32)
        self.weight = np.asarray(weight, dtype=np.float32)
        self.bias = None if bias is None else np.asarray(bias, dtype=np.float32)
        self.gate_type = gate_type
        self.noise_scale = float(noise_scale)
        self.use_noise_network = bool(use_noise_network)
        self.use_fp32 = bool(use_fp32)
        if self.use_noise_network and noise_weight is None:
            noise_weight = rng.uniform(-a, a, size=(num_experts, input_dim)).astype(np.float32)
        self.noise_weight = None if noise_weight is None else np.asarray(noise_weight, dtype=np.float32)
        if noise_seed is None:
            noise_seed = int(rng.integers(0, 2**63)) if self.noise_scale > 0 else 0
        self.noise_seed = int(noise_seed)


def create_experts(config, rng=None):
    """create_experts(config) -- src/core/moe_layer.jl:65-102 (full hidden_dim
    per expert)."""
    if config.use_cur:
        raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, "CUR experts have no device path")
    rng = np.random.default_rng() if rng is None else rng
    wdt = _DTYPES[config.weight_dtype]
    experts = []
    for _ in range(config.num_experts):
        if config.expert_type == "gated":
            experts.append(GatedExpert(config.input_dim, config.hidden_dim, config.output_dim, config.activation,
                                       rng=rng, weight_dtype=wdt))
        else:
            experts.append(StandardExpert(config.input_dim, config.hidden_dim, config.output_dim, config.activation,
                                          dropout=config.expert_dropout, rng=rng, weight_dtype=wdt))
    return experts


class MoELayer:
    """MoELayer(config) -- src/core/moe_layer.jl:34-63."""

    def __init__(self, config, *, rng=None, experts=None, router=None):
        self.config = config
        rng = np.random.default_rng() if rng is None else rng
        self.experts = experts if experts is not None else create_experts(config, rng)
        self.router = router if router is not None else Router(
            config.input_dim, config.num_experts - config.num_shared_experts, config.gate_type,
            noise_scale=config.noise_scale, use_noise_network=config.use_noise_network,
            use_fp32=config.use_fp32_router, rng=rng)
        self.balance_loss = config.balance_loss
        self._drop_seed = int(rng.integers(0, 2**63)) if config.expert_dropout > 0 else 0
        self.training_stats = {
            "tokens_per_expert": np.zeros(config.num_experts, dtype=np.int64),
            "routing_entropy": [],
            "capacity_overflow": 0,
        }
        self._dev = None
        self._noise_error = None  # router noise the device refused (raised by training calls)

    # ---- device state ----------------------------------------------------
    def _new_device(self):
        """A device handle for this layer's configuration (no weights yet)."""
        c = self.config
        if self._dev is not None:
            self._dev.close()
            self._dev = None
        spec = gate_spec(self.router.gate_type, self.router.weight.shape[0])
        return DeviceLayer(
            num_experts=c.num_experts, expert_type=(_lib.MOE_EXPERT_GATED if c.expert_type == "gated"
                                                    else _lib.MOE_EXPERT_STANDARD),
            input_dim=c.input_dim, hidden_dim=c.hidden_dim, output_dim=c.output_dim,
            activation=activation_code(c.activation), gate=spec, weight_dtype=_DTYPES[c.weight_dtype],
            balance_alpha=balance_alpha(self.balance_loss), z_loss_weight=c.z_loss_weight,
            capacity_factor=c.capacity_factor, drop_tokens=c.drop_tokens, max_tokens=c.max_tokens,
            num_shared_experts=c.num_shared_experts)

    def sync_weights(self):
        """(Re)build the device handle and upload router and expert weights."""
        self._dev = self._new_device()
        self._dev.set_router(np.ascontiguousarray(self.router.weight.T), self.router.bias)
        self._noise_error = None
        if self.router.noise_scale > 0:
            nw = self.router.noise_weight if self.router.use_noise_network else None
            try:
                self._dev.set_router_noise(self.router.noise_scale,
                                           None if nw is None else np.ascontiguousarray(nw.T), self.router.noise_seed)
            except _lib.MoeError as err:
                # the noise only enters training calls (router.jl:32): a
                # router whose noise has no device path still runs inference,
                # and its training calls raise this error
                if err.status != _lib.MOE_EUNSUPPORTED:
                    raise
                self._noise_error = err
        for e, ex in enumerate(self.experts):
            ex.upload(self._dev, e)
        p = max([getattr(ex, "dropout", 0.0) for ex in self.experts] + [0.0])
        if p > 0 and self.config.expert_type != "gated":
            # StandardExpert's Dropout(p) in training (standard.jl:49-51),
            # the layer's experts share p (MoEConfig.expert_dropout)
            self._dev.set_expert_dropout(p, self._drop_seed)
        return self._dev

    def close(self):
        if self._dev is not None:
            self._dev.close()
            self._dev = None

    # ---- forward -----------------------------------------------------------
    def __call__(self, x, training=False, return_stats=False, x_dtype="f32", _aux=None):
        """(moe::MoELayer)(x; training, return_stats) -- src/core/moe_layer.jl:107-156.

        With ``num_shared_experts > 0`` this is forward_with_shared_experts
        (src/core/moe_layer.jl:158-185): experts 1..ns run on every token and
        are averaged, the router picks among the others, the output is the
        0.5/0.5 blend, and, as there, the training statistics are not updated.

        x: (input_dim, T) float32, or uint16 bf16 bit patterns with
        ``x_dtype="bf16"``.  Returns (output (output_dim, T) float32,
        balance_loss float32[, training_stats])."""
        xa = np.asarray(x)
        if xa.ndim != 2 or xa.shape[0] != self.config.input_dim:
            raise _lib.MoeError(_lib.MOE_EINVAL, f"x must be ({self.config.input_dim}, T), got {xa.shape}")
        T = xa.shape[1]
        if T > self.config.max_tokens:
            raise _lib.MoeError(_lib.MOE_EINVAL, f"batch of {T} tokens exceeds max_tokens={self.config.max_tokens}")
        if T == 0:
            return self._forward_empty(training, return_stats)
        if x_dtype == "bf16":
            xt = np.ascontiguousarray(xa.T, dtype=np.uint16)
            xcode = _lib.MOE_BF16
        else:
            xt = np.ascontiguousarray(xa.T, dtype=np.float32)
            xcode = _lib.MOE_F32
        dev = self._dev if self._dev is not None else self.sync_weights()
        if training and self._noise_error is not None:
            raise self._noise_error
        aux_free = self.balance_loss if isinstance(self.balance_loss, AuxiliaryFreeLoss) else None
        if aux_free is not None:
            dev.set_aux_free(aux_free)
        gate = self.router.gate_type
        if isinstance(gate, HOST_ROUTED_GATES):
            # the gate's indices come from host code (a hash function, a
            # sampler); the device runs the rest of forward_standard on them
            idx, gates = gate.host_routing(T, self.router.weight.shape[0])
            out, loss, res = dev.forward_routed(xt, xcode, training, idx, gates, None, want_aux=_aux is not None)
        else:
            out, loss, res = dev.forward(xt, xcode, training, want_aux=_aux is not None)
        if aux_free is not None:
            dev.get_aux_free(aux_free)
        if _aux is not None:
            _aux.update(res)
        if self.config.num_shared_experts == 0:
            # update_stats! -- src/core/moe_layer.jl:153, 250-264 (forward_standard only)
            self.training_stats["tokens_per_expert"] += res["counts"].astype(np.int64)
            self.training_stats["routing_entropy"].append(np.float32(res["mean_entropy"]))
        output = out.T
        loss = np.float32(loss)
        if return_stats:
            return output, loss, self.training_stats
        return output, loss


    def _forward_empty(self, training, return_stats):
        """A batch of no tokens, x of shape (input_dim, 0): what the reference's
        forward computes on empty arrays (src/core/moe_layer.jl:107-185), with
        no device work.  The output is (output_dim, 0).  The loss is 0 in
        inference.  In training it is the balance loss over no entries: the
        Switch loss divides zero counts by zero assignments (NaN,
        losses.jl:15-36); NoBalancingLoss gives 0; AuxiliaryFreeLoss counts
        the call in update_bias! and leaves the bias alone (no assignments,
        auxiliary_free.jl:36-55), then gives 0, or NaN with the complementary
        Switch term (:73-83).  A positive z_loss_weight adds the z-loss, a
        mean over no tokens (NaN, losses.jl:103-109).  forward_standard's
        statistics gain no counts and a NaN mean entropy (:250-264)."""
        c = self.config
        balance_alpha(self.balance_loss)  # a loss with no device path raises as in a non-empty call
        loss = np.float32(0.0)
        if training:
            bl = self.balance_loss
            if isinstance(bl, AuxiliaryFreeLoss):
                bl.update_counter += 1
                loss = np.float32(np.nan) if bl.use_complementary_loss else np.float32(0.0)
            elif not isinstance(bl, NoBalancingLoss):
                loss = np.float32(np.nan)
            if c.z_loss_weight > 0:
                loss = np.float32(np.nan)
        if c.num_shared_experts == 0:
            self.training_stats["routing_entropy"].append(np.float32(np.nan))
        output = np.zeros((c.output_dim, 0), dtype=np.float32)
        if return_stats:
            return output, loss, self.training_stats
        return output, loss


def moe_ffn_forward(moe, xb):
    """moe_ffn_forward! -- src/llama2/inference.jl:58-121, the decode caller,
    on this layer's router and gated experts, after the caller's rmsnorm; the
    layer's shared experts (num_shared_experts) are process_shared_experts!
    (:184-216), and an AuxiliaryFreeLoss gets update_bias! per token.  Each token is routed on its own (logits =
    W_router' xb, compute_gates) and its experts are combined in slot order:
    xb2 = 0; xb2 += gate_s * gated_expert_forward!(xb) for s = 1..k, with
    silu(g) = g * (1 / (1 + exp(-g))) (:154-167).

    xb: (input_dim,) or (input_dim, n) float32.  Returns (xb2 of the same
    shape, selected_experts (k[, n]) Int64 1-based, expert_gates (k[, n])
    Float32)."""
    xa = np.asarray(xb, dtype=np.float32)
    vec = xa.ndim == 1
    X = xa.reshape(-1, 1) if vec else xa
    if X.ndim != 2 or X.shape[0] != moe.config.input_dim:
        raise _lib.MoeError(_lib.MOE_EINVAL, f"xb must be ({moe.config.input_dim},) or ({moe.config.input_dim}, n)")
    dev = moe._dev if moe._dev is not None else moe.sync_weights()
    out, _, idx, gates = dev.decode(np.ascontiguousarray(X.T))
    ns = moe.config.num_shared_experts
    if ns > 0:
        # selected_experts as the router numbers them (the shared experts are
        # process_shared_experts!'s, not slots of the routing)
        idx, gates = idx[:, ns:] - ns, gates[:, ns:]
    if isinstance(moe.balance_loss, AuxiliaryFreeLoss):
        # update_bias!(config.moe_balance_loss, selected_experts) per token (:109-111)
        for t in range(idx.shape[0]):
            update_bias(moe.balance_loss, idx[t])
    if vec:
        return out[0], idx[0].astype(np.int64), gates[0]
    return out.T, idx.T.astype(np.int64), gates.T


def reset_stats(moe):
    """reset_stats!(moe) -- src/core/moe_layer.jl:271-276."""
    moe.training_stats["tokens_per_expert"][:] = 0
    moe.training_stats["routing_entropy"].clear()
    moe.training_stats["capacity_overflow"] = 0


def create_moe_layer(input_dim, hidden_dim, output_dim, **kwargs):
    """create_moe_layer(input_dim, hidden_dim, output_dim; kwargs...) --
    src/core/moe_layer.jl:285-293."""
    rng = kwargs.pop("rng", None)
    return MoELayer(MoEConfig(input_dim=input_dim, hidden_dim=hidden_dim, output_dim=output_dim, **kwargs), rng=rng)
