"""Load-balancing losses (src/balancing/losses.jl) computed on the device."""
import ctypes

import numpy as np

from . import _lib


class LoadBalancingLoss:
    """Abstract loss (src/gating/base.jl:14)."""


class SwitchTransformerLoss(LoadBalancingLoss):
    """SwitchTransformerLoss(alpha) -- src/balancing/losses.jl:11-36."""

    def __init__(self, alpha):
        self.alpha = float(np.float32(alpha))

    def __repr__(self):
        return f"SwitchTransformerLoss({self.alpha})"


class ZLoss(LoadBalancingLoss):
    """ZLoss(beta) -- src/balancing/losses.jl:99-114."""

    def __init__(self, beta):
        self.beta = float(np.float32(beta))

    def __repr__(self):
        return f"ZLoss({self.beta})"


class NoBalancingLoss(LoadBalancingLoss):
    """NoBalancingLoss -- src/gating/simple.jl: compute_loss returns 0f0."""

    def __repr__(self):
        return "NoBalancingLoss()"


class DeepSeekLoss(LoadBalancingLoss):
    """DeepSeekLoss(alpha[, balance_type, device_map]) -- src/balancing/losses.jl:46-74.
    The :expert type is the Switch loss; :device and :communication need a
    device map of an expert-parallel deployment and have no device path."""

    def __init__(self, alpha, balance_type="expert", device_map=None):
        self.alpha = float(np.float32(alpha))
        self.balance_type = str(balance_type).lstrip(":")
        self.device_map = device_map

    def __repr__(self):
        return f"DeepSeekLoss({self.alpha}, :{self.balance_type})"


class AuxiliaryFreeLoss(LoadBalancingLoss):
    """AuxiliaryFreeLoss(num_experts; bias_init, learning_rate, momentum,
    update_freq, use_complementary_loss, complementary_weight) --
    src/balancing/auxiliary_free.jl:11-34.  ``bias`` and ``bias_momentum`` are
    float32 vectors of length num_experts, ``update_counter`` counts
    compute_loss calls.  A layer with this loss gates on logits + bias on the
    device and updates the state there (moe_set_aux_free); the layer copies
    the state back after each call."""

    def __init__(self, num_experts, bias_init=0.0, learning_rate=0.01, momentum=0.9, update_freq=1,
                 use_complementary_loss=True, complementary_weight=0.001):
        self.bias = np.full(int(num_experts), np.float32(bias_init), dtype=np.float32)
        self.learning_rate = float(np.float32(learning_rate))
        self.momentum = float(np.float32(momentum))
        self.bias_momentum = np.zeros(int(num_experts), dtype=np.float32)
        self.update_freq = int(update_freq)
        self.update_counter = 0
        self.use_complementary_loss = bool(use_complementary_loss)
        self.complementary_weight = float(np.float32(complementary_weight))

    def __repr__(self):
        return f"AuxiliaryFreeLoss({len(self.bias)})"


def update_bias(loss_fn, expert_indices):
    """update_bias!(loss_fn, expert_indices) -- src/balancing/auxiliary_free.jl:36-69:
    counter += 1, then (every update_freq calls) the momentum / bias step on
    the device over the indices > 0."""
    loss_fn.update_counter += 1
    if loss_fn.update_counter % loss_fn.update_freq != 0:
        return
    idx = np.ascontiguousarray(np.asarray(expert_indices).reshape(-1), dtype=np.int32)
    bias = np.ascontiguousarray(loss_fn.bias, dtype=np.float32)
    mom = np.ascontiguousarray(loss_fn.bias_momentum, dtype=np.float32)
    _lib.check(_lib.lib().moe_aux_free_update_bias(idx.ctypes.data, idx.size, bias.size, loss_fn.learning_rate,
                                                   loss_fn.momentum, bias.ctypes.data, mom.ctypes.data))
    loss_fn.bias = bias
    loss_fn.bias_momentum = mom


def get_biased_logits(loss_fn, router_logits):
    """get_biased_logits -- src/balancing/auxiliary_free.jl:94-96: logits (E, T)
    .+ bias (the layer forward adds the bias on the device instead)."""
    return (np.asarray(router_logits, dtype=np.float32) + loss_fn.bias.reshape(-1, 1)).astype(np.float32)


def balance_alpha(loss):
    """alpha the device applies for the layer's balance loss."""
    if isinstance(loss, SwitchTransformerLoss):
        return loss.alpha
    if isinstance(loss, DeepSeekLoss) and loss.balance_type == "expert":
        return loss.alpha
    if isinstance(loss, NoBalancingLoss):
        return 0.0
    if isinstance(loss, AuxiliaryFreeLoss):
        return 1.0  # the complementary Switch(1) loss; the weight is applied by the device
    raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, f"balance loss {loss!r} has no device path")


def compute_loss(loss_fn, *args):
    """compute_loss(loss, indices, probs) / compute_loss(ZLoss, logits).

    indices (k, T) 1-based, probs (E, T), logits (E, T) -- Julia shapes."""
    if isinstance(loss_fn, NoBalancingLoss):
        return np.float32(0.0)
    out = ctypes.c_float(0.0)
    if isinstance(loss_fn, AuxiliaryFreeLoss):
        # src/balancing/auxiliary_free.jl:78-87
        indices, probs = args
        update_bias(loss_fn, indices)
        if not loss_fn.use_complementary_loss:
            return np.float32(0.0)
        sw = compute_loss(SwitchTransformerLoss(1.0), indices, probs)
        return np.float32(np.float32(loss_fn.complementary_weight) * sw)
    if isinstance(loss_fn, DeepSeekLoss):
        if loss_fn.balance_type != "expert":
            raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, f"DeepSeekLoss :{loss_fn.balance_type} has no device path")
        return compute_loss(SwitchTransformerLoss(loss_fn.alpha), *args)
    if isinstance(loss_fn, SwitchTransformerLoss):
        indices, probs = args
        idx = np.ascontiguousarray(np.asarray(indices).T, dtype=np.int32)
        pr = np.ascontiguousarray(np.asarray(probs, dtype=np.float32).T)
        T, k = idx.shape
        E = pr.shape[1]
        _lib.check(_lib.lib().moe_switch_loss(idx.ctypes.data, T, k, pr.ctypes.data, E, loss_fn.alpha,
                                              ctypes.byref(out)))
        return np.float32(out.value)
    if isinstance(loss_fn, ZLoss):
        (logits,) = args
        lg = np.ascontiguousarray(np.asarray(logits, dtype=np.float32).T)
        T, E = lg.shape
        _lib.check(_lib.lib().moe_z_loss(lg.ctypes.data, T, E, loss_fn.beta, ctypes.byref(out)))
        return np.float32(out.value)
    raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, f"compute_loss for {loss_fn!r} has no device path")
