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


def balance_alpha(loss):
    """alpha the device applies for the layer's balance loss."""
    if isinstance(loss, SwitchTransformerLoss):
        return loss.alpha
    if isinstance(loss, NoBalancingLoss):
        return 0.0
    raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, f"balance loss {loss!r} has no device path")


def compute_loss(loss_fn, *args):
    """compute_loss(loss, indices, probs) / compute_loss(ZLoss, logits).

    indices (k, T) 1-based, probs (E, T), logits (E, T) -- Julia shapes."""
    if isinstance(loss_fn, NoBalancingLoss):
        return np.float32(0.0)
    out = ctypes.c_float(0.0)
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
