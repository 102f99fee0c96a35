"""Gating mechanisms (src/gating/*.jl) and ``compute_gates`` on the device.

Arrays use the reference's Julia shapes: ``logits`` is (E, T), the returned
``indices`` (k, T) are 1-based int64 expert ids, ``gates`` (k, T) float32 and
``probs`` (E, T) float32.
"""
import ctypes

import numpy as np

from . import _lib
from ._device import DeviceLayer, GateSpec


class GatingMechanism:
    """Abstract gate (src/gating/base.jl:7)."""


class TopKGating(GatingMechanism):
    """TopKGating(k) -- src/gating/topk.jl:16-22 (``use_softmax_renorm`` and
    ``use_raw_logits`` are carried but, as in the reference, not read)."""

    def __init__(self, k, use_softmax_renorm=True, use_raw_logits=False):
        self.k = int(k)
        self.use_softmax_renorm = bool(use_softmax_renorm)
        self.use_raw_logits = bool(use_raw_logits)

    def __repr__(self):
        return f"TopKGating({self.k})"


class SwitchGating(GatingMechanism):
    """SwitchGating() = TopKGating(1) -- src/gating/switch.jl:7-11."""

    k = 1

    def __repr__(self):
        return "SwitchGating()"


class SharedExpertGating(GatingMechanism):
    """SharedExpertGating(num_shared, base_gate, num_experts) --
    src/gating/advanced.jl:74-108."""

    def __init__(self, num_shared, base_gate, num_experts):
        self.num_shared = int(num_shared)
        self.base_gate = base_gate
        self.num_experts = int(num_experts)

    def __repr__(self):
        return f"SharedExpertGating({self.num_shared}, {self.base_gate!r}, {self.num_experts})"


def gate_spec(gate, num_router_outputs):
    """Translate a gate object into the ABI's (kind, k, num_shared)."""
    if isinstance(gate, SwitchGating):
        return GateSpec(_lib.MOE_GATE_SWITCH, 1, 0)
    if isinstance(gate, TopKGating):
        return GateSpec(_lib.MOE_GATE_TOPK, gate.k, 0)
    if isinstance(gate, SharedExpertGating):
        if gate.num_experts != num_router_outputs:
            raise _lib.MoeError(_lib.MOE_EINVAL, "SharedExpertGating.num_experts must equal the router outputs")
        base = gate.base_gate
        if isinstance(base, SwitchGating):
            k = 1
        elif isinstance(base, TopKGating):
            k = base.k
        else:
            raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, f"SharedExpertGating base {base!r} has no device path")
        return GateSpec(_lib.MOE_GATE_SHARED, k, gate.num_shared)
    raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, f"gate {gate!r} has no device path")


_gate_handles = {}


def _gating_handle(spec, E, T):
    key = (spec, E)
    dev = _gate_handles.get(key)
    if dev is None or dev.max_tokens < T:
        if dev is not None:
            dev.close()
        dev = DeviceLayer.gating_only(spec, E, max(T, 256))
        _gate_handles[key] = dev
    return dev


def compute_gates(gate, router_logits):
    """compute_gates(gate, router_logits) -> (indices, gates, probs) --
    src/gating/topk.jl:24-44, switch.jl:9-11, advanced.jl:80-108."""
    logits = np.asarray(router_logits, dtype=np.float32)
    if logits.ndim != 2:
        raise _lib.MoeError(_lib.MOE_EINVAL, "router_logits must be a matrix (E, T)")
    E, T = logits.shape
    spec = gate_spec(gate, E)
    kt = spec.num_shared + spec.k
    idx = np.zeros((T, kt), dtype=np.int32)
    gates = np.zeros((T, kt), dtype=np.float32)
    probs = np.zeros((T, E), dtype=np.float32)
    if T > 0:
        dev = _gating_handle(spec, E, T)
        lt = np.ascontiguousarray(logits.T)
        _lib.check(
            _lib.lib().moe_compute_gates(dev.h, lt.ctypes.data, T, idx.ctypes.data, gates.ctypes.data,
                                         probs.ctypes.data),
            dev.h,
        )
    return idx.T.astype(np.int64), gates.T, probs.T


def route_from_logits(gate, router_logits, training=False, capacity_factor=None):
    """compute_gates plus the bucketing of process_expert_forward!
    (src/core/moe_layer.jl:192-203): returns (indices, gates, probs, counts,
    offsets, perm) with perm[pos] = t*k + slot (0-based) for pos <
    offsets[-1].  With ``capacity_factor`` and ``training`` the capacity
    constraint (src/core/moe_layer.jl:221-248) is applied first."""
    logits = np.asarray(router_logits, dtype=np.float32)
    E, T = logits.shape
    spec = gate_spec(gate, E)
    kt = spec.num_shared + spec.k
    dev = DeviceLayer.gating_only(spec, E, max(T, 1), capacity_factor=capacity_factor)
    try:
        idx = np.zeros((T, kt), dtype=np.int32)
        gates = np.zeros((T, kt), dtype=np.float32)
        probs = np.zeros((T, E), dtype=np.float32)
        counts = np.zeros(E, dtype=np.int32)
        offsets = np.zeros(E + 1, dtype=np.int32)
        perm = np.zeros(T * kt, dtype=np.int32)
        lt = np.ascontiguousarray(logits.T)
        _lib.check(
            _lib.lib().moe_route_from_logits(dev.h, lt.ctypes.data, T, int(bool(training)), idx.ctypes.data,
                                             gates.ctypes.data, probs.ctypes.data, counts.ctypes.data,
                                             offsets.ctypes.data, perm.ctypes.data),
            dev.h,
        )
    finally:
        dev.close()
    return idx.T.astype(np.int64), gates.T, probs.T, counts, offsets, perm
