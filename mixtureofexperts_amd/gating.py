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


class SoftMoEGating(GatingMechanism):
    """SoftMoEGating(k, lambda) -- src/gating/advanced.jl:7-33: softmax of
    logits ./ lambda and its top-k; its gate matrix is the (E, T) probability
    matrix, so the dispatch weighs slot j with the probability of expert j."""

    def __init__(self, k, lam):
        self.k = int(k)
        self.lam = float(np.float32(lam))

    def __repr__(self):
        return f"SoftMoEGating({self.k}, {self.lam})"


class ExpertChoiceGating(GatingMechanism):
    """ExpertChoiceGating(capacity_factor) -- src/gating/expert_choice.jl:7-53:
    each expert takes its ceil(T * cf / E) tokens of largest logit."""

    def __init__(self, capacity_factor):
        self.capacity_factor = float(np.float32(capacity_factor))

    def capacity(self, T, E):
        return int(np.ceil(np.float32(np.float32(T) * np.float32(self.capacity_factor)) / np.float32(E)))

    def __repr__(self):
        return f"ExpertChoiceGating({self.capacity_factor})"


def _default_hash(i):
    """A 64-bit integer mix (splitmix64 finaliser) standing in for Julia's
    `hash(::Int)`, whose values depend on the Julia version."""
    z = (int(i) + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
    return z ^ (z >> 31)


class HashGating(GatingMechanism):
    """HashGating(k, num_experts[, hash_fn]) -- src/gating/advanced.jl:37-66:
    token i (1-based) goes to experts (hash_fn(i) + j) % E + 1, j = 0..k-1
    (UInt64 arithmetic), gates 1/k, probabilities 1/E.  hash_fn is user code
    and runs on the host; the layer forward takes the indices from it."""

    def __init__(self, k, num_experts, hash_fn=None):
        self.k = int(k)
        self.num_experts = int(num_experts)
        self.hash_fn = _default_hash if hash_fn is None else hash_fn

    def host_routing(self, T, E):
        idx = np.zeros((T, self.k), dtype=np.int32)
        for i in range(T):
            h = int(self.hash_fn(i + 1)) & 0xFFFFFFFFFFFFFFFF
            for j in range(self.k):
                idx[i, j] = ((h + j) & 0xFFFFFFFFFFFFFFFF) % E + 1
        gates = np.full((T, self.k), np.float32(1) / np.float32(self.k), dtype=np.float32)
        return idx, gates

    def __repr__(self):
        return f"HashGating({self.k}, {self.num_experts})"


class RandomGating(GatingMechanism):
    """RandomGating(k=1) -- src/gating/simple.jl:7-28: k distinct experts per
    token drawn uniformly (StatsBase.sample without replacement; the stream is
    numpy's, not Julia's), gates 1/k, probabilities 1/E."""

    def __init__(self, k=1, rng=None):
        self.k = int(k)
        self.rng = np.random.default_rng() if rng is None else rng

    def host_routing(self, T, E):
        idx = (np.argsort(self.rng.random((T, E)), axis=1)[:, :self.k] + 1).astype(np.int32)
        gates = np.full((T, self.k), np.float32(1) / np.float32(self.k), dtype=np.float32)
        return idx, gates

    def __repr__(self):
        return f"RandomGating({self.k})"


class JitterGating(GatingMechanism):
    """JitterGating(base_gate, eps) -- src/gating/switch.jl:20-33: with
    training=true the logits are multiplied by 1 + (2u - 1) eps, u ~ U[0, 1)
    (numpy's stream), then the base gate.  The layer's router calls
    compute_gates without `training`, so in a layer it is the base gate."""

    def __init__(self, base_gate, eps, rng=None):
        self.base_gate = base_gate
        self.eps = float(np.float32(eps))
        self.rng = np.random.default_rng() if rng is None else rng

    def __repr__(self):
        return f"JitterGating({self.base_gate!r}, {self.eps})"


class StochasticTopKGating(GatingMechanism):
    """StochasticTopKGating(k, train_only) -- src/gating/topk.jl:53-70: with
    noise logits and (training or not train_only), logits .+ randn .*
    softplus(noise_logits) (numpy's stream), then TopKGating(k).  The layer's
    router passes no noise logits, so in a layer it is TopKGating(k)."""

    def __init__(self, k, train_only=True, rng=None):
        self.k = int(k)
        self.train_only = bool(train_only)
        self.rng = np.random.default_rng() if rng is None else rng

    def __repr__(self):
        return f"StochasticTopKGating({self.k}, {self.train_only})"


HOST_ROUTED_GATES = (HashGating, RandomGating)


def gate_spec(gate, num_router_outputs):
    """Translate a gate object into the ABI's (kind, k, num_shared, param).
    Gates whose indices come from host code (Hash, Random) map to a top-k
    handle of their k: the layer passes their routing to moe_forward_routed."""
    if isinstance(gate, JitterGating):
        return gate_spec(gate.base_gate, num_router_outputs)
    if isinstance(gate, StochasticTopKGating):
        return GateSpec(_lib.MOE_GATE_TOPK, gate.k, 0)
    if isinstance(gate, HOST_ROUTED_GATES):
        return GateSpec(_lib.MOE_GATE_TOPK, gate.k, 0)
    if isinstance(gate, SoftMoEGating):
        return GateSpec(_lib.MOE_GATE_SOFT, gate.k, 0, gate.lam)
    if isinstance(gate, ExpertChoiceGating):
        return GateSpec(_lib.MOE_GATE_EXPERT_CHOICE, 1, 0, gate.capacity_factor)
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


def compute_gates(gate, router_logits, noise_logits=None, training=False):
    """compute_gates(gate, router_logits) -> (indices, gates, probs) --
    src/gating/topk.jl:24-70, switch.jl:9-33, advanced.jl:17-108,
    expert_choice.jl:11-53, simple.jl:14-28.  ``training`` (JitterGating,
    StochasticTopKGating) and ``noise_logits`` (StochasticTopKGating) as the
    reference's keyword / optional arguments."""
    logits = np.asarray(router_logits, dtype=np.float32)
    if logits.ndim != 2:
        raise _lib.MoeError(_lib.MOE_EINVAL, "router_logits must be a matrix (E, T)")
    E, T = logits.shape
    if isinstance(gate, JitterGating):
        if training:
            u = gate.rng.random(logits.shape, dtype=np.float32)
            jitter = (np.float32(1) + (np.float32(2) * u - np.float32(1)) * np.float32(gate.eps)).astype(np.float32)
            logits = (logits * jitter).astype(np.float32)
        return compute_gates(gate.base_gate, logits)
    if isinstance(gate, StochasticTopKGating):
        if (training or not gate.train_only) and noise_logits is not None:
            nl = np.asarray(noise_logits, dtype=np.float32)
            sp = np.logaddexp(np.float32(0), nl).astype(np.float32)  # softplus
            noise = (gate.rng.standard_normal(logits.shape, dtype=np.float32) * sp).astype(np.float32)
            logits = (logits + noise).astype(np.float32)
        return compute_gates(TopKGating(gate.k), logits)
    if isinstance(gate, HOST_ROUTED_GATES):
        idx, gates = gate.host_routing(T, E)
        probs = np.full((E, T), np.float32(1) / np.float32(E), dtype=np.float32)
        return idx.T.astype(np.int64), gates.T, probs
    spec = gate_spec(gate, E)
    kt = spec.num_shared + spec.k
    dev = _gating_handle(spec, E, T) if T > 0 else None
    if isinstance(gate, ExpertChoiceGating):
        # the handle's slots: min(capacity at its max_tokens, E), of which a
        # call fills min(capacity, E)
        kt = dev.slots if dev is not None else 0
    idx = np.zeros((T, kt), dtype=np.int32)
    gates = np.zeros((T, kt), dtype=np.float32)
    probs = np.zeros((T, E), dtype=np.float32)
    if T > 0:
        lt = np.ascontiguousarray(logits.T)
        _lib.check(
            _lib.lib().moe_compute_gates(dev.h, lt.ctypes.data, T, idx.ctypes.data, gates.ctypes.data,
                                         probs.ctypes.data),
            dev.h,
        )
    if isinstance(gate, SoftMoEGating):
        return idx.T.astype(np.int64), probs.T.copy(), probs.T  # the gate matrix is the probabilities
    if isinstance(gate, ExpertChoiceGating):
        # (capacity, T) matrices as the reference returns them; rows past the
        # slots a token can hold are empty
        C = gate.capacity(T, E)
        fi = np.zeros((C, T), dtype=np.int64)
        fg = np.zeros((C, T), dtype=np.float32)
        n = min(C, kt)
        fi[:n] = idx.T[:n]
        fg[:n] = gates.T[:n]
        return fi, fg, probs.T
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
    dev = DeviceLayer.gating_only(spec, E, max(T, 1), capacity_factor=capacity_factor)
    kt = dev.slots
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
