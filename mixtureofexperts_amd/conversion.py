"""convert_to_moe's layer conversion and the layer's weight format on disk.

``convert_layer_to_moe`` mirrors src/llama2/conversion.jl:191-331 for one
dense Llama FFN: the experts are derived on the device from the dense weights
(``moe_init_experts_from_dense``: :copy, :perturb, :split, :random) and
prepacked once in the layer's GEMM dtype (fp32, bf16, or fp8-e4m3 with
per-output-channel scales); the router is ``randn(dim, E) .* sqrt(2f0 / dim)``
(create_router_weights, :347-356).

``save_moe_layer`` / ``load_moe_layer`` keep a layer as safetensors: the
prepacked weights in their stored dtype (bf16 as uint16 bits, fp8 as bytes
plus scales) read back from the device (``moe_get_expert``), and the
configuration as JSON metadata.  The reference serialises whole models with
Julia's Serialization (src/llama2/utils.jl:22-67), a format only Julia reads,
and its loader is broken (utils.jl:328-335); this format is the layer's own.
"""
import json

import numpy as np

from . import _lib
from .activations import gelu, identity, relu, silu
from .balancing import NoBalancingLoss, SwitchTransformerLoss
from .experts import GatedExpert, StandardExpert
from .gating import ExpertChoiceGating, SharedExpertGating, SoftMoEGating, SwitchGating, TopKGating
from .layer import MoEConfig, MoELayer, Router

STRATEGIES = {"copy": _lib.MOE_INIT_COPY, "perturb": _lib.MOE_INIT_PERTURB, "split": _lib.MOE_INIT_SPLIT,
              "random": _lib.MOE_INIT_RANDOM}
_WDT = {"f32": (_lib.MOE_F32, np.float32), "bf16": (_lib.MOE_BF16, np.uint16), "fp8": (_lib.MOE_FP8_E4M3, np.uint8)}
_ACTS = {"silu": silu, "gelu": gelu, "relu": relu, "identity": identity}


def _read_experts(layer, dev):
    """Host copies of the device's prepacked expert weights (Flux (out, in))."""
    c = layer.config
    code, dt = _WDT[c.weight_dtype]
    experts = []
    for e in range(c.num_experts):
        w1 = np.zeros((c.hidden_dim, c.input_dim), dt)
        w2 = np.zeros((c.output_dim, c.hidden_dim), dt)
        w3 = np.zeros((c.hidden_dim, c.input_dim), dt)
        s = [np.zeros(c.hidden_dim, np.float32), np.zeros(c.output_dim, np.float32), np.zeros(c.hidden_dim, np.float32)]
        _lib.check(_lib.lib().moe_get_expert(dev.h, e, _lib.MOE_LAYOUT_LLAMA_IN_OUT, w1.ctypes.data, w2.ctypes.data,
                                             w3.ctypes.data, s[0].ctypes.data, s[1].ctypes.data, s[2].ctypes.data),
                   dev.h)
        ex = GatedExpert(c.input_dim, c.hidden_dim, c.output_dim, c.activation, weight_dtype=code, w1=w1, w2=w2, w3=w3)
        if c.weight_dtype == "fp8":
            ex.scales = tuple(s)
        experts.append(ex)
    return experts


def convert_layer_to_moe(w1, w2, w3, *, num_experts=8, top_k=2, expert_init_strategy="perturb",
                         expert_init_noise=0.01, gate_type=None, balance_loss=None, capacity_factor=1.25,
                         drop_tokens=False, weight_dtype="f32", max_tokens=4096, seed=0, rng=None):
    """convert_layer_to_moe(original_layer, moe_config, strategy) --
    src/llama2/conversion.jl:191-233, for the FFN of one Llama layer.

    w1, w3: (dim, hidden_dim) and w2: (hidden_dim, dim) float32, the Llama2
    layout (in, out) the dense FFN computes w2' (silu(w1' x) .* (w3' x)) with.
    Returns an MoELayer of ``num_experts`` gated silu experts whose weights
    were made and packed on the device; ``seed`` keys the device generator of
    the :perturb / :random draws, ``rng`` the router's host draws."""
    if expert_init_strategy not in STRATEGIES:
        raise _lib.MoeError(_lib.MOE_EINVAL, f"Unknown expert initialization strategy: {expert_init_strategy}")
    w1 = np.asarray(w1, np.float32)
    w2 = np.asarray(w2, np.float32)
    w3 = np.asarray(w3, np.float32)
    dim, hidden = w1.shape
    if w3.shape != (dim, hidden) or w2.shape != (hidden, dim):
        raise _lib.MoeError(_lib.MOE_EINVAL, "w1, w3 must be (dim, hidden) and w2 (hidden, dim)")
    rng = np.random.default_rng() if rng is None else rng
    sigma = np.float32(np.sqrt(np.float32(2.0) / np.float32(dim)))
    router_w = (rng.standard_normal((dim, num_experts), dtype=np.float32) * sigma).astype(np.float32)
    cfg = MoEConfig(num_experts=num_experts, expert_type="gated", input_dim=dim, hidden_dim=hidden, output_dim=dim,
                    activation=silu, gate_type=gate_type if gate_type is not None else TopKGating(top_k),
                    top_k=top_k, balance_loss=balance_loss if balance_loss is not None else SwitchTransformerLoss(0.01),
                    capacity_factor=capacity_factor, drop_tokens=drop_tokens, weight_dtype=weight_dtype,
                    max_tokens=max_tokens)
    router = Router(dim, num_experts, cfg.gate_type, weight=np.ascontiguousarray(router_w.T))
    # placeholder host experts (replaced by the device's below); no host draws
    experts = [GatedExpert(dim, hidden, dim, silu, w1=np.zeros((1, 1), np.float32), w2=np.zeros((1, 1), np.float32),
                           w3=np.zeros((1, 1), np.float32)) for _ in range(num_experts)]
    layer = MoELayer(cfg, experts=experts, router=router)
    dev = layer._new_device()
    dev.set_router(np.ascontiguousarray(router.weight.T), None)
    # Llama (in, out) column-major is memory [out][in]: the numpy transposes
    src = [np.ascontiguousarray(m.T) for m in (w1, w2, w3)]
    _lib.check(_lib.lib().moe_init_experts_from_dense(
        dev.h, _lib.MOE_LAYOUT_LLAMA_IN_OUT, _lib.MOE_F32, src[0].ctypes.data, src[1].ctypes.data, src[2].ctypes.data,
        None, None, None, STRATEGIES[expert_init_strategy], float(np.float32(expert_init_noise)), int(seed)), dev.h)
    layer.experts = _read_experts(layer, dev)
    layer._dev = dev
    return layer


# ---- on-disk format ------------------------------------------------------------

def _gate_to_json(g):
    if isinstance(g, SwitchGating):
        return {"type": "SwitchGating"}
    if isinstance(g, TopKGating):
        return {"type": "TopKGating", "k": g.k}
    if isinstance(g, SharedExpertGating):
        return {"type": "SharedExpertGating", "num_shared": g.num_shared, "base": _gate_to_json(g.base_gate),
                "num_experts": g.num_experts}
    if isinstance(g, SoftMoEGating):
        return {"type": "SoftMoEGating", "k": g.k, "lambda": g.lam}
    if isinstance(g, ExpertChoiceGating):
        return {"type": "ExpertChoiceGating", "capacity_factor": g.capacity_factor}
    raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, f"gate {g!r} cannot be saved")


def _gate_from_json(d):
    t = d["type"]
    if t == "SwitchGating":
        return SwitchGating()
    if t == "TopKGating":
        return TopKGating(d["k"])
    if t == "SharedExpertGating":
        return SharedExpertGating(d["num_shared"], _gate_from_json(d["base"]), d["num_experts"])
    if t == "SoftMoEGating":
        return SoftMoEGating(d["k"], d["lambda"])
    if t == "ExpertChoiceGating":
        return ExpertChoiceGating(d["capacity_factor"])
    raise _lib.MoeError(_lib.MOE_EINVAL, f"unknown gate {t}")


def _loss_to_json(loss):
    if isinstance(loss, SwitchTransformerLoss):
        return {"type": "SwitchTransformerLoss", "alpha": loss.alpha}
    if isinstance(loss, NoBalancingLoss):
        return {"type": "NoBalancingLoss"}
    raise _lib.MoeError(_lib.MOE_EUNSUPPORTED, f"balance loss {loss!r} cannot be saved")


def _loss_from_json(d):
    if d["type"] == "SwitchTransformerLoss":
        return SwitchTransformerLoss(d["alpha"])
    return NoBalancingLoss()


def save_moe_layer(layer, path):
    """Write a layer (config, router, the device's prepacked expert weights)
    to a safetensors file."""
    from safetensors.numpy import save_file

    c = layer.config
    dev = layer._dev if layer._dev is not None else layer.sync_weights()
    tensors = {"router.weight": np.ascontiguousarray(layer.router.weight, np.float32)}
    if layer.router.bias is not None:
        tensors["router.bias"] = np.ascontiguousarray(layer.router.bias, np.float32)
    code, dt = _WDT[c.weight_dtype]
    gated = c.expert_type == "gated"
    for e in range(c.num_experts):
        w1 = np.zeros((c.hidden_dim, c.input_dim), dt)
        w2 = np.zeros((c.output_dim, c.hidden_dim), dt)
        w3 = np.zeros((c.hidden_dim, c.input_dim), dt) if gated else None
        s = [np.zeros(c.hidden_dim, np.float32), np.zeros(c.output_dim, np.float32), np.zeros(c.hidden_dim, np.float32)]
        _lib.check(_lib.lib().moe_get_expert(dev.h, e, _lib.MOE_LAYOUT_LLAMA_IN_OUT, w1.ctypes.data, w2.ctypes.data,
                                             None if w3 is None else w3.ctypes.data, s[0].ctypes.data,
                                             s[1].ctypes.data, s[2].ctypes.data), dev.h)
        tensors[f"experts.{e}.w1"] = w1
        tensors[f"experts.{e}.w2"] = w2
        if gated:
            tensors[f"experts.{e}.w3"] = w3
        else:
            ex = layer.experts[e]
            tensors[f"experts.{e}.b1"] = np.ascontiguousarray(ex.b1 if ex.b1 is not None else np.zeros(c.hidden_dim),
                                                              np.float32)
            tensors[f"experts.{e}.b2"] = np.ascontiguousarray(ex.b2 if ex.b2 is not None else np.zeros(c.output_dim),
                                                              np.float32)
        if c.weight_dtype == "fp8":
            for i, nm in enumerate(("s1", "s2", "s3")[:3 if gated else 2]):
                tensors[f"experts.{e}.{nm}"] = s[i]
    meta = dict(num_experts=c.num_experts, expert_type=c.expert_type, input_dim=c.input_dim, hidden_dim=c.hidden_dim,
                output_dim=c.output_dim, activation=repr(c.activation), gate=_gate_to_json(layer.router.gate_type),
                top_k=c.top_k, balance_loss=_loss_to_json(layer.balance_loss), z_loss_weight=c.z_loss_weight,
                capacity_factor=c.capacity_factor, drop_tokens=c.drop_tokens,
                num_shared_experts=c.num_shared_experts, weight_dtype=c.weight_dtype, max_tokens=c.max_tokens)
    save_file(tensors, path, metadata={"moe_layer": json.dumps(meta)})


def load_moe_layer(path, max_tokens=None):
    """Read a layer written by save_moe_layer; the weights go to the device in
    their stored dtype (no requantisation)."""
    from safetensors import safe_open

    with safe_open(path, framework="numpy") as f:
        meta = json.loads(f.metadata()["moe_layer"])
        t = {k: f.get_tensor(k) for k in f.keys()}
    code, dt = _WDT[meta["weight_dtype"]]
    act = _ACTS[meta["activation"]]
    cfg = MoEConfig(num_experts=meta["num_experts"], expert_type=meta["expert_type"], input_dim=meta["input_dim"],
                    hidden_dim=meta["hidden_dim"], output_dim=meta["output_dim"], activation=act,
                    gate_type=_gate_from_json(meta["gate"]), top_k=meta["top_k"],
                    balance_loss=_loss_from_json(meta["balance_loss"]), z_loss_weight=meta["z_loss_weight"],
                    capacity_factor=meta["capacity_factor"], drop_tokens=meta["drop_tokens"],
                    num_shared_experts=meta["num_shared_experts"], weight_dtype=meta["weight_dtype"],
                    max_tokens=max_tokens or meta["max_tokens"])
    router = Router(cfg.input_dim, t["router.weight"].shape[0], cfg.gate_type, weight=t["router.weight"],
                    bias=t.get("router.bias"))
    experts = []
    for e in range(cfg.num_experts):
        if cfg.expert_type == "gated":
            ex = GatedExpert(cfg.input_dim, cfg.hidden_dim, cfg.output_dim, act, weight_dtype=code,
                             w1=t[f"experts.{e}.w1"], w2=t[f"experts.{e}.w2"], w3=t[f"experts.{e}.w3"])
            if meta["weight_dtype"] == "fp8":
                ex.scales = (t[f"experts.{e}.s1"], t[f"experts.{e}.s2"], t[f"experts.{e}.s3"])
        else:
            ex = StandardExpert(cfg.input_dim, cfg.hidden_dim, cfg.output_dim, act, weight_dtype=code,
                                w1=t[f"experts.{e}.w1"], w2=t[f"experts.{e}.w2"], b1=t[f"experts.{e}.b1"],
                                b2=t[f"experts.{e}.b2"])
            if meta["weight_dtype"] == "fp8":
                ex.scales = (t[f"experts.{e}.s1"], t[f"experts.{e}.s2"])
        experts.append(ex)
    return MoELayer(cfg, experts=experts, router=router)
