"""CPU checks of the C ABI boundary: the library loads, exports every symbol
include/moe_mi355x.h declares, and rejects bad configurations before touching
the device.  No compute call is made (no GPU here)."""
import ctypes
import os
import re

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "moe_mi355x.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int|char\s*\*|const char\s*\*)\s*\*?\s*(moe_\w+)\s*\(",
                                 text, flags=re.M)))


def test_header_parses():
    fns = header_functions()
    assert "moe_forward" in fns and "moe_create" in fns and len(fns) >= 20


def test_library_exports_every_declared_symbol(moe):
    from mixtureofexperts_amd import _lib

    L = _lib.lib()
    for name in header_functions():
        assert hasattr(L, name), name
    assert sorted(_lib.EXPORTED_SYMBOLS) == header_functions()


def test_abi_version(moe):
    from mixtureofexperts_amd import _lib

    assert _lib.lib().moe_abi_version() == 1


def _cfg(**kw):
    from mixtureofexperts_amd import _lib

    c = _lib.MoeConfigC()
    c.num_experts, c.expert_type, c.input_dim, c.hidden_dim, c.output_dim = 8, 0, 64, 128, 64
    c.activation, c.gate_kind, c.top_k, c.gate_num_shared, c.weight_dtype = 1, 0, 2, 0, 1
    c.balance_alpha, c.z_loss_weight, c.capacity_factor, c.drop_tokens, c.max_tokens = 0.01, 0.001, 1.25, 0, 64
    for k, v in kw.items():
        setattr(c, k, v)
    return c


@pytest.mark.parametrize("bad,msg", [
    (dict(num_experts=0), "num_experts"),
    (dict(num_experts=513), "num_experts"),
    (dict(top_k=9), "top_k"),
    (dict(top_k=0), "top_k"),
    (dict(top_k=17, num_experts=32), "MOE_MAX_TOPK"),
    (dict(gate_kind=2, gate_num_shared=8), "gate_num_shared"),
    (dict(gate_kind=2, gate_num_shared=2, top_k=15, num_experts=32), "MOE_MAX_TOPK"),
    (dict(gate_kind=7), "gate_kind"),
    (dict(weight_dtype=5), "weight_dtype"),
    (dict(max_tokens=0), "max_tokens"),
    (dict(input_dim=0), "dimensions"),
    (dict(drop_tokens=1, capacity_factor=0.0), "capacity_factor"),
    (dict(num_shared_experts=8), "num_shared_experts"),
    (dict(num_shared_experts=-1), "num_shared_experts"),
    (dict(num_shared_experts=7), "top_k"),
    (dict(num_shared_experts=2, top_k=15, num_experts=32), "MOE_MAX_TOPK"),
    # with the layer's shared experts the gate sees num_experts - num_shared_experts experts
    (dict(num_shared_experts=2, gate_kind=2, gate_num_shared=6), "gate_num_shared"),
    (dict(num_shared_experts=2, gate_kind=2, gate_num_shared=1, top_k=14, num_experts=32), "MOE_MAX_TOPK"),
    (dict(num_shared_experts=2, gate_kind=2, gate_num_shared=3, top_k=4), "top_k"),
    (dict(gate_kind=4, gate_param=0.0), "capacity_factor"),
    (dict(gate_kind=3, top_k=9), "top_k"),
    (dict(gate_kind=3, num_shared_experts=7), "top_k"),
])
def test_create_rejects_bad_config(moe, bad, msg):
    from mixtureofexperts_amd import _lib

    L = _lib.lib()
    h = ctypes.c_void_p()
    rc = L.moe_create(ctypes.byref(_cfg(**bad)), ctypes.byref(h))
    assert rc == _lib.MOE_EINVAL
    assert h.value is None
    assert msg in L.moe_last_error(None).decode()


@pytest.mark.gpu
@pytest.mark.parametrize("kw,slots,router_rows", [
    (dict(num_shared_experts=1, gate_kind=3, top_k=2, gate_param=0.5), 3, 7),      # SoftMoEGating
    (dict(num_shared_experts=2, gate_kind=4, gate_param=1.0), 2 + 6, 6),           # ExpertChoice: 2 + min(C=11, 6)
    (dict(num_shared_experts=2, gate_kind=2, gate_num_shared=1, top_k=2), 5, 6),  # SharedExpertGating
])
def test_create_accepts_shared_experts_with_every_gate(moe, kw, slots, router_rows):
    # forward_with_shared_experts runs whatever gate the layer holds
    # (src/core/moe_layer.jl:158-185): the shared slots plus the gate's
    from mixtureofexperts_amd import _lib

    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.moe_create(ctypes.byref(_cfg(**kw)), ctypes.byref(h)) == _lib.MOE_OK
    try:
        assert L.moe_slots_per_token(h) == slots
        assert L.moe_router_outputs(h) == router_rows
    finally:
        L.moe_destroy(h)


def test_null_handle_calls_fail_cleanly(moe):
    from mixtureofexperts_amd import _lib

    L = _lib.lib()
    assert L.moe_forward(None, None, 0, 1, 0, None, None, None) == _lib.MOE_EINVAL
    assert L.moe_set_router(None, None, None) == _lib.MOE_EINVAL
    assert L.moe_destroy(None) == _lib.MOE_OK
    assert L.moe_router_outputs(None) == -1


def test_loss_argument_checks(moe):
    from mixtureofexperts_amd import _lib

    L = _lib.lib()
    out = ctypes.c_float(0)
    assert L.moe_switch_loss(None, 4, 0, None, 8, 0.01, ctypes.byref(out)) == _lib.MOE_EINVAL
    assert L.moe_z_loss(None, 4, 8, 0.001, ctypes.byref(out)) == _lib.MOE_EINVAL
    # T = 0: means over no tokens are NaN, as Julia's mean of an empty array
    assert L.moe_z_loss(None, 0, 8, 0.001, ctypes.byref(out)) == _lib.MOE_OK and np.isnan(out.value)


def test_host_mirror_config_defaults(moe):
    # MoEConfig defaults mirror src/core/moe_layer.jl:4-29
    c = moe.MoEConfig()
    assert (c.num_experts, c.expert_type, c.input_dim, c.hidden_dim, c.output_dim) == (8, "standard", 768, 3072, 768)
    assert c.activation is moe.gelu and isinstance(c.gate_type, moe.TopKGating) and c.gate_type.k == 2
    assert c.z_loss_weight == 0.001 and c.capacity_factor == 1.25 and c.drop_tokens is False
    assert isinstance(c.balance_loss, moe.SwitchTransformerLoss) and abs(c.balance_loss.alpha - 0.01) < 1e-9
    assert c.num_shared_experts == 0 and c.use_fp32_router is True


def test_host_mirror_rejects_unsupported_before_device(moe):
    from mixtureofexperts_amd import _lib

    with pytest.raises(moe.MoeError):
        moe.MoELayer(moe.MoEConfig(input_dim=8, hidden_dim=16, output_dim=8, use_cur=True))
    with pytest.raises(moe.MoeError):
        moe.gating.gate_spec(object(), 8)
    with pytest.raises(moe.MoeError):
        moe.activations.activation_code(lambda v: v)


def test_layer_empty_batch(moe):
    # x of shape (input_dim, 0): the reference's forward on empty arrays
    # (src/core/moe_layer.jl:107-185) -- an empty output, loss 0 in inference;
    # in training the Switch loss's 0 / 0 and the z-loss's mean over no tokens
    # are NaN.  No device work: the layer never builds its handle.
    def layer(**kw):
        cfg = dict(num_experts=4, expert_type="gated", input_dim=16, hidden_dim=32, output_dim=8,
                   activation=moe.silu, gate_type=moe.TopKGating(2))
        cfg.update(kw)
        return moe.MoELayer(moe.MoEConfig(**cfg), rng=np.random.default_rng(0))

    x = np.zeros((16, 0), np.float32)
    lay = layer()
    out, loss = lay(x)
    assert out.shape == (8, 0) and out.dtype == np.float32 and loss == np.float32(0.0)
    out, loss, stats = lay(x, training=True, return_stats=True)
    assert out.shape == (8, 0) and np.isnan(loss)
    assert stats["tokens_per_expert"].sum() == 0
    assert len(stats["routing_entropy"]) == 2 and all(np.isnan(v) for v in stats["routing_entropy"])
    assert lay._dev is None
    # no balance loss and no z-loss: 0; the z-loss alone: NaN
    assert layer(balance_loss=moe.NoBalancingLoss(), z_loss_weight=0.0)(x, training=True)[1] == np.float32(0.0)
    assert np.isnan(layer(balance_loss=moe.NoBalancingLoss(), z_loss_weight=0.001)(x, training=True)[1])
    # AuxiliaryFreeLoss: update_bias! counts the call, the bias stays (no assignments)
    aux = moe.AuxiliaryFreeLoss(4, bias_init=0.25, use_complementary_loss=False)
    lay = layer(balance_loss=aux, z_loss_weight=0.0)
    assert lay(x, training=True)[1] == np.float32(0.0) and aux.update_counter == 1
    assert np.array_equal(aux.bias, np.full(4, 0.25, np.float32)) and not aux.bias_momentum.any()
    assert lay(x)[1] == np.float32(0.0) and aux.update_counter == 1  # inference: no compute_loss
    aux_c = moe.AuxiliaryFreeLoss(4, use_complementary_loss=True)
    assert np.isnan(layer(balance_loss=aux_c, z_loss_weight=0.0)(x, training=True)[1])
    # forward_with_shared_experts updates no statistics
    lay = layer(num_shared_experts=1)
    out, loss, stats = lay(x, training=True, return_stats=True)
    assert out.shape == (8, 0) and np.isnan(loss) and stats["routing_entropy"] == []
    with pytest.raises(moe.MoeError):
        lay(np.zeros((15, 0), np.float32))


def test_gate_spec_mapping(moe):
    from mixtureofexperts_amd import _lib

    assert tuple(moe.gating.gate_spec(moe.TopKGating(3), 8)) == (_lib.MOE_GATE_TOPK, 3, 0, 0.0)
    assert tuple(moe.gating.gate_spec(moe.SwitchGating(), 8)) == (_lib.MOE_GATE_SWITCH, 1, 0, 0.0)
    g = moe.SharedExpertGating(2, moe.TopKGating(6), 66)
    assert tuple(moe.gating.gate_spec(g, 66)) == (_lib.MOE_GATE_SHARED, 6, 2, 0.0)
    assert tuple(moe.gating.gate_spec(moe.SoftMoEGating(2, 0.5), 8)) == (_lib.MOE_GATE_SOFT, 2, 0, 0.5)
    assert tuple(moe.gating.gate_spec(moe.ExpertChoiceGating(1.25), 8)) == (_lib.MOE_GATE_EXPERT_CHOICE, 1, 0, 1.25)
    # in a layer the router passes no `training` / noise logits: base gate / TopKGating(k)
    assert tuple(moe.gating.gate_spec(moe.JitterGating(moe.SwitchGating(), 0.1), 8))[:3] == (_lib.MOE_GATE_SWITCH, 1, 0)
    assert tuple(moe.gating.gate_spec(moe.StochasticTopKGating(3), 8))[:3] == (_lib.MOE_GATE_TOPK, 3, 0)
    # host-routed gates run on a top-k handle of their k
    assert tuple(moe.gating.gate_spec(moe.HashGating(2, 8), 8))[:3] == (_lib.MOE_GATE_TOPK, 2, 0)
