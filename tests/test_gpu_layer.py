"""GPU parity of the full MoE-layer forward (router GEMM, gating, permute,
grouped expert GEMMs, combine, losses, statistics) through the C ABI against
the oracle on identical seeded inputs.

Tolerances (north star): layer output relative error (Frobenius) <= 1e-4 at
fp32, 2e-2 at bf16, 5e-2 at fp8 weights; balance loss within 1e-5; routing
bit-exact given identical router logits (the oracle is run on the GPU's
logits; the logits themselves are checked against the oracle's fp32 GEMM)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "bf16": 2e-2, "fp8": 5e-2}


def rel_err(a, b):
    return float(np.linalg.norm((a - b).astype(np.float64)) / max(np.linalg.norm(b.astype(np.float64)), 1e-30))


class Case:
    """Seeded weights + inputs, uploaded to a device handle and kept as the
    fp32 values the oracle sees (bf16 / fp8 weights dequantised)."""

    def __init__(self, moe, oracle, *, T, D, H, Dout=None, E, k, gate="topk", ns=0, expert_type="gated", act="silu",
                 wdtype="f32", xdtype="f32", seed=0, router_bias=None, alpha=0.01, z=0.001, drop=False, cf=1.25,
                 max_tokens=None, wscale=None, lsh=0, init="he", gate_param=None):
        from mixtureofexperts_amd import _lib
        from mixtureofexperts_amd._device import DeviceLayer, GateSpec

        self.oracle = oracle
        Dout = D if Dout is None else Dout
        rng = np.random.default_rng(seed)
        self.T, self.D, self.H, self.Dout, self.E, self.k = T, D, H, Dout, E, k
        self.gate, self.ns, self.expert_type, self.act = gate, ns, expert_type, act
        self.alpha, self.z, self.drop, self.cf = alpha, z, drop, cf
        self.lsh = lsh  # MoEConfig.num_shared_experts: the router sees E - lsh experts
        x = rng.standard_normal((T, D)).astype(np.float32)
        if xdtype == "bf16":
            self.x_dev = oracle.f32_to_bf16_bits(x)
            self.x = oracle.bf16_bits_to_f32(self.x_dev)
            self.xcode = _lib.MOE_BF16
        else:
            self.x_dev = self.x = x
            self.xcode = _lib.MOE_F32
        # init "he": experts ~ N(0, 2 / fan_in) as GatedExpert's randn * sqrt(2 / D)
        # (src/experts/gated.jl:16-24), router 1 / sqrt(D); "glorot": Glorot
        # normal, N(0, 2 / (fan_in + fan_out)) for every matrix
        if init == "glorot":
            s_r, s_in, s_h = np.sqrt(2.0 / (D + E - lsh)), np.sqrt(2.0 / (D + H)), np.sqrt(2.0 / (H + Dout))
            s_w2 = s_h
        else:
            s_r = 1.0 / np.sqrt(D)
            s_in = np.sqrt(2.0 / D) if wscale is None else wscale
            s_h = np.sqrt(2.0 / H) if wscale is None else wscale
            s_w2 = s_in if expert_type == "gated" else s_h
        self.wr = (rng.standard_normal((E - lsh, D)) * s_r).astype(np.float32)
        self.rb = router_bias
        self.ex, dev_ex = [], []
        for _ in range(E):
            w1 = (rng.standard_normal((H, D)) * s_in).astype(np.float32)
            w2 = (rng.standard_normal((Dout, H)) * s_w2).astype(np.float32)
            w3 = (rng.standard_normal((H, D)) * s_in).astype(np.float32) if expert_type == "gated" else None
            b1 = (rng.standard_normal(H) * 0.1).astype(np.float32) if expert_type != "gated" else None
            b2 = (rng.standard_normal(Dout) * 0.1).astype(np.float32) if expert_type != "gated" else None
            mats = [w1, w2, w3]
            if wdtype == "bf16":
                dv = [None if m is None else oracle.f32_to_bf16_bits(m) for m in mats]
                ov = [None if m is None else oracle.bf16_bits_to_f32(b) for m, b in zip(mats, dv)]
                dev_ex.append(dict(src=_lib.MOE_BF16, w=dv, s=[None] * 3))
            elif wdtype == "fp8":
                q = [None if m is None else oracle.quantize_fp8_rows(m) for m in mats]
                ov = [None if c is None else oracle.dequantize_fp8_rows(*c) for c in q]
                dev_ex.append(dict(src=_lib.MOE_FP8_E4M3, w=[None if c is None else c[0] for c in q],
                                   s=[None if c is None else c[1] for c in q]))
            else:
                ov = mats
                dev_ex.append(dict(src=_lib.MOE_F32, w=mats, s=[None] * 3))
            self.ex.append(dict(w1=ov[0], w2=ov[1], w3=ov[2], b1=b1, b2=b2))
            dev_ex[-1]["b"] = (b1, b2)
        self.gate_param = gate_param
        spec = {"topk": GateSpec(_lib.MOE_GATE_TOPK, k, 0), "switch": GateSpec(_lib.MOE_GATE_SWITCH, 1, 0),
                "shared": GateSpec(_lib.MOE_GATE_SHARED, k, ns),
                "soft": GateSpec(_lib.MOE_GATE_SOFT, k, 0, gate_param or 0.0),
                "expert_choice": GateSpec(_lib.MOE_GATE_EXPERT_CHOICE, 1, 0, gate_param or 0.0)}[gate]
        acts = {"silu": _lib.MOE_ACT_SILU, "gelu": _lib.MOE_ACT_GELU, "relu": _lib.MOE_ACT_RELU,
                "identity": _lib.MOE_ACT_IDENTITY}
        wcode = {"f32": _lib.MOE_F32, "bf16": _lib.MOE_BF16, "fp8": _lib.MOE_FP8_E4M3}[wdtype]
        print(f"layer case T={T} D={D} H={H} E={E} k={k} gate={gate} ns={ns} lsh={lsh} type={expert_type} "
              f"w={wdtype} x={xdtype}", flush=True)
        self.dev = DeviceLayer(num_experts=E, expert_type=_lib.MOE_EXPERT_GATED if expert_type == "gated"
                               else _lib.MOE_EXPERT_STANDARD, input_dim=D, hidden_dim=H, output_dim=Dout,
                               activation=acts[act], gate=spec, weight_dtype=wcode, balance_alpha=alpha,
                               z_loss_weight=z, capacity_factor=cf, drop_tokens=drop,
                               max_tokens=max_tokens or T, num_shared_experts=lsh)
        self.dev.set_router(np.ascontiguousarray(self.wr.T), router_bias)
        for e, d in enumerate(dev_ex):
            self.dev.set_expert(e, d["w"][0], d["w"][1], d["w"][2], d["b"][0], d["b"][1], src_dtype=d["src"],
                                s1=d["s"][0], s2=d["s"][1], s3=d["s"][2])

    def run(self, training=True, T=None):
        T = self.T if T is None else T
        out, loss, res = self.dev.forward(np.ascontiguousarray(self.x_dev[:T]), self.xcode, training, want_aux=True)
        return out, loss, res

    def oracle_forward(self, logits, training=True, T=None):
        T = self.T if T is None else T
        return self.oracle.moe_forward(self.x[:T], self.wr, self.ex, gate=self.gate, k=self.k, num_shared=self.ns,
                                       expert_type=self.expert_type, act=self.act, alpha=self.alpha,
                                       z_weight=self.z, training=training, drop_tokens=self.drop,
                                       capacity_factor=self.cf, logits=logits, gate_param=self.gate_param)


def check_case(case, tol, training=True, T=None):
    out, loss, res = case.run(training, T)
    # logits: fp32 GEMM vs the oracle's OpenBLAS sgemm
    T = case.T if T is None else T
    ref_logits = (case.x[:T] @ case.wr.T).astype(np.float32)
    if case.rb is not None:
        ref_logits = ref_logits + case.rb
    assert np.max(np.abs(res["logits"] - ref_logits)) <= 1e-5 * max(1.0, np.max(np.abs(ref_logits)))
    # routing bit-exact given the GPU's logits
    ref_out, ref_loss, aux = case.oracle_forward(res["logits"], training, T)
    assert np.array_equal(res["indices"], aux["idx"])
    assert np.array_equal(res["gates"].view(np.uint32), aux["gates"].view(np.uint32))
    assert np.array_equal(res["probs"].view(np.uint32), aux["probs"].view(np.uint32))
    assert np.array_equal(res["counts"], aux["counts"])
    assert np.array_equal(res["offsets"], aux["offsets"])
    n = int(aux["offsets"][-1])
    assert np.array_equal(res["perm"][:n], aux["perm"])
    # layer output and losses
    err = rel_err(out, ref_out)
    assert err <= tol, f"relative error {err:.3e} > {tol}"
    assert abs(loss - ref_loss) <= 1e-5 * max(1.0, abs(float(ref_loss))), (loss, ref_loss)
    assert abs(res["mean_entropy"] - aux["mean_entropy"]) <= 1e-5 * max(1.0, abs(float(aux["mean_entropy"])))
    if not training:
        assert loss == 0.0
    return out, err


def check_shared_experts_case(case, tol, training=True, aux_free=None):
    """forward_with_shared_experts (num_shared_experts = lsh > 0) against the
    oracle on the GPU's router logits; ``aux_free``: an AuxiliaryFreeLoss
    state dict of the oracle's (bias over all E experts), loaded into the
    handle first and compared after the call."""
    import ctypes

    from mixtureofexperts_amd import _lib

    if aux_free is not None:
        st = aux_free
        _lib.check(_lib.lib().moe_set_aux_free(
            case.dev.h, 1, st["bias"].ctypes.data, st["mom"].ctypes.data, st["lr"], st["momentum"],
            st["update_freq"], st["counter"], int(st["use_comp"]), st["cw"]), case.dev.h)
    out, loss, res = case.run(training)
    T, lsh, k, E = case.T, case.lsh, case.k, case.E
    ref_logits = (case.x @ case.wr.T).astype(np.float32)
    assert np.max(np.abs(res["logits"] - ref_logits)) <= 1e-5 * max(1.0, np.max(np.abs(ref_logits)))
    ref_out, ref_loss, aux = case.oracle.moe_forward_shared_experts(
        case.x, case.wr, case.ex, lsh, gate=case.gate, k=k, expert_type=case.expert_type, act=case.act,
        alpha=case.alpha, z_weight=case.z, training=training, logits=res["logits"], gate_param=case.gate_param,
        gate_num_shared=case.ns, aux_free=aux_free)
    # slots: the shared experts 1..lsh, then the gate's shifted ids, bit-exact
    # (ExpertChoice: lsh + min(C, E - lsh) slots, empty ones 0 on the device
    # where the oracle's shifted matrix holds lsh)
    kg = aux["idx"].shape[1]
    kd = res["indices"].shape[1] - lsh
    n = min(kg, kd)
    routed = np.where(aux["routed_idx"] > 0, aux["routed_idx"] + lsh, 0).astype(np.int32)
    if case.gate != "expert_choice":
        assert kd == kg
    assert np.array_equal(res["indices"][:, :lsh], np.tile(np.arange(1, lsh + 1, dtype=np.int32), (T, 1)))
    assert np.array_equal(res["indices"][:, lsh:lsh + n], routed[:, :n])
    assert np.all(routed[:, n:] == 0) and np.all(res["indices"][:, lsh + n:] == 0)
    assert np.array_equal(res["gates"][:, lsh:lsh + n].view(np.uint32), aux["gates"][:, :n].view(np.uint32))
    assert np.array_equal(res["probs"].view(np.uint32), aux["probs"].view(np.uint32))
    assert np.array_equal(res["counts"][:lsh], np.full(lsh, T, np.int32))
    assert np.array_equal(res["counts"][lsh:], aux["routed_counts"])
    err = rel_err(out, ref_out)
    assert err <= tol, f"relative error {err:.3e} > {tol}"
    assert abs(loss - ref_loss) <= 1e-5 * max(1.0, abs(float(ref_loss))), (loss, ref_loss)
    if training:
        assert abs(res["switch_loss"] - aux["switch_loss"]) <= 1e-5 * max(1.0, abs(float(aux["switch_loss"])))
    else:
        assert loss == 0.0
    if aux_free is not None:
        # update_bias! over the shifted ids, the same Float32 / Float64 steps
        bias, mom, cnt = np.zeros(E, np.float32), np.zeros(E, np.float32), ctypes.c_int64(0)
        _lib.check(_lib.lib().moe_get_aux_free(case.dev.h, bias.ctypes.data, mom.ctypes.data, ctypes.byref(cnt)),
                   case.dev.h)
        assert cnt.value == aux_free["counter"]
        assert np.array_equal(bias.view(np.uint32), aux_free["bias"].view(np.uint32)), (bias, aux_free["bias"])
        assert np.array_equal(mom.view(np.uint32), aux_free["mom"].view(np.uint32))
    return out, err


@pytest.mark.parametrize("gate,lsh,k,ns,E,param,wdtype,T", [
    ("soft", 1, 2, 0, 9, 0.5, "bf16", 500),              # SoftMoEGating: slot gate = p of expert `slot`
    ("soft", 2, 3, 0, 8, 1.0, "f32", 300),
    ("expert_choice", 1, 1, 0, 5, 1.0, "f32", 400),      # empty entries count as id lsh in the loss
    ("expert_choice", 2, 1, 0, 10, 1.25, "bf16", 512),   # lsh + min(C, 8) = 10 slots per token
    ("shared", 2, 2, 1, 9, None, "bf16", 500),           # SharedExpertGating(1, TopKGating(2), 7)
    ("shared", 1, 3, 2, 12, None, "fp8", 400),
])
def test_shared_experts_with_every_gate(moe, oracle, gate, lsh, k, ns, E, param, wdtype, T):
    # forward_with_shared_experts runs whatever gate the router holds
    # (src/core/moe_layer.jl:158-185): the gate's ids shifted by lsh, the
    # balance loss on the shifted ids, the output blended 0.5 / 0.5
    c = Case(moe, oracle, T=T, D=128, H=192, E=E, k=k, gate=gate, ns=ns, wdtype=wdtype,
             xdtype="bf16" if wdtype != "f32" else "f32", seed=90 + E, lsh=lsh, gate_param=param)
    try:
        check_shared_experts_case(c, TOL[wdtype], training=True)
        check_shared_experts_case(c, TOL[wdtype], training=False)
    finally:
        c.dev.close()


@pytest.mark.parametrize("gate,lsh,k,E,param,update_freq", [
    ("topk", 1, 2, 7, None, 1),
    ("topk", 2, 2, 8, None, 2),             # the second call updates
    ("expert_choice", 1, 1, 5, 1.0, 1),     # empty entries count for bias index lsh - 1
    ("switch", 3, 1, 9, None, 1),
    ("topk", 1, 4, 300, None, 1),           # bias over 300 experts
])
def test_shared_experts_aux_free_loss(moe, oracle, gate, lsh, k, E, param, update_freq):
    # AuxiliaryFreeLoss with shared experts: the gate sees the plain logits
    # (the bias is not applied: a large bias on one expert does not move the
    # routing), update_bias! and the complementary loss take the shifted ids,
    # and the bias covers all E experts (src/core/moe_layer.jl:158-185,
    # src/balancing/auxiliary_free.jl:36-87).  Three training calls; bias,
    # momentum and counter bit-exact after each.
    c = Case(moe, oracle, T=300, D=64, H=96, E=E, k=k, gate=gate, wdtype="f32", seed=95 + E, lsh=lsh,
             gate_param=param)
    try:
        bias0 = np.zeros(E, np.float32)
        bias0[lsh] = 50.0  # would win every token if the gate added it
        st = dict(bias=bias0, mom=np.zeros(E, np.float32), lr=0.01, momentum=0.9, update_freq=update_freq,
                  counter=0, use_comp=True, cw=0.001)
        for _ in range(3):
            check_shared_experts_case(c, TOL["f32"], training=True, aux_free=st)
    finally:
        c.dev.close()


@pytest.mark.parametrize("lsh,k,E,gate,etype,act,wdtype,xdtype", [
    (1, 2, 6, "topk", "gated", "silu", "f32", "f32"),        # blend fast path, kt = 3
    (2, 2, 10, "topk", "gated", "silu", "bf16", "bf16"),     # kt = 4, 1/ns exact
    (3, 1, 9, "switch", "standard", "gelu", "bf16", "f32"),  # division by 3, Switch gate
    (2, 3, 12, "topk", "gated", "silu", "fp8", "bf16"),      # kt = 5: the general combine path
])
def test_shared_experts_layer(moe, oracle, lsh, k, E, gate, etype, act, wdtype, xdtype):
    c = Case(moe, oracle, T=500, D=128, H=192, E=E, k=k, gate=gate, expert_type=etype, act=act, wdtype=wdtype,
             xdtype=xdtype, seed=30 + lsh, lsh=lsh)
    check_shared_experts_case(c, TOL[wdtype], training=True)
    check_shared_experts_case(c, TOL[wdtype], training=False)


def test_shared_experts_python_api(moe, oracle):
    # MoEConfig(num_shared_experts=2): the router has E - 2 outputs, the
    # training statistics are not updated (forward_with_shared_experts has no
    # update_stats!)
    rng = np.random.default_rng(40)
    cfg = moe.MoEConfig(num_experts=6, expert_type="gated", input_dim=64, hidden_dim=96, output_dim=64,
                        activation=moe.silu, gate_type=moe.TopKGating(2), num_shared_experts=2, max_tokens=64)
    layer = moe.MoELayer(cfg, rng=rng)
    assert layer.router.weight.shape == (4, 64)
    x = rng.standard_normal((64, 40)).astype(np.float32)
    aux = {}
    out, loss = layer(x, training=True, _aux=aux)
    ex = [dict(w1=e.w1, w2=e.w2, w3=e.w3) for e in layer.experts]
    ref, ref_loss, _ = oracle.moe_forward_shared_experts(x.T, layer.router.weight, ex, 2, k=2, training=True,
                                                         logits=aux["logits"])
    assert rel_err(out.T, ref) <= 1e-4
    assert abs(loss - ref_loss) <= 1e-5
    assert layer.training_stats["tokens_per_expert"].sum() == 0
    assert layer.training_stats["routing_entropy"] == []
    layer.close()


@pytest.mark.parametrize("freq,use_comp,drop,wdtype,E,k", [
    (1, True, False, "f32", 8, 2), (2, False, True, "bf16", 8, 2),
    (1, True, False, "bf16", 24, 10),   # more than 8 slots: 32-token route blocks in both gating passes
    (1, False, True, "bf16", 300, 6),   # over 256 router rows: 16-token route blocks
])
def test_aux_free_loss_layer(moe, oracle, freq, use_comp, drop, wdtype, E, k):
    # AuxiliaryFreeLoss as the balance loss: gating on logits + bias, the bias
    # state after every call bit-exact against the oracle's update_bias!
    # restatement, inference calls leave it alone
    rng = np.random.default_rng(50 + freq)
    c = Case(moe, oracle, T=600, D=128, H=192 if E <= 64 else 64, E=E, k=k, wdtype=wdtype, xdtype=wdtype,
             seed=50 + freq + E, drop=drop, cf=1.0)
    lossfn = moe.AuxiliaryFreeLoss(E, learning_rate=0.05, update_freq=freq, use_complementary_loss=use_comp)
    lossfn.bias = (rng.standard_normal(E) * 0.5).astype(np.float32)
    st = dict(bias=lossfn.bias.copy(), mom=np.zeros(E, np.float32), lr=0.05, momentum=0.9, update_freq=freq,
              counter=0, use_comp=use_comp, cw=0.001)
    for step, training in enumerate((True, True, False, True, True)):
        c.dev.set_aux_free(lossfn)
        out, loss, res = c.run(training)
        c.dev.get_aux_free(lossfn)
        ref_out, ref_loss, aux = oracle.moe_forward(c.x, c.wr, c.ex, k=k, training=training, drop_tokens=drop,
                                                    capacity_factor=1.0, z_weight=c.z, logits=res["logits"],
                                                    aux_free=st)
        assert np.array_equal(res["indices"], aux["idx"]), step
        assert np.array_equal(res["gates"].view(np.uint32), aux["gates"].view(np.uint32)), step
        assert np.array_equal(res["probs"].view(np.uint32), aux["probs"].view(np.uint32)), step
        assert np.array_equal(res["counts"], aux["counts"]), step
        assert lossfn.update_counter == st["counter"], step
        assert np.array_equal(lossfn.bias.view(np.uint32), st["bias"].view(np.uint32)), (step, lossfn.bias, st["bias"])
        assert np.array_equal(lossfn.bias_momentum.view(np.uint32), st["mom"].view(np.uint32)), step
        err = rel_err(out, ref_out)
        assert err <= TOL[wdtype], (step, err)
        assert abs(loss - ref_loss) <= 1e-5 * max(1.0, abs(float(ref_loss))), (step, loss, ref_loss)
    assert st["counter"] == 4 and np.any(st["mom"] != 0)


def test_aux_free_python_api(moe, oracle):
    # the layer keeps the loss object's state in step with the device, and
    # update_bias! / compute_loss on given indices match the oracle
    rng = np.random.default_rng(52)
    E = 6
    lossfn = moe.AuxiliaryFreeLoss(E, learning_rate=0.02)
    cfg = moe.MoEConfig(num_experts=E, expert_type="gated", input_dim=64, hidden_dim=96, output_dim=64,
                        activation=moe.silu, gate_type=moe.TopKGating(2), balance_loss=lossfn, max_tokens=64)
    layer = moe.MoELayer(cfg, rng=rng)
    x = rng.standard_normal((64, 50)).astype(np.float32)
    st = dict(bias=np.zeros(E, np.float32), mom=np.zeros(E, np.float32), lr=0.02, momentum=0.9, update_freq=1,
              counter=0, use_comp=True, cw=0.001)
    ex = [dict(w1=e.w1, w2=e.w2, w3=e.w3) for e in layer.experts]
    for _ in range(3):
        aux = {}
        out, loss = layer(x, training=True, _aux=aux)
        ref, ref_loss, _ = oracle.moe_forward(x.T, layer.router.weight, ex, k=2, training=True,
                                              logits=aux["logits"], aux_free=st)
        assert rel_err(out.T, ref) <= 1e-4
        assert abs(loss - ref_loss) <= 1e-5
    assert lossfn.update_counter == 3
    assert np.array_equal(lossfn.bias.view(np.uint32), st["bias"].view(np.uint32))
    layer.close()
    # standalone update_bias! and compute_loss(AuxiliaryFreeLoss, ...)
    idx = rng.integers(0, E + 1, size=(2, 300)).astype(np.int64)  # 0 entries are not counted
    probs = rng.random((E, 300)).astype(np.float32)
    l2 = moe.AuxiliaryFreeLoss(E, bias_init=0.25)
    b, m = l2.bias.copy(), l2.bias_momentum.copy()
    val = moe.compute_loss(l2, idx, probs)
    oracle.aux_free_update_bias(idx.T, b, m, l2.learning_rate, l2.momentum)
    assert np.array_equal(l2.bias.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(l2.bias_momentum.view(np.uint32), m.view(np.uint32))
    # the loss: the balance-loss bar (1e-5); the mean over tokens is summed in another order
    assert abs(val - np.float32(np.float32(0.001) * oracle.switch_loss(idx.T, probs.T, 1.0))) <= 1e-5 * abs(val)
    with pytest.raises(moe.MoeError):
        moe.update_bias(l2, np.array([[E + 1]]))


@pytest.mark.parametrize("gate,param,E,k,wdtype,T", [("soft", 0.5, 8, 2, "bf16", 512), ("soft", 1.0, 6, 3, "f32", 512),
                                                      ("soft", 0.8, 128, 4, "bf16", 1024),
                                                      ("expert_choice", 1.25, 8, 0, "bf16", 512),
                                                      ("expert_choice", 0.125, 16, 0, "f32", 512),
                                                      # more than 8 slots per token: min(capacity, E) = 16, 64, 86
                                                      ("expert_choice", 1.25, 16, 0, "bf16", 4096),
                                                      ("expert_choice", 1.25, 64, 0, "bf16", 4096),
                                                      ("expert_choice", 4.0, 96, 0, "f32", 2048),
                                                      # over 128 experts; 134 slots per token (wide permute)
                                                      ("soft", 0.9, 300, 5, "bf16", 600),
                                                      ("expert_choice", 100.0, 300, 0, "bf16", 400)])
def test_soft_and_expert_choice_layer(moe, oracle, gate, param, E, k, wdtype, T):
    # the layer forward with SoftMoEGating / ExpertChoiceGating against the
    # oracle on the GPU's logits: routing bit-exact, output and loss in tolerance
    from mixtureofexperts_amd import _lib
    from mixtureofexperts_amd._device import DeviceLayer, GateSpec

    rng = np.random.default_rng(70 + E)
    D, H = 128, 192
    print(f"layer gate={gate} param={param} E={E} k={k} w={wdtype} T={T}", flush=True)
    x = rng.standard_normal((T, D)).astype(np.float32)
    wr = (rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32)
    ex, dev_w = [], []
    for _ in range(E):
        mats = [(rng.standard_normal(sh) * np.sqrt(2.0 / D)).astype(np.float32) for sh in ((H, D), (D, H), (H, D))]
        if wdtype == "bf16":
            bits = [oracle.f32_to_bf16_bits(m) for m in mats]
            mats = [oracle.bf16_bits_to_f32(b) for b in bits]
            dev_w.append((bits, _lib.MOE_BF16))
        else:
            dev_w.append((mats, _lib.MOE_F32))
        ex.append(dict(w1=mats[0], w2=mats[1], w3=mats[2]))
    kind = _lib.MOE_GATE_SOFT if gate == "soft" else _lib.MOE_GATE_EXPERT_CHOICE
    dev = DeviceLayer(num_experts=E, expert_type=_lib.MOE_EXPERT_GATED, input_dim=D, hidden_dim=H, output_dim=D,
                      activation=_lib.MOE_ACT_SILU, gate=GateSpec(kind, k if k else 1, 0, param),
                      weight_dtype={"bf16": _lib.MOE_BF16, "f32": _lib.MOE_F32}[wdtype], balance_alpha=0.01,
                      z_loss_weight=0.001, capacity_factor=1.25, drop_tokens=False, max_tokens=T)
    dev.set_router(np.ascontiguousarray(wr.T))
    for e, (w, src) in enumerate(dev_w):
        dev.set_expert(e, w[0], w[1], w[2], src_dtype=src)
    out, loss, res = dev.forward(x, _lib.MOE_F32, True, want_aux=True)
    ref, ref_loss, aux = oracle.moe_forward(x, wr, ex, gate=gate, k=k, gate_param=param, training=True,
                                            logits=res["logits"])
    kt = res["indices"].shape[1]
    n = min(kt, aux["idx"].shape[1])
    assert np.array_equal(res["indices"][:, :n], aux["idx"][:, :n])
    assert np.all(aux["idx"][:, n:] == 0) and np.all(res["indices"][:, n:] == 0)
    assert np.array_equal(res["gates"][:, :n].view(np.uint32), aux["gates"][:, :n].view(np.uint32))
    assert np.array_equal(res["probs"].view(np.uint32), aux["probs"].view(np.uint32))
    assert np.array_equal(res["counts"], aux["counts"])
    # permutation: (token, slot) of each position (entry ids are t * slots + slot)
    m = int(aux["offsets"][-1])
    ko = aux["idx"].shape[1]
    assert np.array_equal(np.divmod(res["perm"][:m], kt), np.divmod(aux["perm"], ko))
    assert rel_err(out, ref) <= TOL[wdtype]
    assert abs(loss - ref_loss) <= 1e-5 * max(1.0, abs(float(ref_loss))), (loss, ref_loss)
    dev.close()


def test_host_routed_gates_layer(moe, oracle):
    # HashGating / RandomGating in a layer: indices from host code, the rest of
    # forward_standard on the device (moe_forward_routed), capacity included
    rng = np.random.default_rng(80)
    for gate, drop in ((moe.HashGating(2, 8, hash_fn=lambda i: 3 * i + i // 7), False),
                       (moe.RandomGating(3, rng=np.random.default_rng(2)), True)):
        cfg = moe.MoEConfig(num_experts=8, expert_type="gated", input_dim=64, hidden_dim=96, output_dim=64,
                            activation=moe.silu, gate_type=gate, max_tokens=128, drop_tokens=drop,
                            capacity_factor=1.0)
        layer = moe.MoELayer(cfg, rng=rng)
        x = rng.standard_normal((64, 100)).astype(np.float32)
        aux = {}
        out, loss = layer(x, training=True, _aux=aux)
        ex = [dict(w1=e.w1, w2=e.w2, w3=e.w3) for e in layer.experts]
        kk = gate.k
        given_idx = aux["indices"] if drop else gate.host_routing(100, 8)[0]
        if not drop:
            assert np.array_equal(aux["indices"], given_idx)
        ref, ref_loss, oa = oracle.moe_forward(x.T, layer.router.weight, ex, k=kk, training=True, drop_tokens=False,
                                               logits=aux["logits"],
                                               given=(aux["indices"], aux["gates"], None))
        assert np.array_equal(aux["counts"], oa["counts"])
        assert rel_err(out.T, ref) <= 1e-4
        if not drop:
            assert abs(loss - ref_loss) <= 1e-5
        layer.close()


def test_readme_config_fp32(moe, oracle):
    # README MoELayer, 8 gated silu experts, 512/2048/512,
    # TopKGating(2), SwitchTransformerLoss(0.01), x randn(512, 32), fp32,
    # weights Glorot-normal from a fixed seed
    c = Case(moe, oracle, T=32, D=512, H=2048, E=8, k=2, wdtype="f32", seed=1, init="glorot")
    check_case(c, TOL["f32"], training=True)
    check_case(c, TOL["f32"], training=False)


@pytest.mark.parametrize("wdtype,xdtype", [("f32", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("fp8", "bf16")])
def test_gated_dtypes(moe, oracle, wdtype, xdtype):
    c = Case(moe, oracle, T=700, D=256, H=384, E=8, k=2, wdtype=wdtype, xdtype=xdtype, seed=2)
    check_case(c, TOL[wdtype])


def test_mixtral_shape_scaled(moe, oracle):
    # C3 structure at reduced size: bf16, skewed router bias
    rng = np.random.default_rng(3)
    bias = rng.standard_normal(8).astype(np.float32)
    c = Case(moe, oracle, T=1024, D=1024, H=1792, E=8, k=2, wdtype="bf16", xdtype="bf16", seed=3,
             router_bias=bias, wscale=0.02)
    check_case(c, TOL["bf16"])


@pytest.mark.parametrize("E,k,etype,act,wdtype", [
    (4, 1, "gated", "silu", "bf16"),
    (4, 1, "gated", "silu", "fp8"),
    (4, 1, "standard", "gelu", "bf16"),
    (4, 1, "standard", "gelu", "fp8"),
    (8, 2, "gated", "silu", "bf16"),
])
def test_256_row_tiles(moe, oracle, E, k, etype, act, wdtype):
    # at most 16 experts averaging >= 384 rows: the 256-row tile kernels (one
    # workgroup per CU; standard experts with fp8 weights stay on 128-row
    # tiles); a skewed router bias gives partial last tiles, and D = 320
    # leaves y rows past the last 256-column block (cut at N)
    rng = np.random.default_rng(70 + E)
    bias = (rng.standard_normal(E) * 0.7).astype(np.float32)
    c = Case(moe, oracle, T=1600, D=320, H=384, E=E, k=k, gate="switch" if k == 1 else "topk", expert_type=etype,
             act=act, wdtype=wdtype, xdtype="bf16", seed=70 + E, router_bias=bias)
    check_case(c, TOL[wdtype])


def test_standard_experts_gelu(moe, oracle):
    # C5 structure at reduced size: StandardExpert + gelu + biases, SwitchGating
    for wd in ("f32", "bf16"):
        c = Case(moe, oracle, T=2048, D=192, H=384, E=32, k=1, gate="switch", expert_type="standard",
                 act="gelu", wdtype=wd, xdtype="bf16" if wd == "bf16" else "f32", seed=4)
        check_case(c, TOL[wd])


def test_shared_expert_gating_fp8(moe, oracle):
    # C4 structure at reduced size: SharedExpertGating(2, TopKGating(6), 18), fp8 weights
    c = Case(moe, oracle, T=1500, D=256, H=192, E=18, k=6, gate="shared", ns=2, wdtype="fp8", xdtype="bf16",
             seed=5)
    check_case(c, TOL["fp8"])


def test_capacity_drop_tokens(moe, oracle):
    rng = np.random.default_rng(6)
    c = Case(moe, oracle, T=600, D=128, H=256, E=8, k=2, wdtype="f32", seed=6, drop=True, cf=0.75,
             router_bias=(rng.standard_normal(8) * 2).astype(np.float32))
    out, _ = check_case(c, TOL["f32"], training=True)
    check_case(c, TOL["f32"], training=False)


def test_other_activations_and_odd_sizes(moe, oracle):
    # dims that are not multiples of the tiles (padding paths)
    c = Case(moe, oracle, T=77, D=100, H=150, Dout=90, E=5, k=3, act="relu", wdtype="f32", seed=7)
    check_case(c, TOL["f32"])
    c = Case(moe, oracle, T=77, D=100, H=150, Dout=90, E=5, k=3, act="identity", wdtype="bf16", seed=8)
    check_case(c, TOL["bf16"])


@pytest.mark.parametrize("E,k,gate,ns", [(96, 3, "topk", 0), (128, 2, "topk", 0), (70, 8, "topk", 0),
                                        (100, 6, "shared", 2)])
def test_over_64_routed_experts(moe, oracle, E, k, gate, ns):
    # more than 64 routed experts with k >= 2: the top-k by per-lane sorted
    # lists and the butterfly merge of the routing kernel, in a full layer
    rng = np.random.default_rng(E + k)
    bias = (rng.standard_normal(E) * 0.5).astype(np.float32)
    c = Case(moe, oracle, T=900, D=128, H=160, E=E, k=k, gate=gate, ns=ns, wdtype="bf16", xdtype="bf16",
             seed=E * 10 + k, router_bias=bias)
    try:
        check_case(c, TOL["bf16"])
        check_case(c, TOL["bf16"], training=False)
    finally:
        c.dev.close()


@pytest.mark.parametrize("E,k,gate,ns,wdtype,drop", [
    (16, 12, "topk", 0, "bf16", False),      # two slots per routing lane, 32-token route blocks
    (24, 16, "topk", 0, "f32", False),       # MOE_MAX_TOPK slots
    (96, 10, "topk", 0, "bf16", False),      # > 64 experts: sorted lists + butterfly merge, k > 8
    (20, 9, "shared", 3, "fp8", False),      # SharedExpertGating: 3 + 9 = 12 slots
    (16, 11, "topk", 0, "bf16", True),       # capacity drop and renormalisation over 11 slots
])
def test_more_than_8_slots(moe, oracle, E, k, gate, ns, wdtype, drop):
    # TopKGating(k) with k up to MOE_MAX_TOPK = 16: routing bit-exact, the
    # combine's general path (slots sorted by expert id) within tolerance
    c = Case(moe, oracle, T=700, D=128, H=160, E=E, k=k, gate=gate, ns=ns, wdtype=wdtype,
             xdtype="f32" if wdtype == "f32" else "bf16", seed=E * 7 + k, drop=drop, cf=1.0)
    try:
        check_case(c, TOL[wdtype])
        check_case(c, TOL[wdtype], training=False)
        check_case(c, TOL[wdtype], T=333)  # a partial last route block
    finally:
        c.dev.close()


@pytest.mark.parametrize("gate,lsh,k,ns,E,param,wdtype", [
    ("topk", 2, 10, 0, 14, None, "bf16"),    # forward_with_shared_experts: 12 slots
    ("soft", 3, 8, 0, 12, 0.75, "f32"),      # 11 slots, SoftMoE gates
    ("shared", 2, 9, 4, 17, None, "bf16"),   # 2 + 4 + 9 = 15 slots
])
def test_shared_experts_more_than_8_slots(moe, oracle, gate, lsh, k, ns, E, param, wdtype):
    c = Case(moe, oracle, T=400, D=128, H=192, E=E, k=k, gate=gate, ns=ns, wdtype=wdtype,
             xdtype="bf16" if wdtype != "f32" else "f32", seed=70 + E, lsh=lsh, gate_param=param)
    try:
        check_shared_experts_case(c, TOL[wdtype], training=True)
        check_shared_experts_case(c, TOL[wdtype], training=False)
    finally:
        c.dev.close()


@pytest.mark.parametrize("E,k,gate,ns,lsh,wdtype,T", [
    (129, 4, "topk", 0, 0, "bf16", 900),     # 32 experts per gating lane, two logits column groups
    (256, 8, "topk", 0, 0, "bf16", 1500),    # DeepSeek-V3's routed expert count
    (300, 6, "shared", 2, 0, "fp8", 700),
    (512, 1, "switch", 0, 0, "bf16", 1200),  # MOE_MAX_EXPERTS: 16-token route blocks, 64 experts per lane
    (160, 3, "topk", 0, 0, "f32", 500),      # fp32 x: the six-term logits GEMM over 10 tiles
    (385, 8, "topk", 0, 1, "bf16", 800),     # 384 routed + 1 shared expert of the layer
    (300, 4, "topk", 0, 0, "f32", 400),      # fp32 x over 256 router rows: 16-token route blocks
])
def test_over_128_experts(moe, oracle, E, k, gate, ns, lsh, wdtype, T):
    # more experts than a 128-row router: the logits GEMM in column groups of
    # 128, the gating with 32 or 64 experts per lane on 32- or 16-token route
    # blocks, the scan's prefix over up to 512 experts; routing bit-exact,
    # output and losses within tolerance
    rng = np.random.default_rng(E + k)
    bias = (rng.standard_normal(E - lsh) * 0.5).astype(np.float32) if lsh == 0 else None
    c = Case(moe, oracle, T=T, D=128, H=96, E=E, k=k, gate=gate, ns=ns, wdtype=wdtype,
             xdtype="f32" if wdtype == "f32" else "bf16", seed=E * 3 + k, router_bias=bias, lsh=lsh)
    try:
        if lsh:
            check_shared_experts_case(c, TOL[wdtype], training=True)
            check_shared_experts_case(c, TOL[wdtype], training=False)
        else:
            check_case(c, TOL[wdtype])
            check_case(c, TOL[wdtype], training=False)
            check_case(c, TOL[wdtype], T=T // 3 + 1)
    finally:
        c.dev.close()


@pytest.mark.parametrize("E,kd,wdtype,T", [(300, 12, "bf16", 500), (40, 16, "f32", 300), (512, 3, "bf16", 700)])
def test_forward_routed_many_experts_and_slots(moe, oracle, E, kd, wdtype, T):
    # moe_forward_routed (the caller's indices and gates, as HashGating /
    # RandomGating hand them over) with up to 512 experts and 16 slots per
    # token; some slots empty (id 0, skipped as the dispatch's expert_id > 0
    # check does, src/core/moe_layer.jl:198); the Switch loss on 1/E
    # probabilities
    # (the handle's routing buffers hold max_tokens * 2 slots: room for T * kd)
    c = Case(moe, oracle, T=T, D=128, H=96, E=E, k=2, wdtype=wdtype, xdtype="f32" if wdtype == "f32" else "bf16",
             seed=E + kd, max_tokens=T * kd // 2)
    try:
        rng = np.random.default_rng(E * kd)
        idx = np.stack([rng.choice(E, kd, replace=False) + 1 for _ in range(T)]).astype(np.int32)
        idx[::17, kd // 2] = 0
        gates = rng.random((T, kd)).astype(np.float32)
        print(f"forward_routed E={E} kd={kd}", flush=True)
        out, loss, res = c.dev.forward_routed(np.ascontiguousarray(c.x_dev), c.xcode, True, idx, gates, want_aux=True)
        ref, ref_loss, aux = oracle.moe_forward(c.x, c.wr, c.ex, k=kd, training=True, logits=res["logits"],
                                                given=(idx, gates, None), alpha=c.alpha, z_weight=c.z)
        assert np.array_equal(res["indices"], idx) and np.array_equal(res["gates"].view(np.uint32), gates.view(np.uint32))
        assert np.array_equal(res["counts"], aux["counts"]) and np.array_equal(res["offsets"], aux["offsets"])
        n = int(aux["offsets"][-1])
        assert np.array_equal(res["perm"][:n], aux["perm"])
        assert rel_err(out, ref) <= TOL[wdtype]
        assert abs(loss - ref_loss) <= 1e-5 * max(1.0, abs(float(ref_loss))), (loss, ref_loss)
    finally:
        c.dev.close()


def test_varying_batch_on_one_handle(moe, oracle):
    c = Case(moe, oracle, T=300, D=128, H=256, E=8, k=2, wdtype="bf16", xdtype="bf16", seed=9)
    for T in (300, 1, 7, 129, 300):
        check_case(c, TOL["bf16"], T=T)


def test_forward_is_deterministic(moe, oracle):
    c = Case(moe, oracle, T=512, D=256, H=512, E=8, k=2, wdtype="bf16", xdtype="bf16", seed=10)
    a = c.run()[0]
    b = c.run()[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_expert_known_answer_dense_llama_ffn(moe, oracle):
    # the reference's known-answer check (test_moeLlama2_integration.jl:132-164):
    # a gated expert equals the dense Llama FFN w2(silu(w1 x) .* (w3 x)) (< 1e-5)
    from mixtureofexperts_amd import _lib
    from mixtureofexperts_amd._device import DeviceLayer, GateSpec

    rng = np.random.default_rng(11)
    dim, hid = 256, 688
    x = rng.standard_normal((5, dim)).astype(np.float32)
    w1 = (rng.standard_normal((dim, hid)) * 0.02).astype(np.float32)  # Llama (in, out)
    w2 = (rng.standard_normal((hid, dim)) * 0.02).astype(np.float32)
    w3 = (rng.standard_normal((dim, hid)) * 0.02).astype(np.float32)
    dev = DeviceLayer(num_experts=1, expert_type=_lib.MOE_EXPERT_GATED, input_dim=dim, hidden_dim=hid,
                      output_dim=dim, activation=_lib.MOE_ACT_SILU, gate=GateSpec(_lib.MOE_GATE_SWITCH, 1, 0),
                      weight_dtype=_lib.MOE_F32, balance_alpha=0.0, z_loss_weight=0.0, capacity_factor=1.0,
                      drop_tokens=False, max_tokens=8)
    # Llama (in, out) column-major == Flux-layout memory [in][out]... pass as FLUX_OUT_IN memory
    dev.set_expert(0, np.ascontiguousarray(w1), np.ascontiguousarray(w2), np.ascontiguousarray(w3),
                   src_dtype=_lib.MOE_F32, layout=_lib.MOE_LAYOUT_FLUX_OUT_IN)
    y = dev.expert_forward(0, x)
    for t in range(5):
        hb1 = w1.T @ x[t]
        hb2 = w3.T @ x[t]
        h = hb1 * (np.float32(1) / (np.float32(1) + np.exp(-hb1))) * hb2
        dense = w2.T @ h
        assert np.max(np.abs(dense - y[t])) < 1e-5
    dev.close()


def test_python_api_readme_flow(moe, oracle):
    # README usage: MoELayer(config)(x; training=true) with silu passed explicitly
    rng = np.random.default_rng(12)
    cfg = moe.MoEConfig(num_experts=8, expert_type="gated", input_dim=512, hidden_dim=2048, output_dim=512,
                        activation=moe.silu, gate_type=moe.TopKGating(2),
                        balance_loss=moe.SwitchTransformerLoss(0.01), max_tokens=64)
    layer = moe.MoELayer(cfg, rng=rng)
    x = rng.standard_normal((512, 32)).astype(np.float32)
    aux = {}
    out, loss = layer(x, training=True, _aux=aux)
    assert out.shape == (512, 32) and out.dtype == np.float32 and np.all(np.isfinite(out))
    assert loss >= 0
    ex = [dict(w1=e.w1, w2=e.w2, w3=e.w3) for e in layer.experts]
    ref, ref_loss, oa = oracle.moe_forward(x.T, layer.router.weight, ex, k=2, training=True, logits=aux["logits"])
    assert rel_err(out.T, ref) <= 1e-4
    assert abs(loss - ref_loss) <= 1e-5
    assert layer.training_stats["tokens_per_expert"].sum() == 64
    assert len(layer.training_stats["routing_entropy"]) == 1
    out2, loss2, stats = layer(x, training=False, return_stats=True)
    assert loss2 == 0.0 and stats["tokens_per_expert"].sum() == 128
    moe.reset_stats(layer)
    assert layer.training_stats["tokens_per_expert"].sum() == 0
    # expert functor on the device: (e::Expert)(x)
    y = layer.experts[3](x[:, :4])
    yref = oracle.gated_expert(x[:, :4].T, layer.experts[3].w1, layer.experts[3].w2, layer.experts[3].w3,
                               oracle.act_silu).T
    assert rel_err(y, yref) <= 1e-4
    layer.close()


def test_async_device_path_matches_host(moe, oracle):
    torch = pytest.importorskip("torch")
    import ctypes

    from mixtureofexperts_amd import _lib

    c = Case(moe, oracle, T=640, D=256, H=512, E=8, k=2, wdtype="bf16", xdtype="bf16", seed=13)
    ref, ref_loss, _ = c.run(training=True)
    x = torch.from_numpy(c.x_dev.view(np.int16)).cuda().view(torch.bfloat16)
    out = torch.empty((c.T, c.Dout), dtype=torch.float32, device="cuda")
    loss = torch.zeros(1, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    _lib.check(_lib.lib().moe_forward_async(c.dev.h, x.data_ptr(), _lib.MOE_BF16, c.T, 1, out.data_ptr(),
                                            loss.data_ptr(), ctypes.c_void_p(stream.cuda_stream)), c.dev.h)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert float(loss.item()) == ref_loss


def test_calls_on_other_streams_are_ordered(moe, oracle):
    # moe_forward_async enqueued on a non-blocking torch stream, then, with no
    # synchronisation in between, a blocking moe_decode and moe_forward (both
    # on the handle's own stream, sharing its workspace): the library orders
    # them after the async work, so every result is bit-identical to the same
    # call made alone
    torch = pytest.importorskip("torch")
    import ctypes

    from mixtureofexperts_amd import _lib

    c = Case(moe, oracle, T=2048, D=512, H=1024, E=8, k=2, wdtype="bf16", xdtype="bf16", seed=15)
    try:
        ref, ref_loss, _ = c.run(training=True)
        xd = np.ascontiguousarray(c.x[:8])
        ref_dec = c.dev.decode(xd)[0]
        x = torch.from_numpy(c.x_dev.view(np.int16)).cuda().view(torch.bfloat16)
        outs = [torch.empty((c.T, c.Dout), dtype=torch.float32, device="cuda") for _ in range(3)]
        stream = torch.cuda.Stream()
        torch.cuda.synchronize()
        L = _lib.lib()
        sp = ctypes.c_void_p(stream.cuda_stream)
        for o in outs:
            _lib.check(L.moe_forward_async(c.dev.h, x.data_ptr(), _lib.MOE_BF16, c.T, 1, o.data_ptr(), None, sp),
                       c.dev.h)
        dec = c.dev.decode(xd)[0]
        fwd, fwd_loss, _ = c.run(training=True)
        torch.cuda.synchronize()
        assert np.array_equal(dec.view(np.uint32), ref_dec.view(np.uint32))
        assert np.array_equal(fwd.view(np.uint32), ref.view(np.uint32)) and fwd_loss == ref_loss
        for o in outs:
            assert np.array_equal(o.cpu().numpy().view(np.uint32), ref.view(np.uint32))
        # and the other way round: a blocking call, then async work on the torch stream
        _lib.check(L.moe_forward_async(c.dev.h, x.data_ptr(), _lib.MOE_BF16, c.T, 1, outs[0].data_ptr(), None, sp),
                   c.dev.h)
        stream.synchronize()
        assert np.array_equal(outs[0].cpu().numpy().view(np.uint32), ref.view(np.uint32))
    finally:
        c.dev.close()


def test_random_layer_shapes(moe, oracle):
    # seeded shapes across the paths the bf16 kernel takes: D / Dout not
    # multiples of 8 (element-wise permute, direct y stores) or of 256 (cut
    # columns), 2..40 experts, top-1..4, gated / standard, bf16 / fp8, batches
    # that give 128- and 256-row tiles, partial tiles and tail-split down tiles
    rng = np.random.default_rng(2026)
    for case in range(14):
        E = int(rng.integers(2, 41))
        k = int(rng.integers(1, min(4, E) + 1))
        D = int(rng.choice([64, 90, 100, 130, 200, 262, 320, 512]))
        Dout = int(rng.choice([D, 72, 90, 130, 136, 262]))
        H = int(rng.choice([96, 200, 384, 688]))
        T = int(rng.integers(16, 700)) if case % 2 == 0 else int(rng.integers(1200, 2400))
        if case % 4 == 1:
            E = int(rng.integers(2, 9))  # few large experts: 256-row tiles
            k = int(rng.integers(1, min(2, E) + 1))
        etype = "gated" if rng.random() < 0.7 else "standard"
        act = "silu" if etype == "gated" else str(rng.choice(["gelu", "relu"]))
        wdtype = str(rng.choice(["bf16", "fp8"]))
        bias = (rng.standard_normal(E) * float(rng.choice([0.0, 1.0]))).astype(np.float32)
        c = Case(moe, oracle, T=T, D=D, H=H, Dout=Dout, E=E, k=k, gate="switch" if k == 1 else "topk",
                 expert_type=etype, act=act, wdtype=wdtype, xdtype="bf16", seed=900 + case, router_bias=bias)
        try:
            check_case(c, TOL[wdtype])
        finally:
            c.dev.close()


def test_random_wide_layers(moe, oracle):
    # seeded layers over the wide ranges: 9..512 experts, up to 16 slots per
    # token, every device gate, the layer's shared experts, fp32 / bf16 / fp8
    # weights, capacity drop; routing bit-exact, output within tolerance
    rng = np.random.default_rng(4243)
    for case in range(12):
        E = int(rng.choice([9, 24, 70, 129, 200, 300, 512]))
        gate = str(rng.choice(["topk", "shared", "soft", "switch"]))
        lsh = int(rng.integers(0, 3)) if case % 3 == 0 else 0
        Er = E - lsh
        ns = int(rng.integers(1, 4)) if gate == "shared" else 0
        kmax = min(16 - lsh - ns, Er - ns)
        k = 1 if gate == "switch" else (kmax if case % 4 == 2 else int(rng.integers(1, kmax + 1)))
        wdtype = str(rng.choice(["f32", "bf16", "fp8"]))
        T = int(rng.integers(40, 900))
        drop = bool(rng.random() < 0.4) and lsh == 0
        param = float(rng.choice([0.6, 1.0, 1.7])) if gate == "soft" else None
        bias = (rng.standard_normal(Er) * 0.5).astype(np.float32) if lsh == 0 else None
        print(f"wide case {case}: E={E} gate={gate} k={k} ns={ns} lsh={lsh} w={wdtype} T={T} drop={drop}", flush=True)
        c = Case(moe, oracle, T=T, D=64, H=64, E=E, k=k, gate=gate, ns=ns, wdtype=wdtype,
                 xdtype="f32" if wdtype == "f32" else "bf16", seed=4242 + case, router_bias=bias, lsh=lsh,
                 drop=drop, cf=1.0, gate_param=param)
        try:
            if lsh:
                check_shared_experts_case(c, TOL[wdtype], training=True)
            else:
                check_case(c, TOL[wdtype], training=bool(case % 2 == 0))
        finally:
            c.dev.close()


def test_router_lse(moe, oracle):
    """Per-token logsumexp of the z-loss (src/balancing/losses.jl:111-114)
    from moe_router_lse after a layer forward: within 2 ulp of the oracle's on
    the GPU's logits, and its squares' mean times beta is the z-loss."""
    case = Case(moe, oracle, T=1000, D=96, H=64, E=12, k=2, seed=41, z=0.01)
    out, loss, res = case.run(training=True)
    lse = case.dev.router_lse(case.T)
    ref = oracle.logsumexp_rows(res["logits"])
    assert np.all(np.abs(lse - ref) <= 2.5e-7 * np.maximum(1.0, np.abs(ref))), np.max(np.abs(lse - ref))
    zl = np.float32(0.01) * np.float32(np.mean((lse.astype(np.float64)) ** 2))
    assert abs(res["z_loss"] - zl) <= 1e-5 * max(1.0, abs(float(zl)))
    from mixtureofexperts_amd import _lib

    with pytest.raises(_lib.MoeError):
        case.dev.router_lse(case.T - 1)


@pytest.mark.parametrize("T", [65536, 131072])
def test_switch_loss_large_batch(moe, oracle, T):
    """The Switch loss at large batches (src/balancing/losses.jl:15-36,
    src/core/moe_layer.jl:151): a router bias makes expert 1 dominant (mean
    probability ~0.8), so at T = 131072 its per-call probability mass passes
    2^16.  The fused loss (the router's fixed-point
    probability sums, totalled in the permute's scan) and the mean entropy
    are checked within 1e-5 against the oracle on the GPU's indices and
    probabilities, and routing bit-exact through check_case."""
    bias = np.zeros(8, np.float32)
    bias[0] = 4.0
    c = Case(moe, oracle, T=T, D=64, H=64, E=8, k=2, wdtype="bf16", xdtype="bf16", seed=131, router_bias=bias)
    try:
        out, loss, res = c.run(training=True)
        p_mean = float(res["probs"][:, 0].astype(np.float64).mean())
        assert p_mean > 0.75, p_mean
        if T > 65536:
            assert p_mean * T > 65536  # the mass a 2^48 fixed-point total would wrap on
        sw = oracle.switch_loss(res["indices"], res["probs"], c.alpha)
        assert abs(res["switch_loss"] - sw) <= 1e-5 * max(1.0, abs(float(sw))), (res["switch_loss"], sw)
        ent = oracle.mean_entropy(res["probs"])
        assert abs(res["mean_entropy"] - ent) <= 1e-5 * max(1.0, abs(float(ent))), (res["mean_entropy"], ent)
        check_case(c, TOL["bf16"])
    finally:
        c.dev.close()


@pytest.mark.parametrize("E,ns", [(10, 1), (11, 3)])
def test_shared_expert_gating_inexact_scales(moe, oracle, E, ns):
    """A layer with SharedExpertGating(ns, TopKGating(2), E): the routed gate
    scale 1 - ns/(ns + 2) (2/3, 2/5) and probability scale 1 - ns/E in
    Float64 (src/gating/advanced.jl:95-105), bit-exact through check_case."""
    c = Case(moe, oracle, T=1200, D=128, H=192, E=E, k=2, gate="shared", ns=ns, wdtype="bf16", xdtype="bf16",
             seed=300 + E)
    try:
        check_case(c, TOL["bf16"])
    finally:
        c.dev.close()
