"""Router noise (src/core/router.jl:32-41) and StandardExpert dropout
(src/experts/standard.jl:49-51) in training, on the GPU.

The noise comes from the library's counter-based generator, not Julia's randn
stream, so the draws are checked by their distribution: the difference of the
training call's logits and the same layer's inference logits, divided by
noise_scale (or by noise_scale .* softplus(noise logits) with a noise
network), must look like N(0, 1).  Everything downstream of the noise is then
checked exactly: the routing on the noisy logits is bit-exact against the
oracle, the Switch loss and the statistics follow the noisy probabilities,
and the z-loss the logits without noise (moe_layer.jl:117-121)."""
import numpy as np
import pytest

from test_gpu_layer import TOL, Case, rel_err

pytestmark = pytest.mark.gpu


def softplus(v):
    v = np.asarray(v, np.float32)
    return (np.log1p(np.exp(-np.abs(v))) + np.maximum(v, 0)).astype(np.float32)


def check_normal(r, what):
    r = np.asarray(r, np.float64).ravel()
    n = r.size
    assert abs(r.mean()) < 5.0 / np.sqrt(n), f"{what}: mean {r.mean():.4f}"
    assert abs(r.std() - 1.0) < 5.0 * np.sqrt(0.5 / n) + 0.01, f"{what}: std {r.std():.4f}"
    # tails of a standard normal: P(|r| > 2) = 4.55 %
    frac = float(np.mean(np.abs(r) > 2.0))
    assert abs(frac - 0.0455) < 0.01, f"{what}: P(|r|>2) {frac:.4f}"


def routed_checks(case, res, out, loss, noisy, clean):
    ref_out, ref_loss, aux = case.oracle.moe_forward(case.x, case.wr, case.ex, gate=case.gate, k=case.k,
                                                     num_shared=case.ns, expert_type=case.expert_type,
                                                     act=case.act, alpha=case.alpha, z_weight=case.z,
                                                     training=True, logits=noisy, z_logits=clean)
    assert np.array_equal(res["indices"], aux["idx"])
    assert np.array_equal(res["gates"].view(np.uint32), aux["gates"].view(np.uint32))
    assert np.array_equal(res["probs"].view(np.uint32), aux["probs"].view(np.uint32))
    assert np.array_equal(res["counts"], aux["counts"])
    n = int(aux["offsets"][-1])
    assert np.array_equal(res["perm"][:n], aux["perm"])
    assert rel_err(out, ref_out) <= TOL["f32"]
    assert abs(loss - ref_loss) <= 1e-5 * max(1.0, abs(float(ref_loss))), (loss, ref_loss)
    assert abs(res["z_loss"] - aux["z_loss"]) <= 1e-5 * max(1.0, abs(float(aux["z_loss"])))
    assert abs(res["mean_entropy"] - aux["mean_entropy"]) <= 1e-5 * max(1.0, abs(float(aux["mean_entropy"])))


@pytest.mark.parametrize("E,k", [(8, 2), (40, 4)])
def test_router_noise(moe, oracle, E, k):
    case = Case(moe, oracle, T=2048, D=128, H=64, E=E, k=k, seed=21)
    scale = 0.5
    case.dev.set_router_noise(scale, None, seed=1234)
    _, _, clean_res = case.run(training=False)
    clean = clean_res["logits"]
    out, loss, res = case.run(training=True)
    noisy = res["logits"]
    check_normal((noisy - clean) / np.float32(scale), f"noise E={E}")
    routed_checks(case, res, out, loss, noisy, clean)
    # a new draw per training call; inference calls stay noise-free
    _, _, res2 = case.run(training=True)
    assert not np.array_equal(res2["logits"], noisy)
    _, _, clean2 = case.run(training=False)
    assert np.array_equal(clean2["logits"], clean)
    # the same seed gives the same draws from a fresh start
    case.dev.set_router_noise(scale, None, seed=1234)
    _, _, res3 = case.run(training=True)
    assert np.array_equal(res3["logits"], noisy)
    # noise_scale 0 turns it off
    case.dev.set_router_noise(0.0, None, seed=1234)
    _, _, res4 = case.run(training=True)
    assert np.array_equal(res4["logits"], clean)


@pytest.mark.parametrize("E,xdtype", [(4, "f32"), (8, "f32"), (24, "f32"), (100, "f32"), (200, "f32"),
                                      (150, "bf16")])
def test_router_noise_network(moe, oracle, E, xdtype):
    # (100: 200 GEMM columns, 32-token route blocks; 150 and 200: over 256
    # columns, 16-token route blocks, on bf16 and fp32 x)
    case = Case(moe, oracle, T=2048, D=128, H=64, E=E, k=2, seed=22, xdtype=xdtype)
    scale = 0.3
    wn = (np.random.default_rng(5).standard_normal((E, case.D)) / np.sqrt(case.D)).astype(np.float32)
    case.dev.set_router_noise(scale, np.ascontiguousarray(wn.T), seed=99)
    _, _, clean_res = case.run(training=False)
    clean = clean_res["logits"]
    out, loss, res = case.run(training=True)
    noisy = res["logits"]
    sp = softplus(case.x @ wn.T)
    check_normal((noisy - clean) / (np.float32(scale) * sp), f"noise network E={E}")
    routed_checks(case, res, out, loss, noisy, clean)


def test_layer_router_noise_python_api(moe):
    cfg = moe.MoEConfig(num_experts=8, expert_type="gated", input_dim=64, hidden_dim=96, output_dim=64,
                        gate_type=moe.TopKGating(2), noise_scale=0.2, use_noise_network=True, max_tokens=256)
    layer = moe.MoELayer(cfg, rng=np.random.default_rng(3))
    x = np.random.default_rng(4).standard_normal((64, 256)).astype(np.float32)
    y0, l0 = layer(x, training=False)
    y1, l1 = layer(x, training=True)
    y2, l2 = layer(x, training=False)
    assert np.array_equal(y0, y2) and l0 == 0.0 and l2 == 0.0
    assert np.isfinite(l1) and l1 > 0
    assert not np.array_equal(y0, y1)  # the noisy gate routes some tokens differently
    layer.close()


@pytest.mark.parametrize("wdtype,p", [("f32", 0.25), ("bf16", 0.25), ("f32", 0.15)])
def test_standard_expert_dropout(moe, oracle, wdtype, p):
    """StandardExpert's Dropout(p) in training (src/experts/standard.jl:49-51):
    with W1 = W2 = I, zero biases, the identity activation and k = 1 (gate
    exactly 1) the layer output is dropout(x): every element is 0 or x times
    the scale 1 / (1 - p) in Float32 arithmetic, as NNlib computes it for the
    Float32 p (fp32: exactly; bf16: x and h rounded to bf16), the zeros are a
    fraction p of the elements, and inference calls keep x.  At p = 0.15 that
    scale is 1 ulp below Float32(1 / (1 - p)) computed in Float64."""
    from mixtureofexperts_amd import _lib
    from mixtureofexperts_amd._device import DeviceLayer, GateSpec

    T, D, E = 512, 64, 4
    rng = np.random.default_rng(31)
    x = rng.standard_normal((T, D)).astype(np.float32)
    if wdtype == "bf16":
        x = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(x))
    wr = rng.standard_normal((E, D)).astype(np.float32)
    eye = np.eye(D, dtype=np.float32)
    wcode = {"f32": _lib.MOE_F32, "bf16": _lib.MOE_BF16}[wdtype]
    dev = DeviceLayer(num_experts=E, expert_type=_lib.MOE_EXPERT_STANDARD, input_dim=D, hidden_dim=D, output_dim=D,
                      activation=_lib.MOE_ACT_IDENTITY, gate=GateSpec(_lib.MOE_GATE_TOPK, 1, 0), weight_dtype=wcode,
                      balance_alpha=0.01, z_loss_weight=0.001, capacity_factor=1.25, drop_tokens=False,
                      max_tokens=T, num_shared_experts=0)
    dev.set_router(np.ascontiguousarray(wr.T), None)
    for e in range(E):
        dev.set_expert(e, eye, eye, None, np.zeros(D, np.float32), np.zeros(D, np.float32), src_dtype=_lib.MOE_F32)
    dev.set_expert_dropout(p, seed=77)
    y_inf, _, _ = dev.forward(x, _lib.MOE_F32, False)
    assert np.array_equal(y_inf, x)
    y, _, _ = dev.forward(x, _lib.MOE_F32, True)
    p32 = np.float32(p)
    scale = np.float32(1) / (np.float32(1) - p32)
    if p == 0.15:
        assert scale != np.float32(1.0 / (1.0 - float(p32)))  # the case tells the two roundings apart
    kept = (x * scale).astype(np.float32)
    if wdtype == "bf16":
        kept = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(kept))
    zero = y == 0
    assert np.array_equal(y[~zero], kept[~zero])
    frac = float(zero.mean())
    assert abs(frac - p) < 5 * np.sqrt(p * (1 - p) / zero.size), frac
    # a new mask per training call, the same one from the same seed
    y2, _, _ = dev.forward(x, _lib.MOE_F32, True)
    assert not np.array_equal(y2 == 0, zero)
    dev.set_expert_dropout(p, seed=77)
    y3, _, _ = dev.forward(x, _lib.MOE_F32, True)
    assert np.array_equal(y3, y)
    dev.set_expert_dropout(0.0, seed=77)
    y4, _, _ = dev.forward(x, _lib.MOE_F32, True)
    assert np.array_equal(y4, x)
    dev.close()


def test_layer_expert_dropout_python_api(moe):
    cfg = moe.MoEConfig(num_experts=4, expert_type="standard", input_dim=64, hidden_dim=128, output_dim=64,
                        gate_type=moe.TopKGating(2), expert_dropout=0.3, max_tokens=128)
    layer = moe.MoELayer(cfg, rng=np.random.default_rng(8))
    x = np.random.default_rng(9).standard_normal((64, 128)).astype(np.float32)
    y0, _ = layer(x, training=False)
    y1, _ = layer(x, training=True)
    y2, _ = layer(x, training=False)
    assert np.array_equal(y0, y2) and not np.array_equal(y0, y1)
    layer.close()


def test_noise_network_many_experts_inference(moe):
    """A noise network on a router of more than 256 outputs has no device path
    (its noise logits would be GEMM columns E .. 2E - 1 past MOE_MAX_EXPERTS).
    The noise only enters training calls (src/core/router.jl:32), so such a
    layer still runs inference, bit-identical to the same layer without
    noise; its training calls raise MOE_EUNSUPPORTED."""
    from mixtureofexperts_amd import _lib

    E, D, H, T = 257, 64, 128, 512
    cfg = moe.MoEConfig(num_experts=E, expert_type="standard", input_dim=D, hidden_dim=H, output_dim=D,
                        gate_type=moe.SwitchGating(), noise_scale=0.2, use_noise_network=True, max_tokens=T,
                        weight_dtype="bf16")
    noisy = moe.MoELayer(cfg, rng=np.random.default_rng(41))
    plain_router = moe.Router(D, E, noisy.router.gate_type, weight=noisy.router.weight)
    plain_cfg = moe.MoEConfig(**{**cfg.__dict__, "noise_scale": 0.0, "use_noise_network": False})
    plain = moe.MoELayer(plain_cfg, experts=noisy.experts, router=plain_router)
    x = np.random.default_rng(42).standard_normal((D, T)).astype(np.float32)
    y0, l0 = noisy(x, training=False)
    y1, l1 = plain(x, training=False)
    assert np.array_equal(y0, y1) and l0 == l1 == 0.0
    with pytest.raises(_lib.MoeError) as err:
        noisy(x, training=True)
    assert err.value.status == _lib.MOE_EUNSUPPORTED
    noisy.close()
    plain.close()
