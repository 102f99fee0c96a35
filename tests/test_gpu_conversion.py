"""GPU checks of convert_to_moe's expert creation on the device
(moe_init_experts_from_dense, src/llama2/conversion.jl:277-331) and of the
layer's on-disk format (moe_get_expert + safetensors).

:copy and :split are deterministic and checked bit-exactly against the
oracle's restatement (after the packed dtype's rounding); :perturb and
:random draw from the library's counter-based generator, which is not
Julia's randn stream: they are checked by their distribution (the noise's
mean and standard deviation), by noise 0 == :copy, and by reproducibility
per seed (parity of the draws themselves is unpinned)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dense(rng, dim=96, hid=200):
    return [(rng.standard_normal(sh) * 0.05).astype(np.float32) for sh in ((dim, hid), (hid, dim), (dim, hid))]


def _expert_f32(oracle, ex):
    """Host copy of an expert's weights as fp32 (Flux (out, in))."""
    if ex.scales is not None:
        return [oracle.dequantize_fp8_rows(w, s) for w, s in zip((ex.w1, ex.w2, ex.w3), ex.scales)]
    if ex.w1.dtype == np.uint16:
        return [oracle.bf16_bits_to_f32(w) for w in (ex.w1, ex.w2, ex.w3)]
    return [ex.w1, ex.w2, ex.w3]


@pytest.mark.parametrize("wdtype", ["f32", "bf16", "fp8"])
def test_copy_and_split(moe, oracle, wdtype):
    rng = np.random.default_rng(90)
    w1, w2, w3 = _dense(rng)
    print(f"convert copy/split w={wdtype}", flush=True)
    for strategy in ("copy", "split"):
        layer = moe.convert_layer_to_moe(w1, w2, w3, num_experts=8, expert_init_strategy=strategy,
                                         weight_dtype=wdtype, max_tokens=64, rng=np.random.default_rng(1))
        for e, ex in enumerate(layer.experts):
            src = (w1, w2, w3) if strategy == "copy" else oracle.split_expert(w1, w2, w3, e, 8)
            flux = [np.ascontiguousarray(m.T) for m in src]  # (out, in)
            if wdtype == "f32":
                expect = [flux[0], flux[1], flux[2]]
                got = [ex.w1, ex.w2, ex.w3]
            elif wdtype == "bf16":
                expect = [oracle.f32_to_bf16_bits(m) for m in flux]
                got = [ex.w1, ex.w2, ex.w3]
            else:
                q = [oracle.quantize_fp8_rows(m) for m in flux]
                expect = [c for c, _ in q] + [s for _, s in q]
                got = [ex.w1, ex.w2, ex.w3] + list(ex.scales)
            for a, b in zip(got, expect):
                assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8)), (strategy, e)
        # the layer runs on the converted weights: output against the oracle
        x = rng.standard_normal((96, 40)).astype(np.float32)
        aux = {}
        out, _ = layer(x, _aux=aux)
        ex = [dict(zip(("w1", "w2", "w3"), _expert_f32(oracle, e))) for e in layer.experts]
        ref, _, _ = oracle.moe_forward(x.T, layer.router.weight, ex, k=2, logits=aux["logits"])
        tol = {"f32": 1e-4, "bf16": 2e-2, "fp8": 5e-2}[wdtype]
        err = np.linalg.norm(out.T - ref) / np.linalg.norm(ref)
        assert err <= tol, (strategy, err)
        layer.close()


def test_split_sum_is_the_dense_ffn(moe, oracle):
    # every expert on every token: the :split experts add up to the dense FFN
    rng = np.random.default_rng(91)
    w1, w2, w3 = _dense(rng)
    layer = moe.convert_layer_to_moe(w1, w2, w3, num_experts=8, expert_init_strategy="split", max_tokens=64)
    x = rng.standard_normal((96, 10)).astype(np.float32)
    total = sum(ex(x).astype(np.float64) for ex in layer.experts)
    dense = oracle.gated_expert(x.T, w1.T, w2.T, w3.T, oracle.act_silu).T
    assert np.max(np.abs(total - dense)) / np.max(np.abs(dense)) < 1e-5
    layer.close()


def test_perturb_and_random_distribution(moe):
    rng = np.random.default_rng(92)
    w1, w2, w3 = _dense(rng, dim=256, hid=512)
    noise = 0.01
    la = moe.convert_layer_to_moe(w1, w2, w3, num_experts=4, expert_init_strategy="perturb",
                                  expert_init_noise=noise, seed=7, max_tokens=16)
    lb = moe.convert_layer_to_moe(w1, w2, w3, num_experts=4, expert_init_strategy="perturb",
                                  expert_init_noise=noise, seed=7, max_tokens=16)
    lc = moe.convert_layer_to_moe(w1, w2, w3, num_experts=4, expert_init_strategy="perturb",
                                  expert_init_noise=noise, seed=8, max_tokens=16)
    l0 = moe.convert_layer_to_moe(w1, w2, w3, num_experts=4, expert_init_strategy="perturb",
                                  expert_init_noise=0.0, seed=7, max_tokens=16)
    base = [np.ascontiguousarray(m.T) for m in (w1, w2, w3)]
    draws = []
    for e in range(4):
        for m, nm in enumerate(("w1", "w2", "w3")):
            a = getattr(la.experts[e], nm)
            assert np.array_equal(a, getattr(lb.experts[e], nm))        # same seed, same weights
            assert not np.array_equal(a, getattr(lc.experts[e], nm))    # another seed, other weights
            assert np.array_equal(getattr(l0.experts[e], nm), base[m])  # noise 0: the copy
            draws.append(((a - base[m]) / noise).ravel())
    z = np.concatenate(draws)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    # experts differ from each other (independent streams)
    assert not np.array_equal(la.experts[0].w1, la.experts[1].w1)
    lr = moe.convert_layer_to_moe(w1, w2, w3, num_experts=2, expert_init_strategy="random", seed=3, max_tokens=16)
    r = np.concatenate([lr.experts[e].w1.ravel() for e in range(2)])
    assert abs(r.std() / np.sqrt(2.0 / 256) - 1.0) < 0.01 and abs(r.mean()) < 0.002
    for lay in (la, lb, lc, l0, lr):
        lay.close()
    with pytest.raises(moe.MoeError):
        moe.convert_layer_to_moe(w1, w2, w3, expert_init_strategy="nope")


@pytest.mark.parametrize("wdtype", ["bf16", "fp8"])
def test_save_load_round_trip(moe, oracle, tmp_path, wdtype):
    rng = np.random.default_rng(93)
    w1, w2, w3 = _dense(rng)
    layer = moe.convert_layer_to_moe(w1, w2, w3, num_experts=8, expert_init_strategy="perturb", seed=11,
                                     weight_dtype=wdtype, max_tokens=64)
    x = rng.standard_normal((96, 48)).astype(np.float32)
    out, loss = layer(x, training=True)
    path = str(tmp_path / "layer.safetensors")
    moe.save_moe_layer(layer, path)
    back = moe.load_moe_layer(path)
    out2, loss2 = back(x, training=True)
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32)) and loss == loss2
    for a, b in zip(layer.experts, back.experts):
        assert np.array_equal(a.w1, b.w1) and np.array_equal(a.w2, b.w2) and np.array_equal(a.w3, b.w3)
    layer.close()
    back.close()
