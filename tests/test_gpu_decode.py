"""GPU parity of the decode caller (moe_ffn_forward!, src/llama2/inference.jl:58-121)
through the C ABI (moe_decode) against the oracle's restatement
(oracle.decode_ffn) on identical seeded inputs.

C2 shapes (stories42M MoE layer: D=512, H=1376, E=8, k=2, fp32).  Routing is
compared bit-exactly on the GPU's own logits (the logits themselves against
fp32 x W'); the output (slot-order combine) within 1e-4 relative at fp32
weights, 2e-2 at bf16, 5e-2 at fp8; two runs are bitwise identical."""
import numpy as np
import pytest

from test_gpu_layer import Case, rel_err

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "bf16": 2e-2, "fp8": 5e-2}


def check_decode(case, oracle, n, tol):
    x = np.ascontiguousarray(case.x[:n])
    print(f"decode n={n} E={case.E} k={case.k} gate={case.gate}", flush=True)
    out, logits, idx, gates = case.dev.decode(x)
    out2, _, _, _ = case.dev.decode(x)
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32)), "not deterministic"
    assert np.all(np.isfinite(out))
    ref_logits = (x.astype(np.float64) @ case.wr.T.astype(np.float64))
    if case.rb is not None:
        ref_logits = ref_logits + np.asarray(case.rb, np.float64)
    assert np.max(np.abs(logits - ref_logits)) <= 1e-5 * max(1.0, float(np.max(np.abs(ref_logits))))
    ref, ridx, rgates, _ = oracle.decode_ffn(x, case.wr, case.ex, gate=case.gate, k=case.k, logits=logits)
    assert np.array_equal(idx, ridx)
    assert np.array_equal(gates.view(np.uint32), rgates.view(np.uint32))
    err = rel_err(out, ref)
    assert err <= tol, f"relative error {err:.3e} > {tol}"
    return out, idx, gates


@pytest.mark.parametrize("n", [1, 8])
def test_decode_c2_fp32(moe, oracle, n):
    c = Case(moe, oracle, T=8, D=512, H=1376, E=8, k=2, wdtype="f32", seed=21)
    try:
        check_decode(c, oracle, n, TOL["f32"])
    finally:
        c.dev.close()


@pytest.mark.parametrize("lsh,k", [(0, 2), (1, 2)])
def test_decode_batch_and_single_calls_agree(moe, oracle, lsh, k):
    # a call over 12 tokens and calls over 1 to 3 of them compute the same
    # products in the same order: each token's output, logits, routing and
    # gates are bitwise equal, over 30 calls in a row
    E = 8 + lsh
    c = Case(moe, oracle, T=12, D=512, H=1376, E=E, k=k, wdtype="f32", seed=31 + lsh, lsh=lsh, max_tokens=12)
    try:
        x = np.ascontiguousarray(c.x[:12])
        print(f"decode n=12 lsh={lsh}", flush=True)
        out12, l12, i12, g12 = c.dev.decode(x)
        ref, ridx, _, _ = oracle.decode_ffn(x, c.wr, c.ex, k=k, logits=l12, num_shared=lsh)
        assert np.array_equal(i12[:, lsh:] - lsh, ridx)
        assert rel_err(out12, ref) <= TOL["f32"]
        for rep in range(30):
            n = 1 + rep % 3
            t = (5 * rep) % (12 - n + 1)
            o, lg, i, g = c.dev.decode(np.ascontiguousarray(x[t:t + n]))
            assert np.array_equal(o.view(np.uint32), out12[t:t + n].view(np.uint32)), (rep, t, n)
            assert np.array_equal(lg.view(np.uint32), l12[t:t + n].view(np.uint32)), (rep, t, n)
            assert np.array_equal(i, i12[t:t + n]) and np.array_equal(g.view(np.uint32), g12[t:t + n].view(np.uint32))
    finally:
        c.dev.close()


@pytest.mark.parametrize("wdtype", ["bf16", "fp8"])
def test_decode_low_precision_weights(moe, oracle, wdtype):
    c = Case(moe, oracle, T=8, D=512, H=1376, E=8, k=2, wdtype=wdtype, seed=22)
    try:
        check_decode(c, oracle, 3, TOL[wdtype])
    finally:
        c.dev.close()


def test_decode_switch_and_wide(moe, oracle):
    # SwitchGating (gate exactly 1.0f0) over 64 experts, D not a multiple of 64
    c = Case(moe, oracle, T=6, D=200, H=300, E=64, k=1, gate="switch", wdtype="f32", seed=23)
    try:
        _, _, gates = check_decode(c, oracle, 6, TOL["f32"])
        assert np.all(gates == np.float32(1.0))
    finally:
        c.dev.close()


def test_decode_many_experts(moe, oracle):
    # E > 64: each lane of the routing wave holds two experts; k = 4 slots;
    # with a router bias
    rb = np.random.default_rng(30).standard_normal(96).astype(np.float32)
    c = Case(moe, oracle, T=5, D=128, H=96, E=96, k=4, wdtype="f32", seed=29, router_bias=rb)
    try:
        check_decode(c, oracle, 5, TOL["f32"])
    finally:
        c.dev.close()


@pytest.mark.parametrize("E,k,lsh", [(20, 12, 0), (96, 16, 0), (14, 10, 3), (200, 8, 0), (384, 8, 1), (512, 6, 0)])
def test_decode_more_than_8_slots(moe, oracle, E, k, lsh):
    # up to MOE_MAX_TOPK = 16 slots per token (routed experts of slots 8..15
    # in the upper words of the wave's slot list), E <= 64 and E > 64 gating
    # (up to 512 experts: 8 per lane), with and without the layer's shared
    # experts
    Et = E + lsh
    c = Case(moe, oracle, T=6, D=256, H=200, E=Et, k=k, wdtype="f32", seed=60 + k, lsh=lsh, max_tokens=8)
    try:
        x = np.ascontiguousarray(c.x[:6])
        print(f"decode E={E} k={k} lsh={lsh}", flush=True)
        out, logits, idx, gates = c.dev.decode(x)
        out2, _, _, _ = c.dev.decode(x)
        assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))
        assert idx.shape == (6, lsh + k)
        ref, ridx, rgates, _ = oracle.decode_ffn(x, c.wr, c.ex, gate="topk", k=k, logits=logits, num_shared=lsh)
        assert np.array_equal(idx[:, :lsh], np.tile(np.arange(1, lsh + 1, dtype=np.int32), (6, 1)))
        assert np.array_equal(idx[:, lsh:] - lsh, ridx)
        assert np.array_equal(gates[:, lsh:].view(np.uint32), rgates.view(np.uint32))
        err = rel_err(out, ref)
        assert err <= TOL["f32"], err
    finally:
        c.dev.close()


@pytest.mark.parametrize("E", [16, 40])
def test_decode_tied_and_infinite_logits(moe, oracle, E):
    # equal probabilities go to the lower expert first (partialsortperm with
    # isless, rev=true): router rows 1, 3 and 7 are equal, so their logits tie
    # bitwise; a +Inf bias on experts 5 and 9 makes p 1/2 there and 0
    # elsewhere (the +Inf-maximum rule), so the third slot is a tie of zeros
    # (expert 0).  Routing and gates bit-exact against the oracle on the GPU's
    # logits; the output within the fp32 tolerance.
    rb = np.zeros(E, np.float32)
    c = Case(moe, oracle, T=6, D=64, H=128, E=E, k=3, wdtype="f32", seed=33, router_bias=rb, max_tokens=6)
    try:
        wr = c.wr.copy()
        wr[3] = wr[1]
        wr[7] = wr[1]
        c.wr = wr
        c.dev.set_router(np.ascontiguousarray(wr.T), rb)
        x = np.ascontiguousarray(c.x[:6])
        out, logits, idx, gates = c.dev.decode(x)
        assert np.array_equal(logits[:, 3].view(np.uint32), logits[:, 1].view(np.uint32))
        ref, ridx, rgates, _ = oracle.decode_ffn(x, wr, c.ex, k=3, logits=logits)
        assert np.array_equal(idx, ridx) and np.array_equal(gates.view(np.uint32), rgates.view(np.uint32))
        assert rel_err(out, ref) <= TOL["f32"]
        rb_inf = rb.copy()
        rb_inf[5] = rb_inf[9] = np.inf
        c.dev.set_router(np.ascontiguousarray(wr.T), rb_inf)
        out, logits, idx, gates = c.dev.decode(x)
        ref, ridx, rgates, _ = oracle.decode_ffn(x, wr, c.ex, k=3, logits=logits)
        assert np.array_equal(idx, ridx) and np.array_equal(gates.view(np.uint32), rgates.view(np.uint32))
        assert np.array_equal(idx, np.tile(np.array([6, 10, 1], np.int32), (6, 1)))
        assert np.array_equal(gates, np.tile(np.array([0.5, 0.5, 0.0], np.float32), (6, 1)))
        assert rel_err(out, ref) <= TOL["f32"]
    finally:
        c.dev.close()


def test_decode_slot_order_differs_from_layer_only_by_rounding(moe, oracle):
    # the layer forward combines in expert order with the NNlib silu, the decode
    # caller in slot order with the inline silu: equal up to fp32 rounding
    c = Case(moe, oracle, T=4, D=512, H=1376, E=8, k=2, wdtype="f32", seed=24)
    try:
        out_dec, _, _, _ = c.dev.decode(np.ascontiguousarray(c.x[:4]))
        out_fwd, _, _ = c.run(training=False, T=4)
        assert rel_err(out_dec, out_fwd) <= 1e-5
    finally:
        c.dev.close()


def test_decode_unsupported_and_bad_args(moe, oracle):
    from mixtureofexperts_amd import _lib

    c = Case(moe, oracle, T=4, D=64, H=128, E=8, k=2, expert_type="standard", act="gelu", wdtype="f32", seed=25)
    try:
        x = np.ascontiguousarray(c.x[:2])
        with pytest.raises(_lib.MoeError) as ei:
            c.dev.decode(x)
        assert ei.value.status == _lib.MOE_EUNSUPPORTED
    finally:
        c.dev.close()
    c = Case(moe, oracle, T=4, D=64, H=128, E=10, k=2, gate="shared", ns=2, wdtype="f32", seed=26)
    try:
        with pytest.raises(_lib.MoeError) as ei:
            c.dev.decode(np.ascontiguousarray(c.x[:2]))
        assert ei.value.status == _lib.MOE_EUNSUPPORTED
    finally:
        c.dev.close()
    c = Case(moe, oracle, T=4, D=64, H=128, E=8, k=2, wdtype="f32", seed=27)
    try:
        with pytest.raises(_lib.MoeError) as ei:
            c.dev.decode(np.zeros((5, 64), np.float32))  # n > max_tokens
        assert ei.value.status == _lib.MOE_EINVAL
    finally:
        c.dev.close()
    # gated_expert_forward! applies silu: a gated layer configured with gelu
    # (MoEConfig's default) is refused instead of silently computing silu
    c = Case(moe, oracle, T=4, D=64, H=128, E=8, k=2, act="gelu", wdtype="f32", seed=29)
    try:
        with pytest.raises(_lib.MoeError) as ei:
            c.dev.decode(np.ascontiguousarray(c.x[:2]))
        assert ei.value.status == _lib.MOE_EUNSUPPORTED and "silu" in str(ei.value)
    finally:
        c.dev.close()


def test_decode_python_api(moe, oracle):
    # moe_ffn_forward(layer, xb) on a vector and on a (D, n) matrix
    rng = np.random.default_rng(28)
    cfg = moe.MoEConfig(num_experts=8, expert_type="gated", input_dim=512, hidden_dim=1376, output_dim=512,
                        activation=moe.silu, gate_type=moe.TopKGating(2), max_tokens=16)
    layer = moe.MoELayer(cfg, rng=rng)
    try:
        xb = rng.standard_normal(512).astype(np.float32)
        y, sel, g = moe.moe_ffn_forward(layer, xb)
        assert y.shape == (512,) and sel.shape == (2,) and sel.dtype == np.int64 and g.shape == (2,)
        ex = [dict(w1=e.w1, w2=e.w2, w3=e.w3) for e in layer.experts]
        ref, ridx, rg, _ = oracle.decode_ffn(xb[None, :], layer.router.weight, ex, k=2)
        assert np.array_equal(sel, ridx[0].astype(np.int64))
        assert rel_err(y, ref[0]) <= 1e-4
        X = rng.standard_normal((512, 5)).astype(np.float32)
        Y, S, G = moe.moe_ffn_forward(layer, X)
        assert Y.shape == (512, 5) and S.shape == (2, 5) and G.shape == (2, 5)
        assert np.allclose(Y[:, 0], moe.moe_ffn_forward(layer, X[:, 0])[0], rtol=0, atol=0)
    finally:
        layer.close()


@pytest.mark.parametrize("lsh,k,wdtype", [(1, 2, "f32"), (2, 2, "bf16"), (3, 1, "fp8")])
def test_decode_shared_experts(moe, oracle, lsh, k, wdtype):
    # process_shared_experts!: shared experts averaged with weight 1f0/ns and
    # blended 0.5 / 0.5 with the slot-order routed combine
    E = 6 + lsh
    c = Case(moe, oracle, T=4, D=256, H=344, E=E, k=k, gate="switch" if k == 1 else "topk", wdtype=wdtype,
             seed=40 + lsh, lsh=lsh, max_tokens=8)
    try:
        x = np.ascontiguousarray(c.x[:4])
        print(f"decode shared lsh={lsh} k={k} w={wdtype}", flush=True)
        out, logits, idx, gates = c.dev.decode(x)
        assert logits.shape == (4, E - lsh)
        ref, ridx, rgates, _ = oracle.decode_ffn(x, c.wr, c.ex, gate=c.gate, k=k, logits=logits, num_shared=lsh)
        assert np.array_equal(idx[:, :lsh], np.tile(np.arange(1, lsh + 1, dtype=np.int32), (4, 1)))
        assert np.array_equal(idx[:, lsh:] - lsh, ridx)
        assert np.array_equal(gates[:, lsh:].view(np.uint32), rgates.view(np.uint32))
        err = rel_err(out, ref)
        assert err <= TOL[wdtype], err
        # and the same routing through the Python mirror: routed ids as the router numbers them
        from mixtureofexperts_amd.layer import moe_ffn_forward  # noqa: F401
    finally:
        c.dev.close()


@pytest.mark.parametrize("wdtype", ["bf16", "fp8"])
def test_decode_between_forwards_leaves_forward_unchanged(moe, oracle, wdtype):
    # the decode caller uses the layer's h workspace as fp32 scratch; the
    # forward call (h as the GEMM's tile image) must come out bit-identical
    # before and after it, on a batch with several tiles per expert
    c = Case(moe, oracle, T=600, D=256, H=688, E=8, k=2, wdtype=wdtype, xdtype="bf16", seed=44)
    try:
        print(f"forward / decode / forward w={wdtype}", flush=True)
        out1, loss1, _ = c.run(training=True)
        c.dev.decode(np.ascontiguousarray(c.x[:8]))
        out2, loss2, _ = c.run(training=True)
        assert np.array_equal(out1.view(np.uint32), out2.view(np.uint32)) and loss1 == loss2
    finally:
        c.dev.close()


def test_stories42m_moe_decode_chain(moe, oracle):
    # BASELINE config 2's MoE part: three stories42M-shaped FFNs (dim 512,
    # hidden 1376) converted with convert_to_moe's :perturb (noise 0.01) into 8
    # gated silu experts, top-2, fp32, then tokens decoded one at a time
    # through the three layers in order (moe_ffn_forward! per layer,
    # src/llama2/inference.jl:58-121; sample_moe's per-token loop,
    # src/llama2/generation.jl:38-128).  Every layer of every token is checked
    # against oracle.decode_ffn on the GPU's logits with the experts read back
    # from the device: routing and gates bit-exact, output within 1e-4; the
    # chain's final output also against the oracle run end to end on its own.
    # 256 tokens: the decode length of BASELINE config 2.
    rng = np.random.default_rng(42)
    dim, hid, E, n_tok = 512, 1376, 8, 256
    layers, host = [], []
    try:
        for li in range(3):
            w1, w3 = [(rng.standard_normal((dim, hid)) * 0.02).astype(np.float32) for _ in range(2)]
            w2 = (rng.standard_normal((hid, dim)) * 0.02).astype(np.float32)
            layer = moe.convert_layer_to_moe(w1, w2, w3, num_experts=E, top_k=2, expert_init_strategy="perturb",
                                             expert_init_noise=0.01, max_tokens=4, seed=100 + li,
                                             rng=np.random.default_rng(li))
            layers.append(layer)
            host.append((layer.router.weight, [dict(w1=e.w1, w2=e.w2, w3=e.w3) for e in layer.experts]))
            # :perturb: each expert is the dense FFN plus N(0, 0.01^2) noise
            d = layers[-1].experts[3].w1 - w1.T
            assert abs(float(d.std()) - 0.01) < 5e-4 and abs(float(d.mean())) < 5e-4
        x = rng.standard_normal((n_tok, dim)).astype(np.float32)
        final = np.zeros((n_tok, dim), np.float32)
        usage = np.zeros((3, E), np.int64)
        for t in range(n_tok):
            print(f"decode chain token {t}", flush=True) if t % 64 == 0 else None
            v = x[t:t + 1]
            for li, layer in enumerate(layers):
                out, logits, idx, gates = layer._dev.decode(np.ascontiguousarray(v))
                wr, ex = host[li]
                ref, ridx, rgates, _ = oracle.decode_ffn(v, wr, ex, k=2, logits=logits)
                assert np.array_equal(idx, ridx), (t, li)
                assert np.array_equal(gates.view(np.uint32), rgates.view(np.uint32)), (t, li)
                assert rel_err(out, ref) <= 1e-4, (t, li)
                usage[li, idx[0] - 1] += 1
                v = out
            final[t] = v[0]
        # end to end on the oracle alone (its own fp32 logits)
        ref = x
        for wr, ex in host:
            ref = oracle.decode_ffn(ref, wr, ex, k=2)[0]
        assert rel_err(final, ref) <= 1e-4
        assert usage.sum() == 3 * n_tok * 2
    finally:
        for layer in layers:
            layer.close()
