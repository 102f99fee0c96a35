"""GPU parity at the benchmark configurations' full sizes (
4, 5): Mixtral-8x7B-shaped bf16 layer, DeepSeek-style fine-grained layer with
fp8-e4m3 weights and SharedExpertGating, Switch-style k=1 layer with 128 GELU
StandardExperts.

The oracle cannot run a whole layer of this size in seconds, so the checks
are split: routing over the whole batch is compared bit-exactly with the
oracle on the GPU's own logits (indices, gates, probs, counts, offsets,
permutation); the layer output is compared on a sample of tokens with the
oracle's fp32 FFNs on the dequantised weights (2e-2 for bf16 weights, 5e-2
for fp8); the losses within 1e-5; and size-independent properties hold:
counts sum to T*k, offsets are their prefix sum, the permutation lists every
entry once, and two runs are bitwise identical."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = {"bf16": 2e-2, "fp8": 5e-2}


def rel_err(a, b):
    return float(np.linalg.norm((a - b).astype(np.float64)) / max(np.linalg.norm(b.astype(np.float64)), 1e-30))


def build(moe, *, T, D, H, E, k, gate, ns, etype, act, wdtype, bias_kind, seed):
    """Weights and inputs generated on the GPU (seeded), uploaded from device
    memory; returns the handle and host copies of everything the oracle needs."""
    import torch

    from mixtureofexperts_amd import _lib
    from mixtureofexperts_amd._device import DeviceLayer, GateSpec

    print(f"fullsize case T={T} D={D} H={H} E={E} k={k} gate={gate} ns={ns} {etype} {act} w={wdtype}", flush=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    spec = {"topk": GateSpec(_lib.MOE_GATE_TOPK, k, 0), "switch": GateSpec(_lib.MOE_GATE_SWITCH, 1, 0),
            "shared": GateSpec(_lib.MOE_GATE_SHARED, k, ns)}[gate]
    gated = etype == "gated"
    dev = DeviceLayer(num_experts=E, expert_type=_lib.MOE_EXPERT_GATED if gated else _lib.MOE_EXPERT_STANDARD,
                      input_dim=D, hidden_dim=H, output_dim=D,
                      activation={"silu": _lib.MOE_ACT_SILU, "gelu": _lib.MOE_ACT_GELU}[act], gate=spec,
                      weight_dtype={"bf16": _lib.MOE_BF16, "fp8": _lib.MOE_FP8_E4M3}[wdtype], balance_alpha=0.01,
                      z_loss_weight=0.001, capacity_factor=1.25, drop_tokens=False, max_tokens=T)
    x = torch.randn(T, D, generator=gen, device="cuda").to(torch.bfloat16)
    if bias_kind == "normal":
        wr = torch.randn(E, D, generator=gen, device="cuda") * 0.02
        rb = torch.randn(E, generator=gen, device="cuda")
    elif bias_kind == "zipf":
        wr = torch.randn(E, D, generator=gen, device="cuda") * 0.02
        r = torch.arange(1, E - ns + 1, device="cuda", dtype=torch.float32)
        rb = torch.cat([torch.zeros(ns, device="cuda"), -1.1 * torch.log(r)])
    else:
        wr = torch.randn(E, D, generator=gen, device="cuda") / (D ** 0.5)
        rb = None
    wr_mem = wr.t().contiguous()
    torch.cuda.synchronize()
    _lib.check(_lib.lib().moe_set_router(dev.h, wr_mem.data_ptr(), None if rb is None else rb.data_ptr()), dev.h)
    host = []
    for e in range(E):
        shapes = [(H, D), (D, H), (H, D)] if gated else [(H, D), (D, H)]
        mats, scales = [], []
        for shp in shapes:
            w = torch.randn(*shp, generator=gen, device="cuda") * 0.02
            if wdtype == "fp8":
                s = (w.abs().amax(dim=1) / 448.0).clamp_min(1e-30)
                q = (w / s[:, None]).to(torch.float8_e4m3fn)
                mats.append(q.view(torch.uint8).contiguous())
                scales.append(s.contiguous())
            else:
                mats.append(w.to(torch.bfloat16).contiguous())
                scales.append(None)
        b1 = b2 = None
        if not gated:
            b1 = (torch.randn(H, generator=gen, device="cuda") * 0.02).contiguous()
            b2 = (torch.randn(D, generator=gen, device="cuda") * 0.02).contiguous()
        w1, w2 = mats[0], mats[1]
        w3 = mats[2] if gated else None
        s1, s2 = scales[0], scales[1]
        s3 = scales[2] if gated else None
        src = _lib.MOE_FP8_E4M3 if wdtype == "fp8" else _lib.MOE_BF16
        ptr = lambda t: None if t is None else t.data_ptr()
        torch.cuda.synchronize()
        _lib.check(_lib.lib().moe_set_expert(dev.h, e, _lib.MOE_LAYOUT_LLAMA_IN_OUT, src, ptr(w1), ptr(w2), ptr(w3),
                                             ptr(b1), ptr(b2), ptr(s1), ptr(s2), ptr(s3)), dev.h)
        host.append(dict(w1=w1, w2=w2, w3=w3, b1=b1, b2=b2, s1=s1, s2=s2, s3=s3))
    torch.cuda.synchronize()
    xh = x.view(torch.int16).cpu().numpy().view(np.uint16)
    return dev, xh, wr.cpu().numpy(), None if rb is None else rb.cpu().numpy(), host


def f32_weights(oracle, host, e, wdtype):
    """Expert e's weights as the fp32 values the device computes with."""
    out = {}
    for n in ("w1", "w2", "w3"):
        t = host[e][n]
        if t is None:
            out[n] = None
        elif wdtype == "fp8":
            out[n] = oracle.dequantize_fp8_rows(t.cpu().numpy(), host[e]["s" + n[1]].cpu().numpy())
        else:
            out[n] = t.float().cpu().numpy()
    for n in ("b1", "b2"):
        out[n] = None if host[e][n] is None else host[e][n].cpu().numpy()
    return out


CASES = {
    "mixtral": dict(T=4096, D=4096, H=14336, E=8, k=2, gate="topk", ns=0, etype="gated", act="silu", wdtype="bf16",
                    bias_kind="normal", seed=31),
    "deepseek": dict(T=8192, D=2048, H=1408, E=66, k=6, gate="shared", ns=2, etype="gated", act="silu", wdtype="fp8",
                     bias_kind="zipf", seed=32),
    "switch": dict(T=16384, D=768, H=3072, E=128, k=1, gate="switch", ns=0, etype="standard", act="gelu",
                   wdtype="bf16", bias_kind=None, seed=33),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_full_size_layer(moe, oracle, name):
    c = CASES[name]
    dev, xh, wr, rb, host = build(moe, **c)
    try:
        T, E, kt = c["T"], c["E"], c["k"] + c["ns"]
        out, loss, res = dev.forward(np.ascontiguousarray(xh), 1, True, want_aux=True)  # x bf16, training
        out2, loss2, _ = dev.forward(np.ascontiguousarray(xh), 1, True, want_aux=False)
        assert np.array_equal(out.view(np.uint32), out2.view(np.uint32)) and loss == loss2, "not deterministic"
        assert np.all(np.isfinite(out))
        logits = res["logits"]
        xf = oracle.bf16_bits_to_f32(xh)
        # router logits: fp32 GEMM against an fp64 product on a token sample
        samp = np.linspace(0, T - 1, 64).astype(np.int64)
        ref_l = (xf[samp].astype(np.float64) @ wr.T.astype(np.float64))
        if rb is not None:
            ref_l = ref_l + rb
        assert np.max(np.abs(logits[samp] - ref_l)) <= 1e-4 * max(1.0, float(np.max(np.abs(ref_l))))
        # routing over the whole batch, bit-exact on identical logits
        if c["gate"] == "shared":
            idx, g, p = oracle.compute_gates_shared(logits, c["ns"], c["k"])
        else:
            idx, g, p = oracle.compute_gates_topk(logits, c["k"])
        counts, offsets, perm = oracle.bucket(idx, E)
        assert np.array_equal(res["indices"], idx)
        assert np.array_equal(res["gates"].view(np.uint32), g.view(np.uint32))
        assert np.array_equal(res["probs"].view(np.uint32), p.view(np.uint32))
        assert np.array_equal(res["counts"], counts) and np.array_equal(res["offsets"], offsets)
        assert np.array_equal(res["perm"][: offsets[-1]], perm)
        # size-independent properties
        assert int(res["counts"].sum()) == T * kt
        assert np.array_equal(np.concatenate([[0], np.cumsum(res["counts"])]), res["offsets"])
        assert np.array_equal(np.sort(res["perm"][: offsets[-1]]), np.arange(T * kt))
        # losses: Switch + z over the whole batch
        ref_loss = np.float32(oracle.switch_loss(idx, p, 0.01) + oracle.z_loss(logits, 0.001))
        assert abs(loss - ref_loss) <= 1e-5 * max(1.0, abs(float(ref_loss))), (loss, ref_loss)
        assert abs(res["mean_entropy"] - oracle.mean_entropy(p)) <= 1e-5 * max(1.0, float(oracle.mean_entropy(p)))
        # layer output on a token sample
        toks = np.linspace(0, T - 1, 48).astype(np.int64)
        used = sorted(set(int(e) for e in idx[toks].ravel() if e > 0))
        ex = [None] * E
        for e1 in used:
            ex[e1 - 1] = f32_weights(oracle, host, e1 - 1, c["wdtype"])
        for e in range(E):
            if ex[e] is None:  # never routed to by the sample, so never read: any expert's arrays stand in
                ex[e] = ex[used[0] - 1]
        ref_out, _, aux = oracle.moe_forward(xf[toks], wr, ex, gate=c["gate"], k=c["k"], num_shared=c["ns"],
                                             expert_type=c["etype"], act=c["act"], logits=logits[toks])
        assert np.array_equal(aux["idx"], idx[toks])
        err = rel_err(out[toks], ref_out)
        print(f"{name}: sampled relative error {err:.3e}", flush=True)
        assert err <= TOL[c["wdtype"]], err
    finally:
        dev.close()
