"""Pins the CPU oracle (oracle/moe_oracle.c + moe_oracle.py) before it is
trusted as the checker of the HIP path.

The reference (MixtureOfExperts.jl) holds no numeric golden vectors (its tests
are unseeded invariant checks, test_moeLlama2_integration.jl), so each oracle
function is pinned by closed forms, brute force with a different algorithm,
crafted exact ties (tests/golden/routing_cases.json) and an independent numpy
float64 restatement.
"""
import itertools
import json
import math
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def isless_sort_key(p):
    """Julia isless order as a sortable tuple (NaN largest)."""
    return (1, 0.0) if math.isnan(p) else (0, p)


# ---- softmax / top-k ---------------------------------------------------------

def test_uniform_logits_closed_form(oracle):
    # all-equal logits: p = 1/E exactly, indices 1..k (ties to the lower index),
    # gates p/(p+...+p) = 1/k for k in {1,2,4}
    for E in (4, 8, 64, 128):
        for k in (1, 2, 4):
            lg = np.full((3, E), 0.37, np.float32)
            idx, g, p = oracle.compute_gates_topk(lg, k)
            assert np.all(p == np.float32(1.0) / np.float32(E))
            assert np.all(idx == np.arange(1, k + 1))
            assert np.all(g == np.float32(1.0) / np.float32(k))


def test_k1_gate_is_exactly_one(oracle):
    rng = np.random.default_rng(1)
    lg = rng.standard_normal((257, 16)).astype(np.float32)
    idx, g, p = oracle.compute_gates_topk(lg, 1)
    assert np.all(g == np.float32(1.0))
    assert np.all(idx[:, 0] == np.argmax(lg, axis=1) + 1)


def test_topk_brute_force(oracle):
    # brute force: full stable sort by (isless desc, index asc) vs the
    # oracle's k-pass selection, over random and tie-heavy inputs
    rng = np.random.default_rng(2)
    for trial in range(300):
        E = int(rng.integers(1, 10))
        k = int(rng.integers(1, E + 1))
        lg = rng.integers(-2, 3, size=(4, E)).astype(np.float32) if trial % 2 else \
            rng.standard_normal((4, E)).astype(np.float32)
        idx, g, p = oracle.compute_gates_topk(lg, k)
        for t in range(4):
            order = sorted(range(E), key=lambda i: (tuple(-v for v in isless_sort_key(float(p[t, i]))), i))
            assert list(idx[t] - 1) == order[:k]
            # all k-subsets: the chosen one has the largest sorted prob vector
            best = max(itertools.combinations(range(E), k),
                       key=lambda c: sorted((float(p[t, i]) for i in c), reverse=True))
            assert sorted(float(p[t, i]) for i in best) == sorted(float(p[t, i - 1]) for i in idx[t])


def test_topk_many_experts_and_slots_sorted_order(oracle):
    # up to 512 experts and 16 slots: the k-pass selection equals the head of
    # a stable sort by (isless desc, index asc) (numpy lexsort), with ties;
    # the gates are p / (sequential slot-order sum), and SharedExpertGating's
    # routed slots are the same top-k over rows ns+1..E
    rng = np.random.default_rng(12)
    for E, k in ((129, 16), (300, 9), (512, 16), (512, 1)):
        for ties in (False, True):
            lg = (rng.integers(-2, 3, size=(40, E)) if ties else rng.standard_normal((40, E))).astype(np.float32)
            idx, g, p = oracle.compute_gates_topk(lg, k)
            keys = np.array([[isless_sort_key(float(v)) for v in row] for row in p])
            for t in range(40):
                order = np.lexsort((np.arange(E), -keys[t][:, 1], -keys[t][:, 0]))
                assert np.array_equal(idx[t] - 1, order[:k])
                sel = p[t, idx[t] - 1]
                s = sel[0]
                for v in sel[1:]:
                    s = np.float32(s + v)
                assert np.array_equal(g[t], (sel / s).astype(np.float32))
            si, sg, sp = oracle.compute_gates_shared(lg, 1, min(k, E - 1))
            ri, _, _ = oracle.compute_gates_topk(lg[:, 1:], min(k, E - 1))
            assert np.array_equal(si[:, 1:], ri + 1) and np.all(si[:, 0] == 1)


def test_softmax_matches_float64(oracle):
    # independent restatement: float64 softmax; oracle within 2 ulp-ish
    rng = np.random.default_rng(3)
    for E in (8, 66, 128):
        lg = (rng.standard_normal((200, E)) * 3).astype(np.float32)
        p = oracle.softmax(lg)
        l64 = lg.astype(np.float64)
        e = np.exp(l64 - l64.max(axis=1, keepdims=True))
        p64 = e / e.sum(axis=1, keepdims=True)
        assert np.max(np.abs(p - p64) / np.maximum(p64, 1e-30)) < 4e-7 * E ** 0.5
        # rows sum to 1 within float32 rounding
        assert np.allclose(p.astype(np.float64).sum(axis=1), 1.0, atol=1e-6)


def test_topk_agrees_with_float64_away_from_ties(oracle):
    rng = np.random.default_rng(4)
    lg = rng.standard_normal((2000, 8)).astype(np.float32)
    idx, g, p = oracle.compute_gates_topk(lg, 2)
    l64 = lg.astype(np.float64)
    order = np.argsort(-l64, axis=1, kind="stable")
    srt = -np.sort(-l64, axis=1)
    clear = (srt[:, 1] - srt[:, 2]) > 1e-5
    assert np.all(idx[clear] - 1 == order[clear, :2])
    # reference test: gates sum to 1 (test_moeLlama2_integration.jl:83, atol 1e-6)
    assert np.allclose(g.astype(np.float64).sum(axis=1), 1.0, atol=1e-6)
    assert np.all((idx >= 1) & (idx <= 8))
    assert np.all(idx[:, 0] != idx[:, 1])


def test_golden_routing_cases(oracle):
    with open(os.path.join(GOLDEN, "routing_cases.json")) as f:
        cases = json.load(f)
    assert len(cases) >= 8
    for c in cases:
        lg = np.array(c["logits"], dtype=np.float32)
        if c.get("num_shared", 0):
            idx, g, p = oracle.compute_gates_shared(lg, c["num_shared"], c["k"])
        else:
            idx, g, p = oracle.compute_gates_topk(lg, c["k"])
        assert idx.tolist() == c["indices"], c["name"]
        if "gates" in c:
            assert g.tolist() == c["gates"], c["name"]
        if "probs" in c:
            assert p.tolist() == c["probs"], c["name"]


def test_nonfinite_logits(oracle):
    # +Inf logit: NNlib's branch gives p = 1 for the +Inf entries (shared equally)
    lg = np.array([[0.0, np.inf, 1.0, np.inf]], np.float32)
    idx, g, p = oracle.compute_gates_topk(lg, 2)
    assert p.tolist() == [[0.0, 0.5, 0.0, 0.5]]
    assert idx.tolist() == [[2, 4]]
    # NaN logit: the sum becomes NaN so every prob is NaN; all NaNs tie under
    # isless, so the lowest indices win
    lg = np.array([[0.0, np.nan, 1.0, 2.0]], np.float32)
    idx, g, p = oracle.compute_gates_topk(lg, 2)
    assert np.all(np.isnan(p))
    assert idx.tolist() == [[1, 2]]


# ---- shared gating ----------------------------------------------------------

def test_shared_gating_closed_form(oracle):
    # SharedExpertGating(2, TopKGating(6), 66) on uniform logits
    lg = np.zeros((5, 66), np.float32)
    idx, g, p = oracle.compute_gates_shared(lg, 2, 6)
    assert idx.tolist() == [[1, 2, 3, 4, 5, 6, 7, 8]] * 5
    assert np.all(g[:, :2] == np.float32(1.0) / np.float32(8))
    # routed gate 1/6 scaled by (1 - 2/8) in Float64, stored Float32
    assert np.all(g[:, 2:] == np.float32(np.float64(np.float32(1.0) / np.float32(6)) * 0.75))
    assert np.all(p[:, :2] == np.float32(1.0) / np.float32(66))
    assert np.all(p[:, 2:] == np.float32(np.float64(np.float32(1.0) / np.float32(64)) * (1 - 2 / 66)))


# ---- bucketing / capacity -----------------------------------------------------

def test_bucket_is_stable_sort(oracle):
    rng = np.random.default_rng(5)
    for _ in range(50):
        T, E = int(rng.integers(1, 60)), int(rng.integers(1, 12))
        k = int(rng.integers(1, min(E, 4) + 1))
        idx = np.stack([rng.permutation(E)[:k] + 1 for _ in range(T)]).astype(np.int32)
        if rng.random() < 0.5:  # some dropped entries
            idx[rng.random(idx.shape) < 0.2] = 0
        counts, offsets, perm = oracle.bucket(idx, E)
        entries = [(int(idx[t, j]), t, j) for t in range(T) for j in range(k) if idx[t, j] > 0]
        expect = [t * k + j for (e, t, j) in sorted(entries)]
        assert perm.tolist() == expect
        assert counts.sum() == len(entries) == offsets[-1]
        assert offsets.tolist() == [0] + np.cumsum(counts).tolist()


def test_capacity_matches_loop(oracle):
    # restated loop of apply_capacity_constraint in plain Python (moe_layer.jl:221-248)
    rng = np.random.default_rng(6)
    for _ in range(30):
        T, E, k = int(rng.integers(1, 80)), int(rng.integers(2, 9)), 2
        lg = rng.standard_normal((T, E)).astype(np.float32)
        lg[:, 0] += 2.0  # overload expert 1
        idx, g, _ = oracle.compute_gates_topk(lg, k)
        cf = float(rng.choice([0.5, 1.0, 1.25]))
        i2, g2, dropped = oracle.capacity(idx, g, E, cf)
        cap = math.ceil(np.float32(np.float32(cf) * np.float32(T)) / np.float32(E))
        cnt = [0] * (E + 1)
        ei, eg, nd = idx.copy(), g.copy(), 0
        for t in range(T):
            for j in range(k):
                e = ei[t, j]
                if e > 0:
                    if cnt[e] >= cap:
                        ei[t, j] = 0
                        eg[t, j] = 0
                        nd += 1
                    else:
                        cnt[e] += 1
            s = np.float32(eg[t, 0])
            for j in range(1, k):
                s = np.float32(s + eg[t, j])
            if s > 0:
                eg[t] = (eg[t] / s).astype(np.float32)
        assert i2.tolist() == ei.tolist()
        assert g2.tolist() == eg.tolist()
        assert dropped == nd


def test_capacity_keeps_the_head_of_each_stable_segment(oracle):
    # An independent characterisation of apply_capacity_constraint: bucket the
    # uncapped routing (stable: tokens ascending inside each expert); the
    # entries kept are exactly the first min(count_e, cap) of expert e's
    # segment, every other entry becomes (0, 0), and each token's surviving
    # gates are its original gates over their slot-order sum.
    rng = np.random.default_rng(9)
    for _ in range(40):
        T, E = int(rng.integers(1, 120)), int(rng.integers(2, 12))
        k = int(rng.integers(1, min(E, 4) + 1))
        lg = rng.standard_normal((T, E)).astype(np.float32)
        lg[:, int(rng.integers(0, E))] += 1.5
        idx, g, _ = oracle.compute_gates_topk(lg, k)
        cf = float(rng.choice([0.25, 0.5, 1.0, 1.25, 2.0]))
        i2, g2, dropped = oracle.capacity(idx, g, E, cf)
        cap = math.ceil(np.float32(np.float32(cf) * np.float32(T)) / np.float32(E))
        counts, offsets, perm = oracle.bucket(idx, E)
        keep = np.zeros(T * k, bool)
        for e in range(E):
            seg = perm[offsets[e]:offsets[e + 1]]
            keep[seg[:cap]] = True
        kept = keep.reshape(T, k)
        assert np.array_equal(i2 != 0, kept)
        assert np.array_equal(i2[kept], idx[kept])
        assert np.all(g2[~kept] == 0)
        assert dropped == int((~kept).sum())
        for t in range(T):
            s = np.float32(0)
            for j in range(k):
                if kept[t, j]:
                    s = np.float32(s + g[t, j])
            if s > 0:
                assert np.array_equal(g2[t, kept[t]], (g[t, kept[t]] / s).astype(np.float32))


# ---- losses / stats ---------------------------------------------------------

def test_switch_loss_closed_forms(oracle):
    # balanced assignments and uniform probs: loss = alpha
    E, T, k = 8, 64, 2
    idx = np.array([[(2 * t) % E + 1, (2 * t + 1) % E + 1] for t in range(T)], np.int32)
    p = np.full((T, E), 1.0 / E, np.float32)
    assert abs(oracle.switch_loss(idx, p, 0.01) - 0.01) < 1e-9
    # everything on expert 1 with P_1 = 1: loss = alpha * N * 1 * 1
    idx = np.ones((T, 1), np.int32)
    p = np.zeros((T, E), np.float32)
    p[:, 0] = 1
    assert oracle.switch_loss(idx, p, 0.01) == np.float32(0.01) * np.float32(E)
    # dropped (0) entries count in length(indices) but not in f
    idx = np.array([[1, 0]] * T, np.int32)
    assert oracle.switch_loss(idx, p, 0.01) == np.float32(0.01) * np.float32(E) * np.float32(0.5)


def test_z_loss_closed_form(oracle):
    for E in (8, 64, 128):
        z = oracle.z_loss(np.zeros((100, E), np.float32), 0.001)
        assert abs(z - 0.001 * math.log(E) ** 2) < 2e-6 * 0.001 * math.log(E) ** 2  # float32 rounding
    # shift invariance of logsumexp minus shift: logits c -> lse = c + ln E
    z = oracle.z_loss(np.full((10, 8), 3.0, np.float32), 1.0)
    assert abs(z - (3.0 + math.log(8)) ** 2) < 1e-4


def test_mean_entropy_closed_form(oracle):
    E = 8
    p = np.full((50, E), 1.0 / E, np.float32)
    h = oracle.mean_entropy(p)
    expect = -E * (1 / E) * math.log(1 / E + 1e-8)
    assert abs(h - expect) < 1e-6
    # one-hot probs: entropy = -log(1 + 1e-8) ~ -1e-8
    p = np.zeros((5, E), np.float32)
    p[:, 3] = 1
    assert abs(oracle.mean_entropy(p)) < 1e-7


# ---- expert FFN / combine ------------------------------------------------------

def test_gated_expert_equals_dense_llama_ffn(oracle):
    # the reference's known-answer check (test_moeLlama2_integration.jl:132-164):
    # gated expert == dense Llama FFN w2(silu(w1 x) * (w3 x)), max diff < 1e-5
    rng = np.random.default_rng(7)
    dim, hid = 64, 160
    x = rng.standard_normal(dim).astype(np.float32)
    w1 = (rng.standard_normal((dim, hid)) * 0.02).astype(np.float32)  # Llama layout (in, out)
    w2 = (rng.standard_normal((hid, dim)) * 0.02).astype(np.float32)
    w3 = (rng.standard_normal((dim, hid)) * 0.02).astype(np.float32)
    hb1 = w1.T @ x
    hb2 = w3.T @ x
    h = hb1 * (np.float32(1) / (np.float32(1) + np.exp(-hb1))) * hb2
    dense = w2.T @ h
    y = oracle.gated_expert(x[None, :], w1.T, w2.T, w3.T, oracle.act_silu)[0]
    assert np.max(np.abs(dense - y)) < 1e-5
    # and against float64
    x64 = x.astype(np.float64)
    g = w1.T.astype(np.float64) @ x64
    y64 = w2.T.astype(np.float64) @ (g / (1 + np.exp(-g)) * (w3.T.astype(np.float64) @ x64))
    assert np.max(np.abs(y - y64)) / np.max(np.abs(y64)) < 1e-5


def test_moe_forward_matches_float64_loops(oracle):
    # full forward vs a float64 per-token restatement (slot loop, no bucketing)
    rng = np.random.default_rng(8)
    T, D, H, E, k = 40, 32, 48, 6, 2
    x = rng.standard_normal((T, D)).astype(np.float32)
    wr = (rng.standard_normal((E, D)) * 0.3).astype(np.float32)
    ex = [dict(w1=(rng.standard_normal((H, D)) * 0.2).astype(np.float32),
               w2=(rng.standard_normal((D, H)) * 0.2).astype(np.float32),
               w3=(rng.standard_normal((H, D)) * 0.2).astype(np.float32)) for _ in range(E)]
    out, loss, aux = oracle.moe_forward(x, wr, ex, k=k, training=True)
    idx, g = aux["idx"], aux["gates"]
    ref = np.zeros((T, D))
    for t in range(T):
        for j in range(k):
            e = idx[t, j] - 1
            w = ex[e]
            xv = x[t].astype(np.float64)
            a = w["w1"].astype(np.float64) @ xv
            hh = a / (1 + np.exp(-a)) * (w["w3"].astype(np.float64) @ xv)
            ref[t] += g[t, j] * (w["w2"].astype(np.float64) @ hh)
    assert np.max(np.abs(out - ref)) / np.max(np.abs(ref)) < 1e-5
    assert loss >= 0  # reference test: balance_loss >= 0 (test_moeLlama2_integration.jl:127)


def test_combine_order_is_ascending_expert(oracle):
    # three entries per token: fl((a + b) + c) in expert order differs from slot order
    y = np.array([[1.0], [1e8], [-1e8]], np.float32)
    # token 0 entries: slot0 -> expert 3, slot1 -> expert 1, slot2 -> expert 2
    idx = np.array([[3, 1, 2]], np.int32)
    gates = np.array([[1.0, 1.0, 1.0]], np.float32)
    counts, offsets, perm = oracle.bucket(idx, 3)
    yp = np.zeros((3, 1), np.float32)
    yp[0] = y[1]  # expert 1 row
    yp[1] = y[2]  # expert 2 row
    yp[2] = y[0]  # expert 3 row
    out = np.zeros((1, 1), np.float32)
    import ctypes
    oracle._lib().oracle_combine(yp.ctypes.data, perm.ctypes.data, 3, gates.ctypes.data, 3, 1, 1,
                                 out.ctypes.data)
    assert out[0, 0] == np.float32(np.float32(1e8 + -1e8) + 1.0)  # (e1 + e2) + e3 = 1


# ---- activations and StandardExpert -------------------------------------------

def test_gelu_is_the_tanh_form_of_the_erf_gelu(oracle):
    # Mathematics of GELU, independent of the oracle's formula:
    #  * odd part: gelu(x) - gelu(-x) = x for both the erf GELU and its tanh
    #    approximation (x Phi(x) + x Phi(-x) = x), so a wrong 0.5 or a wrong
    #    sign of the odd argument fails;
    #  * gelu(0) = 0 and gelu'(0) = 1/2;
    #  * closeness to the exact 0.5 x (1 + erf(x / sqrt 2)) (stdlib math.erf):
    #    the tanh form with sqrt(2/pi) and 0.044715 deviates from it by at most
    #    4.73e-4, reached near |x| = 2.70; the erf form itself (deviation 0)
    #    and a wrong constant (the deviation moves) both fail the window.
    x = np.linspace(-8, 8, 160001).astype(np.float32)
    g = oracle.act_gelu(x)
    assert g.dtype == np.float32
    odd = g.astype(np.float64) - oracle.act_gelu(-x).astype(np.float64) - x.astype(np.float64)
    assert np.max(np.abs(odd) / np.maximum(np.abs(x), 1.0)) < 4e-7
    assert oracle.act_gelu(np.float32(0.0)) == 0.0
    h = np.float32(1e-3)
    assert abs((float(oracle.act_gelu(h)) - float(oracle.act_gelu(-h))) / (2 * float(h)) - 0.5) < 1e-3
    exact = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in x.astype(np.float64)])
    dev = np.abs(g.astype(np.float64) - exact)
    assert 4.6e-4 < dev.max() < 4.9e-4
    assert 2.6 < abs(float(x[dev.argmax()])) < 2.8
    # far tails: x for large positive x, 0 for large negative x
    assert oracle.act_gelu(np.float32(8.0)) == np.float32(8.0)
    assert abs(float(oracle.act_gelu(np.float32(-8.0)))) < 1e-10


def test_relu_and_identity_closed_forms(oracle):
    x = np.array([-np.inf, -3.5, -1e-30, -0.0, 0.0, 1e-30, 2.25, np.inf], np.float32)
    r = oracle.act_relu(x)
    assert r.tolist() == [0.0, 0.0, 0.0, 0.0, 0.0, np.float32(1e-30), 2.25, np.inf]
    assert np.array_equal(oracle.act_identity(x), x)
    # silu(x) = x sigmoid(x): silu(0) = 0, silu(x) - silu(-x) = x, silu(x) -> x
    s = oracle.act_silu(np.linspace(-30, 30, 601).astype(np.float32)).astype(np.float64)
    xs = np.linspace(-30, 30, 601)
    assert s[300] == 0.0
    assert np.max(np.abs(s - s[::-1] - xs) / np.maximum(np.abs(xs), 1.0)) < 4e-7
    assert abs(s[-1] - 30.0) < 1e-10


def test_standard_expert_with_permutation_weights(oracle):
    # W1 and W2 as scaled permutation matrices (not symmetric, so a transposed
    # weight fails): the expert is an index gather, computed here with no
    # matrix product: y[o] = s2 act(s1 x[p1[p2[o]]] + b1[p2[o]]) + b2[o].
    # relu with biases that flip signs catches b1 applied after the
    # activation; s2 != 1 catches b2 added before W2.
    rng = np.random.default_rng(31)
    n = 12
    p1, p2 = rng.permutation(n), rng.permutation(n)
    s1, s2 = np.float32(0.5), np.float32(-2.0)
    w1 = np.zeros((n, n), np.float32)
    w1[np.arange(n), p1] = s1      # (W1 x)[i] = s1 x[p1[i]]
    w2 = np.zeros((n, n), np.float32)
    w2[np.arange(n), p2] = s2      # (W2 h)[o] = s2 h[p2[o]]
    b1 = rng.standard_normal(n).astype(np.float32)
    b2 = rng.standard_normal(n).astype(np.float32)
    x = rng.standard_normal((5, n)).astype(np.float32)
    for name in ("relu", "gelu", "silu", "identity"):
        act = oracle.ACTS[name]
        y = oracle.standard_expert(x, w1, w2, b1, b2, act)
        hid = act((s1 * x[:, p1] + b1).astype(np.float32))
        expect = (s2 * hid[:, p2] + b2).astype(np.float32)
        assert np.array_equal(y, expect), name
    # zero biases (the reference's init, standard.jl:30-31) and missing biases agree
    y0 = oracle.standard_expert(x, w1, w2, np.zeros(n, np.float32), np.zeros(n, np.float32), oracle.act_relu)
    assert np.array_equal(y0, oracle.standard_expert(x, w1, w2, None, None, oracle.act_relu))


def test_standard_moe_forward_matches_float64_loops(oracle):
    # forward_standard with StandardExperts (GELU) against a float64 per-token
    # restatement of the slot loop: W2 act(W1 x + b1) + b2 with the erf-free
    # tanh GELU written from its definition 0.5 v (1 + tanh(sqrt(2/pi)(v +
    # 0.044715 v^3))) in float64
    rng = np.random.default_rng(32)
    T, D, H, Dout, E = 30, 24, 40, 20, 5
    x = rng.standard_normal((T, D)).astype(np.float32)
    wr = (rng.standard_normal((E, D)) * 0.3).astype(np.float32)
    ex = [dict(w1=(rng.standard_normal((H, D)) * 0.2).astype(np.float32),
               w2=(rng.standard_normal((Dout, H)) * 0.2).astype(np.float32),
               b1=(rng.standard_normal(H) * 0.5).astype(np.float32),
               b2=(rng.standard_normal(Dout) * 0.5).astype(np.float32)) for _ in range(E)]
    for gate, k in (("switch", 1), ("topk", 2)):
        out, _, aux = oracle.moe_forward(x, wr, ex, gate=gate, k=k, expert_type="standard", act="gelu")
        ref = np.zeros((T, Dout))
        for t in range(T):
            for j in range(aux["idx"].shape[1]):
                w = ex[aux["idx"][t, j] - 1]
                v = w["w1"].astype(np.float64) @ x[t].astype(np.float64) + w["b1"]
                hid = 0.5 * v * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (v + 0.044715 * v ** 3)))
                ref[t] += float(aux["gates"][t, j]) * (w["w2"].astype(np.float64) @ hid + w["b2"])
        assert np.max(np.abs(out - ref)) / np.max(np.abs(ref)) < 1e-5, gate


# ---- forward_with_shared_experts (num_shared_experts > 0) ----------------------

def _shared_case(rng, T, D, H, E, scale=0.2):
    x = rng.standard_normal((T, D)).astype(np.float32)
    ex = [dict(w1=(rng.standard_normal((H, D)) * scale).astype(np.float32),
               w2=(rng.standard_normal((D, H)) * scale).astype(np.float32),
               w3=(rng.standard_normal((H, D)) * scale).astype(np.float32)) for _ in range(E)]
    return x, ex


def test_shared_experts_identical_experts_give_the_expert(oracle):
    # every expert the same FFN: shared = sum_i y/ns = y, routed = sum_j g_j y
    # = y (gates sum to 1), so out = 0.5 y + 0.5 y = y; a wrong blend weight,
    # a sum instead of the mean over the shared experts or ungated routed
    # outputs all fail this
    rng = np.random.default_rng(21)
    T, D, H, E = 24, 16, 40, 6
    x, ex = _shared_case(rng, T, D, H, 1)
    ex = [ex[0]] * E
    for ns, k in ((1, 2), (2, 2), (3, 1), (2, 4)):
        wr = (rng.standard_normal((E - ns, D)) * 0.5).astype(np.float32)
        out, _, aux = oracle.moe_forward_shared_experts(x, wr, ex, ns, k=k)
        a = ex[0]["w1"].astype(np.float64) @ x.T.astype(np.float64)
        h = a / (1 + np.exp(-a)) * (ex[0]["w3"].astype(np.float64) @ x.T.astype(np.float64))
        y64 = (ex[0]["w2"].astype(np.float64) @ h).T
        assert np.max(np.abs(out - y64)) / np.max(np.abs(y64)) < 1e-5, (ns, k)
        assert aux["idx"].shape == (T, k) and aux["idx"].min() >= ns + 1 and aux["idx"].max() <= E


def test_shared_experts_zero_shared_is_half_the_standard_forward(oracle):
    # shared experts with w2 = 0 output zeros: out = 0.5f0 * forward_standard
    # over the routed experts with the same router, bit for bit
    rng = np.random.default_rng(22)
    T, D, H, E, ns = 30, 16, 24, 7, 2
    x, ex = _shared_case(rng, T, D, H, E)
    for i in range(ns):
        ex[i] = dict(ex[i], w2=np.zeros_like(ex[i]["w2"]))
    wr = (rng.standard_normal((E - ns, D)) * 0.5).astype(np.float32)
    out, _, _ = oracle.moe_forward_shared_experts(x, wr, ex, ns, k=2)
    std, _, _ = oracle.moe_forward(x, wr, ex[ns:], k=2)
    assert np.array_equal(out, (np.float32(0.5) * std).astype(np.float32))


def test_shared_experts_zero_routed_is_half_the_shared_mean(oracle):
    # routed experts with w2 = 0: out = 0.5 * mean of the ns shared outputs
    # (against float64, ns = 3 so 1/ns is inexact)
    rng = np.random.default_rng(23)
    T, D, H, E, ns = 20, 16, 24, 6, 3
    x, ex = _shared_case(rng, T, D, H, E)
    for i in range(ns, E):
        ex[i] = dict(ex[i], w2=np.zeros_like(ex[i]["w2"]))
    wr = (rng.standard_normal((E - ns, D)) * 0.5).astype(np.float32)
    out, _, _ = oracle.moe_forward_shared_experts(x, wr, ex, ns, k=2)
    ref = np.zeros((T, D))
    for i in range(ns):
        a = ex[i]["w1"].astype(np.float64) @ x.T.astype(np.float64)
        h = a / (1 + np.exp(-a)) * (ex[i]["w3"].astype(np.float64) @ x.T.astype(np.float64))
        ref += (ex[i]["w2"].astype(np.float64) @ h).T / ns
    ref *= 0.5
    assert np.max(np.abs(out - ref)) / np.max(np.abs(ref)) < 1e-5


def test_shared_experts_switch_loss_counts_shifted_ids(oracle):
    # the loss sees the router indices shifted by ns against the E - ns
    # probability rows (src/core/moe_layer.jl:172, 182): ids above E - ns are
    # not counted.  E = 4, ns = 2: every shifted id is 3 or 4 > N = 2, so the
    # Switch loss is exactly 0.  E = 5, ns = 1, k = 2: brute-force count of
    # shifted ids 2..4 against the probability means.
    rng = np.random.default_rng(24)
    x, ex = _shared_case(rng, 16, 8, 8, 4)
    wr = rng.standard_normal((2, 8)).astype(np.float32)
    _, loss, aux = oracle.moe_forward_shared_experts(x, wr, ex, 2, k=1, training=True, z_weight=0.0)
    assert loss == 0.0 and aux["switch_loss"] == 0.0
    x, ex = _shared_case(rng, 33, 8, 8, 5)
    wr = rng.standard_normal((4, 8)).astype(np.float32)
    alpha = 0.01
    _, loss, aux = oracle.moe_forward_shared_experts(x, wr, ex, 1, k=2, training=True, alpha=alpha,
                                                     z_weight=0.0)
    N, T, k = 4, 33, 2
    f = [sum(1 for t in range(T) for j in range(k) if aux["idx"][t, j] == e + 1) / (k * T) for e in range(N)]
    P = [float(np.mean(aux["probs"][:, e].astype(np.float64))) for e in range(N)]
    ref = alpha * N * sum(fe * pe for fe, pe in zip(f, P))
    assert f[0] == 0.0 and sum(f) < 1.0  # shared id 1 never counted, id 5 dropped
    assert abs(float(loss) - ref) < 1e-7
    # and the z-loss is the standard one over the router logits
    _, loss_z, aux_z = oracle.moe_forward_shared_experts(x, wr, ex, 1, k=2, training=True, alpha=alpha,
                                                         z_weight=0.001)
    assert aux_z["z_loss"] == oracle.z_loss(aux_z["logits"], 0.001)
    assert loss_z == np.float32(aux_z["switch_loss"] + aux_z["z_loss"])


def test_shared_experts_expert_choice_empty_entries_count_as_id_ns(oracle):
    # ExpertChoiceGating under shared experts: the (C, T) index matrix's empty
    # entries are shifted to id ns like every other entry (:172), so the Switch
    # loss counts them for expert ns when ns <= E - ns.  E = 5, ns = 1, four
    # routed experts, T = 10, capacity_factor 1.0: C = ceil(10 / 4) = 3 rows,
    # brute-force f over the shifted matrix against the probability means; the
    # output ignores the empty entries (process_expert_forward! skips id 0).
    rng = np.random.default_rng(27)
    T, D, H, E, ns = 10, 8, 8, 5, 1
    x, ex = _shared_case(rng, T, D, H, E)
    wr = rng.standard_normal((E - ns, D)).astype(np.float32)
    alpha = 0.01
    out, loss, aux = oracle.moe_forward_shared_experts(x, wr, ex, ns, gate="expert_choice", gate_param=1.0,
                                                       training=True, alpha=alpha, z_weight=0.0)
    C, N = 3, E - ns
    assert aux["idx"].shape == (T, C)
    empty = int(np.sum(aux["routed_idx"] == 0))
    assert empty > 0 and np.sum(aux["idx"] == ns) == empty
    f = [sum(1 for t in range(T) for j in range(C) if aux["idx"][t, j] == e + 1) / (C * T) for e in range(N)]
    assert f[ns - 1] == empty / (C * T)
    P = [float(np.mean(aux["probs"][:, e].astype(np.float64))) for e in range(N)]
    assert abs(float(loss) - alpha * N * sum(fe * pe for fe, pe in zip(f, P))) < 1e-7
    # routed output = the forward_standard of the routed experts on the same gate
    std, _, _ = oracle.moe_forward(x, wr, ex[ns:], gate="expert_choice", gate_param=1.0, logits=aux["logits"])
    assert np.array_equal(aux["routed"], std)


def test_shared_experts_aux_free_updates_over_shifted_ids(oracle):
    # AuxiliaryFreeLoss under shared experts: the gate runs on the plain
    # logits (no bias) and update_bias! counts the shifted ids over a bias of
    # all E experts.  E = 3, ns = 1, k = 1, a router that sends every token to
    # routed expert 1 (shifted id 2): counts (0, T, 0), target T / 3, so the
    # gradient is (-1/3, 2/3, -1/3) and, from zero momentum, the bias moves by
    # -lr (1 - m) grad (mean 0, so the centring step leaves it); the bias
    # (0, -100, 100), which would send every token to id 3 if the gate saw
    # it, does not change the routing.
    rng = np.random.default_rng(28)
    T, D, H, E, ns = 12, 8, 8, 3, 1
    x, ex = _shared_case(rng, T, D, H, E)
    lg = np.tile(np.array([[4.0, -4.0]], np.float32), (T, 1))
    lr, m = 0.01, 0.9
    b0 = np.array([0.0, -100.0, 100.0], np.float32)
    st = dict(bias=b0.copy(), mom=np.zeros(3, np.float32), lr=lr, momentum=m, update_freq=1, counter=0,
              use_comp=True, cw=0.001)
    _, loss, aux = oracle.moe_forward_shared_experts(x, None, ex, ns, k=1, training=True, z_weight=0.0,
                                                     logits=lg, aux_free=st)
    assert np.all(aux["idx"] == 2)
    g = np.array([-1.0 / 3.0, 2.0 / 3.0, -1.0 / 3.0])
    assert np.allclose(st["bias"], b0 - lr * (1 - m) * g, rtol=0, atol=3e-5)
    assert np.allclose(st["mom"], (1 - m) * g, rtol=0, atol=1e-7)
    assert st["counter"] == 1
    # complementary loss: cw * Switch(1) over the shifted ids (id 2 of N = 2)
    p = oracle.softmax(lg)
    assert abs(float(loss) - 0.001 * 1.0 * 2 * 1.0 * float(np.mean(p[:, 1].astype(np.float64)))) < 1e-9


def test_shared_experts_with_shared_expert_gating(oracle):
    # SharedExpertGating(g, TopKGating(k), E - ns) under the layer's ns shared
    # experts: the gate's own shared ids 1..g and its routed ids are shifted
    # by ns; the gate's slot gates are those of compute_gates_shared on the
    # same logits (1/(g + k) and the scaled top-k)
    rng = np.random.default_rng(29)
    T, D, H, E, ns, g, k = 20, 8, 8, 9, 2, 1, 2
    x, ex = _shared_case(rng, T, D, H, E)
    wr = rng.standard_normal((E - ns, D)).astype(np.float32)
    _, _, aux = oracle.moe_forward_shared_experts(x, wr, ex, ns, gate="shared", gate_num_shared=g, k=k)
    i0, g0, _ = oracle.compute_gates_shared(aux["logits"], g, k)
    assert np.array_equal(aux["idx"], i0 + ns) and np.array_equal(aux["gates"], g0)
    assert np.all(aux["idx"][:, 0] == ns + 1)


# ---- SoftMoEGating / ExpertChoiceGating ------------------------------------------

def test_soft_gating_closed_forms(oracle):
    # lambda = 1: the indices of TopKGating; the slot gates are the
    # probabilities of experts 1..k (the reference reads gates[slot, t] of the
    # (E, T) probability matrix), not of the selected experts; lambda = 2
    # flattens the softmax: p = softmax(l / 2)
    rng = np.random.default_rng(26)
    lg = rng.standard_normal((50, 6)).astype(np.float32)
    idx, g, p = oracle.compute_gates_soft(lg, 2, 1.0)
    i2, _, p2 = oracle.compute_gates_topk(lg, 2)
    assert np.array_equal(idx, i2) and np.array_equal(p, p2)
    assert np.array_equal(g, p[:, :2])
    idx, g, p = oracle.compute_gates_soft(lg, 3, 2.0)
    ref = np.exp(lg.astype(np.float64) / 2)
    ref /= ref.sum(axis=1, keepdims=True)
    assert np.max(np.abs(p - ref)) < 1e-6
    assert np.array_equal(g, p[:, :3])


def test_expert_choice_closed_forms(oracle):
    rng = np.random.default_rng(27)
    T, E = 12, 4
    lg = rng.standard_normal((T, E)).astype(np.float32)
    # capacity factor E: capacity T, every expert takes every token, so each
    # token's slots are 1..E and the gates its probabilities
    idx, g, p = oracle.compute_gates_expert_choice(lg, float(E))
    assert idx.shape == (T, T)
    assert np.all(idx[:, :E] == np.arange(1, E + 1)) and np.all(idx[:, E:] == 0)
    assert np.array_equal(g[:, :E], p)
    # capacity 1 (cf = E / T): expert e takes its argmax token
    idx, g, p = oracle.compute_gates_expert_choice(lg, E / T)
    for e in range(E):
        t = int(np.argmax(lg[:, e]))
        assert (e + 1) in idx[t]
    assert int((idx > 0).sum()) == E
    # equal logits: every expert takes the first C tokens (ties to the lower token)
    idx, _, _ = oracle.compute_gates_expert_choice(np.zeros((10, 3), np.float32), 0.9)  # C = ceil(3.0) = 3
    assert np.all(idx[:3, :3] == np.array([1, 2, 3])) and np.all(idx[3:] == 0)
    # brute force on small inputs with ties: the set of (expert, token) pairs
    for trial in range(50):
        T, E = int(rng.integers(1, 9)), int(rng.integers(1, 6))
        cf = float(rng.choice([0.5, 1.0, 1.25, 2.0]))
        lg = rng.integers(-2, 3, size=(T, E)).astype(np.float32)
        idx, _, _ = oracle.compute_gates_expert_choice(lg, cf)
        C = oracle.expert_choice_capacity(T, E, cf)
        chosen = set()
        for e in range(E):
            ranked = sorted(range(T), key=lambda t: (-float(lg[t, e]), t))
            chosen |= {(e + 1, t) for t in ranked[:min(C, T)]}
        got = {(int(idx[t, j]), t) for t in range(T) for j in range(idx.shape[1]) if idx[t, j] > 0}
        expect = set()
        for t in range(T):
            es = sorted(e for e, tt in chosen if tt == t)[:C]
            expect |= {(e, t) for e in es}
        assert got == expect


# ---- convert_to_moe :split ---------------------------------------------------------

def test_split_experts_partition_the_dense_ffn(oracle):
    # the :split experts' hidden units partition the dense FFN's, and silu(0)
    # * 0 = 0, so the sum of the experts' outputs is the dense output
    rng = np.random.default_rng(28)
    dim, hid, E = 24, 50, 8
    w1 = rng.standard_normal((dim, hid)).astype(np.float32)
    w2 = rng.standard_normal((hid, dim)).astype(np.float32)
    w3 = rng.standard_normal((dim, hid)).astype(np.float32)
    x = rng.standard_normal((5, dim)).astype(np.float32)
    dense = oracle.gated_expert(x, w1.T, w2.T, w3.T, oracle.act_silu).astype(np.float64)
    total = np.zeros_like(dense)
    kept = np.zeros(hid, int)
    for e in range(E):
        a, b, c = oracle.split_expert(w1, w2, w3, e, E)
        kept += (np.abs(a).sum(axis=0) > 0).astype(int)
        total += oracle.gated_expert(x, a.T, b.T, c.T, oracle.act_silu)
    assert np.all(kept == 1)  # every hidden unit in exactly one expert
    assert np.max(np.abs(total - dense)) / np.max(np.abs(dense)) < 1e-5


# ---- AuxiliaryFreeLoss ---------------------------------------------------------

def test_aux_free_update_closed_form(oracle):
    # every entry on expert 1 of 4, from momentum 0 and bias 1: total = n,
    # target = n/4, gradient = (0.75, -0.25, -0.25, -0.25); momentum =
    # (1 - 0.9) * gradient; bias = 1 - 0.01 * momentum, then centred (mean 1
    # removed).  A wrong sign, a missing (1 - momentum) factor or a missing
    # centring step fails this.
    idx = np.full((10, 2), 1, np.int32)
    bias = np.ones(4, np.float32)
    mom = np.zeros(4, np.float32)
    oracle.aux_free_update_bias(idx, bias, mom, 0.01, 0.9)
    grad = np.array([0.75, -0.25, -0.25, -0.25])
    assert np.allclose(mom, 0.1 * grad, rtol=1e-6, atol=0)
    assert np.allclose(bias, -0.001 * grad, rtol=1e-4, atol=1e-9)
    assert abs(float(np.sum(bias.astype(np.float64)))) < 2.5e-7  # Float32 rounding of values near 1


def test_aux_free_update_balanced_and_empty(oracle):
    # balanced counts: gradient 0, the momentum decays by `momentum` exactly and
    # the bias moves by -lr * momentum; no entries > 0: nothing changes
    idx = np.array([[1, 2], [3, 4], [2, 1], [4, 3]], np.int32)
    bias = np.zeros(4, np.float32)
    mom = np.array([0.5, -0.5, 0.25, -0.25], np.float32)
    oracle.aux_free_update_bias(idx, bias, mom, 0.01, 0.9)
    assert np.array_equal(mom, (np.float32(0.9) * np.array([0.5, -0.5, 0.25, -0.25], np.float32)))
    assert np.allclose(bias, -0.01 * mom.astype(np.float64), rtol=1e-6)
    b0, m0 = bias.copy(), mom.copy()
    oracle.aux_free_update_bias(np.zeros((3, 2), np.int32), bias, mom, 0.01, 0.9)
    assert np.array_equal(bias, b0) and np.array_equal(mom, m0)


def test_aux_free_forward_regates_on_biased_logits(oracle):
    # a large bias on expert 2 puts it in slot 1 for every token while the
    # probabilities stay those of the plain logits; the update runs every
    # update_freq-th training call; the balance loss is cw * Switch(1)
    rng = np.random.default_rng(25)
    T, D, H, E = 40, 16, 24, 4
    x, ex = _shared_case(rng, T, D, H, E)
    wr = (rng.standard_normal((E, D)) * 0.5).astype(np.float32)
    st = dict(bias=np.array([0, 100, 0, 0], np.float32), mom=np.zeros(E, np.float32), lr=0.01, momentum=0.9,
              update_freq=2, counter=0, use_comp=True, cw=0.001)
    out, loss, aux = oracle.moe_forward(x, wr, ex, k=2, training=True, z_weight=0.0, aux_free=st)
    plain = oracle.moe_forward(x, wr, ex, k=2, training=True, z_weight=0.0)[2]
    assert np.all(aux["idx"][:, 0] == 2)
    assert np.array_equal(aux["probs"], plain["probs"])
    assert st["counter"] == 1 and np.all(st["mom"] == 0)  # first call: no update (freq 2)
    assert loss == np.float32(np.float32(0.001) * oracle.switch_loss(aux["idx"], aux["probs"], 1.0))
    oracle.moe_forward(x, wr, ex, k=2, training=True, z_weight=0.0, aux_free=st)
    assert st["counter"] == 2 and st["mom"][1] > 0 and st["bias"][1] < 100  # expert 2 overloaded: pushed down
    oracle.moe_forward(x, wr, ex, k=2, training=False, aux_free=st)
    assert st["counter"] == 2  # inference calls do not count


# ---- dtype helpers -----------------------------------------------------------

def test_bf16_rounding_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(9)
    a = (rng.standard_normal(10000) * 10 ** rng.uniform(-5, 5, 10000)).astype(np.float32)
    mine = oracle.f32_to_bf16_bits(a)
    ref = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine, ref)


def test_fp8_table_and_quantiser(oracle):
    t = oracle.fp8_e4m3_table()
    assert t[0x7E] == 448.0 and t[0x08] == 2.0 ** -6 and t[0x01] == 2.0 ** -9 and np.isnan(t[0x7F])
    torch = pytest.importorskip("torch")
    if hasattr(torch, "float8_e4m3fn"):
        codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
        ok = ~np.isnan(t)
        assert np.array_equal(codes[ok], t[ok])
    rng = np.random.default_rng(10)
    w = rng.standard_normal((16, 64)).astype(np.float32)
    q, s = oracle.quantize_fp8_rows(w)
    deq = oracle.dequantize_fp8_rows(q, s)
    assert np.max(np.abs(deq - w) / np.abs(w).max(axis=1, keepdims=True)) <= 2.0 ** -4 * 448 / 256 + 1e-6
    # each row's max maps to code 448 (up to the rounding of the fp32 scale)
    assert np.all(np.abs(q & 0x7F).max(axis=1) == 0x7E)
    assert np.allclose(np.abs(deq).max(axis=1), np.abs(w).max(axis=1), rtol=1e-6, atol=0)


def _decode_case(seed, n=6, D=48, H=80, E=8):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, D)).astype(np.float32)
    wr = (rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32)
    ex = [dict(w1=(rng.standard_normal((H, D)) * 0.2).astype(np.float32),
               w2=(rng.standard_normal((D, H)) * 0.2).astype(np.float32),
               w3=(rng.standard_normal((H, D)) * 0.2).astype(np.float32)) for _ in range(E)]
    return x, wr, ex


def test_decode_ffn_matches_float64_loop(oracle):
    # moe_ffn_forward! restated as plain fp64 loops: per token, per slot in order,
    # xb2 += gate * w2 (silu(w1 xb) .* (w3 xb))
    x, wr, ex = _decode_case(40)
    out, idx, gates, logits = oracle.decode_ffn(x, wr, ex, k=2)
    for t in range(x.shape[0]):
        acc = np.zeros(x.shape[1])
        for j in range(idx.shape[1]):
            e = ex[idx[t, j] - 1]
            g = e["w1"].astype(np.float64) @ x[t]
            u = e["w3"].astype(np.float64) @ x[t]
            h = g / (1.0 + np.exp(-g)) * u
            acc += float(gates[t, j]) * (e["w2"].astype(np.float64) @ h)
        assert np.max(np.abs(out[t] - acc)) <= 1e-5 * max(1.0, np.max(np.abs(acc)))
    ref_idx, ref_g, _ = oracle.compute_gates_topk((x @ wr.T).astype(np.float32), 2)
    assert np.array_equal(idx, ref_idx) and np.array_equal(gates, ref_g)


def test_decode_ffn_k1_is_the_expert(oracle):
    # SwitchGating: gate 1.0f0, so xb2 = 0 + 1 * y is the selected expert's output exactly
    x, wr, ex = _decode_case(41)
    out, idx, gates, _ = oracle.decode_ffn(x, wr, ex, gate="switch")
    assert np.all(gates == np.float32(1.0))
    for e in range(len(ex)):
        toks = np.nonzero(idx[:, 0] == e + 1)[0]
        if toks.size:  # the same token batch, so the same sgemm blocking
            y = oracle.gated_expert(x[toks], ex[e]["w1"], ex[e]["w2"], ex[e]["w3"], oracle.silu_inline)
            assert np.array_equal(out[toks], y)


def test_decode_ffn_combines_in_slot_order(oracle):
    # k = 3 with logits that put the experts in slots (6, 2, 4): the fp32 sum
    # ((0 + g1 y6) + g2 y2) + g3 y4 is the result, which expert order would not give
    x, wr, ex = _decode_case(42, n=1)
    logits = np.full((1, 8), -5.0, np.float32)
    logits[0, 5], logits[0, 1], logits[0, 3] = 3.0, 2.9, 2.8
    out, idx, gates, _ = oracle.decode_ffn(x, wr, ex, k=3, logits=logits)
    assert list(idx[0]) == [6, 2, 4]
    ys = [oracle.gated_expert(x, ex[e - 1]["w1"], ex[e - 1]["w2"], ex[e - 1]["w3"], oracle.silu_inline)[0]
          for e in idx[0]]
    slot = np.zeros_like(ys[0])
    for j in range(3):
        slot = (slot + gates[0, j] * ys[j]).astype(np.float32)
    assert np.array_equal(out[0], slot)
    order = np.argsort(idx[0])
    expert = np.zeros_like(ys[0])
    for j in order:
        expert = (expert + gates[0, j] * ys[j]).astype(np.float32)
    assert not np.array_equal(slot, expert)  # the case distinguishes the two orders


def test_logsumexp_rows_closed_forms(oracle):
    # zero logits: lse = ln E; a constant shift c: lse + c; one dominant
    # logit: lse -> that logit; against a float64 restatement on random rows
    E = 7
    z = oracle.logsumexp_rows(np.zeros((3, E), np.float32))
    assert np.allclose(z, np.log(E), rtol=2e-7)
    rng = np.random.default_rng(0)
    lg = rng.standard_normal((50, E)).astype(np.float32)
    a = oracle.logsumexp_rows(lg)
    b = oracle.logsumexp_rows((lg + np.float32(3.0)).astype(np.float32))
    assert np.allclose(b, a + 3.0, rtol=1e-6, atol=1e-6)
    ref = np.log(np.sum(np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True)), 1)) + lg.max(1)
    assert np.allclose(a, ref, rtol=1e-6, atol=1e-6)
    d = np.zeros((1, E), np.float32)
    d[0, 2] = 200.0
    assert oracle.logsumexp_rows(d)[0] == np.float32(200.0)
