"""GPU parity of the routing path: gating, histogram, permutation, capacity and
losses through the C ABI, bit-exact against the oracle on identical fp32
logits (the contract: given identical router logits, expert indices,
per-expert counts and the permutation are bit-exact)."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def same(a, b):
    """Bit-exact equality; NaNs must sit at the same places (payload free)."""
    a, b = np.asarray(a), np.asarray(b)
    if a.shape != b.shape:
        return False
    if a.dtype == np.float32 and b.dtype == np.float32:
        na, nb = np.isnan(a), np.isnan(b)
        return np.array_equal(na, nb) and np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb])
    return np.array_equal(a, b)


def oracle_route(oracle, logits, gate, k, ns, training=False, cf=None):
    if gate == "shared":
        idx, g, p = oracle.compute_gates_shared(logits, ns, k)
    else:
        idx, g, p = oracle.compute_gates_topk(logits, 1 if gate == "switch" else k)
    if cf is not None and training:
        idx, g, _ = oracle.capacity(idx, g, logits.shape[1], cf)
    counts, offsets, perm = oracle.bucket(idx, logits.shape[1])
    return idx, g, p, counts, offsets, perm


def gpu_route(moe, logits, gate, k, ns, training=False, cf=None):
    E = logits.shape[1]
    g = {"topk": moe.TopKGating(k), "switch": moe.SwitchGating(),
         "shared": moe.SharedExpertGating(ns, moe.TopKGating(k), E)}[gate]
    idx, gates, probs, counts, offsets, perm = moe.route_from_logits(g, logits.T, training=training,
                                                                     capacity_factor=cf)
    return idx.T.astype(np.int32), gates.T, probs.T, counts, offsets, perm


def check_route(moe, oracle, logits, gate="topk", k=2, ns=0, training=False, cf=None):
    print(f"route case gate={gate} T={logits.shape[0]} E={logits.shape[1]} k={k} ns={ns} cf={cf}", flush=True)
    o = oracle_route(oracle, logits, gate, k, ns, training, cf)
    d = gpu_route(moe, logits, gate, k, ns, training, cf)
    names = ["indices", "gates", "probs", "counts", "offsets"]
    for nm, a, b in zip(names, d[:5], o[:5]):
        assert same(a, b), f"{nm} differ (gate={gate}, E={logits.shape[1]}, k={k})"
    n = int(o[4][-1])
    assert np.array_equal(d[5][:n], o[5]), "permutation differs"
    return d


@pytest.mark.parametrize("T,E,k", [(4096, 8, 2), (4096, 8, 1), (1000, 8, 8), (8192, 64, 6), (16384, 128, 1),
                                   (1, 8, 2), (255, 16, 3), (257, 16, 3), (513, 5, 2)])
def test_topk_random_logits(moe, oracle, T, E, k):
    rng = np.random.default_rng(T * 131 + E * 7 + k)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    check_route(moe, oracle, logits, "topk", k)


@pytest.mark.parametrize("E", [65, 96, 128, 129, 256, 300, 512])
@pytest.mark.parametrize("k", [2, 3, 6, 8])
def test_topk_over_64_experts(moe, oracle, E, k):
    # more than 64 routed experts with k >= 2: each of a token's 8 lanes keeps
    # the best k of its share in sorted registers, three butterfly steps merge
    # the lists; random, tie-heavy integer and non-finite logits
    rng = np.random.default_rng(E * 100 + k)
    lg = rng.standard_normal((3000, E)).astype(np.float32)
    check_route(moe, oracle, lg, "topk", k)
    lg = rng.integers(-2, 3, size=(2000, E)).astype(np.float32)
    check_route(moe, oracle, lg, "topk", k)
    lg = rng.standard_normal((300, E)).astype(np.float32)
    lg[3, 7] = np.inf
    lg[4, :] = -np.inf
    lg[5, E - 1] = np.nan
    lg[6, [1, E - 2]] = np.inf
    lg[7, ::3] = np.nan
    lg[8, :] = 0.0
    lg[9, :] = np.float32(-0.0)
    check_route(moe, oracle, lg, "topk", k)


@pytest.mark.parametrize("E,ns,k", [(100, 2, 6), (128, 1, 7), (67, 2, 2), (257, 1, 8), (385, 1, 8)])
def test_shared_gating_over_64_routed(moe, oracle, E, ns, k):
    rng = np.random.default_rng(E + ns + k)
    lg = rng.standard_normal((2500, E)).astype(np.float32)
    lg[:, ns:] += np.log(1.0 / np.arange(1, E - ns + 1) ** 1.1).astype(np.float32)
    lg[::5] = np.round(lg[::5])
    d = check_route(moe, oracle, lg, "shared", k, ns)
    assert np.all(d[3][:ns] == 2500)


def test_topk_skewed_and_ties(moe, oracle):
    rng = np.random.default_rng(11)
    # small integer logits: exact ties everywhere
    logits = rng.integers(-3, 4, size=(3000, 8)).astype(np.float32)
    check_route(moe, oracle, logits, "topk", 2)
    # Mixtral-style skew: per-expert bias ~ N(0,1) on top of small logits
    logits = (rng.standard_normal((4096, 8)) * 0.05 + rng.standard_normal(8)).astype(np.float32)
    check_route(moe, oracle, logits, "topk", 2)
    # one expert takes everything
    logits = np.zeros((700, 8), np.float32)
    logits[:, 5] = 10
    d = check_route(moe, oracle, logits, "topk", 2)
    assert d[3][5] == 700


def test_switch_k1_gate_exactly_one(moe, oracle):
    rng = np.random.default_rng(12)
    logits = rng.standard_normal((16384, 128)).astype(np.float32)
    d = check_route(moe, oracle, logits, "switch", 1)
    assert np.all(d[1] == np.float32(1.0))


def test_shared_gating(moe, oracle):
    rng = np.random.default_rng(13)
    bias = np.log(1.0 / np.arange(1, 65) ** 1.1)  # Zipf(1.1)-skewed routed experts
    logits = rng.standard_normal((8192, 66)).astype(np.float32)
    logits[:, 2:] += bias.astype(np.float32)
    d = check_route(moe, oracle, logits, "shared", 6, 2)
    assert np.all(d[3][:2] == 8192)


def test_capacity_constraint(moe, oracle):
    rng = np.random.default_rng(14)
    logits = rng.standard_normal((2000, 8)).astype(np.float32)
    logits[:, 0] += 1.5
    for cf in (0.5, 1.0, 1.25):
        d = check_route(moe, oracle, logits, "topk", 2, training=True, cf=cf)
        cap = int(np.ceil(np.float32(np.float32(cf) * np.float32(2000)) / np.float32(8)))
        assert d[3].max() <= cap
    # capacity is inactive when not training
    check_route(moe, oracle, logits, "topk", 2, training=False, cf=0.5)


def test_golden_cases_on_gpu(moe, oracle):
    with open(os.path.join(GOLDEN, "routing_cases.json")) as f:
        cases = json.load(f)
    for c in cases:
        lg = np.array(c["logits"], dtype=np.float32)
        ns = c.get("num_shared", 0)
        d = gpu_route(moe, lg, "shared" if ns else "topk", c["k"], ns)
        assert d[0].tolist() == c["indices"], c["name"]
        if "gates" in c:
            assert d[1].tolist() == c["gates"], c["name"]
        if "probs" in c:
            assert d[2].tolist() == c["probs"], c["name"]


def test_nonfinite_logits(moe, oracle):
    lg = np.zeros((300, 8), np.float32)
    lg[3, 2] = np.inf
    lg[4, :] = -np.inf
    lg[5, 6] = np.nan
    lg[6, [1, 4]] = np.inf
    check_route(moe, oracle, lg, "topk", 2)


def test_compute_gates_api(moe, oracle):
    rng = np.random.default_rng(15)
    logits = rng.standard_normal((8, 100)).astype(np.float32)  # Julia shape (E, T)
    idx, gates, probs = moe.compute_gates(moe.TopKGating(2), logits)
    assert idx.shape == (2, 100) and idx.dtype == np.int64
    oi, og, op = oracle.compute_gates_topk(logits.T, 2)
    assert np.array_equal(idx, oi.T) and same(gates, og.T) and same(probs, op.T)
    # reference test invariants (test_moeLlama2_integration.jl:82-83)
    assert np.all((idx >= 1) & (idx <= 8))
    assert np.allclose(gates.sum(axis=0), 1.0, atol=1e-6)


def test_standalone_losses(moe, oracle):
    rng = np.random.default_rng(16)
    logits = rng.standard_normal((4096, 8)).astype(np.float32)
    idx, g, p = oracle.compute_gates_topk(logits, 2)
    sw = moe.compute_loss(moe.SwitchTransformerLoss(0.01), idx.T, p.T)
    assert abs(sw - oracle.switch_loss(idx, p, 0.01)) <= 1e-5 * max(1.0, abs(float(sw)))
    z = moe.compute_loss(moe.ZLoss(0.001), logits.T)
    assert abs(z - oracle.z_loss(logits, 0.001)) <= 1e-5 * max(1.0, abs(float(z)))
    assert moe.compute_loss(moe.NoBalancingLoss(), idx.T, p.T) == 0.0


def test_routing_is_deterministic(moe, oracle):
    rng = np.random.default_rng(17)
    logits = rng.standard_normal((5000, 64)).astype(np.float32)
    a = gpu_route(moe, logits, "topk", 6, 0)
    b = gpu_route(moe, logits, "topk", 6, 0)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("T,E,k,lam", [(2048, 8, 2, 0.7), (1000, 64, 6, 2.0), (77, 5, 3, -1.5), (1500, 128, 4, 0.9),
                                       (600, 96, 8, 1.0), (700, 300, 6, 1.3), (300, 512, 12, 0.8)])
def test_soft_moe_gating(moe, oracle, T, E, k, lam):
    # SoftMoEGating: top-k of softmax(logits ./ lambda), the gate matrix is the
    # probabilities (the dispatch reads the probability of expert `slot`)
    rng = np.random.default_rng(T + E)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[::7] = np.round(lg[::7])  # ties
    print(f"soft gating T={T} E={E} k={k} lambda={lam}", flush=True)
    idx, gates, probs = moe.compute_gates(moe.SoftMoEGating(k, lam), lg.T)
    oi, og, op = oracle.compute_gates_soft(lg, k, lam)
    assert same(idx.T.astype(np.int32), oi)
    assert same(probs.T, op) and same(gates, probs)


@pytest.mark.parametrize("T,E,cf,ties", [(4096, 8, 1.25, False), (64, 16, 1.0, True), (300, 8, 0.25, True),
                                         (33, 6, 3.0, True), (4096, 16, 1.25, False), (4096, 64, 1.25, False),
                                         (1000, 64, 2.0, True), (2048, 128, 6.0, False), (2048, 256, 6.0, False),
                                         (500, 512, 3.0, True)])
def test_expert_choice_gating(moe, oracle, T, E, cf, ties):
    # ExpertChoiceGating: the (capacity, T) indices / gates bit-exact
    rng = np.random.default_rng(T * E)
    lg = (rng.integers(-3, 4, size=(T, E)) if ties else rng.standard_normal((T, E))).astype(np.float32)
    print(f"expert choice T={T} E={E} cf={cf}", flush=True)
    idx, gates, probs = moe.compute_gates(moe.ExpertChoiceGating(cf), lg.T)
    oi, og, op = oracle.compute_gates_expert_choice(lg, cf)
    assert idx.shape == (oi.shape[1], T)
    assert same(idx.T.astype(np.int32), oi)
    assert same(gates.T, og) and same(probs.T, op)


def test_expert_choice_many_slots_bucketing(moe, oracle):
    # 16 experts, capacity 16 (equal logits: every expert takes tokens 1..16,
    # so each of them holds all 16 experts); and 64 experts at T = 4096:
    # indices, counts, offsets and the permutation bit-exact
    lg = np.zeros((64, 16), np.float32)
    idx, gates, probs = moe.compute_gates(moe.ExpertChoiceGating(4.0), lg.T)
    assert idx.shape == (16, 64)
    assert np.array_equal(idx[:, :16], np.tile(np.arange(1, 17)[:, None], (1, 16)))
    assert np.all(idx[:, 16:] == 0)
    rng = np.random.default_rng(77)
    # (500, 300, 150.0): 250 slots per token, (300, 512, 600.0): 352 (a lane
    # of the wide permute owns 4 and 6 of them)
    for T, E, cf in ((64, 16, 4.0), (4096, 64, 1.25), (500, 128, 40.0), (500, 300, 150.0), (300, 512, 600.0)):
        lg = rng.standard_normal((T, E)).astype(np.float32)
        g = moe.ExpertChoiceGating(cf)
        print(f"expert choice bucketing T={T} E={E} cf={cf}", flush=True)
        di, dg, dp, counts, offsets, perm = moe.route_from_logits(g, lg.T)
        oi, og, op = oracle.compute_gates_expert_choice(lg, cf)
        kt = di.shape[0]
        n = min(kt, oi.shape[1])
        assert np.array_equal(di.T[:, :n].astype(np.int32), oi[:, :n]) and np.all(oi[:, n:] == 0)
        assert same(dg.T[:, :n], og[:, :n]) and same(dp.T, op)
        oc, oo, opm = oracle.bucket(oi, E)
        assert np.array_equal(counts, oc) and np.array_equal(offsets, oo)
        m = int(oo[-1])
        assert np.array_equal(np.divmod(perm[:m], kt), np.divmod(opm, oi.shape[1]))


def test_jitter_and_stochastic_gates(moe, oracle):
    # without training / noise logits both are their base gate; with them the
    # perturbed logits (numpy's stream, replayed here) go through the base gate
    rng = np.random.default_rng(61)
    lg = rng.standard_normal((8, 500)).astype(np.float32)
    base = moe.compute_gates(moe.TopKGating(2), lg)
    for g in (moe.JitterGating(moe.TopKGating(2), 0.1), moe.StochasticTopKGating(2)):
        out = moe.compute_gates(g, lg)
        assert all(same(a, b) for a, b in zip(out, base))
    jit = moe.JitterGating(moe.TopKGating(2), 0.1, rng=np.random.default_rng(5))
    out = moe.compute_gates(jit, lg, training=True)
    u = np.random.default_rng(5).random(lg.shape, dtype=np.float32)
    jl = (lg * (np.float32(1) + (np.float32(2) * u - np.float32(1)) * np.float32(0.1))).astype(np.float32)
    oi, og, op = oracle.compute_gates_topk(jl.T, 2)
    assert same(out[0].T.astype(np.int32), oi) and same(out[1].T, og) and same(out[2].T, op)
    st = moe.StochasticTopKGating(2, train_only=False, rng=np.random.default_rng(6))
    nl = rng.standard_normal(lg.shape).astype(np.float32)
    out = moe.compute_gates(st, lg, noise_logits=nl)
    noise = (np.random.default_rng(6).standard_normal(lg.shape, dtype=np.float32)
             * np.logaddexp(np.float32(0), nl).astype(np.float32)).astype(np.float32)
    oi, og, op = oracle.compute_gates_topk((lg + noise).astype(np.float32).T, 2)
    assert same(out[0].T.astype(np.int32), oi) and same(out[2].T, op)


def test_host_routed_gates(moe):
    # HashGating: (hash(i) + j) % E + 1 with a user hash; RandomGating: k
    # distinct experts per token; both with gates 1/k and probabilities 1/E
    idx, gates, probs = moe.compute_gates(moe.HashGating(3, 8, hash_fn=lambda i: 5 * i), np.zeros((8, 10), np.float32))
    t = np.arange(1, 11)
    assert np.array_equal(idx, np.stack([(5 * t + j) % 8 + 1 for j in range(3)]))
    assert np.all(gates == np.float32(1) / np.float32(3)) and np.all(probs == np.float32(0.125))
    idx, gates, _ = moe.compute_gates(moe.RandomGating(4, rng=np.random.default_rng(1)), np.zeros((6, 200), np.float32))
    assert idx.shape == (4, 200) and idx.min() >= 1 and idx.max() <= 6
    assert all(len(set(idx[:, i])) == 4 for i in range(200))


@pytest.mark.parametrize("E,ns,k", [(10, 1, 2), (11, 3, 2)])
def test_shared_gating_inexact_scales(moe, oracle, E, ns, k):
    """SharedExpertGating(ns, TopKGating(k), E) with scales that are not
    exact in binary: the routed gates times 1 - ns/total_k (2/3 for ns = 1,
    2/5 for ns = 3) and the routed probabilities times 1 - ns/E (9/10, 8/11),
    both computed in Float64 as Julia promotes `1.0f0 - Int/Int`
    (src/gating/advanced.jl:95-105) and rounded once.  Bit-exact against the
    oracle; the case also shows that a Float32 scale would round some gates
    differently, so a Float32 restatement could not pass it."""
    rng = np.random.default_rng(E * 10 + ns)
    lg = rng.standard_normal((4096, E)).astype(np.float32)
    check_route(moe, oracle, lg, "shared", k, ns)
    # the case tells the Float64 scale from a Float32 one
    _, g, _ = oracle.compute_gates_topk(lg[:, ns:], k)
    s64 = 1.0 - ns / (ns + k)
    f64 = (g.astype(np.float64) * s64).astype(np.float32)
    f32 = g * np.float32(s64)
    assert np.count_nonzero(f64 != f32) > 0
