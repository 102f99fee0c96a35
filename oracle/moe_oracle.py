"""CPU oracle of MixtureOfExperts.jl's MoE-layer forward path.

TEST INFRASTRUCTURE ONLY: the checker the HIP library is compared against.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module; the product (mixtureofexperts_amd) never does.

Routing, bucketing, capacity, losses and statistics call the C restatement in
oracle/moe_oracle.c (libmoe_oracle.so, built by oracle/build.py).  The expert
FFNs are numpy float32 matmuls, which go through OpenBLAS sgemm as the
reference's Flux Dense layers do.  Array layout is token-major ([T][E],
[T][D]), i.e. the memory of the reference's column-major (E, T) / (D, T)
matrices.

Reference lines followed (MixtureOfExperts.jl):
  forward_standard         src/core/moe_layer.jl:107-156
  forward_with_shared_experts src/core/moe_layer.jl:158-185
  process_expert_forward!  src/core/moe_layer.jl:187-219
  Router                   src/core/router.jl:25-46
  GatedExpert              src/experts/gated.jl:29-35
  StandardExpert           src/experts/standard.jl:38-55
  moe_ffn_forward! (decode, slot-order combine) src/llama2/inference.jl:58-121
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmoe_oracle.so")

_L = None


def _lib():
    global _L
    if _L is not None:
        return _L
    if not os.path.exists(LIB_PATH):
        from .build import build_oracle

        build_oracle()
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    L.oracle_softmax.argtypes = [vp, i64, i32, vp]
    L.oracle_compute_gates_topk.argtypes = [vp, i64, i32, i32, vp, vp, vp]
    L.oracle_compute_gates_topk.restype = ctypes.c_int
    L.oracle_compute_gates_shared.argtypes = [vp, i64, i32, i32, i32, vp, vp, vp]
    L.oracle_compute_gates_shared.restype = ctypes.c_int
    L.oracle_capacity.argtypes = [vp, vp, i64, i32, i32, f32]
    L.oracle_capacity.restype = i64
    L.oracle_bucket.argtypes = [vp, i64, i32, i32, vp, vp, vp]
    L.oracle_bucket.restype = i64
    L.oracle_switch_loss.argtypes = [vp, i64, i32, vp, i32, f32]
    L.oracle_switch_loss.restype = f32
    L.oracle_z_loss.argtypes = [vp, i64, i32, f32, vp]
    L.oracle_z_loss.restype = f32
    L.oracle_mean_entropy.argtypes = [vp, i64, i32]
    L.oracle_mean_entropy.restype = f32
    L.oracle_combine.argtypes = [vp, vp, i64, vp, i32, i64, i32, vp]
    _L = L
    return L


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- routing --------------------------------------------------------------

def softmax(logits_TE):
    lg = _c(logits_TE, np.float32)
    T, E = lg.shape
    p = np.empty_like(lg)
    _lib().oracle_softmax(lg.ctypes.data, T, E, p.ctypes.data)
    return p


def compute_gates_topk(logits_TE, k):
    """(idx [T][k] int32 1-based, gates [T][k], probs [T][E]) -- topk.jl:24-44."""
    lg = _c(logits_TE, np.float32)
    T, E = lg.shape
    idx = np.zeros((T, k), np.int32)
    g = np.zeros((T, k), np.float32)
    p = np.zeros((T, E), np.float32)
    if _lib().oracle_compute_gates_topk(lg.ctypes.data, T, E, k, idx.ctypes.data, g.ctypes.data, p.ctypes.data):
        raise ValueError("bad top-k arguments")
    return idx, g, p


def compute_gates_shared(logits_TE, num_shared, k):
    """SharedExpertGating(num_shared, TopKGating(k), E) -- advanced.jl:80-108."""
    lg = _c(logits_TE, np.float32)
    T, E = lg.shape
    kt = num_shared + k
    idx = np.zeros((T, kt), np.int32)
    g = np.zeros((T, kt), np.float32)
    p = np.zeros((T, E), np.float32)
    if _lib().oracle_compute_gates_shared(lg.ctypes.data, T, E, num_shared, k, idx.ctypes.data, g.ctypes.data,
                                          p.ctypes.data):
        raise ValueError("bad shared-gating arguments")
    return idx, g, p


def compute_gates_soft(logits_TE, k, lam):
    """SoftMoEGating(k, lambda) -- advanced.jl:17-33: probs = softmax(logits ./
    lambda), indices = top-k of probs; the returned gate matrix is probs, so
    the dispatch's gates[slot, t] is the probability of expert `slot`.
    Returns (idx [T][k], slot gates [T][k], probs [T][E])."""
    lg = _c(logits_TE, np.float32)
    scaled = (lg / np.float32(lam)).astype(np.float32)
    idx, _, probs = compute_gates_topk(scaled, k)
    return idx, np.ascontiguousarray(probs[:, :k]), probs


def expert_choice_capacity(T, E, capacity_factor):
    """ceil(Int, batch_size * capacity_factor / num_experts) in Float32."""
    return int(np.ceil(np.float32(np.float32(T) * np.float32(capacity_factor)) / np.float32(E)))


def compute_gates_expert_choice(logits_TE, capacity_factor):
    """ExpertChoiceGating -- expert_choice.jl:11-53, by full sorts: expert e
    takes the first min(C, T) tokens of sortperm(scores[:, e], rev=true) with
    Julia's isless order (NaN largest) and ties to the lower token; token t's
    slots list the experts that took it in ascending id order, at most C.
    Returns (idx [T][C], gates [T][C], probs [T][E])."""
    lg = _c(logits_TE, np.float32)
    T, E = lg.shape
    C = expert_choice_capacity(T, E, capacity_factor)
    probs = softmax(lg)
    idx = np.zeros((T, C), np.int32)
    g = np.zeros((T, C), np.float32)
    cnt = np.zeros(T, np.int64)
    for e in range(E):
        col = lg[:, e]
        nan = np.isnan(col)
        # descending isless: NaN first, then by value descending, ties by token ascending
        order = np.lexsort((np.arange(T), -np.where(nan, 0, col).astype(np.float64), ~nan))
        for t in order[:min(C, T)]:
            cnt[t] += 1
            if cnt[t] <= C:
                idx[t, cnt[t] - 1] = e + 1
                g[t, cnt[t] - 1] = probs[t, e]
    return idx, g, probs


def capacity(idx, gates, num_experts, capacity_factor):
    """apply_capacity_constraint (in place on copies) -- moe_layer.jl:221-248."""
    idx = _c(idx, np.int32).copy()
    gates = _c(gates, np.float32).copy()
    T, k = idx.shape
    dropped = _lib().oracle_capacity(idx.ctypes.data, gates.ctypes.data, T, k, num_experts, capacity_factor)
    return idx, gates, int(dropped)


def bucket(idx, E):
    """(counts [E], offsets [E+1], perm [n_valid]) -- moe_layer.jl:192-203."""
    idx = _c(idx, np.int32)
    T, k = idx.shape
    counts = np.zeros(E, np.int32)
    offsets = np.zeros(E + 1, np.int32)
    perm = np.zeros(max(T * k, 1), np.int32)
    n = _lib().oracle_bucket(idx.ctypes.data, T, k, E, counts.ctypes.data, offsets.ctypes.data, perm.ctypes.data)
    return counts, offsets, perm[:n]


def switch_loss(idx, probs, alpha):
    idx = _c(idx, np.int32)
    probs = _c(probs, np.float32)
    T, k = idx.shape
    return np.float32(_lib().oracle_switch_loss(idx.ctypes.data, T, k, probs.ctypes.data, probs.shape[1],
                                                np.float32(alpha)))


def z_loss(logits, beta):
    lg = _c(logits, np.float32)
    T, E = lg.shape
    return np.float32(_lib().oracle_z_loss(lg.ctypes.data, T, E, np.float32(beta), None))


def logsumexp_rows(logits):
    """Per-token lse_t = m + log(sum(exp(l - m))) of the z-loss
    (src/balancing/losses.jl:111-114), the same recipe as z_loss."""
    lg = _c(logits, np.float32)
    T, E = lg.shape
    out = np.zeros(T, np.float32)
    _lib().oracle_z_loss(lg.ctypes.data, T, E, np.float32(1.0), out.ctypes.data)
    return out


def mean_entropy(probs):
    p = _c(probs, np.float32)
    return np.float32(_lib().oracle_mean_entropy(p.ctypes.data, p.shape[0], p.shape[1]))


# ---- experts ----------------------------------------------------------------

def act_silu(x):
    """silu(x) = x * sigmoid(x) (src/experts/gated.jl:35), NNlib sigmoid form."""
    x = np.asarray(x, np.float32)
    t = np.exp(-np.abs(x))
    sig = np.where(x >= 0, np.float32(1) / (np.float32(1) + t), t / (np.float32(1) + t)).astype(np.float32)
    return (x * sig).astype(np.float32)


def act_gelu(x):
    """NNlib gelu, tanh form: 0.5x(1 + tanh(sqrt(2/pi)(x + 0.044715x^3)))."""
    x = np.asarray(x, np.float32)
    c = np.float32(np.sqrt(2.0 / np.pi))
    return (np.float32(0.5) * x * (np.float32(1) + np.tanh(c * (x + np.float32(0.044715) * x ** 3)))).astype(np.float32)


def act_relu(x):
    return np.maximum(np.asarray(x, np.float32), np.float32(0))


def act_identity(x):
    return np.asarray(x, np.float32)


ACTS = {"silu": act_silu, "gelu": act_gelu, "relu": act_relu, "identity": act_identity}


def gated_expert(xb, w1, w2, w3, act):
    """GatedExpert: w2(act(w1 x) .* (w3 x)) on token rows xb [n][D]; weights in
    Flux (out, in) shape.  gated.jl:29-34."""
    g = act(xb @ w1.T)
    u = xb @ w3.T
    return ((g * u).astype(np.float32) @ w2.T).astype(np.float32)


def standard_expert(xb, w1, w2, b1, b2, act):
    """StandardExpert: w2(act(w1 x .+ b1)) .+ b2.  standard.jl:38-55."""
    h = xb @ w1.T
    if b1 is not None:
        h = h + b1
    h = act(h)
    y = h @ w2.T
    if b2 is not None:
        y = y + b2
    return y.astype(np.float32)


def aux_free_update_bias(idx, bias, mom, lr, momentum):
    """The bias step of update_bias!(::AuxiliaryFreeLoss, indices) after its
    counter check (src/balancing/auxiliary_free.jl:44-69), in place, with
    Julia's types: counts Float32; target_count = total / E and the gradient
    Float64; momentum[i] = Float32(Float32(m * momentum[i]) + Float32(1 - m) *
    gradient) (the sum in Float64); bias[i] -= lr * momentum[i] in Float32;
    then bias .-= mean(bias), the Float32 sum in index order (Julia's order
    for fewer than 16 experts)."""
    f32 = np.float32
    E = bias.size
    counts = [f32(0)] * E
    total = 0
    for e in np.asarray(idx).reshape(-1):
        if e > 0:
            counts[int(e) - 1] = f32(counts[int(e) - 1] + f32(1))
            total += 1
    if total == 0:
        return
    target = total / E
    m32, lr32 = f32(momentum), f32(lr)
    for i in range(E):
        grad = (float(counts[i]) - target) / total
        mom[i] = f32(float(f32(m32 * mom[i])) + float(f32(f32(1) - m32)) * grad)
        bias[i] = f32(bias[i] - f32(lr32 * mom[i]))
    s = bias[0]
    for i in range(1, E):
        s = f32(s + bias[i])
    mean = f32(s / f32(E))
    for i in range(E):
        bias[i] = f32(bias[i] - mean)


def moe_forward(x_TD, router_w_ED, experts, *, gate="topk", k=2, num_shared=0, expert_type="gated", act="silu",
                alpha=0.01, z_weight=0.001, training=False, drop_tokens=False, capacity_factor=1.25,
                router_bias=None, logits=None, aux_free=None, gate_param=None, given=None, z_logits=None):
    """forward_standard + the z-loss of MoELayer's call (moe_layer.jl:107-156).

    x_TD: [T][D] float32.  router_w_ED: (E, D) Flux weight.  experts: list of
    dicts with fp32 "w1","w2"(,"w3") in (out, in) shape (+ "b1","b2").
    ``logits`` may be given to route identical logits.  ``gate``: "topk",
    "switch", "shared", "soft" (gate_param = lambda) or "expert_choice"
    (gate_param = capacity factor); ``given`` = (indices, gates, probs or
    None) replaces compute_gates (a gate computed by host code).  ``aux_free``: the
    state of an AuxiliaryFreeLoss balance loss (dict bias, mom, lr, momentum,
    update_freq, counter, use_comp, cw), updated in place: the gating runs on
    logits .+ bias (:137-140) and the balance loss is its compute_loss
    (src/balancing/auxiliary_free.jl:78-87).  ``z_logits``: the logits of the
    z-loss when they differ from the gate's (router noise in training: the
    gate sees the noisy logits, the z-loss reruns the router with
    training=false, moe_layer.jl:117-121).  Returns (out [T][Dout], loss,
    aux dict)."""
    x = np.asarray(x_TD, np.float32)
    T = x.shape[0]
    if logits is None:
        logits = (x @ np.asarray(router_w_ED, np.float32).T).astype(np.float32)
        if router_bias is not None:
            logits = (logits + router_bias).astype(np.float32)
    E = len(experts)

    def gating(lg):
        if gate == "shared":
            return compute_gates_shared(lg, num_shared, k)
        if gate == "soft":
            return compute_gates_soft(lg, k, gate_param)
        if gate == "expert_choice":
            return compute_gates_expert_choice(lg, gate_param)
        return compute_gates_topk(lg, 1 if gate == "switch" else k)

    if given is not None:
        idx, gates = np.asarray(given[0], np.int32), np.asarray(given[1], np.float32)
        probs = given[2] if given[2] is not None else np.full((T, len(experts)), np.float32(1) / np.float32(
            len(experts)), np.float32)
    else:
        idx, gates, probs = gating(logits)
    if aux_free is not None:
        idx, gates, _ = gating((logits + aux_free["bias"].reshape(1, -1)).astype(np.float32))
    if drop_tokens and training:
        idx, gates, _ = capacity(idx, gates, E, capacity_factor)
    counts, offsets, perm = bucket(idx, E)
    kt = idx.shape[1]
    Dout = experts[0]["w2"].shape[0]
    fn = ACTS[act]
    out = np.zeros((T, Dout), np.float32)
    flat_g = gates.reshape(-1)
    for e in range(E):
        lo, hi = offsets[e], offsets[e + 1]
        if hi == lo:
            continue
        ents = perm[lo:hi]
        toks = ents // kt
        xb = x[toks]
        ex = experts[e]
        if expert_type == "gated":
            y = gated_expert(xb, ex["w1"], ex["w2"], ex["w3"], fn)
        else:
            y = standard_expert(xb, ex["w1"], ex["w2"], ex.get("b1"), ex.get("b2"), fn)
        w = flat_g[ents]
        out[toks] = out[toks] + (w[:, None] * y).astype(np.float32)
    loss = np.float32(0.0)
    sw = np.float32(0.0)
    zl = np.float32(0.0)
    if training:
        if aux_free is not None:
            aux_free["counter"] += 1
            if aux_free["counter"] % aux_free["update_freq"] == 0:
                aux_free_update_bias(idx, aux_free["bias"], aux_free["mom"], aux_free["lr"], aux_free["momentum"])
            sw = np.float32(np.float32(aux_free["cw"]) * switch_loss(idx, probs, 1.0)) if aux_free["use_comp"] \
                else np.float32(0.0)
        else:
            sw = switch_loss(idx, probs, alpha)
        loss = sw
        if z_weight > 0:
            zl = z_loss(logits if z_logits is None else z_logits, z_weight)
            loss = np.float32(loss + zl)
    aux = dict(logits=logits, idx=idx, gates=gates, probs=probs, counts=counts, offsets=offsets, perm=perm,
               switch_loss=sw, z_loss=zl, mean_entropy=mean_entropy(probs))
    return out, loss, aux


def moe_forward_shared_experts(x_TD, router_w_ED, experts, num_shared, *, gate="topk", k=2, expert_type="gated",
                               act="silu", alpha=0.01, z_weight=0.001, training=False, router_bias=None, logits=None,
                               gate_param=None, gate_num_shared=0, aux_free=None):
    """forward_with_shared_experts + the z-loss of MoELayer's call
    (src/core/moe_layer.jl:107-128, 158-185), num_shared_experts = ns > 0.

    experts: all E experts, the first ns the shared ones; router_w_ED is the
    (E - ns, D) router.  shared = sum_i (y_i ./ ns) from zeros (:161-166);
    the router's gate (any of moe_forward's, with ``gate_param`` and
    ``gate_num_shared`` for SharedExpertGating) runs on the plain logits (no
    AuxiliaryFreeLoss bias: only forward_standard adds it, :137-140); its
    indices are shifted by ns (:172), every entry, so an ExpertChoice
    matrix's empty entries (0) become ns; the routed experts run through
    process_expert_forward! with the unshifted ids (:174-177), empty entries
    skipped; output = 0.5f0 .* shared .+ 0.5f0 .* routed (:179-180); the
    balance loss takes the shifted indices and the (E - ns) router
    probabilities (:182): the Switch loss counts ids 1..E - ns only
    (src/balancing/losses.jl:22-26); an ``aux_free`` state (moe_forward's
    dict, its bias over all E experts) is updated by update_bias! on the
    shifted indices (src/balancing/auxiliary_free.jl:36-87).  No capacity
    constraint and no update_stats!.  Returns (out, loss, aux)."""
    x = np.asarray(x_TD, np.float32)
    T = x.shape[0]
    ns = int(num_shared)
    fn = ACTS[act]
    shared = np.zeros((T, experts[0]["w2"].shape[0]), np.float32)
    for i in range(ns):
        ex = experts[i]
        if expert_type == "gated":
            y = gated_expert(x, ex["w1"], ex["w2"], ex["w3"], fn)
        else:
            y = standard_expert(x, ex["w1"], ex["w2"], ex.get("b1"), ex.get("b2"), fn)
        shared = (shared + (y / np.float32(ns)).astype(np.float32)).astype(np.float32)
    routed, _, ra = moe_forward(x, router_w_ED, experts[ns:], gate=gate, k=k, num_shared=gate_num_shared,
                                expert_type=expert_type, act=act, alpha=alpha, z_weight=0.0, training=False,
                                router_bias=router_bias, logits=logits, gate_param=gate_param)
    half = np.float32(0.5)
    out = ((half * shared).astype(np.float32) + (half * routed).astype(np.float32)).astype(np.float32)
    shifted = (ra["idx"] + ns).astype(np.int32)
    loss = np.float32(0.0)
    sw = np.float32(0.0)
    zl = np.float32(0.0)
    if training:
        if aux_free is not None:
            aux_free["counter"] += 1
            if aux_free["counter"] % aux_free["update_freq"] == 0:
                aux_free_update_bias(shifted, aux_free["bias"], aux_free["mom"], aux_free["lr"], aux_free["momentum"])
            sw = np.float32(np.float32(aux_free["cw"]) * switch_loss(shifted, ra["probs"], 1.0)) \
                if aux_free["use_comp"] else np.float32(0.0)
        else:
            sw = switch_loss(shifted, ra["probs"], alpha)
        loss = sw
        if z_weight > 0:
            zl = z_loss(ra["logits"], z_weight)
            loss = np.float32(loss + zl)
    aux = dict(logits=ra["logits"], idx=shifted, gates=ra["gates"], probs=ra["probs"], routed_idx=ra["idx"],
               routed_counts=ra["counts"], shared=shared, routed=routed, switch_loss=sw, z_loss=zl,
               mean_entropy=ra["mean_entropy"])
    return out, loss, aux


# ---- decode caller ------------------------------------------------------------

def silu_inline(x):
    """The decode path's inline silu, g * (1 / (1 + exp(-g))) in Float32
    (src/llama2/inference.jl:160)."""
    x = np.asarray(x, np.float32)
    return (x * (np.float32(1) / (np.float32(1) + np.exp(-x)))).astype(np.float32)


def decode_ffn(xb_nD, router_w_ED, experts, *, gate="topk", k=2, router_bias=None, logits=None, num_shared=0):
    """moe_ffn_forward! (src/llama2/inference.jl:58-121) after its rmsnorm,
    for n tokens each routed on its own: logits =
    W_router' xb (:63), compute_gates (:65-66), then xb2 = 0 and, slot by slot
    in order, xb2 += gate * gated_expert_forward!(xb) (:83-104, :154-167).

    xb_nD: [n][D] float32; router_w_ED: (E, D); experts: dicts of fp32 "w1",
    "w3" (H, D) and "w2" (D, H) in (out, in) shape.  ``logits`` may be given
    to route identical logits.  Returns (out [n][Dout], idx, gates, logits)."""
    x = np.asarray(xb_nD, np.float32)
    if logits is None:
        logits = (x @ np.asarray(router_w_ED, np.float32).T).astype(np.float32)
        if router_bias is not None:
            logits = (logits + router_bias).astype(np.float32)
    idx, gates, _ = compute_gates_topk(logits, 1 if gate == "switch" else k)
    n, kt = idx.shape
    ns = int(num_shared)
    routed = experts[ns:]
    Dout = experts[0]["w2"].shape[0]
    out = np.zeros((n, Dout), np.float32)
    for j in range(kt):  # slot order
        for e in range(len(routed)):
            toks = np.nonzero(idx[:, j] == e + 1)[0]
            if toks.size == 0:
                continue
            ex = routed[e]
            y = gated_expert(x[toks], ex["w1"], ex["w2"], ex["w3"], silu_inline)
            out[toks] = (out[toks] + (gates[toks, j][:, None] * y).astype(np.float32)).astype(np.float32)
    if ns > 0:
        # process_shared_experts! (src/llama2/inference.jl:184-216): shared =
        # sum_i (1f0 / ns) * y_i from zeros, xb2 = 0.5f0 * shared + 0.5f0 * xb2
        sw = np.float32(1) / np.float32(ns)
        sh = np.zeros((n, Dout), np.float32)
        for i in range(ns):
            ex = experts[i]
            y = gated_expert(x, ex["w1"], ex["w2"], ex["w3"], silu_inline)
            sh = (sh + (sw * y).astype(np.float32)).astype(np.float32)
        half = np.float32(0.5)
        out = ((half * sh).astype(np.float32) + (half * out).astype(np.float32)).astype(np.float32)
    return out, idx, gates, logits


# ---- convert_to_moe ---------------------------------------------------------------

def split_expert(w1, w2, w3, e, E):
    """create_single_expert(..., :split, expert_idx = e + 1) --
    src/llama2/conversion.jl:296-304: Llama (in, out) matrices w1, w3 (dim,
    hidden), w2 (hidden, dim); expert e keeps hidden units start:end with
    start = (e * hidden) / E + 1 and end = min((e + 1) * hidden / E, hidden)
    (integer division, 1-based), zeros elsewhere."""
    hidden = w1.shape[1]
    start = (e * hidden) // E + 1
    end = min(((e + 1) * hidden) // E, hidden)
    o1 = np.zeros_like(w1)
    o2 = np.zeros_like(w2)
    o3 = np.zeros_like(w3)
    o1[:, start - 1:end] = w1[:, start - 1:end]
    o2[start - 1:end, :] = w2[start - 1:end, :]
    o3[:, start - 1:end] = w3[:, start - 1:end]
    return o1, o2, o3


# ---- dtype helpers used by tests and the bench ------------------------------

def f32_to_bf16_bits(a):
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


_FP8_TABLE = None


def fp8_e4m3_table():
    """All 256 OCP e4m3fn values (NaN at 0x7f/0xff)."""
    global _FP8_TABLE
    if _FP8_TABLE is None:
        t = np.zeros(256, np.float32)
        for b in range(256):
            s = -1.0 if b & 0x80 else 1.0
            e = (b >> 3) & 15
            m = b & 7
            if e == 15 and m == 7:
                t[b] = np.nan
            elif e == 0:
                t[b] = s * m * 2.0 ** -9
            else:
                t[b] = s * (1 + m / 8.0) * 2.0 ** (e - 7)
        _FP8_TABLE = t
    return _FP8_TABLE


def quantize_fp8_rows(w):
    """Per-output-channel (row) e4m3 quantisation: (codes uint8, scales f32)
    with scale = max|row| / 448 and round-to-nearest over the finite codes."""
    w = np.asarray(w, np.float32)
    amax = np.abs(w).max(axis=1)
    scales = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    q = w / scales[:, None]
    table = fp8_e4m3_table()
    pos = np.array(sorted(set(table[:0x7f].tolist())), np.float32)  # finite non-negative codes
    code_of = {float(v): i for i, v in enumerate(table[:0x7f])}
    a = np.abs(q)
    j = np.clip(np.searchsorted(pos, a), 1, len(pos) - 1)
    lo, hi = pos[j - 1], pos[j]
    pick_hi = (a - lo) > (hi - a)
    tie = (a - lo) == (hi - a)
    codes_lo = np.array([code_of[float(v)] for v in pos], np.uint8)
    even_hi = (codes_lo[j] & 1) == 0
    v = np.where(pick_hi | (tie & even_hi), j, j - 1)
    codes = codes_lo[v]
    codes = np.where(q < 0, codes | 0x80, codes).astype(np.uint8)
    return codes, scales


def dequantize_fp8_rows(codes, scales):
    return (fp8_e4m3_table()[codes] * scales[:, None]).astype(np.float32)
