/*
 * moe_oracle.c -- CPU restatement of the MixtureOfExperts.jl routing,
 * bucketing, capacity, loss and statistics semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP library is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path (mixtureofexperts_amd and
 * libmoe_mi355x.so) never calls into it.
 *
 * Layout convention: the reference's Julia arrays are column-major, so a Julia
 * matrix of size (E, T) is stored token-major, i.e. [T][E] row-major here.
 * Expert ids are 1-based (0 marks a dropped entry), exactly as in the
 * reference.
 *
 * Floating-point recipe (the reference's third-party pieces -- Julia's
 * Float32 exp, NNlib.softmax's reduction order -- cannot be run here, so this
 * is the recipe both this oracle and the HIP kernels implement):
 *   m   = max over experts (NaN ignored, NNlib fast_maximum)
 *   e_i = (float)exp((double)(l_i - m))       one rounding of an fp64 exp
 *         (when m == +Inf: e_i = (l_i == +Inf) ? 1 : 0, NNlib's non-finite branch)
 *   s   = ((e_1 + e_2) + e_3) + ...           sequential fp32, expert order
 *   p_i = e_i / s                              IEEE fp32 division
 * Top-k orders by Julia's `isless` (all NaNs largest, -0.0 < +0.0), descending,
 * ties to the lower expert index.
 *
 * Parity pins (tests/test_oracle.py): closed forms (uniform logits -> p = 1/E,
 * gates 1/k, Switch loss = alpha under balance, z-loss = beta*ln(E)^2 for zero
 * logits, entropy = ln E), brute-force top-k / stable sort on tiny inputs,
 * crafted exact ties, and an independent numpy float64 restatement.  Parity
 * with Julia's own Float32 exp and NNlib's summation order is unpinned (no
 * Julia in this environment).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- Julia `isless` total order on Float32, as an unsigned key ---------- */
static inline uint32_t isless_key(float f)
{
    if (isnan(f)) return 0xFFFFFFFFu; /* every NaN is larger than every number */
    uint32_t u;
    memcpy(&u, &f, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* ---- softmax over one token's logits ------------------------------------
 * Follows NNlib.softmax(x; dims=1) as called at src/gating/topk.jl:27
 * (max subtraction, exp, sum, divide). */
static void softmax_row(const float *l, int E, float *p)
{
    float m = -INFINITY;
    for (int i = 0; i < E; ++i)
        if (l[i] > m) m = l[i];
    float s = 0.0f;
    for (int i = 0; i < E; ++i) {
        float e;
        if (m == INFINITY)
            e = (l[i] == INFINITY) ? 1.0f : 0.0f;
        else
            e = (float)exp((double)(l[i] - m));
        p[i] = e;
        s = s + e;
    }
    for (int i = 0; i < E; ++i) p[i] = p[i] / s;
}

void oracle_softmax(const float *logits, int64_t T, int E, float *probs)
{
    for (int64_t t = 0; t < T; ++t) softmax_row(logits + t * E, E, probs + t * E);
}

/* ---- top-k with renormalisation -----------------------------------------
 * src/gating/topk.jl:33-41: partialsortperm(probs[:,t], 1:k, rev=true),
 * then gates = p_sel ./ sum(p_sel), the sum sequential in slot order: Julia's
 * short-array loop for k < 16; for k = 16 its mapreduce_impl adds a1 + a2 and
 * then the other 14 in an @simd loop, too short for a vectorised body (the
 * scalar remainder runs them in order).  `taken`: E bytes of scratch. */
static void topk_row(const float *p, int E, int k, int32_t *idx, float *g, uint8_t *taken)
{
    memset(taken, 0, (size_t)E);
    for (int j = 0; j < k; ++j) {
        int best = -1;
        uint32_t bk = 0;
        for (int i = 0; i < E; ++i) {
            if (taken[i]) continue;
            uint32_t key = isless_key(p[i]);
            if (best < 0 || key > bk) { best = i; bk = key; } /* strict > : lower index wins ties */
        }
        taken[best] = 1;
        idx[j] = best + 1;
    }
    float s = p[idx[0] - 1];
    for (int j = 1; j < k; ++j) s = s + p[idx[j] - 1];
    for (int j = 0; j < k; ++j) g[j] = p[idx[j] - 1] / s;
}

/* compute_gates(::TopKGating) -- src/gating/topk.jl:24-44;
 * compute_gates(::SwitchGating) is k = 1 -- src/gating/switch.jl:9-11. */
int oracle_compute_gates_topk(const float *logits, int64_t T, int E, int k,
                              int32_t *idx, float *gates, float *probs)
{
    if (E < 1 || k < 1 || k > E) return -1;
    uint8_t *taken = (uint8_t *)malloc((size_t)E);
    if (!taken) return -2;
    for (int64_t t = 0; t < T; ++t) {
        softmax_row(logits + t * E, E, probs + t * E);
        topk_row(probs + t * E, E, k, idx + t * k, gates + t * k, taken);
    }
    free(taken);
    return 0;
}

/* compute_gates(::SharedExpertGating) -- src/gating/advanced.jl:80-108.
 * logits: [T][E] (E = gate.num_experts); the softmax/top-k runs over rows
 * ns+1..E only; output has total_k = ns + k slots per token. */
int oracle_compute_gates_shared(const float *logits, int64_t T, int E, int ns, int k,
                                int32_t *idx, float *gates, float *probs)
{
    int Er = E - ns;
    if (ns < 0 || Er < 1 || k < 1 || k > Er) return -1;
    int tk = ns + k;
    float *pr = (float *)malloc(sizeof(float) * (size_t)Er);
    int32_t *ri = (int32_t *)malloc(sizeof(int32_t) * (size_t)k);
    float *rg = (float *)malloc(sizeof(float) * (size_t)k);
    uint8_t *taken = (uint8_t *)malloc((size_t)Er);
    if (!pr || !ri || !rg || !taken) {
        free(pr); free(ri); free(rg); free(taken);
        return -2;
    }
    const double routed_gate_scale = 1.0 - (double)ns / (double)tk; /* 1.0f0 - Int/Int -> Float64 */
    const double routed_prob_scale = 1.0 - (double)ns / (double)E;
    const float shared_gate = 1.0f / (float)tk;
    const float shared_prob = 1.0f / (float)E;
    for (int64_t t = 0; t < T; ++t) {
        softmax_row(logits + t * E + ns, Er, pr);
        topk_row(pr, Er, k, ri, rg, taken);
        for (int j = 0; j < ns; ++j) {
            idx[t * tk + j] = j + 1;
            gates[t * tk + j] = shared_gate;
        }
        for (int j = 0; j < k; ++j) {
            idx[t * tk + ns + j] = ri[j] + ns;
            gates[t * tk + ns + j] = (float)((double)rg[j] * routed_gate_scale);
        }
        for (int i = 0; i < ns; ++i) probs[t * E + i] = shared_prob;
        for (int i = 0; i < Er; ++i) probs[t * E + ns + i] = (float)((double)pr[i] * routed_prob_scale);
    }
    free(pr); free(ri); free(rg); free(taken);
    return 0;
}

/* apply_capacity_constraint -- src/core/moe_layer.jl:221-248.
 * capacity = ceil(Int, capacity_factor * T / num_experts) with Float32
 * arithmetic; entries beyond capacity become (0, 0f0); every token's gates are
 * then renormalised by their slot-order sum when it is positive. */
int64_t oracle_capacity(int32_t *idx, float *gates, int64_t T, int k, int num_experts, float cf)
{
    float capf = ceilf((cf * (float)T) / (float)num_experts);
    int64_t cap = (int64_t)capf;
    int64_t *cnt = (int64_t *)calloc((size_t)num_experts + 1, sizeof(int64_t));
    int64_t dropped = 0;
    if (!cnt) return -1;
    for (int64_t t = 0; t < T; ++t) {
        for (int j = 0; j < k; ++j) {
            int32_t e = idx[t * k + j];
            if (e > 0) {
                if (cnt[e] >= cap) {
                    idx[t * k + j] = 0;
                    gates[t * k + j] = 0.0f;
                    ++dropped;
                } else {
                    cnt[e] += 1;
                }
            }
        }
        float s = gates[t * k];
        for (int j = 1; j < k; ++j) s = s + gates[t * k + j];
        if (s > 0.0f)
            for (int j = 0; j < k; ++j) gates[t * k + j] = gates[t * k + j] / s;
    }
    free(cnt);
    return dropped;
}

/* Bucketing of process_expert_forward! -- src/core/moe_layer.jl:192-203.
 * Entries (t, slot) are visited t-major; each valid entry (1 <= e <= E) is
 * appended to expert e's list.  Output: counts[E], offsets[E+1] (exclusive
 * prefix sum), perm[pos] = t*k + slot (0-based entry id) for pos in
 * [offsets[e], offsets[e]+counts[e]) -- segment order ascending in e, tokens
 * ascending within a segment.  Returns the number of valid entries. */
int64_t oracle_bucket(const int32_t *idx, int64_t T, int k, int E,
                      int32_t *counts, int32_t *offsets, int32_t *perm)
{
    memset(counts, 0, sizeof(int32_t) * (size_t)E);
    for (int64_t t = 0; t < T; ++t)
        for (int j = 0; j < k; ++j) {
            int32_t e = idx[t * k + j];
            if (e > 0 && e <= E) counts[e - 1] += 1;
        }
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t *fill = (int32_t *)calloc((size_t)E, sizeof(int32_t));
    if (!fill) return -1;
    for (int64_t t = 0; t < T; ++t)
        for (int j = 0; j < k; ++j) {
            int32_t e = idx[t * k + j];
            if (e > 0 && e <= E) {
                perm[offsets[e - 1] + fill[e - 1]] = (int32_t)(t * k + j);
                fill[e - 1] += 1;
            }
        }
    free(fill);
    return offsets[E];
}

/* Julia's pairwise reduction (Base.mapreduce_impl, block size 1024) with a
 * sequential base case; used where the reference reduces a long vector with
 * `sum`/`mean` over all elements. */
static float pairwise_sum_f32(const float *a, int64_t lo, int64_t hi) /* [lo, hi] inclusive */
{
    if (hi - lo < 1024) {
        float s = a[lo];
        for (int64_t i = lo + 1; i <= hi; ++i) s = s + a[i];
        return s;
    }
    int64_t mid = (lo + hi) >> 1;
    return pairwise_sum_f32(a, lo, mid) + pairwise_sum_f32(a, mid + 1, hi);
}

static double pairwise_sum_f64(const double *a, int64_t lo, int64_t hi)
{
    if (hi - lo < 1024) {
        double s = a[lo];
        for (int64_t i = lo + 1; i <= hi; ++i) s = s + a[i];
        return s;
    }
    int64_t mid = (lo + hi) >> 1;
    return pairwise_sum_f64(a, lo, mid) + pairwise_sum_f64(a, mid + 1, hi);
}

/* compute_loss(::SwitchTransformerLoss) -- src/balancing/losses.jl:15-36.
 * N = number of prob rows; f_e = count_e / length(indices) (Float32);
 * P_e = mean over tokens (sequential Float32 sum over t, divided by T);
 * loss = (alpha * N) * sum_e f_e * P_e. */
float oracle_switch_loss(const int32_t *idx, int64_t T, int k, const float *probs, int N, float alpha)
{
    float *f = (float *)calloc((size_t)N, sizeof(float));
    float *P = (float *)calloc((size_t)N, sizeof(float));
    float *fp = (float *)calloc((size_t)N, sizeof(float));
    if (!f || !P || !fp) { free(f); free(P); free(fp); return NAN; }
    int64_t total = T * (int64_t)k;
    for (int64_t i = 0; i < total; ++i) {
        int32_t e = idx[i];
        if (e > 0 && e <= N) f[e - 1] += 1.0f;
    }
    if (total > 0)
        for (int e = 0; e < N; ++e) f[e] = f[e] / (float)total;
    for (int64_t t = 0; t < T; ++t)
        for (int e = 0; e < N; ++e) P[e] = P[e] + probs[t * N + e];
    for (int e = 0; e < N; ++e) P[e] = P[e] / (float)T;
    for (int e = 0; e < N; ++e) fp[e] = f[e] * P[e];
    float s = pairwise_sum_f32(fp, 0, N - 1); /* sequential for N < 1024 */
    float r = (alpha * (float)N) * s;
    free(f); free(P); free(fp);
    return r;
}

/* compute_loss(::ZLoss) + logsumexp -- src/balancing/losses.jl:103-114.
 * lse_t = max + log(sum(exp(l - max))) in Float32; loss = beta * mean(lse^2). */
float oracle_z_loss(const float *logits, int64_t T, int E, float beta, float *lse_out)
{
    if (T <= 0) return NAN;
    float *sq = (float *)malloc(sizeof(float) * (size_t)T);
    if (!sq) return NAN;
    for (int64_t t = 0; t < T; ++t) {
        const float *l = logits + t * E;
        float m = -INFINITY;
        for (int i = 0; i < E; ++i) if (l[i] > m) m = l[i];
        float s = 0.0f;
        for (int i = 0; i < E; ++i) s = s + (float)exp((double)(l[i] - m));
        float lse = m + (float)log((double)s);
        if (lse_out) lse_out[t] = lse;
        sq[t] = lse * lse;
    }
    float mean = pairwise_sum_f32(sq, 0, T - 1) / (float)T;
    free(sq);
    return beta * mean;
}

/* update_stats! entropy -- src/core/moe_layer.jl:262-263:
 * mean over tokens of -sum_e p*log(p + 1e-8), evaluated in Float64
 * (1e-8 is a Float64 literal), stored as Float32. */
float oracle_mean_entropy(const float *probs, int64_t T, int E)
{
    if (T <= 0) return NAN;
    double *h = (double *)malloc(sizeof(double) * (size_t)T);
    if (!h) return NAN;
    for (int64_t t = 0; t < T; ++t) {
        double s = 0.0;
        for (int e = 0; e < E; ++e) {
            double p = (double)probs[t * E + e];
            s = s + p * log(p + 1e-8);
        }
        h[t] = -s;
    }
    double m = pairwise_sum_f64(h, 0, T - 1) / (double)T;
    free(h);
    return (float)m;
}

/* Weighted combine of process_expert_forward! -- src/core/moe_layer.jl:205-217:
 * out (zero-initialised Float32) accumulates gate * y for each token in
 * ascending expert order, as separate multiply and add (no fused multiply-add).
 * y: [n_valid][D] rows in permutation order; gate of each row taken from the
 * entry it came from. */
void oracle_combine(const float *y, const int32_t *perm, int64_t n_valid, const float *gates,
                    int k, int64_t T, int D, float *out)
{
    memset(out, 0, sizeof(float) * (size_t)T * (size_t)D);
    for (int64_t pos = 0; pos < n_valid; ++pos) {
        int32_t ent = perm[pos];
        int64_t t = ent / k;
        float g = gates[ent];
        const float *yr = y + pos * D;
        float *o = out + t * D;
        for (int d = 0; d < D; ++d) {
            volatile float prod = g * yr[d];
            o[d] = o[d] + prod;
        }
    }
}
