"""Writes tests/golden/routing_cases.json: known-answer routing cases.

MixtureOfExperts.jl ships no numeric golden vectors (its tests draw unseeded
randn and check invariants), so these cases are crafted so that the expected
indices, gates and probabilities follow by hand from the reference's rules,
without running any implementation:
  - softmax p = exp(l - max) / sum (src/gating/topk.jl:27);
  - top-k on p, descending, ties to the lower expert index
    (partialsortperm(..., rev=true), src/gating/topk.jl:35);
  - gates p_sel / sum(p_sel) (src/gating/topk.jl:39-40);
  - SharedExpertGating (src/gating/advanced.jl:80-108).
Each expected value below is a literal with the derivation in its comment.
"""
import json
import os

INF = float("inf")

CASES = [
    # two equal maxima: p2 == p3, gates p/(p+p) = 0.5 exactly
    dict(name="exact_tie_two_way", logits=[[1.0, 3.0, 3.0, 2.0]], k=2, indices=[[2, 3]], gates=[[0.5, 0.5]]),
    # tie at the k-th place: experts 2,3,4 tie; the lowest index (2) wins
    dict(name="tie_at_kth", logits=[[5.0, 1.0, 1.0, 1.0]], k=2, indices=[[1, 2]]),
    # all equal: p = exp(0)/8 = 0.125 exactly, first k experts, gates 0.5
    dict(name="all_equal_E8_k2", logits=[[0.0] * 8], k=2, indices=[[1, 2]], gates=[[0.5, 0.5]],
         probs=[[0.125] * 8]),
    # strictly increasing logits: top-3 are 8, 7, 6 in that order
    dict(name="descending_pick", logits=[[0.0, 1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0]], k=3, indices=[[8, 7, 6]]),
    # -0.0 and +0.0 give identical exp(0) = 1, p = 0.5 each: tie -> expert 1, gate p/p = 1
    dict(name="signed_zero", logits=[[-0.0, 0.0]], k=1, indices=[[1]], gates=[[1.0]], probs=[[0.5, 0.5]]),
    # k = E: all experts in descending-probability order
    dict(name="k_equals_E", logits=[[3.0, 1.0, 2.0]], k=3, indices=[[1, 3, 2]]),
    # Switch (k = 1) with a tie for the maximum between experts 2 and 4
    dict(name="switch_tie", logits=[[0.0, 2.0, 1.0, 2.0]], k=1, indices=[[2]], gates=[[1.0]]),
    # huge logits: exp(0) = 1 for both 1e30 entries, exp(-1e30 - 1e30) = 0
    dict(name="large_magnitude", logits=[[1e30, -1e30, 0.0, 1e30]], k=2, indices=[[1, 4]], gates=[[0.5, 0.5]],
         probs=[[0.5, 0.0, 0.0, 0.5]]),
    # exp(-200) underflows float32 to 0: experts 2..4 all tie at p = 0 -> 2, 3
    dict(name="underflow_ties", logits=[[0.0, -200.0, -300.0, -250.0]], k=3, indices=[[1, 2, 3]],
         gates=[[1.0, 0.0, 0.0]], probs=[[1.0, 0.0, 0.0, 0.0]]),
    # +Inf logit: NNlib's non-finite branch makes p = 1 on the +Inf entry, 0 elsewhere
    dict(name="plus_inf", logits=[[0.0, INF, 1.0, -1.0]], k=2, indices=[[2, 1]], gates=[[1.0, 0.0]],
         probs=[[0.0, 1.0, 0.0, 0.0]]),
    # SharedExpertGating(2, TopKGating(2), 6): routed rows 3..6 = [0, 4, 4, 1] ->
    # routed picks (4, 5) with gate 0.5 each, scaled by 1 - 2/4 = 0.5 -> 0.25;
    # shared gates 1/4 = 0.25
    dict(name="shared_2_plus_top2", logits=[[9.0, 9.0, 0.0, 4.0, 4.0, 1.0]], k=2, num_shared=2,
         indices=[[1, 2, 4, 5]], gates=[[0.25, 0.25, 0.25, 0.25]]),
    # 256 equal logits: p = exp(0)/256 = 2^-8 exactly; the first 16 experts;
    # their sum 16 * 2^-8 = 2^-4 is exact, so every gate is 2^-8 / 2^-4 = 1/16
    dict(name="all_equal_E256_k16", logits=[[0.0] * 256], k=16, indices=[list(range(1, 17))],
         gates=[[0.0625] * 16], probs=[[0.00390625] * 256]),
    # 512 equal logits: p = 2^-9; the first 9 experts; the partial sums j * 2^-9
    # are exact, so a gate is 2^-9 / (9 * 2^-9) = Float32(1/9) (one rounding)
    dict(name="all_equal_E512_k9", logits=[[0.0] * 512], k=9, indices=[list(range(1, 10))],
         gates=[[0.1111111119389534] * 9]),
    # 300 strictly increasing logits 0, 1, ..., 299: the top 16 are experts
    # 300, 299, ..., 285 in that order
    dict(name="descending_pick_E300_k16", logits=[[float(i) for i in range(300)]], k=16,
         indices=[list(range(300, 284, -1))]),
    # SharedExpertGating(1, TopKGating(8), 257) on equal routed logits: the
    # routed rows 2..257 all have p = 2^-8, the first 8 of them (ids 2..9) with
    # gate 1/8 exactly, times 1 - 1/9 in Float64 = Float32(1/9); the shared
    # expert's gate 1.0f0 / 9 = Float32(1/9) as well
    dict(name="shared_1_plus_top8_E257", logits=[[5.0] + [0.0] * 256], k=8, num_shared=1,
         indices=[list(range(1, 10))], gates=[[0.1111111119389534] * 9]),
    # several tokens at once, each its own case
    dict(name="multi_token", logits=[[1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 1.0], [1.0, 1.0, 1.0]], k=1,
         indices=[[1], [2], [3], [1]], gates=[[1.0], [1.0], [1.0], [1.0]]),
]


def main():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "routing_cases.json")
    with open(path, "w") as f:
        json.dump(CASES, f, indent=1)
    print(path)


if __name__ == "__main__":
    main()
