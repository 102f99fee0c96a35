/*
 * moe_mi355x.h -- C ABI of libmoe_mi355x.so, the MI355X (gfx950) MoE-layer
 * forward path behind MixtureOfExperts.jl's API.
 *
 * The reference has no FFI boundary; its seams are Julia multiple-dispatch
 * points.  Each entry point below names the reference function it replaces
 * (paths relative to the MixtureOfExperts.jl repository).  A host shim (Julia
 * via ccall, Python via ctypes) keeps the reference API and calls these.
 *
 * Conventions
 *  - Plain pointers and sizes only.  Every array is dense and row-major in the
 *    token-major order that Julia's column-major matrices already have:
 *    a Julia matrix of size (D, T) is passed as its own memory, [T][D].
 *  - Expert ids are 1-based, as in the reference; 0 marks an entry dropped by
 *    the capacity constraint.  Entry ids are 0-based: entry = t*k + slot.
 *    Positions, counts and offsets are 0-based.
 *  - Every function returns a moe_status; on failure moe_last_error() holds a
 *    message.  Host-pointer entry points block until results are in host
 *    memory.  *_async entry points take device pointers and a hipStream_t
 *    (passed as void*, NULL = the handle's own stream) and only enqueue.
 *  - Calls on one handle are serialised by the library, across streams too
 *    (a call on another stream than the previous async call's waits for that
 *    call's work); distinct handles may be used from distinct threads.  The
 *    async calls that complete a layer (moe_forward_async, moe_decode_async,
 *    moe_stage_combine_async) mark their end with an event of the handle:
 *    their stream may be destroyed as soon as they return.  The stream of
 *    one of the other stage calls must stay valid until the next call on the
 *    handle has returned.  moe_destroy never uses a caller's stream.
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_ABI_VERSION 1
#define MOE_MAX_TOPK 16       /* maximum slots per token of the top-k gates (shared + routed) */
#define MOE_MAX_EXPERTS 512   /* maximum experts of a layer (shared + routed) */

typedef enum {
    MOE_OK = 0,
    MOE_EINVAL = -1,       /* bad argument (shape, range, null pointer) */
    MOE_EOOM = -2,         /* device allocation failed */
    MOE_EHIP = -3,         /* a HIP runtime call failed */
    MOE_ENOTREADY = -4,    /* router or an expert has no weights yet */
    MOE_EUNSUPPORTED = -5  /* valid in the reference, not implemented here */
} moe_status;

typedef enum { MOE_F32 = 0, MOE_BF16 = 1, MOE_FP8_E4M3 = 2 } moe_dtype;

/* Memory order of a weight matrix as the reference holds it.
 * FLUX_OUT_IN: Flux Dense weight of size (out, in), column-major, i.e. memory
 *              [in][out] (src/experts/gated.jl:15-27, src/core/router.jl:18).
 * LLAMA_IN_OUT: Llama2 weight of size (in, out), column-major, i.e. memory
 *              [out][in] (src/llama2/types.jl:207-210). */
typedef enum { MOE_LAYOUT_FLUX_OUT_IN = 0, MOE_LAYOUT_LLAMA_IN_OUT = 1 } moe_layout;

typedef enum { MOE_EXPERT_GATED = 0, MOE_EXPERT_STANDARD = 1 } moe_expert_type;

/* Elementwise activation of the expert FFN (MoEConfig.activation,
 * src/core/moe_layer.jl:10).  GELU is NNlib's tanh form. */
typedef enum { MOE_ACT_GELU = 0, MOE_ACT_SILU = 1, MOE_ACT_RELU = 2, MOE_ACT_IDENTITY = 3 } moe_activation;

/* Gating mechanism (src/gating/topk.jl:16-22, switch.jl:7-11,
 * advanced.jl:7-108, expert_choice.jl:7-53).
 * SOFT: SoftMoEGating(k, lambda): softmax of logits ./ lambda, top-k indices,
 *   and, as the reference's dispatch reads gates[slot, t] of its (E, T) gate
 *   matrix, slot j's gate is the probability of expert j (advanced.jl:17-33).
 * EXPERT_CHOICE: ExpertChoiceGating(capacity_factor): each expert takes the
 *   capacity = ceil(T * cf / E) tokens of largest logit (ties to the lower
 *   token), gate = its softmax probability; a token's slots hold the experts
 *   that took it in ascending id order, at most capacity of them
 *   (expert_choice.jl:11-53).  Slots per token (moe_slots_per_token):
 *   min(E, capacity at max_tokens); a call fills the first min(capacity, E)
 *   of them (the rest, like the reference's rows past them, are empty). */
typedef enum {
    MOE_GATE_TOPK = 0,
    MOE_GATE_SWITCH = 1,
    MOE_GATE_SHARED = 2,
    MOE_GATE_SOFT = 3,
    MOE_GATE_EXPERT_CHOICE = 4
} moe_gate_kind;

/* Mirror of MoEConfig (src/core/moe_layer.jl:4-29) plus device sizing. */
typedef struct {
    int32_t num_experts;        /* E: experts held by the layer */
    int32_t expert_type;        /* moe_expert_type */
    int32_t input_dim;          /* D */
    int32_t hidden_dim;         /* H */
    int32_t output_dim;         /* D_out */
    int32_t activation;         /* moe_activation */
    int32_t gate_kind;          /* moe_gate_kind */
    int32_t top_k;              /* k of the (base) top-k gate */
    int32_t gate_num_shared;    /* SharedExpertGating.num_shared (gate_kind SHARED) */
    int32_t weight_dtype;       /* moe_dtype the expert GEMMs run on */
    float balance_alpha;        /* SwitchTransformerLoss.alpha */
    float z_loss_weight;        /* MoEConfig.z_loss_weight */
    float capacity_factor;      /* MoEConfig.capacity_factor */
    int32_t drop_tokens;        /* MoEConfig.drop_tokens */
    int32_t max_tokens;         /* largest T a call may pass (workspace size) */
    int32_t num_shared_experts; /* MoEConfig.num_shared_experts: experts 1..ns run on every
                                   token (forward_with_shared_experts,
                                   src/core/moe_layer.jl:158-185); the router then has
                                   num_experts - ns outputs, and any gate and balance loss
                                   runs on those (the gate's ids shifted by ns). */
    float gate_param;           /* SoftMoEGating.lambda (SOFT), ExpertChoiceGating.capacity_factor
                                   (EXPERT_CHOICE); unused otherwise */
    int32_t reserved[5];        /* zero */
} moe_config;

typedef struct moe_handle moe_handle;

/* Optional per-call outputs of moe_forward (any pointer may be NULL). */
typedef struct {
    float *logits;          /* [T][E_router] fp32 router logits */
    float *probs;           /* [T][E_router] router probabilities */
    int32_t *indices;       /* [T][k_total] 1-based expert ids (0 = dropped) */
    float *gates;           /* [T][k_total] */
    int32_t *counts;        /* [E] entries per expert this call */
    int32_t *offsets;       /* [E+1] exclusive prefix sum of counts */
    int32_t *perm;          /* [T*k_total] entry id at each position */
    float *switch_loss;     /* scalar, training only */
    float *z_loss;          /* scalar, training only */
    float *mean_entropy;    /* scalar: update_stats! entropy of this call */
} moe_forward_aux;

/* ---- lifecycle -------------------------------------------------------- */

/* MoELayer(config) -- src/core/moe_layer.jl:44-63.  Allocates the device
 * state for one layer on the current HIP device. */
int moe_create(const moe_config *cfg, moe_handle **out);
int moe_destroy(moe_handle *h);
/* Last error message of h (or of the last failed moe_create when h is NULL). */
const char *moe_last_error(const moe_handle *h);
int moe_abi_version(void);
/* Number of router outputs: E, or E - ns with num_shared_experts = ns > 0. */
int moe_router_outputs(const moe_handle *h);
/* Slots per token: k, 1 (Switch), num_shared + k (SharedExpertGating) or
 * min(capacity at max_tokens, E) (ExpertChoiceGating); with
 * num_shared_experts = ns > 0, ns more: the ns shared slots first, with ids
 * 1..ns, then the gate's slots with ids shifted by ns, as expert_indices .+=
 * ns makes them. */
int moe_slots_per_token(const moe_handle *h);

/* ---- weights (uploaded once, prepacked, device resident) --------------- */
/* Weight sources may be host or device memory.  When any source is device
 * memory the call first waits for the whole device (hipDeviceSynchronize), so
 * kernels that produced it on any stream have finished before it is read. */

/* Router weight -- src/core/router.jl:18 Dense(in, E, bias=false):
 * weight (E_router, D) column-major = memory [D][E_router] fp32.  bias may be
 * NULL (the reference router has none; a bias is Dense(W, b)). */
int moe_set_router(moe_handle *h, const float *weight, const float *bias);

/* Router noise in training -- src/core/router.jl:32-41 (Router(...;
 * noise_scale, use_noise_network)).  In training calls with noise_scale > 0
 * the gate sees logits .+ randn .* noise_scale, or, with a noise network
 * (noise_weight != NULL, memory [D][E_router] like the router weight),
 * logits .+ noise_scale .* (randn .* softplus.(noise_weight' x)).  randn is
 * the library's counter-based generator (seed, the handle's training-call
 * number, token, router row), not Julia's stream.  The Switch loss and the
 * statistics use the noisy probabilities; the z-loss the logits without
 * noise (src/core/moe_layer.jl:117-121).  noise_scale = 0 turns the noise
 * off.  A noise network needs 2 * E_router <= MOE_MAX_EXPERTS. */
int moe_set_router_noise(moe_handle *h, float noise_scale, const float *noise_weight, uint64_t seed);

/* StandardExpert's Dropout(p) in training -- src/experts/standard.jl:26,
 * 49-51: in training calls each element of h = act(W1 x .+ b1) is kept,
 * times 1 / (1 - p) in Float32 arithmetic (1 - p rounded, then the quotient,
 * as NNlib's dropout computes it for a Float32 p), with probability 1 - p (a
 * uniform draw > p), else zeroed, before W2.  Draws: the library's counter-based generator
 * (seed, the handle's training-call number, expert-ordered row, column),
 * not Julia's stream.  p = 0 turns it off; StandardExpert handles only. */
int moe_set_expert_dropout(moe_handle *h, float p, uint64_t seed);

/* Expert e (0-based) weights -- GatedExpert (src/experts/gated.jl:6-27):
 * w1 (H,D), w3 (H,D), w2 (D_out,H); StandardExpert (src/experts/standard.jl):
 * w1 (H,D), w2 (D_out,H), b1 (H), b2 (D_out), w3 NULL.
 * src_dtype: F32 (converted to cfg.weight_dtype; FP8 quantises per output
 * channel), BF16, or FP8_E4M3 with per-output-channel fp32 scales s1/s2/s3
 * (value = fp8 * scale[out]); scales are ignored for other dtypes. */
int moe_set_expert(moe_handle *h, int32_t expert, int32_t layout, int32_t src_dtype,
                   const void *w1, const void *w2, const void *w3,
                   const float *b1, const float *b2,
                   const float *s1, const float *s2, const float *s3);

/* AuxiliaryFreeLoss(E; bias_init, learning_rate, momentum, update_freq,
 * use_complementary_loss, complementary_weight) as the layer's balance loss
 * (src/balancing/auxiliary_free.jl:11-34).  With enable != 0, moe_forward
 * gates on logits + bias (get_biased_logits, forward_standard,
 * src/core/moe_layer.jl:137-140; the probabilities, z-loss and statistics stay
 * those of the plain logits), its balance loss is complementary_weight *
 * Switch(1) or 0 (:78-87), and each training call counts one compute_loss:
 * update_counter += 1 and, when it is a multiple of update_freq, the bias
 * update of update_bias! (:36-69) runs on the device over the kept entries.
 * bias / bias_momentum: E_router floats (host), NULL = zeros.  enable = 0
 * restores the loss set at moe_create.  With num_shared_experts > 0 the layer
 * runs forward_with_shared_experts (src/core/moe_layer.jl:158-185): the gate
 * sees the plain logits (no bias), and the loss and update_bias! receive the
 * gate's ids shifted by num_shared_experts, so bias / bias_momentum then hold
 * num_experts floats (the shared experts' entries count no assignment, and an
 * ExpertChoiceGating matrix's empty entries count as expert
 * num_shared_experts, as the shifted zeros do there). */
int moe_set_aux_free(moe_handle *h, int32_t enable, const float *bias, const float *bias_momentum,
                     float learning_rate, float momentum, int32_t update_freq, int64_t update_counter,
                     int32_t use_complementary_loss, float complementary_weight);
/* Read back the AuxiliaryFreeLoss state (E_router floats each, num_experts
 * with num_shared_experts > 0; any pointer may be NULL).  Blocks until the
 * handle's queued work has finished. */
int moe_get_aux_free(moe_handle *h, float *bias, float *bias_momentum, int64_t *update_counter);

/* Expert initialisation strategies of convert_to_moe / create_single_expert
 * (src/llama2/conversion.jl:277-318). */
typedef enum {
    MOE_INIT_COPY = 0,     /* every expert a copy of the dense FFN */
    MOE_INIT_PERTURB = 1,  /* dense .+ randn .* noise_scale */
    MOE_INIT_SPLIT = 2,    /* expert e keeps hidden units [e H / E, min((e+1) H / E, H)), zeros elsewhere */
    MOE_INIT_RANDOM = 3    /* randn .* sqrt(2f0 / dim) */
} moe_init_strategy;

/* convert_layer_to_moe's experts (create_experts_from_layer /
 * create_single_expert, src/llama2/conversion.jl:262-331) made on the device
 * from one dense gated FFN: the dense w1 (H,D), w2 (D_out,H), w3 (H,D) -- in
 * `layout` and src_dtype as for moe_set_expert, host or device memory (NULL
 * for MOE_INIT_RANDOM) -- are read once and every expert of the handle is
 * derived from them and prepacked in cfg.weight_dtype (fp8: per-output-channel
 * scales of the derived weights).  Normal draws come from a counter-based
 * generator keyed by (seed, expert, matrix, element): reproducible for a seed,
 * not Julia's randn stream.  Gated experts only. */
int moe_init_experts_from_dense(moe_handle *h, int32_t layout, int32_t src_dtype, const void *w1, const void *w2,
                                const void *w3, const float *s1, const float *s2, const float *s3, int32_t strategy,
                                float noise_scale, uint64_t seed);

/* Read expert e's prepacked weights back (the save side of save_moe_model,
 * src/llama2/utils.jl:22-67): w1/w2/w3 as (out, in) matrices in `layout`, in
 * the packed dtype (F32 float, BF16 uint16 bits, FP8_E4M3 bytes), s1/s2/s3 the
 * fp8 per-output-channel scales (ignored otherwise).  Any pointer may be NULL.
 * Host pointers; blocking. */
int moe_get_expert(moe_handle *h, int32_t expert, int32_t layout, void *w1, void *w2, void *w3, float *s1, float *s2,
                   float *s3);

/* ---- host-buffer entry points (blocking) -------------------------------- */

/* compute_gates(gate, logits) -- src/gating/topk.jl:24-44,
 * src/gating/switch.jl:9-11, src/gating/advanced.jl:80-108.
 * logits [T][E_router] -> indices/gates [T][k_total], probs [T][E]. */
int moe_compute_gates(moe_handle *h, const float *logits, int32_t T,
                      int32_t *indices, float *gates, float *probs);

/* compute_gates + the bucketing of process_expert_forward!
 * (src/core/moe_layer.jl:192-203), with the capacity constraint
 * (src/core/moe_layer.jl:221-248) when cfg.drop_tokens && training.
 * counts [E], offsets [E+1], perm [T*k_total] (valid prefix offsets[E]). */
int moe_route_from_logits(moe_handle *h, const float *logits, int32_t T, int32_t training,
                          int32_t *indices, float *gates, float *probs,
                          int32_t *counts, int32_t *offsets, int32_t *perm);

/* (moe::MoELayer)(x; training) -- src/core/moe_layer.jl:107-156.
 * x [T][D] in x_dtype (F32 or BF16); out [T][D_out] fp32; *loss = Switch
 * loss + z-loss when training, else 0.  With num_shared_experts = ns > 0 this
 * is forward_with_shared_experts (src/core/moe_layer.jl:158-185): out =
 * 0.5 * sum_i(y_i / ns) + 0.5 * routed, the routed part combined as in
 * forward_standard over experts ns+1..E, no capacity constraint, and the
 * balance loss over the E - ns router probabilities with the gate's shifted
 * ids (ids above E - ns are not counted, src/balancing/losses.jl:22-26; an
 * ExpertChoiceGating matrix's empty entries become id ns and are counted
 * when ns <= E - ns).  1 <= T <= max_tokens, else MOE_EINVAL. */
int moe_forward(moe_handle *h, const void *x, int32_t x_dtype, int32_t T, int32_t training,
                float *out, float *loss, moe_forward_aux *aux);

/* forward_standard with the gate's compute_gates done by the caller
 * (src/core/moe_layer.jl:130-156 with process_expert_forward!, :187-219): for
 * gates whose indices come from host code -- HashGating's hash function,
 * RandomGating's sampler (src/gating/advanced.jl:37-66, simple.jl:7-28).
 * The router GEMM still runs (logits for aux and the z-loss); indices [T][kd]
 * 1-based (ids outside 1..E are skipped, :198; an id repeated within a token
 * is MOE_EUNSUPPORTED), gates [T][kd], probs [T][E] for the Switch loss and
 * the statistics (NULL: ones ./ E).  The capacity constraint applies as in
 * moe_forward.  kd <= MOE_MAX_TOPK and T * kd <= max_tokens * slots. */
int moe_forward_routed(moe_handle *h, const void *x, int32_t x_dtype, int32_t T, int32_t training,
                       const int32_t *indices, const float *gates, int32_t kd, const float *probs, float *out,
                       float *loss, moe_forward_aux *aux);

/* (e::Expert)(x) on a block of tokens -- src/experts/gated.jl:29-34,
 * src/experts/standard.jl:38-55.  x [n][D] fp32 -> y [n][D_out] fp32 through
 * the device expert path of expert e (0-based). */
int moe_expert_forward(moe_handle *h, int32_t expert, const float *x, int32_t n, float *y);

/* The decode caller: moe_ffn_forward! (src/llama2/inference.jl:58-121)
 * after its rmsnorm.  Each of the n tokens is routed
 * on its own (logits = W_router' xb with the router set by moe_set_router,
 * then compute_gates, src/gating/topk.jl:24-44) and the gated experts of its
 * k slots are combined in slot order on a zero start (:83-104):
 * out = ((0 + g_1 y_1) + g_2 y_2) + ..., y = W2 (silu(W1 xb) .* (W3 xb)),
 * silu(g) = g * (1 / (1 + exp(-g))) (gated_expert_forward!, :154-167).
 * With num_shared_experts = ns > 0 the layer's shared experts are
 * process_shared_experts! (:184-216): shared = sum_i (1f0/ns) * y_i, out =
 * 0.5f0 * shared + 0.5f0 * out; the slots then hold the shared experts 1..ns
 * first and the routed ones shifted by ns.
 * xb [n][D] fp32, out [n][D_out] fp32 (host); logits [n][E_router], indices
 * [n][slots] (1-based), gates [n][slots] may be NULL.  Gated experts with TopKGating or
 * SwitchGating only (else MOE_EUNSUPPORTED); 1 <= n <= max_tokens (handles
 * with bf16 or fp8 weights: max_tokens / 2). */
int moe_decode(moe_handle *h, const float *xb, int32_t n, float *out, float *logits, int32_t *indices,
               float *gates);

/* compute_loss(::SwitchTransformerLoss, indices, probs) --
 * src/balancing/losses.jl:15-36.  indices [T][k] 1-based (entries outside
 * 1..E are not counted), probs [T][E]; no handle needed.  Host pointers. */
int moe_switch_loss(const int32_t *indices, int32_t T, int32_t k, const float *probs, int32_t E, float alpha,
                    float *loss);

/* compute_loss(::ZLoss, logits) -- src/balancing/losses.jl:103-114.
 * logits [T][E]; *loss = beta * mean_t(logsumexp_t^2).  Host pointers. */
int moe_z_loss(const float *logits, int32_t T, int32_t E, float beta, float *loss);

/* The bias step of update_bias!(::AuxiliaryFreeLoss, indices)
 * (src/balancing/auxiliary_free.jl:44-69), without its update_counter check
 * (the caller keeps the counter): indices [n] 1-based (entries <= 0 are not
 * counted, an id above E is MOE_EINVAL as Julia's BoundsError), bias and
 * bias_momentum [E] updated in place.  Host pointers. */
int moe_aux_free_update_bias(const int32_t *indices, int64_t n, int32_t E, float learning_rate, float momentum,
                             float *bias, float *bias_momentum);

/* ---- allocation-free entry point ----------------------------------------- */

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): compute_loss(::SwitchTransformerLoss, indices, probs) as
 * moe_switch_loss computes it (the same kernels, bit for bit), on device
 * buffers indices_dev [T][k], probs_dev [T][E] and loss_dev (1 float),
 * enqueued on `stream` (hipStream_t; NULL = the null stream).  Its partial
 * sums live in a fixed device array of the library,
 * MOE_SWITCH_LOSS_SCRATCH_BYTES per GPU, held until the process ends, instead
 * of a per-call allocation.  E <= MOE_MAX_EXPERTS (else MOE_EINVAL).  Every
 * call on one GPU shares that array: calls that overlap on one GPU (other
 * streams, other threads) race.  The first call on a device looks the array
 * up (hipGetSymbolAddress): make it outside stream capture. */
#define MOE_SWITCH_LOSS_SCRATCH_BYTES (64 * MOE_MAX_EXPERTS * 12)
int moe_switch_loss_noalloc(const int32_t *indices_dev, int32_t T, int32_t k, const float *probs_dev, int32_t E,
                            float alpha, float *loss_dev, void *stream);

/* ---- device-buffer entry points (enqueue only) -------------------------- */

/* moe_forward on device buffers: x_dev [T][D], out_dev [T][D_out] fp32,
 * loss_dev (1 float) may be NULL.  Runs on `stream` (hipStream_t). */
int moe_forward_async(moe_handle *h, const void *x_dev, int32_t x_dtype, int32_t T,
                      int32_t training, float *out_dev, float *loss_dev, void *stream);

/* moe_decode on device buffers: xb_dev [n][D] fp32 (16-byte aligned),
 * out_dev [n][D_out] fp32.  Runs on `stream` (hipStream_t). */
int moe_decode_async(moe_handle *h, const float *xb_dev, int32_t n, float *out_dev, void *stream);

/* Stage-level entry points for profiling: together they issue exactly the
 * kernels of moe_forward_async, one stage per call, on device buffers owned
 * by the handle.  Call them in forward order (router, permute, expert_up,
 * expert_down, combine) after a moe_forward_async on the same handle with the
 * same T.  router = logits GEMM + gating + scan; permute = gather into
 * expert-contiguous rows; expert_up/down = the two grouped GEMMs; combine =
 * the weighted scatter back to token order. */
int moe_stage_router_async(moe_handle *h, const void *x_dev, int32_t x_dtype, int32_t T,
                           int32_t training, void *stream);
int moe_stage_permute_async(moe_handle *h, const void *x_dev, int32_t x_dtype, int32_t T,
                            void *stream);
int moe_stage_expert_up_async(moe_handle *h, int32_t T, void *stream);
int moe_stage_expert_down_async(moe_handle *h, int32_t T, void *stream);
int moe_stage_combine_async(moe_handle *h, int32_t T, float *out_dev, void *stream);

/* Per-token logsumexp of the last routing call's logits (the z-loss's
 * lse_t = max + log(sum(exp(l - max))), src/balancing/losses.jl:111-114;
 * with router noise, of the logits without noise) -> lse [T] float, host
 * memory.  T must be that call's token count.  Blocking. */
int moe_router_lse(moe_handle *h, int32_t T, float *lse);

/* Copy the per-expert counts of the last call to host memory (int32 [E]). */
int moe_read_counts(moe_handle *h, int32_t *counts);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355X_H */
