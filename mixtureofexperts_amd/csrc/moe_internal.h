// moe_internal.h -- device helpers and launcher declarations shared by the
// translation units of libmoe_mi355x.so.  gfx950 (CDNA4) only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_mi355x.h"

namespace moe {

constexpr int kRtThreads = 512;    // threads per router_kernel workgroup (8 per token)
constexpr int kRtMinBlock = 16;    // fewest tokens per router_kernel workgroup
constexpr int kPermThreads = 1024; // threads per permute workgroup: one wave per token
constexpr int kPermTokens = kPermThreads / 64;  // tokens per permute workgroup (divides every route block)
constexpr int kSuper = 16;         // route blocks per super block (rank bases: super rows, then block rows)
// Fixed-point scale of the per-expert probability sums (2^32).  A call's
// total for one expert is at most T * 2^32 < 2^63 for every T the handle
// accepts (max_tokens * slots <= INT_MAX / 2), so the unsigned 64-bit totals
// cannot wrap; each route block's sum is rounded once, by at most 2^-33, far
// below one fp32 ulp of the mean probability.
constexpr double kPsumScale = 4294967296.0;
constexpr int kGemmBM = 128;       // fp32 / fp8-weight grouped-GEMM tile rows (token rows)
constexpr int kGemmBN = 128;       // fp32 / fp8-weight grouped-GEMM tile columns
constexpr int kKPad = 64;          // K padding of packed weights and activation rows
constexpr int kNPadGated = 128;    // N padding of W1/W3 (bf16 gated up tile: 128 h columns)
constexpr int kNPad = 256;         // N padding of every other packed weight (bf16 tile: 256 rows)

enum ComputeType { CT_F32 = 0, CT_BF16 = 1 };
enum WeightType { WT_F32 = 0, WT_BF16 = 1, WT_FP8 = 2 };
enum GemmMode { MODE_GATED_UP = 0, MODE_STD_UP = 1, MODE_DOWN = 2 };

// ---- scalar conversions (host and device) -----------------------------------

// fp32 -> bf16, round to nearest even; NaN stays NaN.
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__host__ __device__ inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
}

// OCP fp8 e4m3fn -> fp32, exact.  Encodings 0x7f/0xff (NaN) are never
// produced by the library's quantiser (it saturates at +-448).
__host__ __device__ inline float fp8e4m3_to_f32(uint8_t b) {
    uint32_t em = b & 0x7fu;
    float v;
    if (em >= 8u) {
        uint32_t u = (em << 20) + (120u << 23);
        __builtin_memcpy(&v, &u, 4);
    } else {
        v = (float)em * 0.001953125f;  // subnormal: m * 2^-9
    }
    return (b & 0x80u) ? -v : v;
}

// Counter-based generator: a splitmix64 hash of (seed, stream, index).
__device__ inline unsigned long long rng_hash(unsigned long long seed, unsigned long long stream, unsigned long long i) {
    unsigned long long z = seed + 0x9E3779B97F4A7C15ull * (stream + 1) + 0xD1B54A32D192ED03ull * i;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// Standard normal for (seed, stream, index): the hash's two 24-bit uniforms
// in (0, 1), Box-Muller gives N(0, 1).
__device__ inline float init_normal(unsigned long long seed, unsigned long long stream, unsigned long long i) {
    const unsigned long long z = rng_hash(seed, stream, i);
    const float u1 = ((float)(z >> 40) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = ((float)(z & 0xFFFFFFull) + 0.5f) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}
// Uniform in (0, 1) for (seed, stream, index): the hash's top 24 bits.
__device__ inline float init_uniform(unsigned long long seed, unsigned long long stream, unsigned long long i) {
    return ((float)(rng_hash(seed, stream, i) >> 40) + 0.5f) * (1.0f / 16777216.0f);
}

// Julia `isless` total order as an unsigned key: every NaN is largest,
// -0.0 < +0.0 (src/gating/topk.jl:35 partialsortperm, rev=true).
__host__ __device__ inline uint32_t isless_key(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---- kernel argument blocks --------------------------------------------------

// Router logits GEMM: x [T][D] (bf16 or fp32) times the router weight split
// into three bf16 parts, held as the fragment image of router_split_kernel
// (Dp = D rounded up to 32).
struct RouterArgs {
    const void *x; int x_bf16; int T, D, Er, Ep, Dp;
    const uint16_t *ws;
};

// Outputs of one gating pass of router_kernel.  A plain forward writes both;
// with an AuxiliaryFreeLoss the probabilities pass runs on the router logits
// and the gating pass on logits + the loss's bias (src/core/moe_layer.jl:137-140).
enum { ROUTE_OUT_PROBS = 1,    // logits, probs, probability sums, per-block z / entropy sums
       ROUTE_OUT_GATING = 2 }; // indices, gates, ranks, per-block and total expert counts

struct RouteArgs {
    const float *part;     // [T][Er] the caller's router logits (when no logits GEMM runs)
    const float *bias;     // [Er] or null
    float *logits;         // [T][Er] out: logits + bias
    int T, Er;
    int E;                 // probability rows (= Er)
    int Eh;                // experts of the histogram: E + lsh
    int gate_kind, k, ns, kt;
    int lsh;               // shared experts of the layer (slots 0..lsh-1 of every token)
    int out_mask;          // ROUTE_OUT_*: which outputs this pass writes
    float soft_lambda;     // SoftMoEGating: the softmax runs on logits / lambda
    int given;             // idx / gates hold the caller's routing (no top-k); probs from
    int given_probs;       //   a.probs when given_probs, else 1/E
    float *probs;          // [T][E]
    float *lse;            // [T] per-token logsumexp of the z-loss's logits (probabilities pass), or null
    int *idx;              // [T][kt]
    float *gates;          // [T][kt]
    int *rank;             // [T][kt] rank of the entry inside its block & expert
    int *blk_counts;       // [nblk][ldc]: entries per expert (columns < Eh)
    int ldc;               // row stride of blk_counts (Eh rounded up to 4)
    double *blk_zh;        // [nblk][2]: the route block's sums of lse^2 and of the entropy
    // totals per super block of kSuper route blocks, by integer atomics
    // (order-free, so deterministic; kSuper route blocks per address instead
    // of all of them): entries per expert sup_cnt [nsup][ldc] and probability
    // sums per router row sup_p [nsup][ldc] in fixed point (kPsumScale).  The
    // call's parity of two buffers, and the other parity's (cleared for the
    // next call: route block b takes the rows b, b + nblk, ... < nsup_max).
    // The permute's scan adds the rows.
    int *sup_cnt;
    unsigned long long *sup_p;
    int *clr_sup;
    unsigned long long *clr_supp;
    int nsup_max;
};

// The scan of a routing call, run by every permute workgroup (its route
// block's rank bases, the offsets and tile starts) and, for the outputs and
// losses, by workgroup 0.
struct ScanArgs {
    const int *blk_counts;  // [nblk][ldc]
    int ldc;
    const double *blk_zh;   // [nblk][2]
    const int *sup_cnt;     // [nsup][ldc] entries per expert of each super block (before capacity)
    const unsigned long long *sup_p;  // [nsup][ldc] probability sums per router row, fixed point
    int nsup;               // super blocks of the call: ceil(nblk / kSuper)
    int nblk, T, E, kt;   // E: experts of the histogram
    int Np, lsh, kl;      // Switch loss: probability rows N, shared experts of the layer, router slots per token
    int ec_empty;          // ExpertChoiceGating with shared experts: the (kl, T) index matrix's empty
                           // entries, shifted to id lsh, count as expert lsh (losses and update_bias!)
    int training, drop, z_enabled;
    float capacity_factor, alpha, beta;
    int bm;                // GEMM tile rows
    int *tile_start;       // [E+1] first M tile of each expert (sum of ceil(count / bm))
    int *item_start;       // [E+1] or null: the up GEMM's paired work items before each expert (pair_nt n-tiles)
    int pair_nt;
    int *counts;           // [E]   (after capacity)
    int *offsets;          // [E+1]
    int *cap_out;          // [1] capacity (INT_MAX when unused)
    int2 *tiles;           // [max_tiles] (expert, m0)
    int *num_tiles;        // [1]
    float *scalars;        // [4]: switch, z, loss, mean entropy
    float *loss_out;       // optional extra destination of the loss
    // AuxiliaryFreeLoss (src/balancing/auxiliary_free.jl): balance loss =
    // complementary_weight * Switch(1) when use_complementary, else 0; the
    // update_bias! step of this call when aux_update (training only)
    int aux_free, aux_use_comp, aux_update;
    float aux_cw, aux_lr, aux_momentum;
    float *aux_bias, *aux_mom;  // [E] device state (the shared experts' entries, lsh > 0, count nothing)
};

// One router_kernel launch: logits (GEMM of g, or r.part), then one or two
// gating passes over TB-token workgroups (route blocks).
struct RtArgs {
    RouteArgs r;           // gating (r.out_mask: outputs of the single pass)
    RouterArgs g;          // logits GEMM (when the kernel computes the logits)
    int TB;                // tokens per workgroup: 16 (paired logits GEMM, over 256 GEMM columns), 32 or 64
    int ncu;               // CUs (64-token workgroups fewer than this: 32-token ones)
    int KP, RB, dma;       // x staging: K columns per pass, LDS bytes per row, by global_load_lds
    int RW;                // LDS row stride of the logits / probability rows (floats)
    int off_L;             // LDS byte offset of the logits rows
    int off_M;             // LDS byte offset of the rank bitmasks (Eh x kRtMaskWords words)
    int npass;             // 2: AuxiliaryFreeLoss (probabilities pass, then gating on logits + aux_bias)
    const float *aux_bias; // [Er]
    int store_rows;        // write logits / probs [T][Er] to global memory
    // router noise in training (src/core/router.jl:32-41): noise_scale > 0
    // adds noise_scale * randn (noise_net: noise_scale * (randn *
    // softplus(noise logits)), the noise logits in GEMM columns Er .. 2 Er - 1)
    // to the logits the gate sees; randn = init_normal(noise_seed,
    // noise_call, token * Er + expert)
    float noise_scale;
    int noise_net;
    unsigned long long noise_seed, noise_call;
};

struct PermuteArgs {
    const void *x; int x_bf16;   // [T][D]
    int T, D, ld_xp, kt, E;
    int ct;                      // compute type of xp
    int *idx; float *gates;      // [T][kt] (rewritten under capacity)
    const int *rank;             // [T][kt] rank inside the route block and expert
    int rb;                      // tokens per route block (a multiple of kPermTokens)
    int tpw;                     // tokens per workgroup (set by launch_permute)
    ScanArgs s;                  // the scan (route-block rows and totals)
    int renorm;                  // capacity active: renormalise gates
    int *perm;                   // [T*kt]
    int *pos_of;                 // [T*kt] (-1 = dropped)
    float *gate_sorted;          // [T*kt]
    void *xp;                    // [rows][ld_xp]
    int copy_rows;               // 0: only the index arrays
    // xp as the bf16 GEMM kernel's A tile image (tiled != 0): the row of
    // expert e's rank rk is row (rk mod bm) of M tile tile_start[e] + rk / bm,
    // ktt = 32-wide K stages per row
    int tiled, bm, ktt;
};

// Tail split of the bf16 GEMMs.  W work items (tiles, or the up GEMM's
// paired items) run on ncu workgroup slots (one per CU for 256-row tiles, two
// for 128-row tiles); the rem = W mod ncu items of the last, partial round
// are each split into S K ranges (the largest S <= smax with S dividing the K
// stages and rem * S <= ncu), so that round is as long as 1/S of a tile.
// Items are numbered in the work list's order (expert-major); items >=
// nfull are split.  Down GEMM: K range 0 of a split tile writes y, range r >= 1
// writes its partial to split_ws block j (S - 1) + r - 1 (j = tile - nfull; a
// block is BM x 256 fp32, row stride 256); fold_split_kernel then adds them
// to y in range order.  With a bf16 y every K range r of a split tile writes
// its partial to block j S + r, and the fold rounds their sum once.  Up GEMM:
// every range writes block j S + r in fragment order, and fold_up_kernel
// sums them and runs the epilogue.
struct TailSplit {
    int nfull;   // tiles not split
    int S;       // K ranges of each split tile (1: none)
};
__host__ __device__ inline TailSplit tail_split(int W, int ncu, int smax, int stages) {
    TailSplit t{W, 1};
    const int rem = (ncu > 0) ? W % ncu : 0;
    if (rem == 0 || smax < 2) return t;
    for (int s = smax; s > 1; --s)
        if (rem * s <= ncu && stages % s == 0) {
            t.nfull = W - rem;
            t.S = s;
            return t;
        }
    return t;
}
constexpr int kDownSplitMax = 4;
// The up GEMM's tail split: K ranges of a split tile (its partials are BM x
// 256 floats per range in fragment order; fold_up_kernel sums them and runs
// the tile's epilogue).
constexpr int kUpSplitMax = 8;
// The fp32 grouped GEMM's K split (small tile grids): at most this many ranges.
constexpr int kF32SplitMax = 8;

struct CombineArgs {
    const void *y; int ld_y;     // [rows][ld_y], fp32 or (y_bf16) bf16
    int y_bf16;
    const int *idx; const int *pos_of; const float *gates;
    int T, D, kt;
    int lsh;                     // > 0: out = 0.5 * sum(y_shared / lsh) + 0.5 * routed
    float *out;                  // [T][D]
    int u, nchunk;               // set by launch_combine: 4-column groups per lane, column chunks per token
};

struct GemmArgs {
    const void *A; long long lda;        // activations [rows][lda] (elements); bf16 kernel: A tile image
    const void *B0; const void *B1;      // packed weights [E][Npad][ldb]; bf16 kernel: B tile images
    long long b_stride;                  // elements per expert
    long long ldb;                       // = padded K
    const float *s0; const float *s1;    // per-output-channel scales [E][Npad] or null
    const float *bias;                   // [E][Npad] or null
    long long s_stride;                  // = Npad
    int N;                               // real N (store bound)
    int K;                               // padded K (multiple of the tile K)
    void *C; long long ldc;              // output [rows][ldc]; bf16 up GEMMs: h as the down GEMM's A
                                         // tile image (ldc = its K)
    const int2 *tiles; const int *num_tiles; const int *counts; const int *offsets;
    const int *tile_start;               // [E+1] (bf16 kernel work list)
    const int *item_start;               // [E+1] or null: the up GEMM's paired items (256-row tiles, n_tiles even)
    int E;
    int m_tiles_grid; int n_tiles;
    int ksplit;                          // bf16 kernel: the most K ranges a tail tile may be split into (tail_split)
    int ncu;                             // workgroup slots of one round (CUs x workgroups per CU)
    float *split_ws;                     // partials of split tiles (ksplit > 1)
    long long split_cap;                 // fp32 kernel: floats of split_ws (its K split fits within)
    int act;
    int c_bf16;                          // MODE_DOWN: y in bf16 (else fp32)
    // MODE_STD_UP in training: StandardExpert's Dropout(drop_p)
    // (src/experts/standard.jl:49-51): element (row pos, column n) of h is
    // kept, times drop_scale = Float32(1 / (1 - p)), when
    // init_uniform(drop_seed, drop_call, pos N + n) > p, else 0
    float drop_p, drop_scale;
    unsigned long long drop_seed, drop_call;
};

__device__ inline float dropout_h(const GemmArgs &g, long long pos, int n, float v) {
    if (g.drop_p > 0.0f) {
        const float u = init_uniform(g.drop_seed, g.drop_call, (unsigned long long)pos * g.N + n);
        v = (u > g.drop_p) ? v * g.drop_scale : 0.0f;
    }
    return v;
}

// Decode (moe_ffn_forward!, src/llama2/inference.jl:58-121): n tokens, each
// routed and combined on its own, slots in order.
struct DecodeArgs {
    const float *x; int D;               // [n][D] fp32 (the rmsnorm'd xb)
    int n, kt, k, E;                     // E: router outputs (routed experts)
    int lsh;                             // shared experts (slots 0..lsh-1, experts 0..lsh-1); routed
                                         // expert e is expert lsh + e of the weights
    const float *wr; int Er_pad;         // router weight [D][Er_pad] fp32
    const float *br;                     // router bias [E] or null
    float *logits, *probs;               // [n][E]
    int *idx; float *gates;              // [n][kt] (1-based expert ids)
    int wt;                              // weight type (WT_*)
    const void *w1, *w3, *w2;            // packed [E][Npad][Kpad]
    long long w1_stride, w2_stride;      // elements per expert
    int Dpad, H, Hpad, Dout;
    const float *s1, *s3, *s2;           // fp8 per-row scales [E][Hpad] / [E][Dout_npad] or null
    int Dout_npad;
    float *h;                            // [n * kt][Hpad] fp32
    float *out;                          // [n][Dout] fp32
};

// ---- launchers ----------------------------------------------------------------
// the router weight [D][Er_pad] fp32 -> the fused router's fragment image of
// its three bf16 parts ((Dp / 32) * tiles per step KB, at most 3 * Ep * Dp * 2 B)
hipError_t launch_router_split(const float *w, int D, int Er, int Er_pad, int Dp, uint16_t *img, hipStream_t s);
// the routing call's router_kernel launch; *tb receives the tokens per
// workgroup (route block) it chose
hipError_t launch_router(RtArgs a, int *tb, hipStream_t s);
// ExpertChoiceGating on logits / probs [T][E] of the E routed experts, after
// the layer's lsh shared experts: sel [T][E] bytes (work), idx / gates
// [T][kt] (kt >= lsh + min(C, E): the shared slots, then the routed ones, ids
// shifted by lsh; the slots past lsh + min(C, E) empty), and the bucketing
// inputs of the scan over the lsh + E experts: rank [T][kt] (rank of each
// entry among its expert's entries in its route block), blk_counts
// [nblk][ldc] and the totals per super block sup_cnt [nsup][ldc] (atomic adds)
hipError_t launch_expert_choice(const float *logits, const float *probs, int T, int E, int lsh, int C, int kt,
                                uint16_t *sel, int *idx, float *gates, int *rank, int *blk_counts, int ldc,
                                int *sup_cnt, int rb, hipStream_t s);
hipError_t launch_permute(PermuteArgs a, hipStream_t s);
hipError_t launch_combine(const CombineArgs &a, hipStream_t s);
// compute_loss(::SwitchTransformerLoss) on device buffers in two launches
// (per-block partial counts and probability sums, then their fold in block
// order); `partials` holds switch_loss_scratch_bytes(T, E) bytes, written
// before they are read (no clearing needed).  E <= MOE_MAX_EXPERTS.
constexpr int kSwitchLossMaxBlocks = 64;
int switch_loss_blocks(long long T);
inline size_t switch_loss_sum_bytes(int nb, int E) { return sizeof(double) * (size_t)nb * E; }
inline size_t switch_loss_scratch_bytes(long long T, int E) {
    const int nb = switch_loss_blocks(T);
    return switch_loss_sum_bytes(nb, E) + sizeof(int) * (size_t)nb * E;
}
hipError_t launch_switch_loss(const int *idx, int T, int k, const float *probs, int E, float alpha, void *partials,
                              float *out, hipStream_t s);
hipError_t launch_z_loss(const float *logits, int T, int E, float beta, float *out, hipStream_t s);
// update_bias!(AuxiliaryFreeLoss, indices) on given indices [n] (entries > 0 counted)
hipError_t launch_aux_free_update(const int *idx, long long n, int E, float lr, float momentum, float *bias,
                                  float *mom, hipStream_t s);
// fp32 activations x fp32 weights (the reference-precision path)
hipError_t launch_grouped_gemm_f32(int mode, const GemmArgs &g, hipStream_t s);
// bf16 activations x bf16 weights; bm = 128 or 256 rows per tile (the scan's bm)
hipError_t launch_grouped_gemm_bf16(int mode, int bm, int wfp8, const GemmArgs &g, hipStream_t s);
// after a MODE_DOWN launch with ksplit > 1: y of each split tile += its partials, in range order
hipError_t launch_fold_split(int bm, const GemmArgs &g, hipStream_t s);
// one expert's packed weight matrix (Npad x Kp, esz-byte elements) -> the
// bf16 kernel's B tile image (RB-row blocks: 128 for gated W1 / W3, else 256)
hipError_t launch_retile_weights(const void *src, void *dst, int Npad, int Kp, int esz, int RB, hipStream_t s);
// decode: routing fused into the gated up products of each selected slot, then
// the down products and the slot-order combine (two kernels); `done`, when not
// null, is recorded at the end of the second
hipError_t launch_decode_ffn(const DecodeArgs &a, int ncu, hipStream_t s, hipEvent_t done = nullptr);

}  // namespace moe
