// moe_route.hip -- router logits, gating (softmax + top-k + renormalisation),
// per-expert histogram / stable ranks, the single-block scan that turns them
// into offsets, GEMM tile lists and the balance losses, the permute (gather)
// into expert-contiguous rows and the deterministic weighted combine.
//
// Semantics follow MixtureOfExperts.jl:
//   Router                src/core/router.jl:25-46
//   compute_gates (TopK)  src/gating/topk.jl:24-44, Switch src/gating/switch.jl:9-11
//   SharedExpertGating    src/gating/advanced.jl:80-108
//   bucketing / combine   src/core/moe_layer.jl:187-219
//   capacity constraint   src/core/moe_layer.jl:221-248
//   Switch loss / z-loss  src/balancing/losses.jl:15-36, 103-114
//   routing entropy       src/core/moe_layer.jl:250-264
#include <algorithm>
#include <climits>

#include "moe_internal.h"

namespace moe {

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// ============================================================================
// Router logits on MFMA at fp32 accuracy.
//
// The fp32 router weight is split once, at upload, into three bf16 parts,
// W = W0 + W1 + W2 exactly (W0 = bf16(W), W1 = bf16(W - W0), W2 = bf16(W - W0
// - W1); each difference is exact in fp32 and the three 8-bit significands
// cover fp32's 24).  bf16 activations are exact in bf16, so x.W = x.W0 + x.W1
// + x.W2 is three bf16 MFMAs per tile whose products are exact and whose sums
// are fp32: the same accuracy as an fp32 dot product, in another summation
// order.  fp32 activations are split the same way and the six cross terms of
// order <= 2^-16 are kept (the three dropped ones are below 2^-24 relative).
// ============================================================================
typedef __bf16 rbf16x8_t __attribute__((ext_vector_type(8)));
typedef float rf32x4_t __attribute__((ext_vector_type(4)));
constexpr int kRouterLdsPieces = 4096;  // 16-byte weight pieces per chunk (64 KB)

__global__ void router_split_kernel(const float *__restrict__ w, int D, int Er, int Er_pad, int Ep, int Dp,
                                    uint16_t *__restrict__ ws) {
#pragma clang fp contract(off)
    const long long n = (long long)Ep * Dp;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
        const int e = (int)(i / Dp), d = (int)(i - (long long)e * Dp);
        const float v = (e < Er && d < D) ? w[(long long)d * Er_pad + e] : 0.0f;
        const uint16_t b0 = f32_to_bf16(v);
        const float r1 = v - bf16_to_f32(b0);
        const uint16_t b1 = f32_to_bf16(r1);
        const float r2 = r1 - bf16_to_f32(b1);
        ws[i] = b0;
        ws[n + i] = b1;
        ws[2 * n + i] = f32_to_bf16(r2);
    }
}

hipError_t launch_router_split(const float *w, int D, int Er, int Er_pad, int Ep, int Dp, uint16_t *ws,
                               hipStream_t s) {
    hipLaunchKernelGGL(router_split_kernel, dim3(256), dim3(256), 0, s, w, D, Er, Er_pad, Ep, Dp, ws);
    return hipGetLastError();
}

// 8 consecutive x values of row t from column k (a multiple of 8) as bf16
// parts (fp32 x: hi, mid, lo).  Otherwise columns >= D read as 0.  ALIGNED
// (D a multiple of 32, so every 32-column block the MFMAs use lies below D):
// one or two 16-byte loads from an address clamped into the row, no branch
// and no select, so the loads of a chunk are all in flight together (a
// select on the loaded value lets the compiler sink the load into a branch).
template <int XBF16, int ALIGNED>
__device__ inline void load_x8(const void *x, int D, int t, int k, rbf16x8_t *p) {
    if (XBF16) {
        const uint16_t *row = (const uint16_t *)x + (long long)t * D;
        uint16_t v[8];
        if (ALIGNED) {
            const uint4 q = *(const uint4 *)(row + min(k, D - 8));
            __builtin_memcpy(v, &q, 16);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (k + i < D) ? row[k + i] : (uint16_t)0;
        }
        __builtin_memcpy(&p[0], v, 16);
    } else {
#pragma clang fp contract(off)
        const float *row = (const float *)x + (long long)t * D;
        float v[8];
        if (ALIGNED) {
            const int kk = min(k, D - 8);
            const float4 q0 = *(const float4 *)(row + kk), q1 = *(const float4 *)(row + kk + 4);
            v[0] = q0.x; v[1] = q0.y; v[2] = q0.z; v[3] = q0.w; v[4] = q1.x; v[5] = q1.y; v[6] = q1.z; v[7] = q1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (k + i < D) ? row[k + i] : 0.0f;
        }
        uint16_t h0[8], h1[8], h2[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            h0[i] = f32_to_bf16(v[i]);
            const float r1 = v[i] - bf16_to_f32(h0[i]);
            h1[i] = f32_to_bf16(r1);
            h2[i] = f32_to_bf16(r1 - bf16_to_f32(h1[i]));
        }
        __builtin_memcpy(&p[0], h0, 16);
        __builtin_memcpy(&p[1], h1, 16);
        __builtin_memcpy(&p[2], h2, 16);
    }
}

// Block: 4 waves x 32 tokens (two 16-token MFMA tiles per wave) over one K
// slice; the slice's weight parts pass through LDS in chunks of KC columns
// (rows padded by 16 bytes so the 16 rows one read touches fall in distinct
// banks).  All global loads of a chunk are issued before any is used: the
// wave's x fragments and the thread's share of the weight chunk (loads past
// the slice use clamped in-bounds addresses and are not used).
// v_mfma_f32_16x16x32_bf16: A = 16 tokens x 32 k (lane l: token l % 16,
// k 8 (l / 16) .. +8), B = 32 k x 16 experts, D lane l: expert l % 16, tokens
// 4 (l / 16) .. +4.
template <int XBF16, int ALIGNED, int KC>
__global__ __launch_bounds__(256) void router_mfma_kernel(RouterArgs r) {
    extern __shared__ __attribute__((aligned(16))) uint8_t rlds[];
    constexpr int NP = XBF16 ? 1 : 3;       // activation parts
    constexpr int RS = KC * 2 + 16;         // LDS row stride
    constexpr int NWP = kRouterLdsPieces / 256;  // weight pieces per thread (upper bound)
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int tb = blockIdx.x * 128 + w * 32;
    const int k_begin = blockIdx.y * r.ks_len, k_end = min(r.Dp, k_begin + r.ks_len);
    const int ET = r.Ep / 16;
    const int l16 = lane & 15, kq = (lane >> 4) * 8;
    const long long np = (long long)r.Ep * r.Dp;
    const int npieces = 3 * r.Ep * (KC / 8);  // 16-byte weight pieces per chunk (<= kRouterLdsPieces)
    rf32x4_t acc[2][8];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int et = 0; et < 8; ++et) acc[ti][et] = rf32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int kc0 = k_begin; kc0 < k_end; kc0 += KC) {
        rbf16x8_t a[KC / 32][2][NP];
#pragma unroll
        for (int kq32 = 0; kq32 < KC / 32; ++kq32)
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
                load_x8<XBF16, ALIGNED>(r.x, r.D, min(tb + ti * 16 + l16, r.T - 1), kc0 + kq32 * 32 + kq, a[kq32][ti]);
        uint4 wv[NWP];
#pragma unroll
        for (int j = 0; j < NWP; ++j) {
            const int i = min((int)threadIdx.x + j * 256, npieces - 1);
            const int row = i / (KC / 8), c = i - row * (KC / 8);  // row = part * Ep + expert
            const int part = row / r.Ep, e = row - part * r.Ep;
            const int col = min(kc0 + c * 8, r.Dp - 8);              // the slice's last chunk may be short
            wv[j] = *(const uint4 *)(r.ws + part * np + (long long)e * r.Dp + col);
        }
#pragma unroll
        for (int j = 0; j < NWP; ++j) {  // clamped pieces rewrite the last piece with its own value
            const int i = min((int)threadIdx.x + j * 256, npieces - 1);
            const int row = i / (KC / 8), c = i - row * (KC / 8);
            *(uint4 *)(rlds + row * RS + c * 16) = wv[j];
        }
        __syncthreads();
        const int kn = min(KC, k_end - kc0);
#pragma unroll
        for (int kq32 = 0; kq32 < KC / 32; ++kq32) {
            const int kk = kq32 * 32;
#pragma unroll
            for (int et = 0; et < 8; ++et) {
                if (kk < kn && et < ET) {
                    rbf16x8_t b[3];
#pragma unroll
                    for (int p = 0; p < 3; ++p)
                        b[p] = *(const rbf16x8_t *)(rlds + (p * r.Ep + et * 16 + l16) * RS + (kk + kq) * 2);
#pragma unroll
                    for (int ti = 0; ti < 2; ++ti) {
                        // x parts i times weight parts j with i + j <= 2
#pragma unroll
                        for (int i = 0; i < NP; ++i)
#pragma unroll
                            for (int j = 0; j + i < 3; ++j)
                                acc[ti][et] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[kq32][ti][i], b[j], acc[ti][et], 0, 0, 0);
                    }
                }
            }
        }
        __syncthreads();
    }
    float *out = r.part + (long long)blockIdx.y * r.T * r.Er;
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int et = 0; et < 8; ++et) {
            const int e = et * 16 + l16;
            if (et < ET && e < r.Er)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int t = tb + ti * 16 + (lane >> 4) * 4 + rr;
                    if (t < r.T) out[(long long)t * r.Er + e] = acc[ti][et][rr];
                }
        }
}

void router_plan(RouterArgs &r) {
    // LDS chunk: three weight parts of Ep rows within 64 KB; 64, 128 or 256
    // columns (64 for fp32 x, whose fragments take three times the registers)
    const int fit = (65536 / (3 * r.Ep) - 16) / 2;
    int kc = fit >= 256 ? 256 : (fit >= 128 ? 128 : 64);
    if (!r.x_bf16) kc = 64;
    // about 256 workgroups: K slices fill in for a small batch
    const int blocks_t = (r.T + 127) / 128;
    int nks = (256 + blocks_t - 1) / blocks_t;
    nks = std::max(1, std::min(std::min(nks, kRouterMaxSlices), r.Dp / 32));
    int ks_len = ((r.Dp + nks - 1) / nks + 31) / 32 * 32;
    if (ks_len > kc) ks_len = (ks_len + kc - 1) / kc * kc;  // whole chunks
    else kc = ks_len <= 64 ? 64 : (ks_len <= 128 ? 128 : 256);
    nks = (r.Dp + ks_len - 1) / ks_len;
    r.nks = nks;
    r.ks_len = ks_len;
    r.kc = kc;
}

hipError_t launch_router_mfma(const RouterArgs &r, int x_bf16, hipStream_t s) {
    if (r.T <= 0) return hipSuccess;
    const size_t lds = (size_t)3 * r.Ep * (r.kc * 2 + 16);
    dim3 grid((r.T + 127) / 128, r.nks), block(256);
    const bool al = (r.D & 31) == 0;
#define MOE_ROUTER_CASE(XB, AL, KC)                                                     \
    if ((x_bf16 != 0) == (XB != 0) && al == (AL != 0) && r.kc == KC) {                  \
        hipLaunchKernelGGL((router_mfma_kernel<XB, AL, KC>), grid, block, lds, s, r);   \
        return hipGetLastError();                                                       \
    }
    MOE_ROUTER_CASE(1, 1, 256) MOE_ROUTER_CASE(1, 1, 128) MOE_ROUTER_CASE(1, 1, 64)
    MOE_ROUTER_CASE(1, 0, 256) MOE_ROUTER_CASE(1, 0, 128) MOE_ROUTER_CASE(1, 0, 64)
    MOE_ROUTER_CASE(0, 1, 64) MOE_ROUTER_CASE(0, 0, 64)
#undef MOE_ROUTER_CASE
    return hipErrorInvalidValue;
}

// ============================================================================
// Gating.  kRouteBlock tokens per block of kRouteThreads threads: TPT lanes
// per token for the per-element work and the top-k, one thread per token for
// the fp32 sum in expert order and the per-token outputs.
// ============================================================================

// LDS row stride of the routing kernel for E rows: a multiple of 4 floats
// (16 B) whose count of 16-byte units is odd, so that 16 token threads
// reading 16 B at one column hit 16 distinct bank quads.
__host__ __device__ inline int route_rw(int E) { return 4 * ((((E + 3) / 4 + 1) | 1)); }

// Fixed-order sum over the TPT consecutive lanes of a token (a butterfly: the
// same tree on every call).
template <int TPT, typename F>
__device__ __forceinline__ F token_sum(F v) {
#pragma unroll
    for (int o = 1; o < TPT; o <<= 1) v = v + __shfl_xor(v, o);
    return v;
}
template <int TPT>
__device__ __forceinline__ float token_max(float v) {  // NaN ignored (v > m is false for NaN)
#pragma unroll
    for (int o = 1; o < TPT; o <<= 1) {
        const float w = __shfl_xor(v, o);
        if (w > v) v = w;
    }
    return v;
}

// The value of the partner lane in butterfly step o (1, 2, 4) of an 8-lane
// group, by DPP: lane ^ 1, lane ^ 2 (quad permutations), then the mirrored
// lane of the other quad (7 - lane within the group; after two steps every
// lane of a quad holds the same list, so any pairing of the two quads works).
__device__ __forceinline__ int lane_swap8(int o, int v) {
    if (o == 1) return __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false);   // quad_perm 1,0,3,2
    if (o == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false);   // quad_perm 2,3,0,1
    return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false);              // row_half_mirror
}

// Entry (key a, index ia) before entry (b, ib) in the top-k order: larger
// isless key, then the lower index (partialsortperm's Perm ordering).
__device__ __forceinline__ bool topk_before(uint32_t a, int ia, uint32_t b, int ib) {
    return a > b || (a == b && ia < ib);
}

// Top-K of row p[lo, n) by the order above, over the TPT consecutive lanes of
// a token: lane rs keeps the best K of elements rs, rs + TPT, ... in K sorted
// register slots, then log2(TPT) butterfly steps merge the lanes' lists (a
// strict total order, so both partners end with the same list).  Every lane
// of the wave must call it (rows of invalid tokens pass active = false).
// Slots past the row's size stay empty (key 0, below every float's key).
template <int K, int TPT>
__device__ __forceinline__ void topk_lanes(const float *__restrict__ p, int lo, int n, int rs, bool active, int *sel,
                                           float *val) {
    uint32_t kb[K];
    int ib[K];
    float vb[K];
#pragma unroll
    for (int q = 0; q < K; ++q) { kb[q] = 0u; ib[q] = 0x7fffffff; vb[q] = 0.0f; }
    auto insert = [&](uint32_t ck, int ci, float cv) {
        if (!topk_before(ck, ci, kb[K - 1], ib[K - 1])) return;
        bool shift = false;  // once inserted, every later slot moves down by one
#pragma unroll
        for (int q = 0; q < K; ++q) {
            const bool ins = shift || topk_before(ck, ci, kb[q], ib[q]);
            const uint32_t tk = kb[q]; const int ti = ib[q]; const float tv = vb[q];
            kb[q] = ins ? ck : tk; ib[q] = ins ? ci : ti; vb[q] = ins ? cv : tv;
            ck = ins ? tk : ck; ci = ins ? ti : ci; cv = ins ? tv : cv;
            shift = ins;
        }
    };
    if (active) {
        for (int i0 = rs; i0 < n; i0 += 4 * TPT) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = p[min(i0 + u * TPT, n - 1)];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * TPT;
                if (i < n && i >= lo) insert(isless_key(v[u]), i, v[u]);
            }
        }
    }
    // a rolled loop: its body is fetched once (the kernel's once-per-block
    // phases are bound by instruction fetch, not by their arithmetic)
#pragma unroll 1
    for (int o = 1; o < TPT; o <<= 1) {
        uint32_t pk[K];
        int pi[K];
        float pv[K];
#pragma unroll
        for (int q = 0; q < K; ++q) {
            pk[q] = (uint32_t)lane_swap8(o, (int)kb[q]);
            pi[q] = lane_swap8(o, ib[q]);
            pv[q] = __int_as_float(lane_swap8(o, __float_as_int(vb[q])));
        }
#pragma unroll
        for (int q = 0; q < K; ++q) insert(pk[q], pi[q], pv[q]);
    }
#pragma unroll
    for (int q = 0; q < K; ++q) {
        sel[q] = ib[q];
        val[q] = vb[q];
    }
}

// Top-k of row p[lo, n) for n - lo <= 8 TPT by ranks: lane rs owns elements
// lo + rs + TPT u and counts, over the row, the elements before each of them
// in the top-k order; an element of rank r < k is slot r.  No lane exchanges
// anything: the owner writes its winners to ksel / kval directly.
template <int TPT>
__device__ __forceinline__ void topk_ranks(const float *__restrict__ p, int lo, int n, int k, int rs, bool active,
                                           int *ksel, float *kval) {
    constexpr int U = 8;
    if (!active) return;
    uint64_t mine[U];  // (key, inverted index): larger is earlier in the order
    int rank[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = lo + rs + TPT * u;
        const float v = p[min(i, n - 1)];
        mine[u] = ((uint64_t)isless_key(v) << 32) | (uint32_t)(0x7fffffff - i);
        rank[u] = 0;
    }
    for (int j0 = lo; j0 < n; j0 += 4) {
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = p[min(j0 + c, n - 1)];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int j = j0 + c;
            const uint64_t kj = ((uint64_t)isless_key(v[c]) << 32) | (uint32_t)(0x7fffffff - j);
#pragma unroll
            for (int u = 0; u < U; ++u) rank[u] += (j < n && kj > mine[u]) ? 1 : 0;
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = lo + rs + TPT * u;
        if (i < n && rank[u] < k) {
            ksel[rank[u]] = i;
            kval[rank[u]] = p[i];
        }
    }
}

template <int TPT>
__device__ __forceinline__ void topk_lanes_k(const float *__restrict__ p, int lo, int n, int k, int rs, bool active,
                                             int *sel, float *val) {
    switch (k) {
    case 1: topk_lanes<1, TPT>(p, lo, n, rs, active, sel, val); break;
    case 2: topk_lanes<2, TPT>(p, lo, n, rs, active, sel, val); break;
    case 3: topk_lanes<3, TPT>(p, lo, n, rs, active, sel, val); break;
    case 4: topk_lanes<4, TPT>(p, lo, n, rs, active, sel, val); break;
    case 5: topk_lanes<5, TPT>(p, lo, n, rs, active, sel, val); break;
    case 6: topk_lanes<6, TPT>(p, lo, n, rs, active, sel, val); break;
    case 7: topk_lanes<7, TPT>(p, lo, n, rs, active, sel, val); break;
    default: topk_lanes<8, TPT>(p, lo, n, rs, active, sel, val); break;
    }
}

__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteArgs a) {
#pragma clang fp contract(off)
    // Block: kRouteBlock tokens, kRouteThreads threads.  The recipe's
    // order-sensitive fp32 softmax sum in expert order and the per-token
    // gates, logsumexp and entropy run one thread per token (threads <
    // kRouteBlock, all in wave 0), reading the token's LDS row 16 B at a
    // time; the rest runs TPT threads per token (max, exp and probability
    // terms, the top-k by ranks or by a lane merge, the fp64 entropy sum and
    // the z-loss exponent sum as fixed-order per-token reductions).  Rows are sized
    // for this layer's E (dynamic LDS).  Every global output is written in the
    // last phase: a store's data register may not be reused before the store
    // has completed, so stores in between would stall the phases that follow.
    constexpr int TPT = kRouteThreads / kRouteBlock;
    static_assert(TPT == 8 && kRouteBlock * TPT == kRouteThreads, "threads per token");
    extern __shared__ __attribute__((aligned(16))) uint8_t rdyn[];
    // stable ranks: bit i of emask[e][i / 32] marks entry i (token * kt + slot)
    // of expert e + 1 in this block; ent_e holds each entry's expert
    __shared__ unsigned emask[MOE_MAX_EXPERTS * MOE_MAX_TOPK];
    __shared__ int ent_e[kRouteBlock * MOE_MAX_TOPK];
    __shared__ int ksel[kRouteBlock][MOE_MAX_TOPK];    // top-k of each token: experts (0-based)
    __shared__ float kval[kRouteBlock][MOE_MAX_TOPK];  // and their probabilities
    __shared__ double red[2][kRouteBlock];
    __shared__ float rmax[kRouteBlock], zmax[kRouteBlock], rsum[kRouteBlock], zsum[kRouteBlock];
    __shared__ double hsum[kRouteBlock];
    const bool shared_gate = a.gate_kind == MOE_GATE_SHARED;
    const bool soft = a.gate_kind == MOE_GATE_SOFT;
    const bool zsep = shared_gate || soft;  // z-loss from a softmax of its own (all rows, unscaled)
    const bool out_probs = (a.out_mask & ROUTE_OUT_PROBS) != 0;
    const bool out_gating = (a.out_mask & ROUTE_OUT_GATING) != 0;
    // a gating pass on the caller's routing needs none of the softmax phases
    const bool softmax = out_probs || !a.given;
    const int EM = max(a.Er, a.E);
    const int RW = route_rw(EM);
    float *lrow = (float *)rdyn;            // [kRouteBlock][RW] logits
    float *prow = lrow + kRouteBlock * RW;  // exp terms, then probabilities (before the shared-gating scale)
    float *srow = prow + kRouteBlock * RW;  // output probabilities (after it)

    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * kRouteBlock;
    const int t = t0 + tid;
    const int ntok = min(kRouteBlock, a.T - t0);
    const bool tok = tid < kRouteBlock;         // a token thread
    const bool valid = tok && t < a.T;
    const int ns = shared_gate ? a.ns : 0;      // rows before the routed ones
    const int rt = tid / TPT, rs = tid - rt * TPT;  // row-parallel phases: token rt, lane rs of it
    const bool rvalid = rt < ntok;

    for (int i = tid; i < MOE_MAX_EXPERTS * MOE_MAX_TOPK; i += kRouteThreads) emask[i] = 0u;

    // (1) router logits: the K-slice partial sums in slice order, then the
    // bias.  Elements q = tid + 256 u; the slices (and biases) of 4 elements
    // are loaded, from clamped addresses, before any is summed.
    if (softmax) {
    const int nq = ntok * a.Er;
    const long long sstride = (long long)a.T * a.Er;
    // elements per thread per round (block-uniform): up to 8, with the
    // partials of 4 slices each in flight, but never more than the block has
    constexpr int RU = 8;
    const int nu = min(RU, (nq + kRouteThreads - 1) / kRouteThreads);
    for (int q0 = 0; q0 < nq; q0 += RU * kRouteThreads) {
        long long o[RU];
        int qq[RU];
        float v[RU];
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            qq[u] = min(q0 + u * kRouteThreads + tid, nq - 1);
            const int tt = qq[u] / a.Er;
            o[u] = (long long)(t0 + tt) * a.Er + (qq[u] - tt * a.Er);
            v[u] = 0.0f;
        }
        // slices in groups of 4 (clamped to the last slice): every load of a
        // group is issued before the group's sums, which run in slice order
        for (int sg = 0; sg < a.nks; sg += 4) {
            float pv[RU][4];
#pragma unroll
            for (int u = 0; u < RU; ++u)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (u < nu) pv[u][c] = a.part[min(sg + c, a.nks - 1) * sstride + o[u]];
#pragma unroll
            for (int u = 0; u < RU; ++u)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (u < nu && sg + c < a.nks) v[u] = (sg + c == 0) ? pv[u][c] : v[u] + pv[u][c];
        }
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            const int q = q0 + u * kRouteThreads + tid;
            if (u < nu && q < nq) {
                const int tt = q / a.Er, i = q - tt * a.Er;
                float w = v[u];
                if (a.bias) w = w + a.bias[i];
                lrow[tt * RW + i] = w;
            }
        }
    }
    __syncthreads();
    // (2) per token: max of the routed logits and, for shared gating, of all
    // rows (z-loss); NaN ignored.  The order does not matter: only the sign of
    // a zero maximum could, and exp(l - m) is the same for m = +0 and -0.
    {
        float m = -INFINITY, mz = -INFINITY;
        if (rvalid)
            for (int i = rs; i < EM; i += TPT) {
                const float v = lrow[rt * RW + i];
                const float sv = soft ? v / a.soft_lambda : v;  // logits ./ lambda (advanced.jl:18)
                if (i >= ns && i < a.E && sv > m) m = sv;
                if (i < a.Er && v > mz) mz = v;
            }
        m = token_max<TPT>(m);
        mz = token_max<TPT>(mz);
        if (rvalid && rs == 0) {
            rmax[rt] = m;
            zmax[rt] = mz;
        }
    }
    __syncthreads();
    // (3) exp terms e = (float)exp((double)(l - m)) (NNlib's branch for m ==
    // +Inf); shared gating: the z-loss exponent sum over all rows
    {
        float zs = 0.0f;
        if (rvalid) {
            const float m = rmax[rt], mz = zmax[rt];
            for (int i = rs; i < a.Er; i += TPT) {
                const float v = lrow[rt * RW + i];
                const float sv = soft ? v / a.soft_lambda : v;
                if (i >= ns && i < a.E)
                    prow[rt * RW + i] = (m == INFINITY) ? ((sv == INFINITY) ? 1.0f : 0.0f) : (float)exp((double)(sv - m));
                if (zsep) zs = zs + (float)exp((double)(v - mz));
            }
        }
        if (zsep) {
            zs = token_sum<TPT>(zs);
            if (rvalid && rs == 0) zsum[rt] = zs;
        }
    }
    __syncthreads();
    // (4) per token: sum in expert order
    if (valid) {
        const float *row = prow + tid * RW;
        float s = 0.0f;
        for (int i0 = ns & ~3; i0 < a.E; i0 += 8) {
            const float4 va = *(const float4 *)(row + i0), vb = *(const float4 *)(row + i0 + 4);
            const float vv[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int i = i0 + c;
                if (i >= ns && i < a.E) s = s + vv[c];
            }
        }
        rsum[tid] = s;
    }
    __syncthreads();
    // (5) probabilities p = e / s; output rows (shared gating: shared rows 1/E,
    // routed rows p scaled by 1 - ns/E in Float64); the entropy terms
    // p log(p + 1e-8) summed in fp64 per token (a fixed order)
    {
        double hs = 0.0;
        if (rvalid) {
            const float s = rsum[rt];
            for (int i = rs; i < a.E; i += TPT) {
                float pv;
                if (a.given) {
                    // the caller's gate: its probabilities, or ones ./ E
                    pv = a.given_probs ? a.probs[(long long)(t0 + rt) * a.E + i] : 1.0f / (float)a.E;
                } else if (i < ns) {
                    pv = 1.0f / (float)a.E;
                } else {
                    const float pu = prow[rt * RW + i] / s;
                    prow[rt * RW + i] = pu;
                    pv = shared_gate ? (float)((double)pu * (1.0 - (double)ns / (double)a.E)) : pu;
                }
                srow[rt * RW + i] = pv;
                // p * log(p + 1e-8) with p + 1e-8 in Float64 as Julia
                // promotes it; the log in fp32 (a statistic: the mean entropy
                // is checked to 1e-5)
                const double pd = (double)pv;
                hs = hs + pd * (double)logf((float)(pd + 1e-8));
            }
        }
        hs = token_sum<TPT>(hs);
        if (rvalid && rs == 0) hsum[rt] = hs;
    }
    __syncthreads();
    }  // softmax phases

    // (6a) top-k of each token's probabilities over its TPT lanes; the shared
    // rows of SharedExpertGating are left out (the base gate sees the routed
    // rows only)
    if (!a.given) {
        if (a.E - ns <= 8 * TPT) {
            // up to 64 routed experts: ranks (no cross-lane dependence chain)
            topk_ranks<TPT>(prow + rt * RW, ns, a.E, a.k, rs, rvalid, ksel[rt], kval[rt]);
        } else {
            int sl[MOE_MAX_TOPK];
            float vl[MOE_MAX_TOPK];
            topk_lanes_k<TPT>(prow + rt * RW, ns, a.E, a.k, rs, rvalid, sl, vl);
            if (rvalid && rs == 0) {
#pragma unroll
                for (int q = 0; q < MOE_MAX_TOPK; ++q)
                    if (q < a.k) {
                        ksel[rt][q] = sl[q];
                        kval[rt][q] = vl[q];
                    }
            }
        }
    }
    __syncthreads();

    int ex[MOE_MAX_TOPK];     // 1-based expert ids of this token's slots
    float gx[MOE_MAX_TOPK];   // their gates
    double zterm = 0.0, hterm = 0.0;
#pragma unroll
    for (int j = 0; j < MOE_MAX_TOPK; ++j) {
        ex[j] = 0;
        gx[j] = 0.0f;
    }

    // (6) per token: top-k and gates, logsumexp, entropy
    if (valid && a.given) {
        // the caller's routing: ids outside 1..E are skipped, as the
        // dispatch's `expert_id > 0 && expert_id <= length(experts)` does
        // (src/core/moe_layer.jl:198)
#pragma unroll
        for (int j = 0; j < MOE_MAX_TOPK; ++j)
            if (j < a.kt) {
                const long long ent = (long long)t * a.kt + j;
                const int e = a.idx[ent];
                ex[j] = (e >= 1 && e <= a.Eh) ? e : 0;
                gx[j] = a.gates[ent];
            }
        if (softmax) {
            const float lse = zsep ? zmax[tid] + logf(zsum[tid])
                                   : rmax[tid] + logf(rsum[tid]);
            zterm = (double)(lse * lse);
            hterm = -hsum[tid];
        }
    } else if (valid) {
        float *p = prow + tid * RW;
        int sel[MOE_MAX_TOPK];
        float g[MOE_MAX_TOPK];
        {
            // the winners in slot order; gates: p of the slots over their sum
            // in slot order
            float v[MOE_MAX_TOPK];
#pragma unroll
            for (int q = 0; q < MOE_MAX_TOPK; ++q) {
                sel[q] = (q < a.k) ? ksel[tid][q] : 0;
                v[q] = (q < a.k) ? kval[tid][q] : 0.0f;
            }
            float sg = v[0];
#pragma unroll
            for (int q = 1; q < MOE_MAX_TOPK; ++q)
                if (q < a.k) sg = sg + v[q];
#pragma unroll
            for (int q = 0; q < MOE_MAX_TOPK; ++q) g[q] = v[q] / sg;
        }
        if (soft) {
            // SoftMoEGating: top-k of the scaled-softmax probabilities; the
            // dispatch reads row `slot` of the (E, T) gate matrix, i.e. the
            // probability of expert `slot` (advanced.jl:24-33, moe_layer.jl:200)
#pragma unroll
            for (int j = 0; j < MOE_MAX_TOPK; ++j)
                if (j < a.k) {
                    ex[j] = sel[j] + 1;
                    gx[j] = p[j];
                }
            const float lse = zmax[tid] + logf(zsum[tid]);
            zterm = (double)(lse * lse);
        } else if (shared_gate) {
            // top-k and gates on the routed probabilities as the base gate
            // returns them (before the 1 - ns/E scaling)
            const double gscale = 1.0 - (double)ns / (double)a.kt;
            const float gshared = 1.0f / (float)a.kt;
#pragma unroll
            for (int j = 0; j < MOE_MAX_TOPK; ++j) {
                if (j < ns) {
                    ex[j] = j + 1;
                    gx[j] = gshared;
                }
                if (j < a.k) {
                    // slot ns + j (ns + k <= MOE_MAX_TOPK)
#pragma unroll
                    for (int q = 0; q < MOE_MAX_TOPK; ++q)
                        if (q == ns + j) {
                            ex[q] = sel[j] + 1;
                            gx[q] = (float)((double)g[j] * gscale);
                        }
                }
            }
            const float lse = zmax[tid] + logf(zsum[tid]);
            zterm = (double)(lse * lse);
        } else {
            if (a.lsh == 0) {
#pragma unroll
                for (int j = 0; j < MOE_MAX_TOPK; ++j)
                    if (j < a.k) {
                        ex[j] = sel[j] + 1;
                        gx[j] = g[j];
                    }
            } else {
                // forward_with_shared_experts: shared experts 1..lsh in slots
                // 0..lsh-1 (their outputs are averaged, the gate is only
                // reported), then the routed ids shifted by lsh (expert_indices
                // .+= num_shared_experts, src/core/moe_layer.jl:172)
                const float gsh = 1.0f / (float)a.lsh;
#pragma unroll
                for (int j = 0; j < MOE_MAX_TOPK; ++j) {
                    if (j < a.lsh) {
                        ex[j] = j + 1;
                        gx[j] = gsh;
                    }
                    if (j < a.k) {
#pragma unroll
                        for (int q = 0; q < MOE_MAX_TOPK; ++q)
                            if (q == a.lsh + j) {
                                ex[q] = sel[j] + 1 + a.lsh;
                                gx[q] = g[j];
                            }
                    }
                }
            }
            // logsumexp (src/balancing/losses.jl:111-114) from the same exp recipe,
            // the log in Float32 as Julia takes it of the Float32 sum
            const float lse = rmax[tid] + logf(rsum[tid]);
            zterm = (double)(lse * lse);
        }
        hterm = -hsum[tid];  // entropy of update_stats!, Float64
    }
    __syncthreads();

    // ---- stable rank of each entry among the block's entries of its expert ----
    // (entries in token-then-slot order, as the bucket loop visits them; a
    // gating pass only: kt <= MOE_MAX_TOPK there)
    int my_e = 0, my_r = 0;
    if (out_gating) {
        const int nent = kRouteBlock * a.kt;
        if (tok) {
#pragma unroll
            for (int j = 0; j < MOE_MAX_TOPK; ++j)
                if (j < a.kt) ent_e[tid * a.kt + j] = ex[j];
        }
        __syncthreads();
        if (tid < nent) {
            my_e = ent_e[tid];
            if (my_e > 0) atomicOr(&emask[(my_e - 1) * MOE_MAX_TOPK + (tid >> 5)], 1u << (tid & 31));
        }
        __syncthreads();
        if (tid < nent && my_e > 0) {
            const unsigned *m = &emask[(my_e - 1) * MOE_MAX_TOPK];
            int rr = __popc(m[tid >> 5] & ((1u << (tid & 31)) - 1u));
            for (int w = 0; w < (tid >> 5); ++w) rr += __popc(m[w]);
            my_r = rr;
        }
    }
    if (tok) {
        red[0][tid] = zterm;
        red[1][tid] = hterm;
    }
    __syncthreads();
    for (int st = kRouteBlock / 2; st > 0; st >>= 1) {
        if (tid < st) {
            red[0][tid] += red[0][tid + st];
            red[1][tid] += red[1][tid + st];
        }
        __syncthreads();
    }

    // ---- outputs --------------------------------------------------------------
    if (out_probs) {
        for (int q = tid; q < ntok * a.Er; q += kRouteThreads) {
            const int tt = q / a.Er, i = q - tt * a.Er;
            a.logits[(long long)(t0 + tt) * a.Er + i] = lrow[tt * RW + i];
        }
        for (int q = tid; q < ntok * a.E; q += kRouteThreads) {
            const int tt = q / a.E, i = q - tt * a.E;
            a.probs[(long long)(t0 + tt) * a.E + i] = srow[tt * RW + i];
        }
    }
    if (valid && out_gating) {
#pragma unroll
        for (int j = 0; j < MOE_MAX_TOPK; ++j) {
            if (j < a.kt) {
                const long long ent = (long long)t * a.kt + j;
                a.idx[ent] = ex[j];
                a.gates[ent] = gx[j];
            }
        }
    }
    if (out_gating && tid < ntok * a.kt) a.rank[(long long)t0 * a.kt + tid] = my_r;
    const int nb = blockIdx.x;
    for (int e = tid; e < a.Eh; e += kRouteThreads) {
        if (out_gating) {
            int c = 0;
#pragma unroll
            for (int w = 0; w < MOE_MAX_TOPK; ++w) c += __popc(emask[e * MOE_MAX_TOPK + w]);
            a.blk_counts[(long long)nb * a.Eh + e] = c;
        }
        if (out_probs) {
            // per-row probability sums (Switch loss P_e) in fp64, token order
            double ps = 0.0;
            if (e < a.E) {
#pragma unroll 8
                for (int i = 0; i < ntok; ++i) ps += (double)srow[i * RW + e];
            }
            a.blk_stats[(long long)nb * (a.Eh + 2) + e] = ps;
        }
    }
    if (tid == 0 && out_probs) {
        a.blk_stats[(long long)nb * (a.Eh + 2) + a.Eh] = red[0][0];
        a.blk_stats[(long long)nb * (a.Eh + 2) + a.Eh + 1] = red[1][0];
    }
}

hipError_t launch_route(const RouteArgs &a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    const int nblk = (a.T + kRouteBlock - 1) / kRouteBlock;
    // three rows of route_rw(E) floats per token: 50.7 KB at E = MOE_MAX_EXPERTS,
    // within the 64 KB of dynamic LDS a launch gets without an attribute
    const size_t lds = (size_t)kRouteBlock * sizeof(float) * route_rw(std::max(a.Er, a.E)) * 3;
    if (lds > 65536) return hipErrorInvalidValue;
    hipLaunchKernelGGL(route_kernel, dim3(nblk), dim3(kRouteThreads), lds, s, a);
    return hipGetLastError();
}

// ============================================================================
// ExpertChoiceGating (src/gating/expert_choice.jl:11-53).
// ============================================================================
// Block e: expert e takes the min(C, T) tokens of largest logit,
// partialsortperm(scores[:, e], 1:C, rev=true): Julia's isless order (NaN
// largest), ties to the lower token.  A 4-pass 8-bit radix select finds the
// C-th largest key K and how many tokens of key K to take; the tokens of key
// > K and the first of key == K in token order are marked in sel[t][e].
__global__ __launch_bounds__(256) void expert_choice_select_kernel(const float *__restrict__ logits, int T, int E,
                                                                   int C, uint8_t *__restrict__ sel) {
    __shared__ unsigned hist[256];
    __shared__ unsigned s_prefix, s_rem;
    __shared__ unsigned wties[4];
    const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t prefix = 0, mask = 0;
    unsigned rem = (unsigned)min(C, T);
    for (int pos = 24; pos >= 0; pos -= 8) {
        hist[tid] = 0;
        __syncthreads();
        for (int t = tid; t < T; t += 256) {
            const uint32_t key = isless_key(logits[(long long)t * E + e]);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> pos) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            unsigned cum = 0;
            int d = 255;
            for (; d > 0; --d) {
                if (cum + hist[d] >= rem) break;
                cum += hist[d];
            }
            s_prefix = prefix | ((uint32_t)d << pos);
            s_rem = rem - cum;
        }
        __syncthreads();
        prefix = s_prefix;
        rem = s_rem;
        mask |= 255u << pos;
    }
    // take key > K, and the first `rem` tokens of key == K in token order
    unsigned ties_before = 0;
    for (int t0 = 0; t0 < T; t0 += 256) {
        const int t = t0 + tid;
        const uint32_t key = (t < T) ? isless_key(logits[(long long)t * E + e]) : 0u;
        const bool eq = t < T && key == prefix;
        const uint64_t b = __ballot(eq);
        if (lane == 0) wties[wave] = __popcll(b);
        __syncthreads();
        unsigned r = ties_before + __popcll(b & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
        for (int w = 0; w < wave; ++w) r += wties[w];
        if (t < T) sel[(long long)t * E + e] = (key > prefix || (eq && r < rem)) ? 1 : 0;
        ties_before += wties[0] + wties[1] + wties[2] + wties[3];
        __syncthreads();
    }
}

// One thread per token: its slots hold the experts that took it in ascending
// id order, at most kcap = min(C, E) of them (a later expert past the
// capacity rows is left out, expert_choice.jl:40-50), gate = probability of
// the expert for the token; the remaining slots of the kt are empty (id 0).
// sel[t][e] becomes the slot + 1 of entry (t, e) (<= kcap <= 128), or 0 when
// expert e did not take token t or the entry was left out.
__global__ __launch_bounds__(256) void expert_choice_assemble_kernel(uint8_t *__restrict__ sel,
                                                                     const float *__restrict__ probs, int T, int E,
                                                                     int kt, int kcap, int *idx, float *gates) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= T) return;
    int c = 0;
    for (int e = 0; e < E; ++e) {
        const long long o = (long long)t * E + e;
        if (sel[o]) {
            if (c < kcap) {
                idx[(long long)t * kt + c] = e + 1;
                gates[(long long)t * kt + c] = probs[o];
                sel[o] = (uint8_t)(c + 1);
            } else {
                sel[o] = 0;
            }
            ++c;
        }
    }
    for (int j = min(c, kcap); j < kt; ++j) {
        idx[(long long)t * kt + j] = 0;
        gates[(long long)t * kt + j] = 0.0f;
    }
}

// The bucketing inputs of the kept entries, per route block of kRouteBlock
// tokens: thread e walks the block's tokens in order; a token holds expert e
// in at most one slot, so the entry's rank among expert e's entries of the
// block (token-then-slot order, the bucket loop's) is the count of earlier
// tokens that hold e.
__global__ __launch_bounds__(MOE_MAX_EXPERTS) void expert_choice_rank_kernel(const uint8_t *__restrict__ sel, int T,
                                                                            int E, int kt, int *rank,
                                                                            int *blk_counts) {
    const int e = threadIdx.x;
    if (e >= E) return;
    const int t0 = blockIdx.x * kRouteBlock;
    const int ntok = min(kRouteBlock, T - t0);
    int c = 0;
    for (int i = 0; i < ntok; ++i) {
        const int sl = sel[(long long)(t0 + i) * E + e];
        if (sl) {
            rank[(long long)(t0 + i) * kt + sl - 1] = c;
            ++c;
        }
    }
    blk_counts[(long long)blockIdx.x * E + e] = c;
}

hipError_t launch_expert_choice(const float *logits, const float *probs, int T, int E, int C, int kt, uint8_t *sel,
                                int *idx, float *gates, int *rank, int *blk_counts, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    if (E > MOE_MAX_EXPERTS || kt < min(C, E) || kt > 255) return hipErrorInvalidValue;
    hipLaunchKernelGGL(expert_choice_select_kernel, dim3(E), dim3(256), 0, s, logits, T, E, C, sel);
    hipLaunchKernelGGL(expert_choice_assemble_kernel, dim3((T + 255) / 256), dim3(256), 0, s, sel, probs, T, E, kt,
                       min(C, E), idx, gates);
    hipLaunchKernelGGL(expert_choice_rank_kernel, dim3((T + kRouteBlock - 1) / kRouteBlock), dim3(MOE_MAX_EXPERTS),
                       0, s, sel, T, E, kt, rank, blk_counts);
    return hipGetLastError();
}

// ============================================================================
// Scan: per-expert totals, per-block rank bases (many blocks), then the
// capacity clamp, offsets, the (expert, m0) GEMM tile list and the loss
// scalars (one block).
// ============================================================================
// update_bias!(::AuxiliaryFreeLoss, expert_indices) after its counter check
// (src/balancing/auxiliary_free.jl:36-69), one thread, with Julia's types:
// counts Float32, target = total / E and the gradient in Float64, the
// momentum stored as Float32 of a Float64 sum, the bias step in Float32, then
// bias .-= mean(bias) with the Float32 sum taken in index order.
__device__ inline void aux_free_step(const int *cnt, long long total, int E, float lr, float momentum,
                                     float *bias, float *mom) {
#pragma clang fp contract(off)
    if (total <= 0) return;
    const double target = (double)total / (double)E;
    for (int e = 0; e < E; ++e) {
        const double grad = ((double)(float)cnt[e] - target) / (double)total;
        const float m = (float)((double)(momentum * mom[e]) + (double)(1.0f - momentum) * grad);
        mom[e] = m;
        bias[e] = bias[e] - lr * m;
    }
    float s = bias[0];
    for (int e = 1; e < E; ++e) s = s + bias[e];
    const float mean = s / (float)E;
    for (int e = 0; e < E; ++e) bias[e] = bias[e] - mean;
}

// Scan, part 1: many blocks.  Block b takes kScanCols columns (expert
// counts and fp64 statistics of column c; columns E, E + 1: the z and
// entropy sums) and splits the nblk route-block rows into kScanChunks
// contiguous chunks, one thread per (chunk, column): the chunk sums go to
// LDS, every thread then writes the rank bases of its chunk's rows (the
// counts of the earlier chunks, then of the chunk's earlier rows), and the
// first chunk's threads the column totals, chunk sums added in chunk order.
constexpr int kScanCols = 8;
constexpr int kScanChunks = 32;

__global__ __launch_bounds__(kScanCols * kScanChunks) void scan_columns_kernel(ScanArgs a) {
#pragma clang fp contract(off)
    __shared__ int csum[kScanChunks][kScanCols];
    __shared__ double ssum[kScanChunks][kScanCols];
    const int NC = a.E + 2;
    const int c = blockIdx.x * kScanCols + (threadIdx.x % kScanCols);
    const int g = threadIdx.x / kScanCols;
    const int R = (a.nblk + kScanChunks - 1) / kScanChunks;
    const int b0 = min(a.nblk, g * R), b1 = min(a.nblk, b0 + R);
    const bool col = c < NC, cnt_col = c < a.E;
    int cs = 0;
    double ss = 0.0;
    if (col) {
        for (int b = b0; b < b1; b += 8) {
            int cv[8];
            double sv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int bb = min(b + u, b1 - 1);
                cv[u] = cnt_col ? a.blk_counts[(long long)bb * a.E + c] : 0;
                sv[u] = a.blk_stats[(long long)bb * NC + c];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (b + u < b1) {
                    cs += cv[u];
                    ss += sv[u];
                }
        }
    }
    csum[g][threadIdx.x % kScanCols] = cs;
    ssum[g][threadIdx.x % kScanCols] = ss;
    __syncthreads();
    if (cnt_col) {
        int base = 0;
        for (int q = 0; q < g; ++q) base += csum[q][threadIdx.x % kScanCols];
        for (int b = b0; b < b1; b += 8) {
            int cv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) cv[u] = a.blk_counts[(long long)min(b + u, b1 - 1) * a.E + c];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (b + u < b1) {
                    a.rank_base[(long long)(b + u) * a.E + c] = base;
                    base += cv[u];
                }
        }
    }
    if (col && g == 0) {
        int tc = 0;
        double ts = 0.0;
        for (int q = 0; q < kScanChunks; ++q) {
            tc += csum[q][threadIdx.x % kScanCols];
            ts += ssum[q][threadIdx.x % kScanCols];
        }
        if (cnt_col) a.tot_counts[c] = tc;
        a.tot_stats[c] = ts;
    }
}

// Scan, part 2: one block.  Capacity clamp, offsets, per-expert GEMM tile
// starts and the (expert, m0) tile list, the Switch and z losses, the mean
// entropy and the AuxiliaryFreeLoss step, from the column totals.
__global__ __launch_bounds__(256) void scan_finish_kernel(ScanArgs a) {
#pragma clang fp contract(off)
    __shared__ int cnt[MOE_MAX_EXPERTS];
    __shared__ int off[MOE_MAX_EXPERTS + 1];
    __shared__ int tstart[MOE_MAX_EXPERTS + 1];
    __shared__ float fp[MOE_MAX_EXPERTS];
    __shared__ int cap_s;
    const int tid = threadIdx.x;
    if (tid == 0) {
        int cap = INT_MAX;
        if (a.training && a.drop) {
            // capacity = ceil(Int, capacity_factor * batch_size / num_experts), Float32
            const float cf = ceilf((a.capacity_factor * (float)a.T) / (float)a.E);
            cap = (cf >= 2147483647.0f) ? INT_MAX : (int)cf;
        }
        cap_s = cap;
        a.cap_out[0] = cap;
    }
    __syncthreads();
    const float total = (float)((long long)a.T * a.kl);
    for (int e = tid; e < a.E; e += 256) {
        const int ce = min(a.tot_counts[e], cap_s);
        cnt[e] = ce;
        // the terms f_e * P_e of the Switch loss (src/balancing/losses.jl:15-36)
        // over the a.Np probability rows; with shared experts of the layer the
        // ids are the shifted routed ids and expert e < lsh holds none of them
        if (e < a.Np) {
            float f = (e < a.lsh) ? 0.0f : (float)ce;
            if (a.T * a.kl > 0) f = f / total;
            const float P = (float)a.tot_stats[e] / (float)a.T;
            fp[e] = f * P;
        }
    }
    __syncthreads();
    // offsets and GEMM tile starts: exclusive prefixes over the experts by
    // wave 0 (lane l holds experts 2 l and 2 l + 1; E <= 128)
    __shared__ float lsum_s;
    if (tid < 64) {
        const int e0 = 2 * tid, e1 = e0 + 1;
        const int c0 = (e0 < a.E) ? cnt[e0] : 0, c1 = (e1 < a.E) ? cnt[e1] : 0;
        const int n0 = (c0 + a.bm - 1) / a.bm, n1 = (c1 + a.bm - 1) / a.bm;
        int cs = c0 + c1, ns = n0 + n1;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int cu = __shfl_up(cs, o), nu = __shfl_up(ns, o);
            if (tid >= o) {
                cs += cu;
                ns += nu;
            }
        }
        const int ce = cs - (c0 + c1), ne = ns - (n0 + n1);  // exclusive
        if (e0 <= a.E) {
            off[e0] = ce;
            tstart[e0] = ne;
        }
        if (e1 <= a.E) {
            off[e1] = ce + c0;
            tstart[e1] = ne + n0;
        }
        if (tid == 63) {  // the totals (also for E = 128, past the last pair)
            off[a.E] = cs;
            tstart[a.E] = ns;
        }
        // the Switch-loss sum over the a.Np terms: in expert order up to 16
        // experts (Julia's sequential sum), else a fixed tree (Julia's order
        // for longer arrays is its SIMD reduction, not reproduced)
        float part = 0.0f;
        if (a.Np > 16) {
            part = (e0 < a.Np) ? fp[e0] : 0.0f;
            if (e1 < a.Np) part = part + fp[e1];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) part = part + __shfl_xor(part, o);
        } else if (tid == 0) {
            part = fp[0];
            for (int e = 1; e < a.Np; ++e) part = part + fp[e];
        }
        if (tid == 0) lsum_s = part;
    }
    __syncthreads();
    if (tid == 0) {
        const int ts = tstart[a.E];
        a.num_tiles[0] = ts;
        const double zs = a.tot_stats[a.E], hs = a.tot_stats[a.E + 1];
        const float s = lsum_s;
        // AuxiliaryFreeLoss: complementary_weight * Switch(1.0f0) or 0.0f0
        // (src/balancing/auxiliary_free.jl:78-87)
        float sw;
        if (a.aux_free) sw = a.aux_use_comp ? a.aux_cw * ((1.0f * (float)a.Np) * s) : 0.0f;
        else sw = (a.alpha * (float)a.Np) * s;
        const float z = a.beta * ((float)zs / (float)a.T);
        float loss = 0.0f;
        if (a.training) loss = a.z_enabled ? sw + z : sw;
        a.scalars[0] = a.training ? sw : 0.0f;
        a.scalars[1] = (a.training && a.z_enabled) ? z : 0.0f;
        a.scalars[2] = loss;
        a.scalars[3] = (float)(hs / (double)a.T);
        if (a.loss_out) a.loss_out[0] = loss;
        if (a.aux_free && a.training && a.aux_update) {
            // the kept entries of each expert are the counts after capacity
            long long kept = 0;
            for (int e = 0; e < a.E; ++e) kept += cnt[e];
            aux_free_step(cnt, kept, a.E, a.aux_lr, a.aux_momentum, a.aux_bias, a.aux_mom);
        }
    }
    __syncthreads();
    for (int e = tid; e <= a.E; e += 256) {
        a.offsets[e] = off[e];
        a.tile_start[e] = tstart[e];
    }
    for (int e = tid; e < a.E; e += 256) {
        a.counts[e] = cnt[e];
        const int nt = tstart[e + 1] - tstart[e];
        for (int i = 0; i < nt; ++i) a.tiles[tstart[e] + i] = make_int2(e, i * a.bm);
    }
}

hipError_t launch_scan(const ScanArgs &a, hipStream_t s) {
    const int NC = a.E + 2;
    hipLaunchKernelGGL(scan_columns_kernel, dim3((NC + kScanCols - 1) / kScanCols), dim3(kScanCols * kScanChunks), 0, s,
                       a);
    hipLaunchKernelGGL(scan_finish_kernel, dim3(1), dim3(256), 0, s, a);
    return hipGetLastError();
}

// Element offset in xp of column col of row q: row-major (row stride ld_xp),
// or, for the bf16 GEMM kernel (tiled), its place in the A tile image: row
// q mod bm of M tile q / bm, K stage col / 32 of 64 B, 16-byte chunk
// (col mod 32) / 8 at chunk position chunk ^ ((row >> 2) & 3).
__device__ __forceinline__ long long xp_index(const PermuteArgs &a, long long q, int col) {
    if (!a.tiled) return q * a.ld_xp + col;
    const long long mt = q / a.bm;
    const int lr = (int)(q - mt * a.bm);
    const int chunk = ((col & 31) >> 3) ^ ((lr >> 2) & 3);
    return ((mt * a.ktt + (col >> 5)) * a.bm + lr) * 32 + chunk * 8 + (col & 7);
}

// Store U chunks of 8 bf16 per lane into the xp row of every position the
// token holds (row of lane j: xp row of entry j, < 0 if dropped).  Chunk u of
// a lane is column min(d0 + 512 u + 8 lane, D - 8), the column its value was
// loaded from: a lane past the row's end rewrites the last chunk with that
// chunk's own value, so no store is conditional.
template <int U>
__device__ __forceinline__ void store_row_chunk(const PermuteArgs &a, int row, int d0, int lane,
                                                const u32x4_t (&v)[U]) {
    int cols[U];
#pragma unroll
    for (int u = 0; u < U; ++u) cols[u] = min(d0 + u * 512 + lane * 8, a.D - 8);
#pragma nounroll
    for (int j = 0; j < a.kt; ++j) {
        const int q = __shfl(row, j);
        if (q >= 0) {
#pragma unroll
            for (int u = 0; u < U; ++u) *(u32x4_t *)((uint16_t *)a.xp + xp_index(a, q, cols[u])) = v[u];
        }
    }
}

// ============================================================================
// Permute: one wave per token.  Lanes < kt finalise the token's entries
// (capacity drop + renormalisation, position), then the wave copies the
// token's row into every position it owns, converting to the GEMM type.
// ============================================================================
__global__ __launch_bounds__(256) void permute_kernel(PermuteArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    const int blk = t / kRouteBlock;
    const int cap = a.cap[0];
    int e = 0, pos = -1, row = -1;  // position in expert order; xp row (tile image row when tiled)
    float g = 0.0f;
    if (lane < a.kt) {
        const long long ent = (long long)t * a.kt + lane;
        e = a.idx[ent];
        g = a.gates[ent];
        if (e > 0 && e <= a.E) {
            const int rk = a.rank_base[(long long)blk * a.E + (e - 1)] + a.rank[ent];
            if (rk < cap) {
                pos = a.offsets[e - 1] + rk;
                row = a.tiled ? a.tile_start[e - 1] * a.bm + rk : pos;
            } else {
                e = 0;
                g = 0.0f;
            }
        }
    }
    if (a.renorm) {
        // gate_sum = sum(expert_gates[:, j]) in slot order; divide when > 0
        float s = __shfl(g, 0);
        for (int j = 1; j < a.kt; ++j) s = s + __shfl(g, j);
        if (s > 0.0f) g = g / s;
    }
    if (lane < a.kt) {
        const long long ent = (long long)t * a.kt + lane;
        if (a.renorm) {
            a.idx[ent] = e;
            a.gates[ent] = g;
        }
        a.pos_of[ent] = pos;
        if (pos >= 0) {
            a.perm[pos] = (int)ent;
            a.gate_sorted[pos] = g;
        }
    }
    if (!a.copy_rows) return;
    if (a.ct == CT_BF16 && a.x_bf16 && (a.D & 7) == 0) {
        // 8 bf16 per lane per chunk; the loads of 8 chunks (8 KB per wave) are
        // issued together from clamped in-row addresses, then stored to every
        // position the token holds.
        const uint16_t *__restrict__ src = (const uint16_t *)a.x + (long long)t * a.D;
        constexpr int U = 8;
        for (int d0 = 0; d0 < a.D; d0 += 512 * U) {
            u32x4_t v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = *(const u32x4_t *)(src + min(d0 + u * 512 + lane * 8, a.D - 8));
            store_row_chunk<U>(a, row, d0, lane, v);
        }
        return;
    }
    if (a.ct == CT_BF16 && !a.x_bf16 && (a.D & 7) == 0) {
        const float *__restrict__ src = (const float *)a.x + (long long)t * a.D;
        constexpr int U = 4;
        for (int d0 = 0; d0 < a.D; d0 += 512 * U) {
            u32x4_t v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int d = min(d0 + u * 512 + lane * 8, a.D - 8);
                const float4 f0 = *(const float4 *)(src + d), f1 = *(const float4 *)(src + d + 4);
                v[u] = u32x4_t{f32_to_bf16(f0.x) | ((uint32_t)f32_to_bf16(f0.y) << 16),
                                  f32_to_bf16(f0.z) | ((uint32_t)f32_to_bf16(f0.w) << 16),
                                  f32_to_bf16(f1.x) | ((uint32_t)f32_to_bf16(f1.y) << 16),
                                  f32_to_bf16(f1.z) | ((uint32_t)f32_to_bf16(f1.w) << 16)};
            }
            store_row_chunk<U>(a, row, d0, lane, v);
        }
        return;
    }
    for (int j = 0; j < a.kt; ++j) {
        const int p = __shfl(row, j);
        if (p < 0) continue;
        if (a.ct == CT_BF16) {
            uint16_t *dst = (uint16_t *)a.xp;
            if (a.x_bf16) {
                const uint16_t *src = (const uint16_t *)a.x + (long long)t * a.D;
                for (int d = lane; d < a.D; d += 64) dst[xp_index(a, p, d)] = src[d];
            } else {
                const float *src = (const float *)a.x + (long long)t * a.D;
                for (int d = lane; d < a.D; d += 64) dst[xp_index(a, p, d)] = f32_to_bf16(src[d]);
            }
        } else {
            float *dst = (float *)a.xp + (long long)p * a.ld_xp;
            if (a.x_bf16) {
                const uint16_t *src = (const uint16_t *)a.x + (long long)t * a.D;
                for (int d = lane; d < a.D; d += 64) dst[d] = bf16_to_f32(src[d]);
            } else {
                const float *src = (const float *)a.x + (long long)t * a.D;
                if ((a.D & 3) == 0) {
                    for (int d = lane * 4; d < a.D; d += 256)
                        *(float4 *)(dst + d) = *(const float4 *)(src + d);
                } else {
                    for (int d = lane; d < a.D; d += 64) dst[d] = src[d];
                }
            }
        }
    }
}

// Permute for more slots per token than a wave has lanes (ExpertChoiceGating
// with min(capacity, E) > 64; kt <= MOE_MAX_EXPERTS): lane l owns entries l
// and l + 64; same finalisation as permute_kernel, then one row copy per kept
// entry, element by element (most of these slots are empty).
__global__ __launch_bounds__(256) void permute_wide_kernel(PermuteArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    const int blk = t / kRouteBlock;
    const int cap = a.cap[0];
    int ee[2], pos[2], row[2];
    float g[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int j = lane + 64 * c;
        ee[c] = 0; pos[c] = -1; row[c] = -1; g[c] = 0.0f;
        if (j < a.kt) {
            const long long ent = (long long)t * a.kt + j;
            ee[c] = a.idx[ent];
            g[c] = a.gates[ent];
            if (ee[c] > 0 && ee[c] <= a.E) {
                const int rk = a.rank_base[(long long)blk * a.E + (ee[c] - 1)] + a.rank[ent];
                if (rk < cap) {
                    pos[c] = a.offsets[ee[c] - 1] + rk;
                    row[c] = a.tiled ? a.tile_start[ee[c] - 1] * a.bm + rk : pos[c];
                } else {
                    ee[c] = 0;
                    g[c] = 0.0f;
                }
            }
        }
    }
    if (a.renorm) {
        // gate_sum over the slots in slot order; divide when > 0
        float sum = __shfl(g[0], 0);
        for (int j = 1; j < a.kt; ++j) sum = sum + __shfl(g[j >> 6], j & 63);
        if (sum > 0.0f) {
            g[0] = g[0] / sum;
            g[1] = g[1] / sum;
        }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int j = lane + 64 * c;
        if (j < a.kt) {
            const long long ent = (long long)t * a.kt + j;
            if (a.renorm) {
                a.idx[ent] = ee[c];
                a.gates[ent] = g[c];
            }
            a.pos_of[ent] = pos[c];
            if (pos[c] >= 0) {
                a.perm[pos[c]] = (int)ent;
                a.gate_sorted[pos[c]] = g[c];
            }
        }
    }
    if (!a.copy_rows) return;
    for (int j = 0; j < a.kt; ++j) {
        const int p = __shfl(row[j >> 6], j & 63);
        if (p < 0) continue;
        for (int d = lane; d < a.D; d += 64) {
            const float v = a.x_bf16 ? bf16_to_f32(((const uint16_t *)a.x)[(long long)t * a.D + d])
                                     : ((const float *)a.x)[(long long)t * a.D + d];
            if (a.ct == CT_BF16) ((uint16_t *)a.xp)[xp_index(a, p, d)] = f32_to_bf16(v);
            else ((float *)a.xp)[(long long)p * a.ld_xp + d] = v;
        }
    }
}

hipError_t launch_permute(const PermuteArgs &a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    if (a.kt > 2 * 64) return hipErrorInvalidValue;
    if (a.kt > 64) hipLaunchKernelGGL(permute_wide_kernel, dim3((a.T + 3) / 4), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(permute_kernel, dim3((a.T + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ============================================================================
// Combine: one wave per token.  out[t] = sum over the token's entries in
// ascending expert order of gate * y, as separate fp32 multiply and add on a
// zero start (src/core/moe_layer.jl:132, 205-217).  No atomics.
//
// With shared experts of the layer (lsh > 0, forward_with_shared_experts,
// src/core/moe_layer.jl:158-185) the token's first lsh entries in expert
// order are the shared experts: shared = sum of y / lsh (IEEE division,
// `expert_out ./ num_shared_experts`, :164-166), routed = the sum above over
// the rest, out = 0.5f * shared + 0.5f * routed (:179-180).
//
// y is fp32, or bf16 (a.y_bf16) where the down GEMM ran on the bf16 kernel;
// each term is widened to fp32 before it is scaled and summed.
//
// Fast path (every one of the token's KT entries kept, rows 16-byte
// aligned): the entries are sorted by expert in registers, and all y loads of
// a chunk of U groups of 4 per lane are issued before any is summed.
// ============================================================================
template <bool YB>
__device__ __forceinline__ float4 load_y4(const void *y, long long off) {
    if (YB) {
        const uint2 r = *(const uint2 *)((const uint16_t *)y + off);
        return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                           __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
    }
    return *(const float4 *)((const float *)y + off);
}

template <int KT, bool BLEND, bool YB>
__device__ __forceinline__ void combine_fast(const CombineArgs &a, int t, int lane) {
#pragma clang fp contract(off)
    constexpr int U = (KT >= 8) ? 2 : (KT >= 4 ? 4 : 8);
    int ee[KT], pp[KT];
    float gg[KT];
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        const long long ent = (long long)t * KT + j;
        ee[j] = a.idx[ent];
        pp[j] = a.pos_of[ent];
        gg[j] = a.gates[ent];
    }
    // stable sort by expert id (distinct ids; a fixed compare-exchange network)
#pragma unroll
    for (int i = 0; i < KT; ++i)
#pragma unroll
        for (int j = 0; j + 1 < KT - i; ++j) {
            const bool sw = ee[j] > ee[j + 1];
            const int e0 = ee[j], p0 = pp[j];
            const float g0 = gg[j];
            ee[j] = sw ? ee[j + 1] : e0; ee[j + 1] = sw ? e0 : ee[j + 1];
            pp[j] = sw ? pp[j + 1] : p0; pp[j + 1] = sw ? p0 : pp[j + 1];
            gg[j] = sw ? gg[j + 1] : g0; gg[j + 1] = sw ? g0 : gg[j + 1];
        }
    float *__restrict__ o = a.out + (long long)t * a.D;
    for (int d0 = 0; d0 < a.D; d0 += 256 * U) {
        float4 v[KT][U];
#pragma unroll
        for (int i = 0; i < KT; ++i)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int d = min(d0 + u * 256 + lane * 4, a.D - 4);
                v[i][u] = load_y4<YB>(a.y, (long long)pp[i] * a.ld_y + d);
            }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float4 sh = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int i = 0; i < KT; ++i) {
                if (BLEND && i < a.lsh) {
                    const float n = (float)a.lsh;
                    sh.x = sh.x + v[i][u].x / n;
                    sh.y = sh.y + v[i][u].y / n;
                    sh.z = sh.z + v[i][u].z / n;
                    sh.w = sh.w + v[i][u].w / n;
                } else {
                    const float g = gg[i];
                    acc.x = acc.x + g * v[i][u].x;
                    acc.y = acc.y + g * v[i][u].y;
                    acc.z = acc.z + g * v[i][u].z;
                    acc.w = acc.w + g * v[i][u].w;
                }
            }
            if (BLEND) {
                acc.x = 0.5f * sh.x + 0.5f * acc.x;
                acc.y = 0.5f * sh.y + 0.5f * acc.y;
                acc.z = 0.5f * sh.z + 0.5f * acc.z;
                acc.w = 0.5f * sh.w + 0.5f * acc.w;
            }
            const int d = d0 + u * 256 + lane * 4;
            if (d < a.D) *(float4 *)(o + d) = acc;
        }
    }
}

template <int KT>
__device__ __forceinline__ bool try_combine_fast(const CombineArgs &a, int t, int lane) {
    if (a.kt != KT) return false;
    if (a.y_bf16) combine_fast<KT, false, true>(a, t, lane);
    else combine_fast<KT, false, false>(a, t, lane);
    return true;
}

template <int KT>
__device__ __forceinline__ bool try_combine_blend(const CombineArgs &a, int t, int lane) {
    if (a.kt != KT) return false;
    if (a.y_bf16) combine_fast<KT, true, true>(a, t, lane);
    else combine_fast<KT, true, false>(a, t, lane);
    return true;
}

__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    if (a.kt > MOE_MAX_TOPK) {
        // more slots than a token's sort network holds: ExpertChoiceGating,
        // whose slots list the token's experts in ascending id order (empty
        // and dropped slots have no position), so slot order is expert order
        float *o = a.out + (long long)t * a.D;
        for (int d = lane; d < a.D; d += 64) {
            float acc = 0.0f;
            for (int j = 0; j < a.kt; ++j) {
                const long long ent = (long long)t * a.kt + j;
                const int p = a.pos_of[ent];
                if (p < 0) continue;
                const long long off = (long long)p * a.ld_y + d;
                const float v = a.y_bf16 ? bf16_to_f32(((const uint16_t *)a.y)[off]) : ((const float *)a.y)[off];
                acc = acc + a.gates[ent] * v;
            }
            o[d] = acc;
        }
        return;
    }
    bool all_kept = (a.D & 3) == 0 && (a.ld_y & 3) == 0;
    for (int j = 0; j < a.kt; ++j) all_kept = all_kept && a.pos_of[(long long)t * a.kt + j] >= 0;
    if (all_kept) {
        if (a.lsh > 0) {
            if (try_combine_blend<2>(a, t, lane) || try_combine_blend<3>(a, t, lane) ||
                try_combine_blend<4>(a, t, lane))
                return;
        } else if (try_combine_fast<2>(a, t, lane) || try_combine_fast<1>(a, t, lane) ||
                   try_combine_fast<8>(a, t, lane) || try_combine_fast<4>(a, t, lane) ||
                   try_combine_fast<6>(a, t, lane)) {
            return;
        }
    }
    int ee[MOE_MAX_TOPK], pp[MOE_MAX_TOPK];
    float gg[MOE_MAX_TOPK];
    int n = 0;
    for (int j = 0; j < a.kt; ++j) {
        const long long ent = (long long)t * a.kt + j;
        const int p = a.pos_of[ent];
        if (p < 0) continue;
        const int e = a.idx[ent];
        const float g = a.gates[ent];
        int i = n;
        while (i > 0 && ee[i - 1] > e) {
            ee[i] = ee[i - 1];
            pp[i] = pp[i - 1];
            gg[i] = gg[i - 1];
            --i;
        }
        ee[i] = e;
        pp[i] = p;
        gg[i] = g;
        ++n;
    }
    float *o = a.out + (long long)t * a.D;
    for (int d = lane; d < a.D; d += 64) {
        float acc = 0.0f, sh = 0.0f;
        for (int i = 0; i < n; ++i) {
            const long long off = (long long)pp[i] * a.ld_y + d;
            const float v = a.y_bf16 ? bf16_to_f32(((const uint16_t *)a.y)[off]) : ((const float *)a.y)[off];
            if (i < a.lsh) sh = sh + v / (float)a.lsh;
            else acc = acc + gg[i] * v;
        }
        if (a.lsh > 0) acc = 0.5f * sh + 0.5f * acc;
        o[d] = acc;
    }
}

hipError_t launch_combine(const CombineArgs &a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    hipLaunchKernelGGL(combine_kernel, dim3((a.T + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ============================================================================
// Standalone losses on given routing (compute_loss seams).
// ============================================================================
// compute_loss(::SwitchTransformerLoss, indices, probs) in two launches.
// Part 1: block b of nb takes the contiguous token range [b R, (b + 1) R),
// R = ceil(T / nb): its entries' expert counts (LDS histogram) and, per
// expert e (thread e), the fp64 sum of probs[t][e] over the range in token
// order; both go to the block's row of the partials (cnt [nb][E], sum
// [nb][E]).  Every row is written (zeros for an empty range), so the
// partials need no clearing.
__global__ __launch_bounds__(256) void switch_loss_partial_kernel(const int *__restrict__ idx, int T, int k,
                                                                  const float *__restrict__ probs, int E,
                                                                  int *__restrict__ cnt_part,
                                                                  double *__restrict__ sum_part) {
    __shared__ int cnt[MOE_MAX_EXPERTS];
    const int tid = threadIdx.x;
    const int R = (T + gridDim.x - 1) / gridDim.x;
    const int t0 = min(T, (int)blockIdx.x * R), t1 = min(T, t0 + R);
    for (int e = tid; e < E; e += 256) cnt[e] = 0;
    __syncthreads();
    for (long long i = (long long)t0 * k + tid; i < (long long)t1 * k; i += 256) {
        const int e = idx[i];
        if (e > 0 && e <= E) atomicAdd(&cnt[e - 1], 1);
    }
    for (int e = tid; e < E; e += 256) {
        double ps = 0.0;
        for (int t = t0; t < t1; ++t) ps += (double)probs[(long long)t * E + e];
        sum_part[(long long)blockIdx.x * E + e] = ps;
    }
    __syncthreads();
    for (int e = tid; e < E; e += 256) cnt_part[(long long)blockIdx.x * E + e] = cnt[e];
}

// Part 2, one block: thread e adds its expert's partials in block order;
// f_e = count / (T k) (the length of indices counts every entry,
// src/balancing/losses.jl:17,30), P_e = mean_t probs[t][e] (:33), and the
// f_e P_e terms are summed in expert order (:35).  T = 0 gives NaN, the mean
// over no tokens.
__global__ __launch_bounds__(256) void switch_loss_finish_kernel(const int *__restrict__ cnt_part,
                                                                 const double *__restrict__ sum_part, int nb, int T,
                                                                 int k, int E, float alpha, float *out) {
#pragma clang fp contract(off)
    __shared__ float fp[MOE_MAX_EXPERTS];
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += 256) {
        long long c = 0;
        double ps = 0.0;
        for (int b = 0; b < nb; ++b) {
            c += cnt_part[(long long)b * E + e];
            ps += sum_part[(long long)b * E + e];
        }
        float f = (float)c;
        if ((long long)T * k > 0) f = f / (float)((long long)T * k);
        const float P = (float)ps / (float)T;
        fp[e] = f * P;
    }
    __syncthreads();
    if (tid == 0) {
        float s = fp[0];
        for (int e = 1; e < E; ++e) s = s + fp[e];
        out[0] = (alpha * (float)E) * s;
    }
}

int switch_loss_blocks(long long T) {
    // about 512 tokens per block, at most kSwitchLossMaxBlocks blocks
    return (int)std::max<long long>(1, std::min<long long>(kSwitchLossMaxBlocks, (T + 511) / 512));
}

hipError_t launch_switch_loss(const int *idx, int T, int k, const float *probs, int E, float alpha, void *partials,
                              float *out, hipStream_t s) {
    if (E < 1 || E > MOE_MAX_EXPERTS || T < 0 || k < 1) return hipErrorInvalidValue;
    const int nb = switch_loss_blocks(T);
    int *cnt_part = (int *)((uint8_t *)partials + switch_loss_sum_bytes(nb, E));
    double *sum_part = (double *)partials;
    hipLaunchKernelGGL(switch_loss_partial_kernel, dim3(nb), dim3(256), 0, s, idx, T, k, probs, E, cnt_part, sum_part);
    hipLaunchKernelGGL(switch_loss_finish_kernel, dim3(1), dim3(256), 0, s, cnt_part, sum_part, nb, T, k, E, alpha,
                       out);
    return hipGetLastError();
}

// compute_loss(::ZLoss, logits): beta * mean_t(logsumexp_t^2), one block.
__global__ __launch_bounds__(256) void z_loss_kernel(const float *logits, int T, int E, float beta, float *out) {
#pragma clang fp contract(off)
    __shared__ double red[256];
    const int tid = threadIdx.x;
    double acc = 0.0;
    for (int t = tid; t < T; t += 256) {
        const float *l = logits + (long long)t * E;
        float m = -INFINITY;
        for (int i = 0; i < E; ++i) if (l[i] > m) m = l[i];
        float s = 0.0f;
        for (int i = 0; i < E; ++i) s = s + (float)exp((double)(l[i] - m));
        const float lse = m + logf(s);
        acc += (double)(lse * lse);
    }
    red[tid] = acc;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) red[tid] += red[tid + st];
        __syncthreads();
    }
    if (tid == 0) out[0] = beta * ((float)red[0] / (float)T);
}

// update_bias! on given indices: one block counts entries 1..E, one thread steps.
__global__ __launch_bounds__(256) void aux_free_update_kernel(const int *idx, long long n, int E, float lr,
                                                              float momentum, float *bias, float *mom) {
    __shared__ int cnt[MOE_MAX_EXPERTS];
    __shared__ unsigned long long tot;
    const int tid = threadIdx.x;
    for (int e = tid; e < MOE_MAX_EXPERTS; e += 256) cnt[e] = 0;
    if (tid == 0) tot = 0;
    __syncthreads();
    unsigned long long mine = 0;
    for (long long i = tid; i < n; i += 256) {
        const int e = idx[i];
        if (e > 0 && e <= E) {  // the host checked that no id exceeds E
            atomicAdd(&cnt[e - 1], 1);
            ++mine;
        }
    }
    atomicAdd(&tot, mine);
    __syncthreads();
    if (tid == 0) aux_free_step(cnt, (long long)tot, E, lr, momentum, bias, mom);
}

hipError_t launch_aux_free_update(const int *idx, long long n, int E, float lr, float momentum, float *bias,
                                  float *mom, hipStream_t s) {
    hipLaunchKernelGGL(aux_free_update_kernel, dim3(1), dim3(256), 0, s, idx, n, E, lr, momentum, bias, mom);
    return hipGetLastError();
}

hipError_t launch_z_loss(const float *logits, int T, int E, float beta, float *out, hipStream_t s) {
    hipLaunchKernelGGL(z_loss_kernel, dim3(1), dim3(256), 0, s, logits, T, E, beta, out);
    return hipGetLastError();
}

}  // namespace moe
