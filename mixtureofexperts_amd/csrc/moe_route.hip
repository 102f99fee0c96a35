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
#include <mutex>

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

// The router weight's three parts as the fused router's B-fragment image:
// for each 32-wide K step s and each of its NTS 16-column tiles q, the 64
// lanes' 16-byte fragments in lane order (1 KB), so that every fragment load
// is one contiguous read.  Lane l of tile q holds column c = l % 16 at K
// s * 32 + 8 (l / 16) .. +8.  Paired (Er <= 8): tile 0 holds part 0 of the
// experts in columns 0..7 and part 1 in columns 8..15, tile 1 part 2 in
// columns 0..7 (8..15 zero); otherwise tile q = 3 et + p holds part p of
// experts 16 et .. 16 et + 15.  Past Er or D: zero.
__global__ void router_split_kernel(const float *__restrict__ w, int D, int Er, int Er_pad, int S, int NTS,
                                    int paired, uint16_t *__restrict__ img) {
#pragma clang fp contract(off)
    const long long n = (long long)S * NTS * 64 * 8;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
        const int m = (int)(i & 7), l = (int)((i >> 3) & 63);
        const long long qs = i >> 9;
        const int q = (int)(qs % NTS), st = (int)(qs / NTS);
        const int k = st * 32 + 8 * (l >> 4) + m, c = l & 15;
        int part, e;
        if (paired) {
            e = c & 7;
            part = (q == 0) ? (c >> 3) : ((c < 8) ? 2 : -1);
        } else {
            part = q % 3;
            e = (q / 3) * 16 + c;
        }
        const float v = (part >= 0 && e < Er && k < D) ? w[(long long)k * Er_pad + e] : 0.0f;
        const uint16_t b0 = f32_to_bf16(v);
        const float r1 = v - bf16_to_f32(b0);
        const uint16_t b1 = f32_to_bf16(r1);
        const float r2 = r1 - bf16_to_f32(b1);
        img[i] = (part <= 0) ? b0 : (part == 1 ? b1 : f32_to_bf16(r2));
    }
}

static int router_tiles_per_step(int Er) { return Er <= 8 ? 2 : 3 * ((Er + 15) / 16); }

hipError_t launch_router_split(const float *w, int D, int Er, int Er_pad, int Dp, uint16_t *img, hipStream_t s) {
    if (Dp % 32 != 0 || Er < 1 || Er > MOE_MAX_EXPERTS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(router_split_kernel, dim3(512), dim3(256), 0, s, w, D, Er, Er_pad, Dp / 32,
                       router_tiles_per_step(Er), Er <= 8 ? 1 : 0, img);
    return hipGetLastError();
}

// ============================================================================
// The router kernel (router_kernel): one launch per routing call.  Workgroup
// b of kRtThreads threads owns the TB = 16 or 64 tokens [b TB, b TB + TB)
// (its route block) and
//   1. computes their router logits on MFMA into LDS rows (or reads the
//      caller's logits), plus the router bias;
//   2. gates them, 8 lanes per token (softmax, top-k, gates);
//   3. writes the entries, the stable rank of each inside the route block
//      and expert, the route block's expert histogram and z-loss / entropy
//      sums, and adds its expert counts and probability sums (fixed point)
//      to the call's totals with integer atomics (the permute kernel's scan
//      turns them into rank bases, offsets, tile lists and losses).
// With an AuxiliaryFreeLoss the gating runs twice on the same LDS logits:
// the probabilities pass on the logits, then the gating pass on logits + the
// loss's bias.
// ============================================================================
#define RT_LDS __attribute__((address_space(3)))

// LDS byte address of a pointer into the workgroup's LDS (the M0 operand of
// global_load_lds).
__device__ __forceinline__ uint32_t rt_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const RT_LDS uint8_t *)p;
}

// global_load_lds_dwordx4: lane l copies 16 bytes from its own global address
// to LDS byte lds + 16 l (lds wave-uniform, an input operand bound to M0).
// The staging below waits for these with rt_wait_vm0 and a barrier before any
// LDS read of the bytes.
__device__ __forceinline__ void rt_dma16(const void *gaddr, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gaddr), "{m0}"(lds));
}
__device__ __forceinline__ void rt_wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

constexpr int kRtMaskWords = 16;  // rank bitmask words per expert: TB * kt <= 512 entries (TB <= 32 when kt > 8)

// The partner lane of butterfly step 1, 2, 3 inside an 8-lane group, by DPP:
// lane ^ 1, lane ^ 2 (quad permutations), then the mirrored lane of the other
// quad (7 - lane within the group).  After the first two steps every lane of
// a quad holds the quad's value, so the third pairs the two quads.
__device__ __forceinline__ int dpp_x1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false); }
__device__ __forceinline__ int dpp_x2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false); }
__device__ __forceinline__ int dpp_m8(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false); }
template <int STEP>
__device__ __forceinline__ int dpp_step(int v) {
    if constexpr (STEP == 0) return dpp_x1(v);
    else if constexpr (STEP == 1) return dpp_x2(v);
    else return dpp_m8(v);
}
template <int STEP>
__device__ __forceinline__ float dpp_stepf(float v) { return __int_as_float(dpp_step<STEP>(__float_as_int(v))); }
template <int STEP>
__device__ __forceinline__ double dpp_stepd(double v) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)dpp_step<STEP>((int)(unsigned)u), hi = (unsigned)dpp_step<STEP>((int)(unsigned)(u >> 32));
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
template <int STEP>
__device__ __forceinline__ uint64_t dpp_stepu64(uint64_t v) {
    const unsigned lo = (unsigned)dpp_step<STEP>((int)(unsigned)v), hi = (unsigned)dpp_step<STEP>((int)(unsigned)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Max over the 8 lanes of a token (NaN never enters: the callers' maxima
// start at -Inf and take a value only when it compares greater).
__device__ __forceinline__ float lanes8_max(float v) {
    float w = dpp_stepf<0>(v); v = (w > v) ? w : v;
    w = dpp_stepf<1>(v); v = (w > v) ? w : v;
    w = dpp_stepf<2>(v); v = (w > v) ? w : v;
    return v;
}
// Sum over the 8 lanes of a token as a fixed tree (lane pairs, then quads,
// then the two quads); every lane ends with the same bits.
__device__ __forceinline__ float lanes8_sum(float v) {
    v = v + dpp_stepf<0>(v);
    v = v + dpp_stepf<1>(v);
    return v + dpp_stepf<2>(v);
}
__device__ __forceinline__ double lanes8_sum(double v) {
    v = v + dpp_stepd<0>(v);
    v = v + dpp_stepd<1>(v);
    return v + dpp_stepd<2>(v);
}

// ---- router logits ----------------------------------------------------------
// Logits of the workgroup's TB tokens into LDS rows L[t][RW] (plus the router
// bias).  K runs in passes of KP columns.  A pass's x tile is staged in LDS
// (row r at byte r RB; 16-byte unit u of the row at unit position u ^ (r & 15),
// so the 16 rows of one fragment read hit 16 distinct bank groups): by
// global_load_lds when x is 16-byte aligned and D is a multiple of 32, else
// by register copies that write zeros past D.  Waves split the expert tiles
// (ET groups; paired tiles: one) and the pass's K steps (KG = 8 / ET
// groups).  A wave reads its weight fragments from the fragment image in
// groups of kRtSG steps (4; fp32 x: 2) through a ring of three register
// groups: the first two load with the x tile, then each group's loads are
// issued two groups ahead of its MFMAs.  Per step and 16-token row
// tile: acc += x . W0 + x . W1 + x . W2 (v_mfma_f32_16x16x32_bf16; fp32 x:
// each part of x times the weight parts of combined order <= 2).  A: 16
// tokens x 32 k (lane l: token l % 16, k 8 (l / 16) .. +8); B: the image
// tile; D lane l: column l % 16, tokens 4 (l / 16) .. +4.  The accumulators
// then go to LDS partials P[kg][t][col] and each logit is their sum in
// K-group order (paired tiles: the three parts' columns added in part order).
// More than 8 expert tiles (over 128 GEMM columns): column groups of 8 tiles
// in turn, one tile per wave and one K group, x staged again for each group.
template <int XBF16, int PAIRED, int RT>
__device__ __forceinline__ void rt_logits(const RtArgs &a, int t0, uint8_t *lds, float *L) {
#pragma clang fp contract(off)
    constexpr int ESZ = XBF16 ? 2 : 4;
    constexpr int NPT = PAIRED ? 2 : 3;   // image tiles per expert tile and step
    constexpr int NP = XBF16 ? 1 : 3;     // activation parts
    constexpr int NACC = PAIRED ? 2 : 1;  // accumulator tiles per row tile
    // RT: 16-token row tiles (the workgroup's TB = 16 RT tokens)
    constexpr int kRtSG = XBF16 ? 4 : 2;  // K steps per group of prefetched weight fragments
    // weight groups in the register ring: all of a paired wave's 16 steps in
    // flight at once for bf16 x; otherwise two groups ahead of the MFMAs
    constexpr int NRING = (PAIRED && XBF16) ? 5 : (XBF16 || PAIRED ? 3 : 2);
    // the next step's x fragments read during this step's MFMAs (bf16 x; the
    // three parts of fp32 x over four row tiles would not fit the registers)
    constexpr bool XPF = XBF16 || PAIRED;
    const RouterArgs &g = a.g;
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int TB = RT * 16, RB = a.RB, PPR = RB >> 4;
    const int ETA = PAIRED ? 1 : (g.Er + 15) >> 4;  // expert tiles of the GEMM
    const int NTS = PAIRED ? 2 : 3 * ETA;
    for (int cgo = 0; cgo < ETA; cgo += 8) {  // column group: tiles cgo .. cgo + 7
        const int ET = PAIRED ? 1 : min(ETA - cgo, 8);
        const int KG = ETA > 8 ? 1 : 8 / ET;
        const int cg = w % ET, kg = w / ET;
        const bool mw = kg < KG;  // this wave runs MFMAs

        rf32x4_t acc[RT][NACC];
#pragma unroll
        for (int ti = 0; ti < RT; ++ti)
#pragma unroll
            for (int j = 0; j < NACC; ++j) acc[ti][j] = rf32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

        using WF = rbf16x8_t[kRtSG][NPT];
        for (int k0 = 0; k0 < g.Dp; k0 += a.KP) {
            const int kp = min(a.KP, g.Dp - k0);
            const int UPR = kp * ESZ / 16;  // data units per staged row
            // ---- stage x[t0 .. t0 + TB)[k0 .. k0 + kp) (rows past T: row T - 1) ----
            if (a.dma) {
                const int NCH = TB * PPR / 64;  // 1 KB pieces of LDS
                for (int c = w; c < NCH; c += kRtThreads / 64) {
                    const int p = c * 64 + lane;
                    const int r = p / PPR, pu = p - r * PPR, u = pu ^ (r & 15);
                    const long long t = min(t0 + r, g.T - 1);
                    const uint8_t *src = (const uint8_t *)g.x + (t * g.D + k0) * ESZ + (u < UPR ? u : 0) * 16;
                    rt_dma16(src, __builtin_amdgcn_readfirstlane(rt_lds_addr(lds + c * 1024)));
                }
            } else {
                for (int p = tid; p < TB * PPR; p += kRtThreads) {
                    const int r = p / PPR, pu = p - r * PPR, u = pu ^ (r & 15);
                    const long long t = min(t0 + r, g.T - 1);
                    uint32_t q[4] = {0u, 0u, 0u, 0u};
                    if (u < UPR) {
                        const int kb = k0 + u * (16 / ESZ);
                        if (XBF16) {
                            const uint16_t *row = (const uint16_t *)g.x + t * g.D;
                            uint16_t hv[8];
#pragma unroll
                            for (int i = 0; i < 8; ++i) hv[i] = (kb + i < g.D) ? row[min(kb + i, g.D - 1)] : (uint16_t)0;
                            __builtin_memcpy(q, hv, 16);
                        } else {
                            const float *row = (const float *)g.x + t * g.D;
                            float fv[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i) fv[i] = (kb + i < g.D) ? row[min(kb + i, g.D - 1)] : 0.0f;
                            __builtin_memcpy(q, fv, 16);
                        }
                    }
                    *(u32x4_t *)(lds + p * 16) = u32x4_t{q[0], q[1], q[2], q[3]};
                }
            }
            // ---- this wave's K steps of the pass: [sb, se) ----
            const int sp = kp >> 5, spw = (sp + KG - 1) / KG;
            const int sb = (k0 >> 5) + kg * spw, se = min((k0 >> 5) + sp, sb + spw);
            const bool act = mw && sb < se;
            auto load_w = [&](int s0, WF &wf) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < kRtSG; ++i) {
                    const int st = min(s0 + i, se - 1);
#pragma unroll
                    for (int p = 0; p < NPT; ++p) {
                        const int q = PAIRED ? p : 3 * (cgo + cg) + p;
                        const rbf16x8_t *src = (const rbf16x8_t *)(g.ws + (((long long)st * NTS + q) * 64 + lane) * 8);
                        if (PAIRED && p == 1) {
                            // paired tile 1: columns 8..15 are zero in the image; those lanes skip the load
                            rbf16x8_t z = {};
                            if ((lane & 8) == 0) z = *src;
                            wf[i][p] = z;
                        } else {
                            wf[i][p] = *src;
                        }
                    }
                }
            };
            // the x fragments (parts) of step st of the pass, every row tile
            auto load_x = [&](int st, rbf16x8_t (&xa)[RT][NP]) __attribute__((always_inline)) {
                const int u = st - (k0 >> 5);  // step inside the pass
#pragma unroll
                for (int ti = 0; ti < RT; ++ti) {
                    const int r = ti * 16 + l16;
                    const uint8_t *row = lds + r * RB;
                    if (XBF16) {
                        xa[ti][0] = *(const rbf16x8_t *)(row + (((u * 4 + (lane >> 4)) ^ (r & 15)) << 4));
                    } else {
                        const int u0 = u * 8 + (lane >> 4) * 2;
                        const float4 f0 = *(const float4 *)(row + ((u0 ^ (r & 15)) << 4));
                        const float4 f1 = *(const float4 *)(row + (((u0 + 1) ^ (r & 15)) << 4));
                        const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
                        uint16_t h0[8], h1[8], h2[8];
#pragma unroll
                        for (int m = 0; m < 8; ++m) {
                            h0[m] = f32_to_bf16(v[m]);
                            const float r1 = v[m] - bf16_to_f32(h0[m]);
                            h1[m] = f32_to_bf16(r1);
                            h2[m] = f32_to_bf16(r1 - bf16_to_f32(h1[m]));
                        }
                        __builtin_memcpy(&xa[ti][0], h0, 16);
                        __builtin_memcpy(&xa[ti][NP > 1 ? 1 : 0], h1, 16);
                        __builtin_memcpy(&xa[ti][NP > 2 ? 2 : 0], h2, 16);
                    }
                }
            };
            // one group: the next step's x fragments are read while this step's
            // MFMAs run; the MFMAs of a step go part by part over the row tiles,
            // so consecutive ones write different accumulators
            auto mma = [&](int s0, const WF &wf) __attribute__((always_inline)) {
                rbf16x8_t xc[RT][NP], xn[XPF ? RT : 1][NP];
                if constexpr (XPF) load_x(min(s0, se - 1), xc);
#pragma unroll
                for (int i = 0; i < kRtSG; ++i) {
                    if (s0 + i >= se) break;
                    if constexpr (!XPF) load_x(s0 + i, xc);
                    else if (i + 1 < kRtSG) load_x(min(s0 + i + 1, se - 1), xn);
                    if constexpr (PAIRED) {
                        // tile 0 (parts 0 | 1): every x part; tile 1 (part 2): x part 0
#pragma unroll
                        for (int xi = 0; xi < NP; ++xi)
#pragma unroll
                            for (int ti = 0; ti < RT; ++ti)
                                acc[ti][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xc[ti][xi], wf[i][0], acc[ti][0], 0, 0, 0);
#pragma unroll
                        for (int ti = 0; ti < RT; ++ti)
                            acc[ti][NACC - 1] =
                                __builtin_amdgcn_mfma_f32_16x16x32_bf16(xc[ti][0], wf[i][NPT - 1], acc[ti][NACC - 1], 0, 0, 0);
                    } else {
#pragma unroll
                        for (int p = 0; p < 3; ++p)
#pragma unroll
                            for (int xi = 0; xi + p < 3 && xi < NP; ++xi)
#pragma unroll
                                for (int ti = 0; ti < RT; ++ti)
                                    acc[ti][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xc[ti][xi], wf[i][p < NPT ? p : 0],
                                                                                         acc[ti][0], 0, 0, 0);
                    }
                    if constexpr (XPF) {
                        if (i + 1 < kRtSG) {
#pragma unroll
                            for (int ti = 0; ti < RT; ++ti)
#pragma unroll
                                for (int xi = 0; xi < NP; ++xi) xc[ti][xi] = xn[ti][xi];
                        }
                    }
                }
            };
            // the ring: NRING - 1 groups in flight with the x tile, then each
            // group's loads issued NRING - 1 groups ahead of its MFMAs
            WF wr[NRING];
            if (act) {
#pragma unroll
                for (int j = 0; j + 1 < NRING; ++j)
                    if (sb + j * kRtSG < se) load_w(sb + j * kRtSG, wr[j]);
            }
            rt_wait_vm0();  // this wave's x pieces (and its first weight groups) have landed
            __syncthreads();
            if (act) {
                for (int s0 = sb; s0 < se; s0 += NRING * kRtSG) {
#pragma unroll
                    for (int j = 0; j < NRING; ++j) {
                        const int sj = s0 + j * kRtSG;
                        if (sj >= se) break;
                        const int nx = sj + (NRING - 1) * kRtSG;
                        if (nx < se) load_w(nx, wr[(j + NRING - 1) % NRING]);
                        mma(sj, wr[j]);
                    }
                }
            }
            __syncthreads();  // the pass's x tile is consumed
        }

        const float *bias = a.r.bias;
        if (!PAIRED && KG == 1) {
            // one K group: each logit is one wave's accumulator, written with the
            // bias straight into its row (the values the partial-sum pass gives)
            if (mw) {
#pragma unroll
                for (int ti = 0; ti < RT; ++ti) {
                    const int e = (cgo + cg) * 16 + l16;
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        const int t = ti * 16 + (lane >> 4) * 4 + rr;
                        float v = acc[ti][0][rr];
                        if (bias && e < a.r.Er) v = v + bias[e];
                        if (e < g.Er) L[t * a.RW + e] = v;
                    }
                }
            }
            continue;  // the next column group (ETA > 8), else done
        }
        // accumulators -> LDS partials P[kg][t][col] (over the staging region),
        // col = image column of the expert tile (paired: 16 j + c)
        const int NCOL = PAIRED ? 32 : ET * 16;
        float *P = (float *)lds;
        if (mw) {
#pragma unroll
            for (int ti = 0; ti < RT; ++ti) {
#pragma unroll
                for (int j = 0; j < NACC; ++j) {
                    const int col = PAIRED ? j * 16 + l16 : cg * 16 + l16;
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        const int t = ti * 16 + (lane >> 4) * 4 + rr;
                        P[(kg * TB + t) * NCOL + col] = acc[ti][j][rr];
                    }
                }
            }
        }
        __syncthreads();
        for (int q = tid; q < TB * g.Er; q += kRtThreads) {
            const int t = q / g.Er, e = q - t * g.Er;
            auto col_sum = [&](int col) __attribute__((always_inline)) {
                float v = P[t * NCOL + col];
                for (int k = 1; k < KG; ++k) v = v + P[(k * TB + t) * NCOL + col];
                return v;
            };
            float v = PAIRED ? (col_sum(e) + col_sum(8 + e)) + col_sum(16 + e) : col_sum(e);
            if (bias && e < a.r.Er) v = v + bias[e];  // (not on the noise network's columns)
            L[t * a.RW + e] = v;
        }
    }  // column groups (one when ETA <= 8: this path)
}

// ---- gating -------------------------------------------------------------------
// One gating pass over the route block's tokens: lane rs of token rt = tid /
// 8 owns the contiguous experts rs EPL .. +EPL of the token's row.  Logits:
// the LDS row L[rt] (plus xbias, the second pass's bias).  Per token: the
// max; exp terms e = (float)exp((double)(l - m)) (NNlib's branch for m ==
// +Inf); their fp32 sum in expert order (a chain through the lanes: lane r
// adds its experts, in order, to lane r - 1's running sum, passed on by DPP
// row_shr:1); probabilities e / s; the fp64 entropy terms and the
// logsumexp.  Top-k: k rounds, each taking the largest (isless key, then
// lower index) element below the previous round's, by a per-lane scan and a
// 3-step DPP butterfly; the gates.  Then per entry (lane rs = slot rs): its
// stable rank among the route block's entries of its expert (LDS bitmask per
// expert, bit = entry), and the route block's histogram, probability sums
// and loss terms.  Pr: LDS rows [TB][RW] for the output probabilities; G:
// LDS rows [TB][RW], the gate's working row (its logits, then the exp terms,
// then the probabilities).
//
// The per-expert work with long instruction sequences (fp64 exp, IEEE
// division, the entropy log, the noise draws) runs in loops over the lane's
// EPL experts through G, so that its code is executed EPL times from the
// instruction cache instead of being laid out EPL times (up to 16: tens of KB
// of straight-line code, fetched once per workgroup at L2 latency); only the
// ordered chain sum and the top-k compares work on registers (pr).
template <int EPL>
__device__ __forceinline__ void rt_gate(const RtArgs &A, int out_mask, const float *xbias, int blk, int t0, int ntok,
                                        const float *L, float *Pr, float *G, unsigned *emask,
                                        double (*wred)[kRtThreads / 64]) {
#pragma clang fp contract(off)
    const RouteArgs &a = A.r;
    const int RW = A.RW;
    const bool shared_gate = a.gate_kind == MOE_GATE_SHARED;
    const bool soft = a.gate_kind == MOE_GATE_SOFT;
    const bool zsep = shared_gate || soft;  // z-loss from a softmax of its own (all rows, unscaled)
    const bool out_probs = (out_mask & ROUTE_OUT_PROBS) != 0;
    const bool out_gating = (out_mask & ROUTE_OUT_GATING) != 0;
    // a gating pass on the caller's routing needs none of the softmax phases
    const bool softmax = out_probs || !a.given;
    const int E = a.E;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int rt = tid >> 3, rs = tid & 7;
    const bool rvalid = rt < ntok;
    const long long t = (long long)t0 + rt;
    const int ns = shared_gate ? a.ns : 0;  // rows before the routed ones
    const int base = rs * EPL;
    const int row = rt * RW;

    __syncthreads();  // a previous pass is done with emask and the rows
    for (int i = tid; i < a.Eh * kRtMaskWords; i += kRtThreads) emask[i] = 0u;

    const bool noise = A.noise_scale > 0.0f;
    // z-loss from a softmax of its own: over all rows, unscaled, and on the
    // logits without router noise (the reference's z-loss reruns the router
    // with training=false, src/core/moe_layer.jl:117-121)
    const bool zs_own = zsep || noise;
    float pr[EPL];  // exp terms, then probabilities
#pragma unroll
    for (int j = 0; j < EPL; ++j) pr[j] = 0.0f;
    // G[row + i] into pr (the lane's experts in range)
    auto load_pr = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const bool ok = rvalid && base + j < E;
            pr[j] = ok ? G[ok ? row + base + j : 0] : 0.0f;
        }
    };
    float lse = 0.0f;
    double hs = 0.0;
    if (softmax) {
        // ---- the gate's logits (router noise, the aux bias) into G; the
        // max of the routed rows (zs_own: also of all rows' plain logits) ----
        float m = -INFINITY, mz = -INFINITY;
#pragma unroll 4
        for (int j = 0; j < EPL; ++j) {
            const int i = base + j;
            const bool ok = rvalid && i < E;
            const float v = ok ? L[ok ? row + i : 0] : 0.0f;
            float x = v;
            if (noise) {
                // logits .+ randn .* noise_scale, or logits .+ noise_scale .*
                // (randn .* softplus.(noise logits)) (router.jl:32-41)
                const float r = init_normal(A.noise_seed, A.noise_call, (unsigned long long)t * E + (ok ? i : 0));
                if (A.noise_net) {
                    const float nl = ok ? L[ok ? row + E + i : 0] : 0.0f;
                    const float sp = log1pf(expf(-fabsf(nl))) + fmaxf(nl, 0.0f);  // NNlib softplus
                    x = x + A.noise_scale * (r * sp);
                } else {
                    x = x + r * A.noise_scale;
                }
            }
            // AuxiliaryFreeLoss gating pass: (noisy) logits .+ bias
            if (xbias) x = ok ? x + xbias[ok ? i : 0] : x;
            const float vg = ok ? x : 0.0f;
            if (ok) {
                G[row + i] = vg;
                if (A.store_rows && out_probs) a.logits[t * E + i] = vg;
            }
            const float sv = soft ? vg / a.soft_lambda : vg;  // logits ./ lambda for SoftMoEGating (advanced.jl:18)
            m = (ok && i >= ns && sv > m) ? sv : m;
            mz = (ok && v > mz) ? v : mz;
        }
        m = lanes8_max(m);
        if (zs_own) mz = lanes8_max(mz);
        // ---- exp terms into G (0 for the shared rows); zs_own: the z-loss
        // exponent sum over all rows ----
        float zs = 0.0f;
#pragma unroll 4
        for (int j = 0; j < EPL; ++j) {
            const int i = base + j;
            const bool ok = rvalid && i < E;
            const bool okr = ok && i >= ns;
            const float vg = ok ? G[ok ? row + i : 0] : 0.0f;
            const float sv = soft ? vg / a.soft_lambda : vg;
            const float ex = (m == INFINITY) ? ((sv == INFINITY) ? 1.0f : 0.0f) : (float)exp((double)(sv - m));
            if (ok) G[row + i] = okr ? ex : 0.0f;
            if (zs_own && ok) zs = zs + (float)exp((double)(L[row + i] - mz));
        }
        if (zs_own) zs = lanes8_sum(zs);
        load_pr();
        // ---- sum in expert order: a chain through the token's lanes ----
        float s;
        {
            float c = 0.0f;
#pragma unroll
            for (int j = 0; j < EPL; ++j) c = c + pr[j];
            s = (rs == 0) ? c : 0.0f;
#pragma unroll
            for (int r = 1; r < 8; ++r) {
                // lane i receives lane i - 1's running sum (row_shr:1 inside each 16-lane row)
                float c2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x111, 0xf, 0xf, false));
#pragma unroll
                for (int j = 0; j < EPL; ++j) c2 = c2 + pr[j];
                s = (rs == r) ? c2 : s;
            }
            // every lane of the token takes lane 7's total (swizzle: lane (i & 0x18) | 7)
            s = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(s), 0xF8));
        }
        // ---- probabilities (into G for the top-k; outputs: shared gating's
        // shared rows 1/E, routed rows p scaled by 1 - ns/E in Float64; the
        // caller's gate: its probabilities or ones ./ E); entropy terms p
        // log(p + 1e-8) with p + 1e-8 in Float64 as Julia promotes it, the
        // log as the hardware log2 (v_log_f32, about 1 ulp) times ln 2 in
        // fp32 (a statistic: the mean entropy is checked to 1e-5 relative) ----
        const float invE = 1.0f / (float)E;
        const double pscale = 1.0 - (double)ns / (double)E;
#pragma unroll 4
        for (int j = 0; j < EPL; ++j) {
            const int i = base + j;
            const bool ok = rvalid && i < E;
            float pv;
            if (a.given) {
                pv = a.given_probs ? (ok ? a.probs[ok ? t * E + i : 0] : 0.0f) : invE;
            } else {
                const float p = (ok ? G[ok ? row + i : 0] : 0.0f) / s;
                if (ok) G[row + i] = p;
                pv = (i < ns) ? invE : (shared_gate ? (float)((double)p * pscale) : p);
            }
            if (ok) {
                Pr[row + i] = pv;
                if (A.store_rows && out_probs) a.probs[t * E + i] = pv;
            }
            const double pd = (double)pv;
            const float lg = __builtin_amdgcn_logf((float)(pd + 1e-8)) * 0.693147180559945309f;
            const double term = pd * (double)lg;
            hs = ok ? hs + term : hs;
        }
        hs = lanes8_sum(hs);
        // logsumexp (src/balancing/losses.jl:111-114) from the same exp recipe,
        // the log in Float32 as Julia takes it of the Float32 sum
        lse = zs_own ? mz + logf(zs) : m + logf(s);
        if (!a.given) load_pr();
    }

    // ---- top-k and gates; the entries of this lane: slots rs and rs + 8 of
    // its token (kt <= 16 = 2 x 8 lanes) ----
    constexpr int SPL = 2;
    const int spl = a.kt > 8 ? 2 : 1;  // slot passes in use
    int my_e[SPL] = {0, 0};            // 1-based expert of entry (rt, rs + 8 p), 0: none
    float my_g[SPL] = {0.0f, 0.0f};
    if (out_gating && !a.given) {
        // routed slot of each pass: its slot minus the shared slots before it
        // (the layer's lsh shared experts, then SharedExpertGating's ns)
        int jr[SPL];
#pragma unroll
        for (int p = 0; p < SPL; ++p) jr[p] = rs + 8 * p - a.lsh - ns;
        uint64_t thr = ~0ull;
        float sg = 0.0f;
        float sel_v[SPL] = {0.0f, 0.0f};
        int sel_i[SPL] = {-1, -1};
#pragma unroll 1
        for (int r = 0; r < a.k; ++r) {
            uint64_t best = 0ull;
            float bv = 0.0f;
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const int i = base + j;
                const bool okr = rvalid && i >= ns && i < E;
                const uint64_t c = okr ? (((uint64_t)isless_key(pr[j]) << 32) | (uint32_t)~(uint32_t)i) : 0ull;
                const bool take = (r == 0 || c < thr) && c > best;
                best = take ? c : best;
                bv = take ? pr[j] : bv;
            }
            {
                uint64_t ob = dpp_stepu64<0>(best); float ov = dpp_stepf<0>(bv);
                bool tk = ob > best; best = tk ? ob : best; bv = tk ? ov : bv;
                ob = dpp_stepu64<1>(best); ov = dpp_stepf<1>(bv);
                tk = ob > best; best = tk ? ob : best; bv = tk ? ov : bv;
                ob = dpp_stepu64<2>(best); ov = dpp_stepf<2>(bv);
                tk = ob > best; best = tk ? ob : best; bv = tk ? ov : bv;
            }
            thr = best;
            sg = (r == 0) ? bv : sg + bv;  // gate sum in slot order
#pragma unroll
            for (int p = 0; p < SPL; ++p) {
                const bool mine = r == jr[p];
                sel_i[p] = mine ? (int)~(uint32_t)best : sel_i[p];
                sel_v[p] = mine ? bv : sel_v[p];
            }
        }
#pragma unroll
        for (int p = 0; p < SPL; ++p) {
            if (p >= spl) break;
            const int q = rs + 8 * p;  // the slot of this pass
            const bool routed = jr[p] >= 0 && jr[p] < a.k;
            if (a.lsh > 0 && q < a.lsh) {
                // forward_with_shared_experts: the layer's shared experts 1..lsh in
                // slots 0..lsh-1 (their outputs are averaged, the gate is only
                // reported); the gate's ids below are shifted by lsh
                // (expert_indices .+= num_shared_experts, src/core/moe_layer.jl:172)
                my_e[p] = q + 1;
                my_g[p] = 1.0f / (float)a.lsh;
            }
            if (soft) {
                // SoftMoEGating: top-k of the scaled-softmax probabilities; the
                // dispatch reads row `slot` of the (E, T) gate matrix, i.e. the
                // probability of expert `slot` (advanced.jl:24-33, moe_layer.jl:200)
                // for the routed slot jr
                float pj = 0.0f;
                const int jq = max(jr[p], 0);
                const int src = (lane & ~7) | (jq / EPL);  // the lane holding expert jq (jq < k <= E)
#pragma unroll
                for (int u = 0; u < EPL; ++u) {
                    const float wv2 = __shfl(pr[u], src);
                    pj = (u == jq % EPL) ? wv2 : pj;
                }
                if (routed) {
                    my_e[p] = sel_i[p] + 1 + a.lsh;
                    my_g[p] = pj;
                }
            } else if (shared_gate) {
                // the gate's shared slots (ids 1..ns, gate 1/kt of the gate's kt =
                // ns + k), then the routed top-k with gates scaled by 1 - ns/kt
                // in Float64 (advanced.jl:80-108)
                const int kg = a.kt - a.lsh;
                if (q >= a.lsh && q < a.lsh + ns) {
                    my_e[p] = q + 1;
                    my_g[p] = 1.0f / (float)kg;
                } else if (routed) {
                    my_e[p] = sel_i[p] + 1 + a.lsh;
                    my_g[p] = (float)((double)(sel_v[p] / sg) * (1.0 - (double)ns / (double)kg));
                }
            } else if (routed) {
                my_e[p] = sel_i[p] + 1 + a.lsh;
                my_g[p] = sel_v[p] / sg;
            }
            if (!rvalid || (routed && sel_i[p] < 0)) my_e[p] = 0;
        }
    } else if (out_gating && rvalid) {
        // the caller's routing: ids outside 1..E are skipped, as the
        // dispatch's `expert_id > 0 && expert_id <= length(experts)` does
        // (src/core/moe_layer.jl:198)
#pragma unroll
        for (int p = 0; p < SPL; ++p) {
            const int q = rs + 8 * p;
            if (q < a.kt) {
                const long long ent = t * a.kt + q;
                const int e = a.idx[ent];
                my_e[p] = (e >= 1 && e <= a.Eh) ? e : 0;
                my_g[p] = a.gates[ent];
            }
        }
    }

    // ---- stable rank of each entry among the route block's entries of its
    // expert (entries in token-then-slot order, as the bucket loop visits them)
    int ent[SPL];
    bool has_ent[SPL];
#pragma unroll
    for (int p = 0; p < SPL; ++p) {
        const int q = rs + 8 * p;
        ent[p] = rt * a.kt + q;  // entry of this pass (q < kt)
        has_ent[p] = out_gating && rvalid && q < a.kt && my_e[p] > 0;
    }
    __syncthreads();  // emask cleared
#pragma unroll
    for (int p = 0; p < SPL; ++p)
        if (has_ent[p]) atomicOr(&emask[(my_e[p] - 1) * kRtMaskWords + (ent[p] >> 5)], 1u << (ent[p] & 31));
    // route-block sums of the per-token loss terms (tokens rt: lane rs == 0),
    // in a fixed order: within a wave its 8 tokens in order (read lane by
    // lane: no LDS round trip per step), then the waves in order
    double zterm = 0.0, hterm = 0.0;
    if (softmax && rvalid && rs == 0) {
        zterm = (double)(lse * lse);
        hterm = -hs;
        if (out_probs && a.lse) a.lse[t] = lse;
    }
    {
        auto lane_d = [](double v, int l) __attribute__((always_inline)) {
            const unsigned long long u = (unsigned long long)__double_as_longlong(v);
            const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, l);
            const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), l);
            return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
        };
        double zw = lane_d(zterm, 0), hw = lane_d(hterm, 0);
#pragma unroll
        for (int q = 1; q < 8; ++q) {
            zw = zw + lane_d(zterm, 8 * q);
            hw = hw + lane_d(hterm, 8 * q);
        }
        zterm = zw;
        hterm = hw;
    }
    if (lane == 0) {
        wred[0][wv] = zterm;
        wred[1][wv] = hterm;
    }
    __syncthreads();  // emask complete, wred and the probability rows written
#pragma unroll
    for (int p = 0; p < SPL; ++p) {
        const int q = rs + 8 * p;
        if (has_ent[p]) {
            const unsigned *mk = &emask[(my_e[p] - 1) * kRtMaskWords];
            int rr = __popc(mk[ent[p] >> 5] & ((1u << (ent[p] & 31)) - 1u));
            for (int wd = 0; wd < (ent[p] >> 5); ++wd) rr += __popc(mk[wd]);
            a.rank[t * a.kt + q] = rr;
        }
        if (out_gating && rvalid && q < a.kt) {
            a.idx[t * a.kt + q] = my_e[p];
            a.gates[t * a.kt + q] = my_g[p];
        }
    }
    const int TW = (ntok * a.kt + 31) >> 5;  // mask words in use
    for (int e = tid; e < a.Eh; e += kRtThreads) {
        if (out_gating) {
            int c = 0;
            for (int wd = 0; wd < TW; ++wd) c += __popc(emask[e * kRtMaskWords + wd]);
            a.blk_counts[(long long)blk * a.ldc + e] = c;
            if (c) atomicAdd(&a.sup_cnt[(long long)(blk / kSuper) * a.ldc + e], c);
        }
        if (out_probs && e < E) {
            // per-row probability sums (Switch loss P_e): fp64 over the route
            // block's tokens in token order, added to the super block's sum
            // in fixed point (kPsumScale = 2^32, at most 2^38 per route block)
            double ps = 0.0;
#pragma unroll 8
            for (int i = 0; i < ntok; ++i) ps += (double)Pr[i * RW + e];
            const unsigned long long fx = __double2ull_rn(ps * kPsumScale);
            if (fx) atomicAdd(&a.sup_p[(long long)(blk / kSuper) * a.ldc + e], fx);
        }
    }
    if (tid == 0 && out_probs) {
        double zb = 0.0, hb = 0.0;
#pragma unroll
        for (int wd = 0; wd < kRtThreads / 64; ++wd) {
            zb += wred[0][wd];
            hb += wred[1][wd];
        }
        a.blk_zh[(long long)blk * 2] = zb;
        a.blk_zh[(long long)blk * 2 + 1] = hb;
    }
}

// LDS row stride of the logits and probability rows for E experts: a multiple
// of 4 floats (16 B) whose count of 16-byte units is odd, so that token
// threads reading 16 B at one column hit distinct bank quads.
__host__ __device__ inline int route_rw(int E) { return 4 * ((((E + 3) / 4 + 1) | 1)); }

// LG: 0 = the caller's logits (r.part), 1 = logits GEMM on bf16 x, 2 = on fp32
// x.  PAIRED: Er <= 8 (the paired weight tiles).  EPL: experts per lane.
// RT: 16-token row tiles of the logits GEMM (TB = 16 RT).
template <int LG, int PAIRED, int EPL, int RT>
__global__ __launch_bounds__(kRtThreads) void router_kernel(RtArgs A) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t rdyn[];
    __shared__ double wred[2][kRtThreads / 64];
    const int blk = blockIdx.x;
    const int t0 = blk * A.TB;
    const int ntok = min(A.TB, A.r.T - t0);
    float *L = (float *)(rdyn + A.off_L);
    // the rank bitmasks, Eh x kRtMaskWords words after the logits rows
    unsigned *emask = (unsigned *)(rdyn + A.off_M);
    // over the staging region, free once the logits are in L: the output
    // probability rows, then the gate's working rows
    float *Pr = (float *)rdyn;
    float *G = Pr + A.TB * A.RW;
    // the other parity's super-block totals, last read by the previous call's permute
    for (int s = blk; s < A.r.nsup_max; s += gridDim.x)
        for (int e = threadIdx.x; e < A.r.ldc; e += kRtThreads) {
            A.r.clr_sup[(long long)s * A.r.ldc + e] = 0;
            A.r.clr_supp[(long long)s * A.r.ldc + e] = 0ull;
        }
    if constexpr (LG > 0) {
        rt_logits<LG == 1, PAIRED, RT>(A, t0, rdyn, L);
    } else {
        const int Er = A.r.Er;
        for (int q = threadIdx.x; q < ntok * Er; q += kRtThreads) {
            const int t = q / Er, e = q - t * Er;
            float v = A.r.part[(long long)(t0 + t) * Er + e];
            if (A.r.bias) v = v + A.r.bias[e];
            L[t * A.RW + e] = v;
        }
    }
    if (A.npass == 2) {
        rt_gate<EPL>(A, ROUTE_OUT_PROBS, nullptr, blk, t0, ntok, L, Pr, G, emask, wred);
        rt_gate<EPL>(A, ROUTE_OUT_GATING, A.aux_bias, blk, t0, ntok, L, Pr, G, emask, wred);
    } else {
        rt_gate<EPL>(A, A.r.out_mask, nullptr, blk, t0, ntok, L, Pr, G, emask, wred);
    }
}

// experts per lane of a token's 8 (the gating's register blocks)
static int route_epl(int E) {
    return E <= 8 ? 1 : (E <= 16 ? 2 : (E <= 32 ? 4 : (E <= 64 ? 8 : (E <= 80 ? 10 : (E <= 96 ? 12 :
           (E <= 128 ? 16 : (E <= 256 ? 32 : 64)))))));
}

// dynamic LDS of a router workgroup (the static wred is 128 B of the 160 KB)
constexpr size_t kRtLdsMax = 159 * 1024;

template <int LG, int PAIRED, int EPL, int RT>
static hipError_t launch_router_case(const RtArgs &A, int nblk, size_t lds, hipStream_t s) {
    auto kern = router_kernel<LG, PAIRED, EPL, RT>;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [&] {
        attr = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRtLdsMax);
    });
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, dim3(nblk), dim3(kRtThreads), lds, s, A);
    return hipGetLastError();
}

hipError_t launch_router(RtArgs A, int *tb, hipStream_t s) {
    const RouteArgs &a = A.r;
    if (a.T <= 0) {
        *tb = kRtMinBlock;
        return hipSuccess;
    }
    const bool gemm = A.g.x != nullptr;
    if (a.E != a.Er || a.E < 1 || a.E > MOE_MAX_EXPERTS || a.Eh > MOE_MAX_EXPERTS || a.k > MOE_MAX_TOPK ||
        ((a.out_mask & ROUTE_OUT_GATING) && a.kt > MOE_MAX_TOPK) || (!gemm && !a.part))
        return hipErrorInvalidValue;
    const int Er = a.Er;
    // the GEMM's columns: the router logits, then (noise network) the noise logits
    const int Eg = gemm ? A.g.Er : Er;
    const bool paired = gemm && Eg <= 8;
    const int ET = paired ? 1 : (Eg + 15) / 16;
    // tokens per workgroup: 16 for the paired (few-expert) GEMM, whose x tile
    // is widest; otherwise 64 (the weight image is read once per workgroup:
    // the more tokens share it the better; 64 tokens fill the gating lanes),
    // or 32 when 64-token workgroups would leave CUs idle (their x tile then
    // also takes fewer K passes) (the logits GEMM's row tiles are
    // compile-time: 1, 2 or 4)
    // more than 8 slots per token: 32-token workgroups at most (the rank
    // bitmasks hold kRtMaskWords * 32 = 512 entries per expert); the three
    // LDS rows of a token (logits, probabilities, gate) over 128 columns: 32
    // tokens, over 256 columns: 16
    const bool wide = (a.out_mask & ROUTE_OUT_GATING) && a.kt > 8;
    const bool half = (gemm && !paired && A.ncu > 0 && (a.T + 63) / 64 < A.ncu) || wide || Eg > 128;
    const int TB = (gemm && paired) || Eg > 256 ? 16 : (half ? 32 : 64);
    *tb = TB;
    A.TB = TB;
    A.RW = route_rw(Eg);
    const size_t rows = sizeof(float) * (size_t)TB * A.RW;
    const size_t mask_bytes = sizeof(unsigned) * (size_t)a.Eh * kRtMaskWords;
    // the x tile, rows and partials within 150 KB (the bitmasks of up to 128
    // experts beside them), less for more experts
    const size_t lds_max = std::min<size_t>(150 * 1024, kRtLdsMax - mask_bytes);
    size_t region0 = 2 * rows;  // the gating's Pr and G rows
    if (gemm) {
        const RouterArgs &g = A.g;
        if (g.Dp % 32 != 0 || g.Dp < g.D || g.Er != (A.noise_net ? 2 * Er : Er) || g.Er > MOE_MAX_EXPERTS)
            return hipErrorInvalidValue;
        const int ESZ = g.x_bf16 ? 2 : 4;
        // x tile bytes per row: what LDS holds beside the logits rows, in 256 B units
        const size_t avail = lds_max - rows - 1024;
        const int maxRB = (int)((avail / TB) & ~(size_t)255);
        const int KPmax = maxRB / ESZ;
        A.KP = std::min(g.Dp, KPmax);
        A.RB = ((A.KP * ESZ + 255) / 256) * 256;
        A.dma = (g.D % 32 == 0) && (((uintptr_t)g.x & 15) == 0);
        // the partial sums of the K groups (one column group of at most 8
        // tiles: more tiles write their logits directly)
        const int KG = ET > 8 ? 0 : 8 / ET;
        const size_t part = sizeof(float) * (size_t)KG * TB * (paired ? 32 : ET * 16);
        region0 = std::max(region0, std::max((size_t)TB * A.RB, part));
    }
    A.off_L = (int)((region0 + 1023) & ~(size_t)1023);
    A.off_M = (int)(A.off_L + rows);
    const size_t lds = (size_t)A.off_M + mask_bytes;
    const int nblk = (a.T + TB - 1) / TB;
    if (lds > lds_max + mask_bytes || a.ldc < a.Eh || !a.blk_zh || !a.sup_cnt || !a.sup_p || !a.clr_sup || !a.clr_supp ||
        a.nsup_max * kSuper < nblk)
        return hipErrorInvalidValue;
    const int epl = route_epl(Er);
#define MOE_RT(LG_, P_, EPL_, RT_) return launch_router_case<LG_, P_, EPL_, RT_>(A, nblk, lds, s)
#define MOE_RT_EPL(LG_, RT_)            \
    switch (epl) {                      \
    case 2: MOE_RT(LG_, 0, 2, RT_);     \
    case 4: MOE_RT(LG_, 0, 4, RT_);     \
    case 8: MOE_RT(LG_, 0, 8, RT_);     \
    case 10: MOE_RT(LG_, 0, 10, RT_);   \
    case 12: MOE_RT(LG_, 0, 12, RT_);   \
    default: MOE_RT(LG_, 0, 16, RT_);   \
    }
    // over 128 router rows: 32 experts per lane on 32-token workgroups, over
    // 256: 64 on 16-token ones (a noise network's GEMM columns can make the
    // workgroups smaller than the gating needs: the TB they get is used)
    if (epl == 64) {
        if (!gemm) MOE_RT(0, 0, 64, 4);
        if (A.g.x_bf16) MOE_RT(1, 0, 64, 1);
        MOE_RT(2, 0, 64, 1);
    }
    if (epl == 32) {
        if (!gemm) MOE_RT(0, 0, 32, 4);
        if (TB == 16) {
            if (A.g.x_bf16) MOE_RT(1, 0, 32, 1);
            MOE_RT(2, 0, 32, 1);
        }
        if (A.g.x_bf16) MOE_RT(1, 0, 32, 2);
        MOE_RT(2, 0, 32, 2);
    }
    if (!gemm) {
        // (RT only shapes the logits GEMM, which this case does not run)
        if (epl == 1) MOE_RT(0, 0, 1, 4);
        MOE_RT_EPL(0, 4)
    }
    if (A.g.x_bf16) {
        if (paired) MOE_RT(1, 1, 1, 1);
        if (half) MOE_RT_EPL(1, 2)
        MOE_RT_EPL(1, 4)
    }
    if (paired) MOE_RT(2, 1, 1, 1);
    if (half) MOE_RT_EPL(2, 2)
    MOE_RT_EPL(2, 4)
#undef MOE_RT_EPL
#undef MOE_RT
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
                                                                   int C, uint16_t *__restrict__ sel) {
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

// One thread per token: with shared experts of the layer (lsh > 0) its
// first lsh slots hold them (ids 1..lsh, gate 1/lsh reported); the next
// slots hold the routed experts that took it in ascending id order, ids
// shifted by lsh (src/core/moe_layer.jl:172), at most kcap = min(C, E) of
// them (a later expert past the capacity rows is left out,
// expert_choice.jl:40-50), gate = probability of the expert for the token;
// the remaining slots of the kt are empty (id 0).  sel[t][e] becomes the
// routed slot + 1 of entry (t, e) (<= kcap <= MOE_MAX_EXPERTS), or 0 when expert e did
// not take token t or the entry was left out.
__global__ __launch_bounds__(256) void expert_choice_assemble_kernel(uint16_t *__restrict__ sel,
                                                                     const float *__restrict__ probs, int T, int E,
                                                                     int kt, int kcap, int lsh, int *idx,
                                                                     float *gates) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= T) return;
    for (int j = 0; j < lsh; ++j) {
        idx[(long long)t * kt + j] = j + 1;
        gates[(long long)t * kt + j] = 1.0f / (float)lsh;
    }
    int c = 0;
    for (int e = 0; e < E; ++e) {
        const long long o = (long long)t * E + e;
        if (sel[o]) {
            if (c < kcap) {
                idx[(long long)t * kt + lsh + c] = lsh + e + 1;
                gates[(long long)t * kt + lsh + c] = probs[o];
                sel[o] = (uint16_t)(c + 1);
            } else {
                sel[o] = 0;
            }
            ++c;
        }
    }
    for (int j = lsh + min(c, kcap); j < kt; ++j) {
        idx[(long long)t * kt + j] = 0;
        gates[(long long)t * kt + j] = 0.0f;
    }
}

// The bucketing inputs of the kept entries, per route block of rb
// tokens: thread e (of the lsh + E experts of the layer) walks the block's
// tokens in order; a token holds expert e in at most one slot, so the
// entry's rank among expert e's entries of the block (token-then-slot order,
// the bucket loop's) is the count of earlier tokens that hold e.  A shared
// expert e < lsh is held by every token, in slot e.
__global__ __launch_bounds__(MOE_MAX_EXPERTS) void expert_choice_rank_kernel(const uint16_t *__restrict__ sel, int T,
                                                                            int E, int kt, int lsh, int *rank,
                                                                            int *blk_counts, int ldc,
                                                                            int *sup_cnt, int rb) {
    const int e = threadIdx.x;
    if (e >= lsh + E) return;
    const int t0 = blockIdx.x * rb;
    const int ntok = min(rb, T - t0);
    int c = 0;
    if (e < lsh) {
        for (int i = 0; i < ntok; ++i) rank[(long long)(t0 + i) * kt + e] = i;
        c = ntok;
    } else {
        for (int i = 0; i < ntok; ++i) {
            const int sl = sel[(long long)(t0 + i) * E + (e - lsh)];
            if (sl) {
                rank[(long long)(t0 + i) * kt + lsh + sl - 1] = c;
                ++c;
            }
        }
    }
    blk_counts[(long long)blockIdx.x * ldc + e] = c;
    if (c) atomicAdd(&sup_cnt[(long long)(blockIdx.x / kSuper) * ldc + e], c);
}

hipError_t launch_expert_choice(const float *logits, const float *probs, int T, int E, int lsh, int C, int kt,
                                uint16_t *sel, int *idx, float *gates, int *rank, int *blk_counts, int ldc,
                                int *sup_cnt, int rb, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    if (lsh < 0 || lsh + E > MOE_MAX_EXPERTS || kt < lsh + min(C, E) || kt > MOE_MAX_EXPERTS || ldc < lsh + E)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(expert_choice_select_kernel, dim3(E), dim3(256), 0, s, logits, T, E, C, sel);
    hipLaunchKernelGGL(expert_choice_assemble_kernel, dim3((T + 255) / 256), dim3(256), 0, s, sel, probs, T, E, kt,
                       min(C, E), lsh, idx, gates);
    hipLaunchKernelGGL(expert_choice_rank_kernel, dim3((T + rb - 1) / rb), dim3(MOE_MAX_EXPERTS), 0, s, sel, T, E,
                       kt, lsh, rank, blk_counts, ldc, sup_cnt, rb);
    return hipGetLastError();
}

// ============================================================================
// Scan: the route blocks' rank bases, the capacity clamp, offsets, the
// (expert, m0) GEMM tile list and the loss scalars, at the start of the
// permute kernel.
// ============================================================================
// update_bias!(::AuxiliaryFreeLoss, expert_indices) after its counter check
// (src/balancing/auxiliary_free.jl:36-69), one thread, with Julia's types:
// counts Float32, target = total / E and the gradient in Float64, the
// momentum stored as Float32 of a Float64 sum, the bias step in Float32, then
// bias .-= mean(bias) with the Float32 sum taken in index order.
// With the layer's shared experts (lsh > 0) the indices are the gate's ids
// shifted by lsh (forward_with_shared_experts, src/core/moe_layer.jl:172,
// 182): the shared experts e < lsh hold none of them, except that `extra`
// entries (an ExpertChoice matrix's empty entries, shifted to id lsh) count
// for expert lsh - 1 (0-based).
__device__ inline void aux_free_step(const int *cnt, int lsh, long long extra, long long total, int E, float lr,
                                     float momentum, float *bias, float *mom) {
#pragma clang fp contract(off)
    if (total <= 0) return;
    const double target = (double)total / (double)E;
    for (int e = 0; e < E; ++e) {
        const long long ce = (e < lsh) ? (e == lsh - 1 ? extra : 0) : cnt[e];
        const double grad = ((double)(float)ce - target) / (double)total;
        const float m = (float)((double)(momentum * mom[e]) + (double)(1.0f - momentum) * grad);
        mom[e] = m;
        bias[e] = bias[e] - lr * m;
    }
    float s = bias[0];
    for (int e = 1; e < E; ++e) s = s + bias[e];
    const float mean = s / (float)E;
    for (int e = 0; e < E; ++e) bias[e] = bias[e] - mean;
}

// Scan, run by every permute workgroup for its route block blk: the
// capacity, the expert counts after capacity (from the call's totals), their
// offsets and GEMM tile starts (exclusive prefixes over the experts), and the
// route block's rank bases (the counts of the route blocks before it, summed
// with integer LDS atomics).  The writer (workgroup 0) also writes the
// offsets, counts, tile starts, the (expert, m0) GEMM tile
// list and the capacity, computes the Switch and z losses and the mean
// entropy, and runs the AuxiliaryFreeLoss step.  Ends with a barrier.
struct ScanLds {
    int cnt[MOE_MAX_EXPERTS];
    int base[MOE_MAX_EXPERTS];
    int tot[MOE_MAX_EXPERTS];                  // the call's entries per expert (before capacity)
    unsigned long long ptot[MOE_MAX_EXPERTS];  // the call's probability sums (fixed point), workgroup 0
    int off[MOE_MAX_EXPERTS + 1];
    int tstart[MOE_MAX_EXPERTS + 1];
    float fp[MOE_MAX_EXPERTS];
    double zh[2];
    int cap;
    float lsum;
};

__device__ __forceinline__ void scan_block(const ScanArgs &a, int blk, ScanLds &L, bool writer) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x, nth = blockDim.x;
    if (tid == 0) {
        int cap = INT_MAX;
        if (a.training && a.drop) {
            // capacity = ceil(Int, capacity_factor * batch_size / num_experts), Float32
            const float cf = ceilf((a.capacity_factor * (float)a.T) / (float)a.E);
            cap = (cf >= 2147483647.0f) ? INT_MAX : (int)cf;
        }
        L.cap = cap;
    }
    for (int e = tid; e < a.E; e += nth) {
        L.base[e] = 0;
        L.tot[e] = 0;
        L.ptot[e] = 0ull;
    }
    __syncthreads();
    {
        // rank bases: the super blocks before blk's, then the route blocks
        // of its own super block before it (at most 2 kSuper - 1 rows); the
        // totals: every super block's row (workgroup 0 also the probability
        // sums).  Thread (g, j) adds row j's experts 4 g .. 4 g + 3, all
        // rows' loads in flight at once (integer LDS atomics: any order)
        const int ng = (a.E + 3) / 4;
        const int ns = blk / kSuper, nrow = ns + (blk - ns * kSuper);
        const int nq = ng * (nrow + a.nsup * (writer ? 2 : 1));
        for (int q = tid; q < nq; q += nth) {
            const int g = q % ng, j = q / ng;
            if (j < nrow + a.nsup) {
                const bool bj = j < nrow;
                const int *src = !bj ? a.sup_cnt + (long long)(j - nrow) * a.ldc
                                     : (j < ns) ? a.sup_cnt + (long long)j * a.ldc
                                                : a.blk_counts + (long long)(ns * kSuper + j - ns) * a.ldc;
                const int4 v = *(const int4 *)(src + 4 * g);
                const int s[4] = {v.x, v.y, v.z, v.w};
                int *dst = bj ? L.base : L.tot;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (4 * g + i < a.E && s[i]) atomicAdd(&dst[4 * g + i], s[i]);
            } else {
                const unsigned long long *src = a.sup_p + (long long)(j - nrow - a.nsup) * a.ldc + 4 * g;
                const ulonglong2 v0 = *(const ulonglong2 *)src, v1 = *(const ulonglong2 *)(src + 2);
                const unsigned long long s[4] = {v0.x, v0.y, v1.x, v1.y};
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (4 * g + i < a.Np && s[i]) atomicAdd(&L.ptot[4 * g + i], s[i]);
            }
        }
    }
    const float total = (float)((long long)a.T * a.kl);
    __syncthreads();
    for (int e = tid; e < a.E; e += nth) {
        const int ce = min(L.tot[e], L.cap);
        L.cnt[e] = ce;
        // the terms f_e * P_e of the Switch loss (src/balancing/losses.jl:15-36)
        // over the a.Np probability rows; with shared experts of the layer the
        // ids are the shifted routed ids and expert e < lsh holds none of them
        if (writer && e < a.Np) {
            float f = (float)ce;
            if (e < a.lsh) {
                // ExpertChoice's empty entries, shifted to id lsh (ec_empty)
                long long empty = 0;
                if (a.ec_empty && e == a.lsh - 1) {
                    empty = (long long)a.T * a.kl;
                    for (int r = a.lsh; r < a.E; ++r) empty -= L.tot[r];
                }
                f = (float)empty;
            }
            if (a.T * a.kl > 0) f = f / total;
            const float P = (float)((double)L.ptot[e] / kPsumScale) / (float)a.T;
            L.fp[e] = f * P;
        }
    }
    if (writer && tid >= 64 && tid < 128) {
        // the z and entropy sums over the route blocks: lane l takes rows
        // l, l + 64, ... in order, then a fixed butterfly over the lanes
        const int l = tid - 64;
        double z = 0.0, hh = 0.0;
        for (int b = l; b < a.nblk; b += 64) {
            z += a.blk_zh[(long long)b * 2];
            hh += a.blk_zh[(long long)b * 2 + 1];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            z = z + __shfl_xor(z, o);
            hh = hh + __shfl_xor(hh, o);
        }
        if (l == 0) {
            L.zh[0] = z;
            L.zh[1] = hh;
        }
    }
    __syncthreads();
    // offsets and GEMM tile starts: exclusive prefixes over the experts by
    // wave 0, in groups of 64 experts (lane l: expert g0 + l of group g0)
    if (tid < 64) {
        int cbase = 0, nbase = 0;  // totals of the groups before
        for (int g0 = 0; g0 < a.E; g0 += 64) {
            const int e = g0 + tid;
            const int c = (e < a.E) ? L.cnt[e] : 0;
            const int n = (c + a.bm - 1) / a.bm;
            int cs = c, ns = n;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int cu = __shfl_up(cs, o), nu = __shfl_up(ns, o);
                if (tid >= o) {
                    cs += cu;
                    ns += nu;
                }
            }
            if (e <= a.E) {  // (e == E: the totals)
                L.off[e] = cbase + cs - c;
                L.tstart[e] = nbase + ns - n;
            }
            cbase += __shfl(cs, 63);
            nbase += __shfl(ns, 63);
        }
        if (tid == 0 && (a.E & 63) == 0) {  // the totals, past the last group's lanes
            L.off[a.E] = cbase;
            L.tstart[a.E] = nbase;
        }
        if (writer) {
            // the Switch-loss sum over the a.Np terms: in expert order up to 16
            // experts (Julia's sequential sum), else a fixed tree: lane l adds
            // the pairs (2 l, 2 l + 1) of each 128 experts in turn, then a
            // butterfly over the lanes (Julia's order for longer arrays is its
            // SIMD reduction, not reproduced)
            float part = 0.0f;
            if (a.Np > 16) {
#pragma unroll
                for (int q = 0; q < MOE_MAX_EXPERTS / 128; ++q) {
                    const int e0 = 128 * q + 2 * tid, e1 = e0 + 1;
                    float pq = (e0 < a.Np) ? L.fp[e0] : 0.0f;
                    if (e1 < a.Np) pq = pq + L.fp[e1];
                    part = (q == 0) ? pq : part + pq;
                }
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) part = part + __shfl_xor(part, o);
            } else if (tid == 0) {
                part = L.fp[0];
                for (int e = 1; e < a.Np; ++e) part = part + L.fp[e];
            }
            if (tid == 0) L.lsum = part;
        }
    }
    __syncthreads();
    if (!writer) return;
    if (tid == 0) {
        a.cap_out[0] = L.cap;
        a.num_tiles[0] = L.tstart[a.E];
        const double zs = L.zh[0], hs = L.zh[1];
        const float s = L.lsum;
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
            // the kept entries of each expert are the counts after capacity;
            // with shared experts the loss's index matrix holds the routed
            // entries (and ExpertChoice's empty ones, as id lsh)
            long long kept = 0;
            for (int e = a.lsh; e < a.E; ++e) kept += L.cnt[e];
            const long long empty = a.ec_empty ? (long long)a.T * a.kl - kept : 0;
            aux_free_step(L.cnt, a.lsh, empty, kept + empty, a.E, a.aux_lr, a.aux_momentum, a.aux_bias, a.aux_mom);
        }
    }
    for (int e = tid; e <= a.E; e += nth) {
        a.offsets[e] = L.off[e];
        a.tile_start[e] = L.tstart[e];
    }
    if (a.item_start && tid < 64) {
        // the up GEMM's work items per expert: pair_nt n-tiles times its M
        // tiles, except that a last M tile of at most bm / 2 rows serves two
        // n-tiles in one item (pair_nt even); exclusive prefix by wave 0
        auto items = [&](int e) {
            if (e >= a.E) return 0;
            const int c = L.cnt[e], f = c / a.bm, r = c - f * a.bm;
            return (r > 0 && 2 * r <= a.bm) ? a.pair_nt * f + a.pair_nt / 2 : a.pair_nt * (f + (r > 0 ? 1 : 0));
        };
        int nbase = 0;
        for (int g0 = 0; g0 < a.E; g0 += 64) {
            const int e = g0 + tid;
            const int n = items(e);
            int ns = n;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int nu = __shfl_up(ns, o);
                if (tid >= o) ns += nu;
            }
            if (e <= a.E) a.item_start[e] = nbase + ns - n;
            nbase += __shfl(ns, 63);
        }
        if (tid == 0 && (a.E & 63) == 0) a.item_start[a.E] = nbase;
    }
    for (int e = tid; e < a.E; e += nth) {
        a.counts[e] = L.cnt[e];
        const int nt = L.tstart[e + 1] - L.tstart[e];
        for (int i = 0; i < nt; ++i) a.tiles[L.tstart[e] + i] = make_int2(e, i * a.bm);
    }
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
// Permute: workgroups of kPermTokens tokens of one route block (its scan
// first), one wave per token.  Lanes < kt finalise the token's entries (capacity drop +
// renormalisation, position), then the wave copies the token's row into
// every position it owns, converting to the GEMM type.
// ============================================================================
// bf16 rows into the bf16 tile image: UB 16-byte chunks per lane per batch
// (UB * 512 columns, the smallest power of two covering D up to 2048, so that
// few lanes rewrite the row's last chunk), loaded together from clamped
// in-row addresses, then stored to every position the token holds.
__device__ __forceinline__ bool permute_bf16_rows(const PermuteArgs &a) {
    return a.copy_rows && a.ct == CT_BF16 && a.x_bf16 && (a.D & 7) == 0;
}
template <int UB>
__device__ __forceinline__ void load_row_chunk(const PermuteArgs &a, int t, int d0, int lane, u32x4_t (&v)[UB]) {
    const uint16_t *__restrict__ src = (const uint16_t *)a.x + (long long)t * a.D;
#pragma unroll
    for (int u = 0; u < UB; ++u) v[u] = *(const u32x4_t *)(src + min(d0 + u * 512 + lane * 8, a.D - 8));
}

// The entry of lane j < kt of a token (its expert id, gate and rank inside
// the route block), loaded ahead of the scan that gives its position.
struct EntryMeta {
    int e, rk;
    float g;
};
__device__ __forceinline__ EntryMeta load_meta(const PermuteArgs &a, int t, int lane) {
    EntryMeta m{0, 0, 0.0f};
    if (t >= 0 && lane < a.kt) {
        const long long ent = (long long)t * a.kt + lane;
        m.e = a.idx[ent];
        m.g = a.gates[ent];
        m.rk = a.rank[ent];
    }
    return m;
}

// A token's entries after the scan: capacity drop and renormalisation,
// positions (pos_of, perm, gate_sorted); returns the xp row of lane j's entry
// j (< 0: none).
__device__ __forceinline__ int permute_entries(const PermuteArgs &a, int t, int lane, const ScanLds &L, EntryMeta m) {
#pragma clang fp contract(off)
    const int cap = L.cap;
    int e = 0, pos = -1, row = -1;  // position in expert order; xp row (tile image row when tiled)
    float g = 0.0f;
    if (lane < a.kt) {
        e = m.e;
        g = m.g;
        if (e > 0 && e <= a.E) {
            const int rk = L.base[e - 1] + m.rk;
            if (rk < cap) {
                pos = L.off[e - 1] + rk;
                row = a.tiled ? L.tstart[e - 1] * a.bm + rk : pos;
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
    return row;
}

// The token's row into every xp row it owns, converting to the GEMM type.
// bf16 rows: `first` holds the row's first batch (loaded by the caller);
// each further batch is loaded before the previous one is stored.
template <int UB>
__device__ __forceinline__ void permute_copy(const PermuteArgs &a, int t, int lane, int row,
                                             const u32x4_t (&first)[UB]) {
    if (permute_bf16_rows(a)) {
        u32x4_t cur[UB];
#pragma unroll
        for (int u = 0; u < UB; ++u) cur[u] = first[u];
        for (int d0 = 0;; d0 += 512 * UB) {
            const bool more = d0 + 512 * UB < a.D;
            u32x4_t nx[UB];
            if (more) load_row_chunk<UB>(a, t, d0 + 512 * UB, lane, nx);
            store_row_chunk<UB>(a, row, d0, lane, cur);
            if (!more) break;
#pragma unroll
            for (int u = 0; u < UB; ++u) cur[u] = nx[u];
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

// Workgroup w takes the tpw tokens [w tpw, w tpw + tpw) of one route block,
// a wave per token in turn, after that route block's scan (workgroup 0 is
// also the scan's writer: a workgroup of its own would not fit beside the
// others and would run after them).  Each wave loads its first token's
// entries and first row batch before the scan (they do not depend on it), so
// their latency overlaps the scan's.  Batches are at most 4 chunks per lane
// (2048 columns): a row of 8 chunks held through the scan exceeds the 128
// registers of a 1024-thread workgroup.  Then the loads that the next stores
// need are in flight before the current stores: rows of one batch (PIPE) the
// next token's entries and first batch; longer rows (one token per wave at
// the usual sizes) the row's next batch (permute_copy).
template <int UB, bool PIPE>
__global__ __launch_bounds__(kPermThreads) void permute_kernel(PermuteArgs a) {
    static_assert(UB <= 4, "row batch held through the scan");
    __shared__ ScanLds L;
    const int lane = threadIdx.x & 63;
    const int t1 = min(a.T, (int)(blockIdx.x + 1) * a.tpw);
    int t = blockIdx.x * a.tpw + (threadIdx.x >> 6);
    const bool rows16 = permute_bf16_rows(a);
    EntryMeta m = load_meta(a, t < t1 ? t : -1, lane);
    u32x4_t cur[UB];
    if (rows16 && t < t1) load_row_chunk<UB>(a, t, 0, lane, cur);
    scan_block(a.s, (int)(((long long)blockIdx.x * a.tpw) / a.rb), L, blockIdx.x == 0);
    for (; t < t1; t += kPermThreads / 64) {
        const int tn = t + kPermThreads / 64;
        const EntryMeta mn = load_meta(a, tn < t1 ? tn : -1, lane);
        u32x4_t nxt[PIPE ? UB : 1];
        if (PIPE && rows16 && tn < t1) load_row_chunk<PIPE ? UB : 1>(a, tn, 0, lane, nxt);
        const int row = permute_entries(a, t, lane, L, m);
        if (a.copy_rows) permute_copy<UB>(a, t, lane, row, cur);
        m = mn;
        if constexpr (PIPE) {
#pragma unroll
            for (int u = 0; u < UB; ++u) cur[u] = nxt[u];
        } else if (rows16 && tn < t1) {
            load_row_chunk<UB>(a, tn, 0, lane, cur);
        }
    }
}

// Permute for more slots per token than a wave has lanes (ExpertChoiceGating
// with min(capacity, E) > 64; kt <= MOE_MAX_EXPERTS): lane l owns entries l,
// l + 64, ... (kWideEnt of them); same finalisation as permute_kernel, then
// one row copy per kept entry, element by element (most of these slots are
// empty).
constexpr int kWideEnt = MOE_MAX_EXPERTS / 64;

__device__ __forceinline__ void permute_wide_token(const PermuteArgs &a, int t, int lane, const ScanLds &L) {
#pragma clang fp contract(off)
    const int cap = L.cap;
    int ee[kWideEnt], pos[kWideEnt], row[kWideEnt];
    float g[kWideEnt];
#pragma unroll
    for (int c = 0; c < kWideEnt; ++c) {
        const int j = lane + 64 * c;
        ee[c] = 0; pos[c] = -1; row[c] = -1; g[c] = 0.0f;
        if (j < a.kt) {
            const long long ent = (long long)t * a.kt + j;
            ee[c] = a.idx[ent];
            g[c] = a.gates[ent];
            if (ee[c] > 0 && ee[c] <= a.E) {
                const int rk = L.base[ee[c] - 1] + a.rank[ent];
                if (rk < cap) {
                    pos[c] = L.off[ee[c] - 1] + rk;
                    row[c] = a.tiled ? L.tstart[ee[c] - 1] * a.bm + rk : pos[c];
                } else {
                    ee[c] = 0;
                    g[c] = 0.0f;
                }
            }
        }
    }
    // (slot 64 c + l is lane l's entry c: the loops over slots run c-major
    // with c a compile-time index, so no register array is indexed at run time)
    if (a.renorm) {
        // gate_sum over the slots in slot order; divide when > 0
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < kWideEnt; ++c)
            for (int l = 0; l < 64 && 64 * c + l < a.kt; ++l) {
                const float v = __shfl(g[c], l);
                sum = (c == 0 && l == 0) ? v : sum + v;
            }
        if (sum > 0.0f) {
#pragma unroll
            for (int c = 0; c < kWideEnt; ++c) g[c] = g[c] / sum;
        }
    }
#pragma unroll
    for (int c = 0; c < kWideEnt; ++c) {
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
#pragma unroll
    for (int c = 0; c < kWideEnt; ++c)
        for (int l = 0; l < 64 && 64 * c + l < a.kt; ++l) {
            const int p = __shfl(row[c], l);
            if (p < 0) continue;
            for (int d = lane; d < a.D; d += 64) {
                const float v = a.x_bf16 ? bf16_to_f32(((const uint16_t *)a.x)[(long long)t * a.D + d])
                                         : ((const float *)a.x)[(long long)t * a.D + d];
                if (a.ct == CT_BF16) ((uint16_t *)a.xp)[xp_index(a, p, d)] = f32_to_bf16(v);
                else ((float *)a.xp)[(long long)p * a.ld_xp + d] = v;
            }
        }
}

__global__ __launch_bounds__(kPermThreads) void permute_wide_kernel(PermuteArgs a) {
    __shared__ ScanLds L;
    scan_block(a.s, (int)(((long long)blockIdx.x * a.tpw) / a.rb), L, blockIdx.x == 0);
    const int t1 = min(a.T, (int)(blockIdx.x + 1) * a.tpw);
    for (int t = blockIdx.x * a.tpw + (threadIdx.x >> 6); t < t1; t += kPermThreads / 64)
        permute_wide_token(a, t, threadIdx.x & 63, L);
}

hipError_t launch_permute(PermuteArgs a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    const int nblk = (a.T + a.rb - 1) / a.rb;
    if (a.kt > kWideEnt * 64 || a.rb < kPermTokens || a.rb % kPermTokens || a.s.nblk != nblk || a.s.E > MOE_MAX_EXPERTS ||
        a.s.ldc < a.s.E || a.s.ldc % 4)
        return hipErrorInvalidValue;
    // tokens per workgroup: kPermTokens (one per wave) while that leaves at
    // most 512 workgroups, else 2 or 4 per wave (dividing the route block):
    // each workgroup runs its route block's scan first
    a.tpw = kPermTokens;
    while (a.tpw * 2 <= a.rb && a.tpw < 4 * kPermTokens && (a.T + a.tpw - 1) / a.tpw > 512) a.tpw *= 2;
    const int nwg = (a.T + a.tpw - 1) / a.tpw;
    if (a.kt > 64) hipLaunchKernelGGL(permute_wide_kernel, dim3(nwg), dim3(kPermThreads), 0, s, a);
    else if (a.D > 2048) hipLaunchKernelGGL((permute_kernel<4, false>), dim3(nwg), dim3(kPermThreads), 0, s, a);
    else if (a.D > 1024) hipLaunchKernelGGL((permute_kernel<4, true>), dim3(nwg), dim3(kPermThreads), 0, s, a);
    else if (a.D > 512) hipLaunchKernelGGL((permute_kernel<2, true>), dim3(nwg), dim3(kPermThreads), 0, s, a);
    else hipLaunchKernelGGL((permute_kernel<1, true>), dim3(nwg), dim3(kPermThreads), 0, s, a);
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
// Fast path (every entry kept, rows 16-byte aligned): the entries are sorted
// by expert in registers, then the token's columns are walked in chunks of
// 256 u columns (lane l: columns 4 l .. 4 l + 3 of each group of 256), the
// loads of chunk c + 1 issued before chunk c is summed and stored.  Every
// wave then reads and writes at the same time: a wave that first loaded its
// whole row and only then stored it would leave the HBM with a phase of
// reads only, then a phase of writes only.  u = 8 / kt groups per chunk (at
// least 1; lowered to the smallest power of two covering D), so a chunk is
// kt u loads of 8 bytes (bf16 y) per lane.
// ============================================================================
__host__ __device__ constexpr int combine_umax(int kt) { return kt >= 8 ? 1 : 8 / kt; }

template <bool YB>
struct YRaw {
    uint2 v;  // 4 bf16
    __device__ __forceinline__ void load(const void *y, long long off) { v = *(const uint2 *)((const uint16_t *)y + off); }
    __device__ __forceinline__ float4 f() const {
        return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                           __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
    }
};
template <>
struct YRaw<false> {
    float4 v;
    __device__ __forceinline__ void load(const void *y, long long off) { v = *(const float4 *)((const float *)y + off); }
    __device__ __forceinline__ float4 f() const { return v; }
};

// pp / gg: positions and gates of the token's KT entries in expert order
template <int KT, bool BLEND, bool YB>
__device__ __forceinline__ void combine_fast(const CombineArgs &a, long long t, int lane, const int (&pp)[KT],
                                             const float (&gg)[KT]) {
#pragma clang fp contract(off)
    constexpr int UM = combine_umax(KT);
    const int cw = 256 * a.u;
    YRaw<YB> cur[KT][UM], nxt[KT][UM];
    auto load = [&](YRaw<YB>(&r)[KT][UM], int d0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < KT; ++i)
#pragma unroll
            for (int u = 0; u < UM; ++u)
                if (u < a.u) r[i][u].load(a.y, (long long)pp[i] * a.ld_y + min(d0 + u * 256 + lane * 4, a.D - 4));
    };
    float *__restrict__ o = a.out + t * a.D;
    load(cur, 0);
    for (int d0 = 0; d0 < a.D; d0 += cw) {
        if (d0 + cw < a.D) load(nxt, d0 + cw);
#pragma unroll
        for (int u = 0; u < UM; ++u) {
            if (u >= a.u) break;
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float4 sh = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int i = 0; i < KT; ++i) {
                const float4 v = cur[i][u].f();
                if (BLEND && i < a.lsh) {
                    const float n = (float)a.lsh;
                    sh.x = sh.x + v.x / n;
                    sh.y = sh.y + v.y / n;
                    sh.z = sh.z + v.z / n;
                    sh.w = sh.w + v.w / n;
                } else {
                    const float g = gg[i];
                    acc.x = acc.x + g * v.x;
                    acc.y = acc.y + g * v.y;
                    acc.z = acc.z + g * v.z;
                    acc.w = acc.w + g * v.w;
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
#pragma unroll
        for (int i = 0; i < KT; ++i)
#pragma unroll
            for (int u = 0; u < UM; ++u) cur[i][u] = nxt[i][u];
    }
}

// The token's entries (all KT slots), then the fast path when every one is
// kept and the rows are 16-byte aligned.  Returns false otherwise.
template <int KT, bool BLEND>
__device__ __forceinline__ bool try_combine_fast(const CombineArgs &a, long long t, int lane) {
    if (a.kt != KT) return false;
    int ee[KT], pp[KT];
    float gg[KT];
    bool all_kept = (a.D & 3) == 0 && (a.ld_y & 3) == 0;
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        const long long ent = t * KT + j;
        ee[j] = a.idx[ent];
        pp[j] = a.pos_of[ent];
        gg[j] = a.gates[ent];
        all_kept = all_kept && pp[j] >= 0;
    }
    if (!all_kept) return false;
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
    if (a.y_bf16) combine_fast<KT, BLEND, true>(a, t, lane, pp, gg);
    else combine_fast<KT, BLEND, false>(a, t, lane, pp, gg);
    return true;
}

__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const long long t = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    if (a.kt > MOE_MAX_TOPK) {
        // more slots than a token's sort network holds: ExpertChoiceGating,
        // whose slots list the token's experts in ascending id order (empty
        // and dropped slots have no position), so slot order is expert order;
        // the layer's shared experts, if any, are slots 0..lsh-1 (ids 1..lsh)
        float *o = a.out + t * a.D;
        for (int d = lane; d < a.D; d += 64) {
            float acc = 0.0f, sh = 0.0f;
            for (int j = 0; j < a.kt; ++j) {
                const long long ent = t * a.kt + j;
                const int p = a.pos_of[ent];
                if (p < 0) continue;
                const long long off = (long long)p * a.ld_y + d;
                const float v = a.y_bf16 ? bf16_to_f32(((const uint16_t *)a.y)[off]) : ((const float *)a.y)[off];
                if (j < a.lsh) sh = sh + v / (float)a.lsh;
                else acc = acc + a.gates[ent] * v;
            }
            if (a.lsh > 0) acc = 0.5f * sh + 0.5f * acc;
            o[d] = acc;
        }
        return;
    }
    if (a.lsh > 0) {
        if (try_combine_fast<2, true>(a, t, lane) || try_combine_fast<3, true>(a, t, lane) ||
            try_combine_fast<4, true>(a, t, lane))
            return;
    } else if (try_combine_fast<2, false>(a, t, lane) || try_combine_fast<1, false>(a, t, lane) ||
               try_combine_fast<8, false>(a, t, lane) || try_combine_fast<4, false>(a, t, lane) ||
               try_combine_fast<6, false>(a, t, lane)) {
        return;
    }
    int ee[MOE_MAX_TOPK], pp[MOE_MAX_TOPK];
    float gg[MOE_MAX_TOPK];
    int n = 0;
    for (int j = 0; j < a.kt; ++j) {
        const long long ent = t * a.kt + j;
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
    float *o = a.out + t * a.D;
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

hipError_t launch_combine(const CombineArgs &a0, hipStream_t s) {
    if (a0.T <= 0) return hipSuccess;
    CombineArgs a = a0;
    // 256-column groups per chunk of the fast path: combine_umax(kt), lowered
    // to the smallest power of two that covers D
    const int groups = (a.D + 255) / 256;
    a.u = combine_umax(std::min(a.kt, MOE_MAX_TOPK));
    while (a.u > 1 && a.u / 2 >= groups) a.u /= 2;
    a.nchunk = (a.D + 256 * a.u - 1) / (256 * a.u);
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((a.T + 3) / 4)), dim3(256), 0, s, a);
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
    if (tid == 0) aux_free_step(cnt, 0, 0, (long long)tot, E, lr, momentum, bias, mom);
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
