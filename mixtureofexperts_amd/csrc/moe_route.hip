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

// The router logits of TM tokens (32 or 64) over all of K, into LDS rows
// lrow[t][RW].  K runs in chunks of 256 (8 MFMA steps of 32): the block
// stages each chunk of x in LDS with coalesced loads (each 16-lane pass
// reads 256 contiguous bytes; rows padded by 16 B so the fragment reads hit
// distinct banks), double-buffered so the next chunk's loads are in flight
// during this chunk's MFMAs.  The split router weight is read from its
// fragment image (router_split_kernel): one contiguous 1 KB per fragment.
// Waves split the expert tiles NG ways and the K steps of each chunk
// 4 / NG ways; per step, row tile and expert tile: acc += x . W0 + x . W1 +
// x . W2 as v_mfma_f32_16x16x32_bf16 (fp32 x: each of its three parts times
// the weight parts).  The waves' accumulators then go to an LDS buffer and
// each logit is their sum in K-group order (paired tiles: the three parts'
// columns added in part order), plus the router bias.
// A: 16 tokens x 32 k (lane l: token l % 16, k 8 (l / 16) .. +8); B: the
// image tile; D lane l: column l % 16, tokens 4 (l / 16) .. +4.
constexpr int kRouterKC = 256;  // K per staged chunk

template <int XBF16, int TM>
__host__ __device__ constexpr int router_stage_row_bytes() { return kRouterKC * (XBF16 ? 2 : 4) + 16; }

template <int XBF16, int TM, int PAIRED, int NG, int TPW, typename Out>
__device__ __forceinline__ void fused_logits(const RouterArgs &r, int t0, int ntok, int s_begin, int s_end,
                                             uint8_t *stage, Out &&out) {
#pragma clang fp contract(off)
    constexpr int RT = TM / 16;                 // 16-token row tiles
    constexpr int ESZ = XBF16 ? 2 : 4;
    constexpr int ROWB = router_stage_row_bytes<XBF16, TM>();
    constexpr int UPR = kRouterKC * ESZ / 16;   // 16-byte units per staged row
    constexpr int NU = TM * UPR / kRouteThreads;  // units per thread per chunk
    constexpr int KG = 4 / NG;                  // K groups
    constexpr int SPW = 8 / KG;                 // steps per wave per chunk
    constexpr int NPT = PAIRED ? 2 : 3;         // image tiles per expert tile
    constexpr int NP = XBF16 ? 1 : 3;           // activation parts
    constexpr int NACC = PAIRED ? 2 : TPW;      // accumulator tiles per row tile
    static_assert(NU * kRouteThreads == TM * UPR, "staging units");
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15;
    const int ET = PAIRED ? 1 : (r.Er + 15) / 16;
    const int NTS = PAIRED ? 2 : 3 * ET;
    const int gn = w % NG, gk = w / NG;         // this wave's expert-tile group and K group
    // K steps [s_begin, s_end) (a multiple of 8 apart unless s_end = Dp / 32)
    const int S = s_end;
    const int NCH = (s_end - s_begin + 7) / 8;
    uint8_t *buf[2] = {stage, stage + TM * ROWB};

    // staging: unit u = tid + 256 j is row u / UPR, 16 bytes at column unit u % UPR
    auto load_chunk = [&](int ch, u32x4_t (&v)[NU]) {
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const int u = tid + j * kRouteThreads;
            const int row = u / UPR, cu = u - row * UPR;
            const int k0 = s_begin * 32 + ch * kRouterKC + cu * (16 / ESZ);
            const long long t = min(t0 + row, r.T - 1);
            if (k0 + 16 / ESZ <= r.D && (r.D % (16 / ESZ)) == 0) {
                v[j] = *(const u32x4_t *)((const uint8_t *)r.x + (t * r.D + k0) * ESZ);
            } else {
                uint32_t q[4] = {0u, 0u, 0u, 0u};
                if (XBF16) {
                    uint16_t h[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) h[i] = (k0 + i < r.D) ? ((const uint16_t *)r.x)[t * r.D + k0 + i] : 0;
                    __builtin_memcpy(q, h, 16);
                } else {
                    float f[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) f[i] = (k0 + i < r.D) ? ((const float *)r.x)[t * r.D + k0 + i] : 0.0f;
                    __builtin_memcpy(q, f, 16);
                }
                v[j] = u32x4_t{q[0], q[1], q[2], q[3]};
            }
        }
    };
    auto store_chunk = [&](uint8_t *b, const u32x4_t (&v)[NU]) {
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const int u = tid + j * kRouteThreads;
            const int row = u / UPR, cu = u - row * UPR;
            *(u32x4_t *)(b + row * ROWB + cu * 16) = v[j];
        }
    };
    // the x fragment (parts) of step u of a staged chunk, row tile ti
    auto x_frag = [&](const uint8_t *b, int u, int ti, rbf16x8_t *xa) {
        const uint8_t *row = b + (ti * 16 + l16) * ROWB;
        if (XBF16) {
            xa[0] = *(const rbf16x8_t *)(row + u * 64 + (lane >> 4) * 16);
        } else {
            const float4 f0 = *(const float4 *)(row + (u * 32 + (lane >> 4) * 8) * 4);
            const float4 f1 = *(const float4 *)(row + (u * 32 + (lane >> 4) * 8 + 4) * 4);
            const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
            uint16_t h0[8], h1[8], h2[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                h0[i] = f32_to_bf16(v[i]);
                const float r1 = v[i] - bf16_to_f32(h0[i]);
                h1[i] = f32_to_bf16(r1);
                h2[i] = f32_to_bf16(r1 - bf16_to_f32(h1[i]));
            }
            __builtin_memcpy(&xa[0], h0, 16);
            __builtin_memcpy(&xa[1], h1, 16);
            __builtin_memcpy(&xa[2], h2, 16);
        }
    };

    rf32x4_t acc[RT][NACC];
#pragma unroll
    for (int ti = 0; ti < RT; ++ti)
#pragma unroll
        for (int j = 0; j < NACC; ++j) acc[ti][j] = rf32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // weight fragments of a chunk for this wave (independent of LDS); with
    // few of them (small E) the next chunk's are loaded a chunk ahead
    constexpr bool WPF = SPW * TPW * NPT <= 16;
    using WFrag = rbf16x8_t[SPW][TPW][NPT];
    auto load_w = [&](int ch, WFrag &wb) {
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int st = min(s_begin + ch * 8 + gk * SPW + i, S - 1);
#pragma unroll
            for (int j = 0; j < TPW; ++j) {
                const int et = min(gn + j * NG, ET - 1);
#pragma unroll
                for (int p = 0; p < NPT; ++p) {
                    const int q = PAIRED ? p : et * 3 + p;
                    wb[i][j][p] = *(const rbf16x8_t *)(r.ws + (((long long)st * NTS + q) * 64 + lane) * 8);
                }
            }
        }
    };
    // x of chunk 0 staged; chunks 1 and 2 in flight in registers (each chunk
    // is stored one iteration after its loads were issued)
    u32x4_t va[NU], vb[NU];
    load_chunk(0, va);
    store_chunk(buf[0], va);
    if (NCH > 1) load_chunk(1, va);
    WFrag wn;
    if constexpr (WPF) load_w(0, wn);
    __syncthreads();
    for (int ch = 0; ch < NCH; ++ch) {
        WFrag wb;
        if constexpr (WPF) {
#pragma unroll
            for (int i = 0; i < SPW; ++i)
#pragma unroll
                for (int j = 0; j < TPW; ++j)
#pragma unroll
                    for (int p = 0; p < NPT; ++p) wb[i][j][p] = wn[i][j][p];
            if (ch + 1 < NCH) load_w(ch + 1, wn);
        } else {
            load_w(ch, wb);
        }
        if (ch + 2 < NCH) load_chunk(ch + 2, vb);
        const uint8_t *b = buf[ch & 1];
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int u = gk * SPW + i;
            if (s_begin + ch * 8 + u >= S) break;
#pragma unroll
            for (int ti = 0; ti < RT; ++ti) {
                rbf16x8_t xa[NP];
                x_frag(b, u, ti, xa);
                if constexpr (PAIRED) {
                    // tile 0 (parts 0, 1): every x part; tile 1 (part 2): x part 0
#pragma unroll
                    for (int xi = 0; xi < NP; ++xi)
                        acc[ti][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[xi], wb[i][0][0], acc[ti][0], 0, 0, 0);
                    acc[ti][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[0], wb[i][0][1], acc[ti][1], 0, 0, 0);
                } else {
#pragma unroll
                    for (int j = 0; j < TPW; ++j) {
                        if (gn + j * NG >= ET) break;
#pragma unroll
                        for (int p = 0; p < 3; ++p)
#pragma unroll
                            for (int xi = 0; xi + p < 3 && xi < NP; ++xi)
                                acc[ti][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[xi], wb[i][j][p], acc[ti][j],
                                                                                     0, 0, 0);
                    }
                }
            }
        }
        if (ch + 1 < NCH) store_chunk(buf[(ch + 1) & 1], va);
#pragma unroll
        for (int j = 0; j < NU; ++j) va[j] = vb[j];
        __syncthreads();
    }

    // accumulators -> LDS partials P[gk][t][col] (the staging buffers are
    // free now), col = image column of the expert tile (paired: 16 q + c)
    const int NCOL = PAIRED ? 32 : ET * 16;
    float *P = (float *)stage;
#pragma unroll
    for (int ti = 0; ti < RT; ++ti)
#pragma unroll
        for (int j = 0; j < NACC; ++j) {
            const int col = PAIRED ? j * 16 + l16 : (gn + j * NG) * 16 + l16;
            if (PAIRED || gn + j * NG < ET)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int t = ti * 16 + (lane >> 4) * 4 + rr;
                    P[((long long)gk * TM + t) * NCOL + col] = acc[ti][j][rr];
                }
        }
    __syncthreads();
    // logit (of this K range) = the K groups' partials in order (paired: per
    // part column, the parts then added in part order), to out(t, e, value)
    for (int q = tid; q < ntok * r.Er; q += kRouteThreads) {
        const int t = q / r.Er, e = q - t * r.Er;
        auto col_sum = [&](int col) {
            float v = P[(long long)t * NCOL + col];
#pragma unroll
            for (int g = 1; g < KG; ++g) v = v + P[((long long)g * TM + t) * NCOL + col];
            return v;
        };
        out(t, e, PAIRED ? (col_sum(e) + col_sum(8 + e)) + col_sum(16 + e) : col_sum(e));
    }
}

// ============================================================================
// Gating.  kRouteBlock tokens per routing block of kRouteThreads threads, 8
// lanes per token, each holding a contiguous block of the token's experts in
// registers (gate_block).
// ============================================================================

// LDS row stride of the routing kernel for E rows: a multiple of 4 floats
// (16 B) whose count of 16-byte units is odd, so that 16 token threads
// reading 16 B at one column hit 16 distinct bank quads.
__host__ __device__ inline int route_rw(int E) { return 4 * ((((E + 3) / 4 + 1) | 1)); }

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

// Top-K of a token's routed probabilities held in registers: lane rs of the
// token's 8 keeps elements base + j (j < EPL) of the row; each lane keeps the
// best K of its elements in sorted register slots (larger isless key, then
// the lower index), then three butterfly steps merge the lanes' lists (a
// strict total order, so every lane ends with the same list).  Every lane of
// the wave must call it (inactive rows pass active = false).  Slots past the
// row's routed size stay empty (key 0, below every float's key).
template <int K, int EPL>
__device__ __forceinline__ void topk_reg(const float (&p)[EPL], int base, int lo, int n, bool active, int *sel,
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
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int i = base + j;
            if (i >= lo && i < n) insert(isless_key(p[j]), i, p[j]);
        }
    }
#pragma unroll 1
    for (int o = 1; o < 8; o <<= 1) {
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

template <int EPL>
__device__ __forceinline__ void topk_reg_k(const float (&p)[EPL], int base, int lo, int n, int k, bool active,
                                           int *sel, float *val) {
    // K >= k slots: the first k of the best K are the top-k
    if (k == 1) topk_reg<1, EPL>(p, base, lo, n, active, sel, val);
    else if (k == 2) topk_reg<2, EPL>(p, base, lo, n, active, sel, val);
    else if (k <= 4) topk_reg<4, EPL>(p, base, lo, n, active, sel, val);
    else topk_reg<8, EPL>(p, base, lo, n, active, sel, val);
}

// Butterfly sum / max over the 8 lanes of a token (the same tree every call).
template <typename F>
__device__ __forceinline__ F lanes8_sum(F v) {
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) v = v + __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float lanes8_max(float v) {  // NaN ignored (v > m is false for NaN)
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        const float w = __shfl_xor(v, o);
        if (w > v) v = w;
    }
    return v;
}

// One routing block, number blk: kRouteBlock tokens, 8 lanes per token (lane
// rs of token rt = tid / 8 holds the contiguous experts rs EPL .. +EPL of the
// row in registers).  Logits: the token's row of lin (LDS rows, stride RW)
// when FROM_LDS, else the sum of a.part's nks K slices in slice order plus
// the bias, read straight from global memory (each token's 8 lanes read its
// row contiguously).  Per token, in registers: max; exp terms e =
// (float)exp((double)(l - m)) (NNlib's branch for m == +Inf); their fp32 sum
// in expert order (the recipe's order: lane r adds its experts after lane
// r - 1's running sum); probabilities e / s; the fp64 entropy terms and the
// logsumexp; the top-k by per-lane sorted lists and a butterfly merge; the
// gates.  Then per entry (lane rs = slot rs): its stable rank among the
// block's entries of its expert (LDS bitmask per expert, bit = entry), and
// the block's histogram, probability sums and loss terms.  sl: LDS rows
// [kRouteBlock][RW] for the output probabilities (the block sums).
template <int EPL, bool FROM_LDS>
__device__ __forceinline__ void gate_block(const RouteArgs &a, int blk, const float *lin, int RW, float *sl) {
#pragma clang fp contract(off)
    // stable ranks: bit i of emask[e][i / 32] marks entry i (token * kt + slot)
    // of expert e + 1 in this block
    __shared__ unsigned emask[MOE_MAX_EXPERTS * MOE_MAX_TOPK];
    __shared__ double wred[2][kRouteThreads / 64];
    const bool shared_gate = a.gate_kind == MOE_GATE_SHARED;
    const bool soft = a.gate_kind == MOE_GATE_SOFT;
    const bool zsep = shared_gate || soft;  // z-loss from a softmax of its own (all rows, unscaled)
    const bool out_probs = (a.out_mask & ROUTE_OUT_PROBS) != 0;
    const bool out_gating = (a.out_mask & ROUTE_OUT_GATING) != 0;
    // a gating pass on the caller's routing needs none of the softmax phases
    const bool softmax = out_probs || !a.given;
    const int E = a.E;                       // router rows (= a.Er)
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int rt = tid >> 3, rs = tid & 7;   // token rt of the block, lane rs of it
    const int t0 = blk * kRouteBlock;
    const int ntok = min(kRouteBlock, a.T - t0);
    const bool rvalid = rt < ntok;
    const long long t = (long long)t0 + rt;
    const int ns = shared_gate ? a.ns : 0;   // rows before the routed ones
    const int base = rs * EPL;

    __syncthreads();  // the previous routing block of this workgroup is done with the LDS
    for (int i = tid; i < MOE_MAX_EXPERTS * MOE_MAX_TOPK; i += kRouteThreads) emask[i] = 0u;

    float v[EPL], pr[EPL];  // logits; exp terms, then probabilities (before the shared-gating scale)
#pragma unroll
    for (int j = 0; j < EPL; ++j) { v[j] = 0.0f; pr[j] = 0.0f; }
    float m = -INFINITY, s = 0.0f, lse = 0.0f;
    double hs = 0.0;
    if (softmax) {
        // ---- logits ----
        if (rvalid) {
            if constexpr (FROM_LDS) {
#pragma unroll
                for (int j = 0; j < EPL; ++j)
                    if (base + j < E) v[j] = lin[rt * RW + base + j];
            } else {
                const long long sstride = (long long)a.T * a.Er;
                const float *row = a.part + t * a.Er + base;
                float pv[EPL];
#pragma unroll
                for (int j = 0; j < EPL; ++j) pv[j] = (base + j < E) ? row[j] : 0.0f;
                for (int sl_ = 1; sl_ < a.nks; ++sl_) {
                    float q[EPL];
#pragma unroll
                    for (int j = 0; j < EPL; ++j) q[j] = (base + j < E) ? row[sl_ * sstride + j] : 0.0f;
#pragma unroll
                    for (int j = 0; j < EPL; ++j) pv[j] = pv[j] + q[j];
                }
#pragma unroll
                for (int j = 0; j < EPL; ++j) {
                    float w = pv[j];
                    if (a.bias && base + j < E) w = w + a.bias[base + j];
                    v[j] = w;
                }
            }
        }
        // ---- max (of the routed rows; zsep: also of all rows) ----
        float mz = -INFINITY;
        float sv[EPL];  // logits ./ lambda for SoftMoEGating (advanced.jl:18)
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int i = base + j;
            sv[j] = soft ? v[j] / a.soft_lambda : v[j];
            if (rvalid && i >= ns && i < E && sv[j] > m) m = sv[j];
            if (rvalid && i < E && v[j] > mz) mz = v[j];
        }
        m = lanes8_max(m);
        mz = lanes8_max(mz);
        // ---- exp terms; zsep: the z-loss exponent sum over all rows ----
        float zs = 0.0f;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int i = base + j;
            if (rvalid && i >= ns && i < E)
                pr[j] = (m == INFINITY) ? ((sv[j] == INFINITY) ? 1.0f : 0.0f) : (float)exp((double)(sv[j] - m));
            if (zsep && rvalid && i < E) zs = zs + (float)exp((double)(v[j] - mz));
        }
        if (zsep) zs = lanes8_sum(zs);
        // ---- sum in expert order ----
        if constexpr (EPL == 1) {
            float ev[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) ev[r] = __shfl(pr[0], (lane & ~7) | r);
#pragma unroll
            for (int r = 0; r < 8; ++r)
                if (r >= ns && r < E) s = s + ev[r];
        } else {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                float c = s;
                if (rs == r) {
#pragma unroll
                    for (int j = 0; j < EPL; ++j) {
                        const int i = r * EPL + j;
                        if (i >= ns && i < E) c = c + pr[j];
                    }
                }
                s = __shfl(c, (lane & ~7) | r);
            }
        }
        // ---- probabilities (outputs: shared gating's shared rows 1/E, routed
        // rows p scaled by 1 - ns/E in Float64; the caller's gate: its
        // probabilities or ones ./ E); entropy terms p log(p + 1e-8) with
        // p + 1e-8 in Float64 as Julia promotes it, the log in fp32 (a
        // statistic: the mean entropy is checked to 1e-5) ----
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int i = base + j;
            if (!rvalid || i >= E) continue;
            float pv;
            if (a.given) {
                pv = a.given_probs ? a.probs[t * E + i] : 1.0f / (float)E;
            } else if (i < ns) {
                pv = 1.0f / (float)E;
            } else {
                pr[j] = pr[j] / s;
                pv = shared_gate ? (float)((double)pr[j] * (1.0 - (double)ns / (double)E)) : pr[j];
            }
            sl[rt * RW + i] = pv;
            const double pd = (double)pv;
            hs = hs + pd * (double)logf((float)(pd + 1e-8));
        }
        hs = lanes8_sum(hs);
        // logsumexp (src/balancing/losses.jl:111-114) from the same exp recipe,
        // the log in Float32 as Julia takes it of the Float32 sum
        lse = zsep ? mz + logf(zs) : m + logf(s);
        if (out_probs && rvalid) {
#pragma unroll
            for (int j = 0; j < EPL; ++j)
                if (base + j < E) {
                    a.logits[t * E + base + j] = v[j];
                    a.probs[t * E + base + j] = sl[rt * RW + base + j];
                }
        }
    }

    // ---- top-k and gates; the entries' experts (slot rs of the token) ----
    int my_e = 0;     // 1-based expert of entry (rt, rs), 0: none
    float my_g = 0.0f;
    if (!a.given) {
        int sel[MOE_MAX_TOPK];
        float val[MOE_MAX_TOPK];
#pragma unroll
        for (int q = 0; q < MOE_MAX_TOPK; ++q) { sel[q] = 0; val[q] = 0.0f; }
        topk_reg_k<EPL>(pr, base, ns, E, a.k, rvalid, sel, val);
        // gates: p of the slots over their sum in slot order
        float sg = val[0];
#pragma unroll
        for (int q = 1; q < MOE_MAX_TOPK; ++q)
            if (q < a.k) sg = sg + val[q];
        // the slot this lane reports: rs (slots 0 .. kt-1)
        const int j = rs;
        if (soft) {
            // SoftMoEGating: top-k of the scaled-softmax probabilities; the
            // dispatch reads row `slot` of the (E, T) gate matrix, i.e. the
            // probability of expert `slot` (advanced.jl:24-33, moe_layer.jl:200)
            float pj = 0.0f;
            const int src = (lane & ~7) | (j / EPL);  // the lane holding expert j (j < 8)
#pragma unroll
            for (int u = 0; u < EPL; ++u) {
                const float w = __shfl(pr[u], src);
                if (u == j % EPL) pj = w;
            }
            if (j < a.k) {
#pragma unroll
                for (int q = 0; q < MOE_MAX_TOPK; ++q)
                    if (q == j) my_e = sel[q] + 1;
                my_g = pj;
            }
        } else if (shared_gate) {
            // shared slots 0 .. ns-1 (gate 1/kt), then the routed top-k with
            // gates scaled by 1 - ns/kt in Float64 (advanced.jl:80-108)
            if (j < ns) {
                my_e = j + 1;
                my_g = 1.0f / (float)a.kt;
            } else if (j < ns + a.k) {
                const double gscale = 1.0 - (double)ns / (double)a.kt;
#pragma unroll
                for (int q = 0; q < MOE_MAX_TOPK; ++q)
                    if (q == j - ns) {
                        my_e = sel[q] + 1;
                        my_g = (float)((double)(val[q] / sg) * gscale);
                    }
            }
        } else if (a.lsh > 0) {
            // forward_with_shared_experts: shared experts 1..lsh in slots
            // 0..lsh-1 (their outputs are averaged, the gate is only
            // reported), then the routed ids shifted by lsh (expert_indices
            // .+= num_shared_experts, src/core/moe_layer.jl:172)
            if (j < a.lsh) {
                my_e = j + 1;
                my_g = 1.0f / (float)a.lsh;
            } else if (j < a.lsh + a.k) {
#pragma unroll
                for (int q = 0; q < MOE_MAX_TOPK; ++q)
                    if (q == j - a.lsh) {
                        my_e = sel[q] + 1 + a.lsh;
                        my_g = val[q] / sg;
                    }
            }
        } else if (j < a.k) {
#pragma unroll
            for (int q = 0; q < MOE_MAX_TOPK; ++q)
                if (q == j) {
                    my_e = sel[q] + 1;
                    my_g = val[q] / sg;
                }
        }
        if (!rvalid) my_e = 0;
    } else if (rvalid && rs < a.kt) {
        // the caller's routing: ids outside 1..E are skipped, as the
        // dispatch's `expert_id > 0 && expert_id <= length(experts)` does
        // (src/core/moe_layer.jl:198)
        const long long ent = t * a.kt + rs;
        const int e = a.idx[ent];
        my_e = (e >= 1 && e <= a.Eh) ? e : 0;
        my_g = a.gates[ent];
    }

    // ---- stable rank of each entry among the block's entries of its expert ----
    // (entries in token-then-slot order, as the bucket loop visits them)
    const int ent = rt * a.kt + rs;  // entry of this lane (rs < kt)
    const bool has_ent = out_gating && rs < a.kt && my_e > 0;
    __syncthreads();  // emask cleared
    if (has_ent) atomicOr(&emask[(my_e - 1) * MOE_MAX_TOPK + (ent >> 5)], 1u << (ent & 31));
    // block sums of the per-token loss terms (tokens rt: lane rs == 0), in a
    // fixed order: within a wave by a butterfly over its 8 tokens, then the
    // waves in order
    double zterm = 0.0, hterm = 0.0;
    if (softmax && rvalid && rs == 0) {
        zterm = (double)(lse * lse);
        hterm = -hs;
    }
#pragma unroll
    for (int o = 8; o < 64; o <<= 1) {
        zterm = zterm + __shfl_xor(zterm, o);
        hterm = hterm + __shfl_xor(hterm, o);
    }
    if (lane == 0) {
        wred[0][wv] = zterm;
        wred[1][wv] = hterm;
    }
    __syncthreads();  // emask complete, wred and the probability rows written
    if (has_ent && rvalid) {
        const unsigned *mk = &emask[(my_e - 1) * MOE_MAX_TOPK];
        int rr = __popc(mk[ent >> 5] & ((1u << (ent & 31)) - 1u));
        for (int w = 0; w < (ent >> 5); ++w) rr += __popc(mk[w]);
        a.rank[t * a.kt + rs] = rr;
    }
    if (out_gating && rvalid && rs < a.kt) {
        a.idx[t * a.kt + rs] = my_e;
        a.gates[t * a.kt + rs] = my_g;
    }
    for (int e = tid; e < a.Eh; e += kRouteThreads) {
        if (out_gating) {
            int c = 0;
#pragma unroll
            for (int w = 0; w < MOE_MAX_TOPK; ++w) c += __popc(emask[e * MOE_MAX_TOPK + w]);
            a.blk_counts[(long long)blk * a.Eh + e] = c;
        }
        if (out_probs) {
            // per-row probability sums (Switch loss P_e) in fp64, token order
            double ps = 0.0;
            if (e < E) {
#pragma unroll 8
                for (int i = 0; i < ntok; ++i) ps += (double)sl[i * RW + e];
            }
            a.blk_stats[(long long)blk * (a.Eh + 2) + e] = ps;
        }
    }
    if (tid == 0 && out_probs) {
        double zb = 0.0, hb = 0.0;
#pragma unroll
        for (int w = 0; w < kRouteThreads / 64; ++w) {
            zb += wred[0][w];
            hb += wred[1][w];
        }
        a.blk_stats[(long long)blk * (a.Eh + 2) + a.Eh] = zb;
        a.blk_stats[(long long)blk * (a.Eh + 2) + a.Eh + 1] = hb;
    }
}

template <int EPL>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t rdyn[];
    const int RW = route_rw(a.E);
    gate_block<EPL, false>(a, blockIdx.x, nullptr, RW, (float *)rdyn);
}

// The router's MFMA logits GEMM and the gating of route_kernel in one
// launch: a workgroup computes the logits of TM = 32 or 64 tokens over all of
// K into LDS, then gates them as TM / 32 routing blocks (no partial sums
// through HBM).  Dynamic LDS: the logit rows of the TM tokens, then one
// routing block's probability rows, which the x staging of the logits phase
// shares.
template <int XBF16, int TM, int PAIRED, int NG, int TPW, int EPL>
__global__ __launch_bounds__(kRouteThreads) void router_fused_kernel(RouteArgs a, RouterArgs r) {
    extern __shared__ __attribute__((aligned(16))) uint8_t rdyn[];
    const int RW = route_rw(a.E);
    float *lrows = (float *)rdyn;
    float *srow = lrows + TM * RW;
    const int t0 = blockIdx.x * TM;
    const float *bias = a.bias;
    fused_logits<XBF16, TM, PAIRED, NG, TPW>(r, t0, min(TM, a.T - t0), 0, r.Dp / 32, (uint8_t *)srow,
                                            [&](int t, int e, float v) {
                                                if (bias) v = v + bias[e];
                                                lrows[t * RW + e] = v;
                                            });
    constexpr int NSUB = TM / kRouteBlock;
#pragma unroll 1
    for (int sb = 0; sb < NSUB; ++sb) {
        const int blk = blockIdx.x * NSUB + sb;
        if (blk * kRouteBlock >= a.T) break;  // uniform over the workgroup
        gate_block<EPL, true>(a, blk, lrows + sb * kRouteBlock * RW, RW, srow);
    }
}

// The router's logits GEMM on its own: workgroup (token tile, K slice)
// computes the partial logits of TM tokens over K steps [z S8, (z + 1) S8)
// (S8 = r.kslice steps) into part[z][T][Er]; the routing kernel adds the
// slices in slice order and the bias.  K slices spread a small batch over
// every CU, and keep the x tile each workgroup streams small.
template <int XBF16, int TM, int PAIRED, int NG, int TPW>
__global__ __launch_bounds__(kRouteThreads) void router_logits_kernel(RouterArgs r, float *part) {
    extern __shared__ __attribute__((aligned(16))) uint8_t rdyn[];
    const int t0 = blockIdx.x * TM;
    const int z = blockIdx.y;
    const int S = r.Dp / 32;
    const int sb = z * r.kslice, se = min(S, sb + r.kslice);
    float *dst = part + (long long)z * r.T * r.Er + (long long)t0 * r.Er;
    fused_logits<XBF16, TM, PAIRED, NG, TPW>(r, t0, min(TM, r.T - t0), sb, se, rdyn,
                                            [&](int t, int e, float v) { dst[(long long)t * r.Er + e] = v; });
}

static size_t route_lds_bytes(const RouteArgs &a) {
    // the probability rows of one routing block
    return (size_t)kRouteBlock * sizeof(float) * route_rw(a.E);
}

// experts per lane of a token's 8 (the gating body's register blocks)
static int route_epl(int E) { return E <= 8 ? 1 : (E <= 16 ? 2 : (E <= 32 ? 4 : (E <= 64 ? 8 : 16))); }

template <int XBF16, int TM, int PAIRED, int NG, int TPW, int EPL>
static hipError_t launch_fused_case(const RouteArgs &a, const RouterArgs &r, hipStream_t s) {
    const int RW = route_rw(a.E);
    const int ET = PAIRED ? 1 : (r.Er + 15) / 16;
    const size_t stage = std::max<size_t>((size_t)2 * TM * router_stage_row_bytes<XBF16, TM>(),
                                          sizeof(float) * (size_t)(4 / NG) * TM * (PAIRED ? 32 : ET * 16));
    const size_t lds = sizeof(float) * (size_t)TM * RW + std::max<size_t>(sizeof(float) * kRouteBlock * RW, stage);
    if (lds > 150 * 1024) return hipErrorInvalidValue;
    auto kern = router_fused_kernel<XBF16, TM, PAIRED, NG, TPW, EPL>;
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3((a.T + TM - 1) / TM), dim3(kRouteThreads), lds, s, a, r);
    return hipGetLastError();
}

hipError_t launch_router_fused(const RouteArgs &a, const RouterArgs &r, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    if (r.Er < 1 || r.Er > MOE_MAX_EXPERTS || r.Er != a.Er || a.E != a.Er || r.Dp % 32 != 0 || r.Dp < r.D ||
        ((a.out_mask & ROUTE_OUT_GATING) && a.kt > MOE_MAX_TOPK))
        return hipErrorInvalidValue;
    const int ET = (r.Er + 15) / 16;
    // 64-token workgroups for bf16 x when that still gives at least 256 of them
    const bool tm64 = r.x_bf16 && a.T >= 64 * 256;
    // expert tiles -> (paired, waves along N, tiles per wave) and the gating's
    // experts per lane: E <= 8 | <= 16 | <= 32 (ET 2) | <= 48 / 64 (ET 3, 4) | more
#define MOE_FUSED(XB, TM_, P, NG_, TPW_, EPL_) return launch_fused_case<XB, TM_, P, NG_, TPW_, EPL_>(a, r, s)
#define MOE_FUSED_TILES(XB, TM_)                                  \
    if (r.Er <= 8) MOE_FUSED(XB, TM_, 1, 1, 1, 1);                \
    if (ET == 1) MOE_FUSED(XB, TM_, 0, 1, 1, 2);                  \
    if (ET == 2) MOE_FUSED(XB, TM_, 0, 2, 1, 4);                  \
    if (ET == 3) MOE_FUSED(XB, TM_, 0, 2, 2, 8);                  \
    if (ET == 4) MOE_FUSED(XB, TM_, 0, 4, 1, 8);                  \
    MOE_FUSED(XB, TM_, 0, 4, 2, 16);
    if (!r.x_bf16) { MOE_FUSED_TILES(0, 32) }
    if (tm64) { MOE_FUSED_TILES(1, 64) }
    MOE_FUSED_TILES(1, 32)
#undef MOE_FUSED_TILES
#undef MOE_FUSED
}

template <int XBF16, int TM, int PAIRED, int NG, int TPW>
static hipError_t launch_logits_case(const RouterArgs &r, float *part, int nks, hipStream_t s) {
    const int ET = PAIRED ? 1 : (r.Er + 15) / 16;
    const size_t lds = std::max<size_t>((size_t)2 * TM * router_stage_row_bytes<XBF16, TM>(),
                                        sizeof(float) * (size_t)(4 / NG) * TM * (PAIRED ? 32 : ET * 16));
    if (lds > 150 * 1024) return hipErrorInvalidValue;
    auto kern = router_logits_kernel<XBF16, TM, PAIRED, NG, TPW>;
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3((r.T + TM - 1) / TM, nks), dim3(kRouteThreads), lds, s, r, part);
    return hipGetLastError();
}

hipError_t launch_router_logits(RouterArgs r, float *part, int max_slices, int *nks, hipStream_t s) {
    *nks = 1;
    if (r.T <= 0) return hipSuccess;
    if (r.Er < 1 || r.Er > MOE_MAX_EXPERTS || r.Dp % 32 != 0 || r.Dp < r.D || max_slices < 1)
        return hipErrorInvalidValue;
    const int ET = (r.Er + 15) / 16;
    const bool tm64 = r.x_bf16 != 0;  // 64-token tiles for bf16 x (fp32 x: 32, its staging is twice as wide)
    const int TM = tm64 ? 64 : 32;
    const int tiles = (r.T + TM - 1) / TM;
    // K slices of whole 8-step chunks so that tiles x slices reaches 256 workgroups
    const int S = r.Dp / 32, chunks = (S + 7) / 8;
    int want = std::max(1, std::min(std::min(max_slices, chunks), (256 + tiles - 1) / tiles));
    const int per = (chunks + want - 1) / want;
    r.kslice = per * 8;
    const int n = (S + r.kslice - 1) / r.kslice;
    *nks = n;
#define MOE_LOGITS(XB, TM_, P, NG_, TPW_) return launch_logits_case<XB, TM_, P, NG_, TPW_>(r, part, n, s)
#define MOE_LOGITS_TILES(XB, TM_)                                   \
    if (r.Er <= 8) MOE_LOGITS(XB, TM_, 1, 1, 1);                    \
    if (ET == 1) MOE_LOGITS(XB, TM_, 0, 1, 1);                      \
    if (ET == 2) MOE_LOGITS(XB, TM_, 0, 2, 1);                      \
    if (ET == 3) MOE_LOGITS(XB, TM_, 0, 2, 2);                      \
    if (ET == 4) MOE_LOGITS(XB, TM_, 0, 4, 1);                      \
    MOE_LOGITS(XB, TM_, 0, 4, 2);
    if (tm64) { MOE_LOGITS_TILES(1, 64) }
    MOE_LOGITS_TILES(0, 32)
#undef MOE_LOGITS_TILES
#undef MOE_LOGITS
}

hipError_t launch_route(const RouteArgs &a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    if (a.E != a.Er || a.E < 1 || a.E > MOE_MAX_EXPERTS || ((a.out_mask & ROUTE_OUT_GATING) && a.kt > MOE_MAX_TOPK))
        return hipErrorInvalidValue;
    const int nblk = (a.T + kRouteBlock - 1) / kRouteBlock;
    const size_t lds = route_lds_bytes(a);
    switch (route_epl(a.E)) {
    case 1: hipLaunchKernelGGL(route_kernel<1>, dim3(nblk), dim3(kRouteThreads), lds, s, a); break;
    case 2: hipLaunchKernelGGL(route_kernel<2>, dim3(nblk), dim3(kRouteThreads), lds, s, a); break;
    case 4: hipLaunchKernelGGL(route_kernel<4>, dim3(nblk), dim3(kRouteThreads), lds, s, a); break;
    case 8: hipLaunchKernelGGL(route_kernel<8>, dim3(nblk), dim3(kRouteThreads), lds, s, a); break;
    default: hipLaunchKernelGGL(route_kernel<16>, dim3(nblk), dim3(kRouteThreads), lds, s, a); break;
    }
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

__device__ __forceinline__ void scan_finish_block(const ScanArgs &a);

__global__ __launch_bounds__(kScanCols * kScanChunks) void scan_kernel(ScanArgs a) {
#pragma clang fp contract(off)
    static_assert(kScanCols * kScanChunks == 256, "the finish phase runs on 256 threads");
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
    // The block that finishes last runs the finish phase on all the column
    // totals: every block publishes its totals (release fence), then takes a
    // ticket; the last ticket's block acquires them and resets the ticket for
    // the next launch (which stream order puts after this one).
    __shared__ bool last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(a.ticket, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    if (threadIdx.x == 0) *a.ticket = 0u;
    scan_finish_block(a);
}

// Scan, part 2: one block (the last of part 1).  Capacity clamp, offsets,
// per-expert GEMM tile starts and the (expert, m0) tile list, the Switch and
// z losses, the mean entropy and the AuxiliaryFreeLoss step, from the column
// totals.
__device__ __forceinline__ void scan_finish_block(const ScanArgs &a) {
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
    if (!a.ticket || a.E > MOE_MAX_EXPERTS) return hipErrorInvalidValue;
    const int NC = a.E + 2;
    hipLaunchKernelGGL(scan_kernel, dim3((NC + kScanCols - 1) / kScanCols), dim3(kScanCols * kScanChunks), 0, s, a);
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
