// moe_gemm.hip -- grouped GEMM over variable-size expert segments on CDNA4
// MFMA, with the expert FFN's elementwise work fused into the epilogues.
//
//   MODE_GATED_UP : h = act(s1 .* (A W1^T)) .* (s3 .* (A W3^T))   GatedExpert
//                   (src/experts/gated.jl:29-34)
//   MODE_STD_UP   : h = act(s1 .* (A W1^T) + b1)                  StandardExpert
//                   (src/experts/standard.jl:38-47)
//   MODE_DOWN     : y = s2 .* (h W2^T) (+ b2)                     both
//
// A rows are one expert's contiguous segment of the permuted activations; the
// (expert, m0) tile list comes from the device-side scan, so no host round
// trip is needed.  Weights are prepacked [E][Npad][Kpad] (K contiguous) so a
// tile row is 128 contiguous bytes: 64 bf16 or 32 fp32 (fp8 weights are
// widened to bf16 on their way into LDS; the per-output-channel scale is
// applied in the epilogue).
//
// Tile: 128 x 128 outputs per B matrix, 4 waves in a 2 x 2 layout, each wave
// 64 x 64 = 2 x 2 blocks of the 32x32 MFMA.  bf16 uses
// v_mfma_f32_32x32x16_bf16; fp32 uses v_mfma_f32_32x32x2_f32 four times per
// 16-byte fragment.  LDS rows of 128 B are XOR-swizzled in 16-byte chunks so
// both the stores and the fragment reads are bank-conflict free.
#include "moe_internal.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ inline float act_apply(int act, float x) {
    switch (act) {
    case MOE_ACT_SILU:  // x * sigmoid(x)
        return x / (1.0f + expf(-x));
    case MOE_ACT_GELU: {  // NNlib gelu, tanh form
        const float c = 0.7978845608028654f;  // sqrt(2/pi)
        const float u = c * (x + 0.044715f * x * x * x);
        return 0.5f * x * (1.0f + tanhf(u));
    }
    case MOE_ACT_RELU:
        return x > 0.0f ? x : 0.0f;
    default:
        return x;
    }
}

// Two fp8 e4m3 bytes (low half of w) -> two bf16 packed in a uint32 (exact).
__device__ inline uint32_t fp8x2_to_bf16x2(uint32_t w) {
    const uint32_t v0 = (uint32_t)f32_to_bf16(fp8e4m3_to_f32((uint8_t)(w & 0xffu)));
    const uint32_t v1 = (uint32_t)f32_to_bf16(fp8e4m3_to_f32((uint8_t)((w >> 8) & 0xffu)));
    return v0 | (v1 << 16);
}

// 16 fp8 e4m3 bytes -> 16 bf16 (exact) packed in two uint4.
__device__ inline void fp8x16_to_bf16(const u32x4_t &in, u32x4_t &lo, u32x4_t &hi) {
    lo.x = fp8x2_to_bf16x2(in.x);
    lo.y = fp8x2_to_bf16x2(in.x >> 16);
    lo.z = fp8x2_to_bf16x2(in.y);
    lo.w = fp8x2_to_bf16x2(in.y >> 16);
    hi.x = fp8x2_to_bf16x2(in.z);
    hi.y = fp8x2_to_bf16x2(in.z >> 16);
    hi.z = fp8x2_to_bf16x2(in.w);
    hi.w = fp8x2_to_bf16x2(in.w >> 16);
}

__device__ __forceinline__ int lds_off(int r, int chunk) { return r * 128 + ((chunk ^ (r & 7)) << 4); }

template <int MODE, int CT, int WT, int OUT_BF16>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GemmArgs g) {
    constexpr int NB = (MODE == MODE_GATED_UP) ? 2 : 1;
    constexpr int BM = kGemmBM, BN = kGemmBN;
    constexpr int ROWB = 128;                     // bytes per LDS tile row
    constexpr int ESZ = (CT == CT_F32) ? 4 : 2;   // compute element size
    constexpr int BK = ROWB / ESZ;                // K elements per tile
    __shared__ __attribute__((aligned(16))) uint8_t lds[(BM + NB * BN) * ROWB];

    // ---- XCD-aware tile order: consecutive tiles (same weights, next rows)
    // land on the same XCD (blocks are dealt round-robin over 8 XCDs).
    const int L = blockIdx.x;
    const int per = gridDim.x >> 3;
    const int id = (L & 7) * per + (L >> 3);
    const int mt = id % g.m_tiles_grid;
    const int nt = id / g.m_tiles_grid;
    if (nt >= g.n_tiles) return;
    if (mt >= g.num_tiles[0]) return;
    const int2 te = g.tiles[mt];
    const int e = te.x, m0 = te.y;
    const int rows = min(BM, g.counts[e] - m0);
    const long long arow0 = (long long)g.offsets[e] + m0;
    const int n0 = nt * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = (wave & 1) * 64;
    const int wn = (wave >> 1) * 64;

    const uint8_t *Ab = (const uint8_t *)g.A;
    const long long lda_b = g.lda * ESZ;
    constexpr int WSZ = (WT == WT_FP8) ? 1 : ESZ;  // stored weight element size
    const long long ldb_b = g.ldb * WSZ;
    // packed weights [E][Npad][ldb]: this tile's first row is n0 of expert e
    const uint8_t *Bb0 = (const uint8_t *)g.B0 + ((long long)e * g.b_stride + (long long)n0 * g.ldb) * WSZ;
    const uint8_t *Bb1 =
        (NB == 2) ? (const uint8_t *)g.B1 + ((long long)e * g.b_stride + (long long)n0 * g.ldb) * WSZ : Bb0;

#define MOE_LOAD_TILES(KT_)                                                                            \
    do {                                                                                              \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                               \
            const int c = tid + i * 256;                                                              \
            const int rr = min(c >> 3, rows - 1);                                                     \
            ra[i] = *(const u32x4_t *)(Ab + (arow0 + rr) * lda_b + (long long)(KT_) * ROWB + (c & 7) * 16); \
        }                                                                                             \
        _Pragma("unroll") for (int i = 0; i < NBCH; ++i) {                                            \
            const int c = tid + i * 256;                                                              \
            const long long o = (WT == WT_FP8) ? (long long)(c >> 2) * ldb_b + (long long)(KT_) * 64 + (c & 3) * 16 \
                                               : (long long)(c >> 3) * ldb_b + (long long)(KT_) * ROWB + (c & 7) * 16; \
            rb0[i] = *(const u32x4_t *)(Bb0 + o);                                                       \
            if (NB == 2) rb1[i] = *(const u32x4_t *)(Bb1 + o);                                          \
        }                                                                                             \
    } while (0)

#define MOE_STORE_B(RB_, LB_)                                                                         \
    do {                                                                                              \
        _Pragma("unroll") for (int i = 0; i < NBCH; ++i) {                                            \
            const int c = tid + i * 256;                                                              \
            if (WT == WT_FP8) {                                                                       \
                u32x4_t lo, hi;                                                                       \
                fp8x16_to_bf16(RB_[i], lo, hi);                                                       \
                *(u32x4_t *)((LB_) + lds_off(c >> 2, 2 * (c & 3))) = lo;                              \
                *(u32x4_t *)((LB_) + lds_off(c >> 2, 2 * (c & 3) + 1)) = hi;                          \
            } else {                                                                                  \
                *(u32x4_t *)((LB_) + lds_off(c >> 3, c & 7)) = RB_[i];                                  \
            }                                                                                         \
        }                                                                                             \
    } while (0)

#define MOE_STORE_TILES()                                                                             \
    do {                                                                                              \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                               \
            const int c = tid + i * 256;                                                              \
            *(u32x4_t *)(lds + lds_off(c >> 3, c & 7)) = ra[i];                                         \
        }                                                                                             \
        MOE_STORE_B(rb0, lds + BM * ROWB);                                                            \
        if (NB == 2) MOE_STORE_B(rb1, lds + (BM + BN) * ROWB);                                        \
    } while (0)

    // global -> register staging; chunk c = tid + i*256: row c>>3, 16B chunk c&7
    // (fp8 weights: row c>>2, 16 fp8 bytes = two bf16 LDS chunks)
    constexpr int NBCH = (WT == WT_FP8) ? 2 : 4;
    u32x4_t ra[4], rb0[NBCH], rb1[NBCH];

    f32x16_t acc[NB][2][2];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[b][i][j][q] = 0.0f;

    const int KT = g.K / BK;
    const int half = lane >> 5;
    const int r32 = lane & 31;
    MOE_LOAD_TILES(0);
    for (int kt = 0; kt < KT; ++kt) {
        __syncthreads();
        MOE_STORE_TILES();
        __syncthreads();
        MOE_LOAD_TILES(min(kt + 1, KT - 1));  // the last iteration re-reads a resident tile
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int chunk = ks * 2 + half;
            if constexpr (CT == CT_BF16) {
                bf16x8_t af[2], bfr[NB][2];
#pragma unroll
                for (int i = 0; i < 2; ++i) af[i] = *(const bf16x8_t *)(lds + lds_off(wm + i * 32 + r32, chunk));
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        bfr[b][j] = *(const bf16x8_t *)(lds + (BM + b * BN) * ROWB + lds_off(wn + j * 32 + r32, chunk));
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[b][j], acc[b][i][j], 0, 0, 0);
            } else {
                f32x4_t af[2], bfr[NB][2];
#pragma unroll
                for (int i = 0; i < 2; ++i) af[i] = *(const f32x4_t *)(lds + lds_off(wm + i * 32 + r32, chunk));
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        bfr[b][j] = *(const f32x4_t *)(lds + (BM + b * BN) * ROWB + lds_off(wn + j * 32 + r32, chunk));
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i].x, bfr[b][j].x, acc[b][i][j], 0, 0, 0);
                            acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i].y, bfr[b][j].y, acc[b][i][j], 0, 0, 0);
                            acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i].z, bfr[b][j].z, acc[b][i][j], 0, 0, 0);
                            acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i].w, bfr[b][j].w, acc[b][i][j], 0, 0, 0);
                        }
            }
        }
    }

    // ---- epilogue: lane holds column r32 of each 32x32 block, rows
    // 8*(q/4) + 4*half + q%4.
    const long long sofs = (long long)e * g.s_stride;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int nl = wn + j * 32 + r32;
        const int n = n0 + nl;
        if (n >= g.N) continue;
        float sc0 = 1.0f, sc1 = 1.0f, bias = 0.0f;
        if (g.s0) sc0 = g.s0[sofs + n];
        if (NB == 2 && g.s1) sc1 = g.s1[sofs + n];
        if (g.bias) bias = g.bias[sofs + n];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int ml = wm + i * 32 + 8 * (q >> 2) + 4 * half + (q & 3);
                if (ml >= rows) continue;
                float v;
                if (MODE == MODE_GATED_UP) {
                    const float gv = acc[0][i][j][q] * sc0;
                    const float uv = acc[NB - 1][i][j][q] * sc1;
                    v = act_apply(g.act, gv) * uv;
                } else if (MODE == MODE_STD_UP) {
                    v = act_apply(g.act, acc[0][i][j][q] * sc0 + bias);
                } else {
                    v = acc[0][i][j][q] * sc0 + bias;
                }
                const long long off = (arow0 + ml) * g.ldc + n;
                if (OUT_BF16)
                    ((uint16_t *)g.C)[off] = f32_to_bf16(v);
                else
                    ((float *)g.C)[off] = v;
            }
    }
}

template <int MODE, int CT, int WT, int OB>
static hipError_t launch_one(const GemmArgs &g, hipStream_t s) {
    long long total = (long long)g.m_tiles_grid * g.n_tiles;
    total = (total + 7) / 8 * 8;
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE, CT, WT, OB>), dim3((unsigned)total), dim3(256), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_grouped_gemm(int mode, int ct, int wt, int out_bf16, const GemmArgs &g,
                               hipStream_t s) {
    if (g.m_tiles_grid <= 0 || g.n_tiles <= 0) return hipSuccess;
#define MOE_GEMM_CASE(M, C, W, O)                                            \
    if (mode == M && ct == C && wt == W && out_bf16 == O) return launch_one<M, C, W, O>(g, s);
    // gated / standard up-projection: bf16 path writes bf16 h, fp32 path fp32 h
    MOE_GEMM_CASE(MODE_GATED_UP, CT_BF16, WT_BF16, 1)
    MOE_GEMM_CASE(MODE_GATED_UP, CT_BF16, WT_FP8, 1)
    MOE_GEMM_CASE(MODE_GATED_UP, CT_F32, WT_F32, 0)
    MOE_GEMM_CASE(MODE_STD_UP, CT_BF16, WT_BF16, 1)
    MOE_GEMM_CASE(MODE_STD_UP, CT_BF16, WT_FP8, 1)
    MOE_GEMM_CASE(MODE_STD_UP, CT_F32, WT_F32, 0)
    MOE_GEMM_CASE(MODE_DOWN, CT_BF16, WT_BF16, 0)
    MOE_GEMM_CASE(MODE_DOWN, CT_BF16, WT_FP8, 0)
    MOE_GEMM_CASE(MODE_DOWN, CT_F32, WT_F32, 0)
#undef MOE_GEMM_CASE
    return hipErrorInvalidValue;
}

}  // namespace moe
