// moe_gemm.hip -- the fp32 (reference-precision) grouped GEMM over
// variable-size expert segments on CDNA4 MFMA, with the expert FFN's
// elementwise work fused into the epilogues.  Handles with bf16 or fp8
// weights run the LDS-DMA kernel of moe_gemm_bf16.hip instead.
//
//   MODE_GATED_UP : h = act(A W1^T) .* (A W3^T)      GatedExpert
//                   (src/experts/gated.jl:29-34)
//   MODE_STD_UP   : h = act(A W1^T + b1)             StandardExpert
//                   (src/experts/standard.jl:38-47)
//   MODE_DOWN     : y = h W2^T (+ b2)                both
//
// A rows are one expert's contiguous segment of the permuted activations; the
// (expert, m0) tile list comes from the device-side scan, so no host round
// trip is needed.  Weights are prepacked [E][Npad][Kpad] (K contiguous) so a
// tile row is 128 contiguous bytes (32 fp32).
//
// Tile: 128 x 128 outputs per B matrix, 4 waves in a 2 x 2 layout, each wave
// 64 x 64 = 2 x 2 blocks of v_mfma_f32_32x32x2_f32, four per 16-byte
// fragment (a tile of at most 32 rows: 1 x 4 waves of one 32 x 32 block; the
// blocks past the tile's rows run no MFMAs).  LDS rows of 128 B are XOR-swizzled in 16-byte chunks so both the
// stores and the fragment reads are bank-conflict free.
//
// K split (g.ksplit = S > 1, chosen by the launch when the tile grid cannot
// fill the GPU: small expert segments stream their weights one K stage at a
// time per workgroup): workgroup (tile, ks) covers K stages [ks KT / S,
// (ks + 1) KT / S) and stores its raw accumulators (rows of the tile only) to
// split_ws block (tile, ks) = NB x BM x BN floats, [b][row][col];
// fold_f32_kernel sums the S ranges in order and runs the epilogue.
#include <algorithm>

#include "moe_internal.h"

namespace moe {

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

__device__ __forceinline__ int lds_off(int r, int chunk) { return r * 128 + ((chunk ^ (r & 7)) << 4); }

template <int MODE>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GemmArgs g) {
    constexpr int NB = (MODE == MODE_GATED_UP) ? 2 : 1;
    constexpr int BM = kGemmBM, BN = kGemmBN;
    constexpr int ROWB = 128;                     // bytes per LDS tile row
    constexpr int BK = ROWB / 4;                  // K elements per tile
    __shared__ __attribute__((aligned(16))) uint8_t lds[(BM + NB * BN) * ROWB];

    // ---- XCD-aware tile order: consecutive tiles (same weights, next rows)
    // land on the same XCD (blocks are dealt round-robin over 8 XCDs); the K
    // ranges of a tile are consecutive
    const int L = blockIdx.x;
    const int per = gridDim.x >> 3;
    const int S = g.ksplit;
    const int id0 = (L & 7) * per + (L >> 3);
    const int ks = id0 % S, id = id0 / S;
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
    // Wave layout: 2 x 2 waves of 64 x 64 outputs; a tile of at most 32 rows
    // (a small expert segment) runs 1 x 4 waves of 32 x 32, so that all four
    // SIMDs share its MFMAs.
    const bool skinny = rows <= 32;
    const int wm = skinny ? 0 : (wave & 1) * 64;
    const int wn = skinny ? wave * 32 : (wave >> 1) * 64;
    const int nj = skinny ? 1 : 2;  // 32-column blocks of the wave

    const uint8_t *Ab = (const uint8_t *)g.A;
    const long long lda_b = g.lda * 4;
    const long long ldb_b = g.ldb * 4;
    // packed weights [E][Npad][ldb]: this tile's first row is n0 of expert e
    const uint8_t *Bb0 = (const uint8_t *)g.B0 + ((long long)e * g.b_stride + (long long)n0 * g.ldb) * 4;
    const uint8_t *Bb1 =
        (NB == 2) ? (const uint8_t *)g.B1 + ((long long)e * g.b_stride + (long long)n0 * g.ldb) * 4 : Bb0;

    // global -> register staging; chunk c = tid + i*256: row c>>3, 16B chunk c&7
    u32x4_t ra[4], rb0[4], rb1[4];
#define MOE_LOAD_TILES(KT_)                                                                            \
    do {                                                                                              \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                               \
            const int c = tid + i * 256;                                                              \
            const int rr = min(c >> 3, rows - 1);                                                     \
            ra[i] = *(const u32x4_t *)(Ab + (arow0 + rr) * lda_b + (long long)(KT_) * ROWB + (c & 7) * 16); \
            const long long o = (long long)(c >> 3) * ldb_b + (long long)(KT_) * ROWB + (c & 7) * 16;   \
            rb0[i] = *(const u32x4_t *)(Bb0 + o);                                                       \
            if (NB == 2) rb1[i] = *(const u32x4_t *)(Bb1 + o);                                          \
        }                                                                                             \
    } while (0)

#define MOE_STORE_TILES()                                                                             \
    do {                                                                                              \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                               \
            const int c = tid + i * 256;                                                              \
            *(u32x4_t *)(lds + lds_off(c >> 3, c & 7)) = ra[i];                                         \
            *(u32x4_t *)(lds + BM * ROWB + lds_off(c >> 3, c & 7)) = rb0[i];                            \
            if (NB == 2) *(u32x4_t *)(lds + (BM + BN) * ROWB + lds_off(c >> 3, c & 7)) = rb1[i];        \
        }                                                                                             \
    } while (0)

    f32x16_t acc[NB][2][2];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[b][i][j][q] = 0.0f;

    const int KTT = g.K / BK;
    const int kb = (ks * KTT) / S, ke = ((ks + 1) * KTT) / S;  // this workgroup's K stages
    const int half = lane >> 5;
    const int r32 = lane & 31;
    // 32-row blocks of this wave that hold rows of the tile (wave-uniform): an
    // expert's last tile runs MFMAs only on those; the other accumulators stay
    // 0 and their rows are not stored
    const int nv = __builtin_amdgcn_readfirstlane(min(2, max(0, rows - wm + 31) >> 5));
    MOE_LOAD_TILES(kb);
    for (int kt = kb; kt < ke; ++kt) {
        __syncthreads();
        MOE_STORE_TILES();
        __syncthreads();
        MOE_LOAD_TILES(min(kt + 1, ke - 1));  // the last iteration re-reads a resident tile
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int chunk = ks * 2 + half;
            f32x4_t af[2], bfr[NB][2];
#pragma unroll
            for (int i = 0; i < 2; ++i) af[i] = *(const f32x4_t *)(lds + lds_off(wm + i * 32 + r32, chunk));
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    if (j < nj) bfr[b][j] = *(const f32x4_t *)(lds + (BM + b * BN) * ROWB + lds_off(wn + j * 32 + r32, chunk));
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        if (i >= nv || j >= nj) continue;  // no row of the tile, or not the wave's
                        acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i].x, bfr[b][j].x, acc[b][i][j], 0, 0, 0);
                        acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i].y, bfr[b][j].y, acc[b][i][j], 0, 0, 0);
                        acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i].z, bfr[b][j].z, acc[b][i][j], 0, 0, 0);
                        acc[b][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i].w, bfr[b][j].w, acc[b][i][j], 0, 0, 0);
                    }
        }
    }
#undef MOE_LOAD_TILES
#undef MOE_STORE_TILES

    // ---- epilogue: lane holds column r32 of each 32x32 block, rows
    // 8*(q/4) + 4*half + q%4.
    if (S > 1) {
        // a K range: the raw sums of the tile's rows
        float *ws = g.split_ws + ((long long)(mt * g.n_tiles + nt) * S + ks) * (NB * BM * BN);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (j >= nj) continue;
                const int nl = wn + j * 32 + r32;
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        const int ml = wm + i * 32 + 8 * (q >> 2) + 4 * half + (q & 3);
                        if (ml < rows) ws[(b * BM + ml) * BN + nl] = acc[b][i][j][q];
                    }
            }
        return;
    }
    const long long sofs = (long long)e * g.s_stride;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if (j >= nj) continue;
        const int nl = wn + j * 32 + r32;
        const int n = n0 + nl;
        if (n >= g.N) continue;
        const float bias = g.bias ? g.bias[sofs + n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int ml = wm + i * 32 + 8 * (q >> 2) + 4 * half + (q & 3);
                if (ml >= rows) continue;
                float v;
                if (MODE == MODE_GATED_UP) {
                    v = act_apply(g.act, acc[0][i][j][q]) * acc[NB - 1][i][j][q];
                } else if (MODE == MODE_STD_UP) {
                    v = dropout_h(g, arow0 + ml, n, act_apply(g.act, acc[0][i][j][q] + bias));
                } else {
                    v = acc[0][i][j][q] + bias;
                }
                ((float *)g.C)[(arow0 + ml) * g.ldc + n] = v;
            }
    }
}

// Fold of the K-split tiles: block (tile, y) covers elements 256 y .. of the
// tile; a thread sums its element's S partial sums in range order (a fixed
// order, so results are deterministic; all S loads in flight first) and
// applies the kernel's epilogue to it.
template <int MODE>
__global__ __launch_bounds__(256) void fold_f32_kernel(GemmArgs g) {
    constexpr int NB = (MODE == MODE_GATED_UP) ? 2 : 1;
    constexpr int BM = kGemmBM, BN = kGemmBN;
    const int mt = blockIdx.x % g.m_tiles_grid, nt = blockIdx.x / g.m_tiles_grid;
    if (nt >= g.n_tiles || mt >= g.num_tiles[0]) return;
    const int2 te = g.tiles[mt];
    const int e = te.x, m0 = te.y;
    const int rows = min(BM, g.counts[e] - m0);
    const long long arow0 = (long long)g.offsets[e] + m0;
    const int S = g.ksplit;
    const float *ws = g.split_ws + (long long)(mt * g.n_tiles + nt) * S * (NB * BM * BN);
    const long long sofs = (long long)e * g.s_stride;
    const int q = blockIdx.y * 256 + threadIdx.x;
    if (q < rows * BN) {
        const int ml = q / BN, nl = q - ml * BN, n = nt * BN + nl;
        if (n >= g.N) return;
        float p0[kF32SplitMax], p1[kF32SplitMax];
#pragma unroll
        for (int k = 0; k < kF32SplitMax; ++k)
            if (k < S) {
                const float *p = ws + (long long)k * (NB * BM * BN);
                p0[k] = p[ml * BN + nl];
                p1[k] = NB == 2 ? p[(BM + ml) * BN + nl] : 0.0f;
            }
        float v0 = p0[0], v1 = p1[0];
#pragma unroll
        for (int k = 1; k < kF32SplitMax; ++k)
            if (k < S) {
                v0 = v0 + p0[k];
                v1 = v1 + p1[k];
            }
        const float bias = g.bias ? g.bias[sofs + n] : 0.0f;
        float v;
        if (MODE == MODE_GATED_UP) v = act_apply(g.act, v0) * v1;
        else if (MODE == MODE_STD_UP) v = dropout_h(g, arow0 + ml, n, act_apply(g.act, v0 + bias));
        else v = v0 + bias;
        ((float *)g.C)[(arow0 + ml) * g.ldc + n] = v;
    }
}

template <int MODE>
static hipError_t launch_one(const GemmArgs &g, hipStream_t s) {
    long long total = (long long)g.m_tiles_grid * g.n_tiles * g.ksplit;
    total = (total + 7) / 8 * 8;
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE>), dim3((unsigned)total), dim3(256), 0, s, g);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && g.ksplit > 1) {
        hipLaunchKernelGGL((fold_f32_kernel<MODE>), dim3((unsigned)(g.m_tiles_grid * g.n_tiles), kGemmBM * kGemmBN / 256),
                           dim3(256), 0, s, g);
        e = hipGetLastError();
    }
    return e;
}

// K ranges of the fp32 GEMM: about two workgroups per CU over the tile grid,
// at most kF32SplitMax, at most one per K stage, and within the split
// workspace (g.split_cap floats; none: 1).
static int f32_ksplit(const GemmArgs &g, int nb) {
    const long long tiles = (long long)g.m_tiles_grid * g.n_tiles;
    if (!g.split_ws || g.ncu < 1 || tiles <= 0) return 1;
    long long S = std::min<long long>(kF32SplitMax, (2LL * g.ncu) / tiles);
    S = std::min<long long>(S, g.K / 32);
    S = std::min<long long>(S, g.split_cap / (tiles * nb * kGemmBM * kGemmBN));
    return (int)std::max<long long>(1, S);
}

hipError_t launch_grouped_gemm_f32(int mode, const GemmArgs &g0, hipStream_t s) {
    if (g0.m_tiles_grid <= 0 || g0.n_tiles <= 0) return hipSuccess;
    GemmArgs g = g0;
    g.ksplit = f32_ksplit(g, mode == MODE_GATED_UP ? 2 : 1);
    if (mode == MODE_GATED_UP) return launch_one<MODE_GATED_UP>(g, s);
    if (mode == MODE_STD_UP) return launch_one<MODE_STD_UP>(g, s);
    if (mode == MODE_DOWN) return launch_one<MODE_DOWN>(g, s);
    return hipErrorInvalidValue;
}

}  // namespace moe
