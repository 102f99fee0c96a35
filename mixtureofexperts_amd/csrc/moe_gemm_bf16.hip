// moe_gemm_bf16.hip -- the bf16 grouped expert GEMM (the layer's MFMA-bound
// hot spot) for CDNA4: direct global->LDS loads into a ring of LDS stages,
// 256-column block tiles on v_mfma_f32_32x32x16_bf16, with the expert FFN's
// elementwise work in the epilogue.
//
//   MODE_GATED_UP : h = act(A W1^T) .* (A W3^T)       GatedExpert (src/experts/gated.jl:29-34)
//   MODE_STD_UP   : h = act(A W1^T + b1)              StandardExpert (src/experts/standard.jl:38-47)
//   MODE_DOWN     : y = h W2^T (+ b2)                 both
//
// A (the permuted tokens, or h) and the weights (bf16 or fp8 e4m3, WF8) are
// read as tile images: each LDS stage's bytes stored contiguously in the
// order the DMA writes them (load_plan), so every load is a whole-line 1 KB
// read.  The permute writes xp and the up GEMM's epilogue writes h in that
// form; the weights are retiled from their packed rows once per upload.
// fp8 weights stay fp8 in HBM and LDS (half the load bytes); each lane widens
// its fragments to bf16 with v_cvt_scalef32_pk_bf16_fp8 (exact for e4m3, scale
// 1) and the per-output-channel scale s multiplies the fp32 accumulator in
// the epilogue: s[n] * sum_k a[k] q[n][k] = sum_k a[k] (s[n] q[n][k]).
//
// Work list.  The device-side scan writes tile_start[e] = sum over e' < e of
// ceil(count_e' / BM).  Work item id is ordered expert-major, then blocks of
// kMBlock M tiles, then n-tile, then M tile (the up GEMM on 256-row tiles:
// pairs of n-tiles with a paired last M tile; split items: K range), so
// consecutive items share one weight tile and a block's rows serve its
// n-tiles.  Workgroups are dealt round-robin to the 8 XCDs, so item ids are
// assigned in contiguous per-XCD ranges: the blocks that share a weight tile
// and walk K in step run behind the same L2.
//
// Block: 4 waves, one per SIMD, as 2 (M) x 2 (N); each wave owns a (BM/2) x 128
// sub-tile and interleaves its MFMAs with the fragment reads of the next
// sub-step and the loads NS-1 stages ahead.  A wave runs MFMAs only on its
// 32-row blocks that hold rows of the tile: the last tile of an expert skips
// the padding past the expert's last row.
//
// For MODE_GATED_UP the 256 B-tile rows are 128 rows of W1 followed by the
// same 128 rows of W3, and each wave's four 32-column blocks are (gate, up)
// pairs for 64 h columns, so the silu-mul pairs sit in the same lane's
// registers.
//
// LDS: per stage an A tile (BM rows) and a B tile (256 rows) of 32 bf16 =
// 64 B per row; the 16-byte chunks of row r are stored at chunk ^ ((r >> 2) & 3)
// so the fragment reads (32 rows, one chunk) spread over all 64 banks.  Each
// global_load_lds_dwordx4 writes 1 KB = 16 rows linearly (lane l -> offset
// 16 l), so the swizzle is part of the tile images.
#include <algorithm>
#include <type_traits>

#include "moe_internal.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
#define MOE_LDS_AS __attribute__((address_space(3)))

// Activation in the epilogue of the bf16 path (outputs are rounded to bf16 or
// checked at bf16 tolerance): silu(x) = x * sigmoid(x) and NNlib's tanh-form
// gelu(x) = 0.5 x (1 + tanh(u)) = x * sigmoid(2u), u = sqrt(2/pi)(x + 0.044715 x^3),
// both as x * rcp(1 + exp(-z)) with the hardware exp and reciprocal.
template <int ACT>
__device__ __forceinline__ float act_fast(float x) {
    if constexpr (ACT == MOE_ACT_SILU) {
        return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
    } else if constexpr (ACT == MOE_ACT_GELU) {
        const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
        return x * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * u));
    } else if constexpr (ACT == MOE_ACT_RELU) {
        return x > 0.0f ? x : 0.0f;
    } else {
        return x;
    }
}

// Four fp32 -> four bf16 (round to nearest even, v_cvt_pk_bf16_f32), packed.
__device__ __forceinline__ uint2 pack_bf16x4(float a, float b, float c, float d) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t lo = {(__bf16)a, (__bf16)b}, hi = {(__bf16)c, (__bf16)d};
    uint2 r;
    __builtin_memcpy(&r.x, &lo, 4);
    __builtin_memcpy(&r.y, &hi, 4);
    return r;
}

// Eight fp8 e4m3 bytes (lo: bytes 0-3, hi: bytes 4-7) -> eight bf16 (exact).
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16x8_t widen_fp8x8(uint32_t lo, uint32_t hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    return bf16x8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Wait until at most N vector-memory operations of this wave are outstanding.
// The LDS writes of global_load_lds are counted by vmcnt.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Workgroup barrier that is also a compiler memory barrier (LDS accesses are
// not moved across it); the LDS reads of this wave are complete before it.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// global_load_lds_dwordx4: lane l copies 16 bytes from its own global address
// to LDS byte lds + 16 l (lds is wave-uniform, passed in M0: an input operand
// bound to M0, so the compiler itself writes M0 before the load and knows it
// is used).  Issued as inline assembly that the compiler does not see as a
// memory access: its wait insertion would otherwise treat every later LDS
// read as possibly reading these bytes and wait for all loads in flight.
// Correct ordering is kept by the kernels themselves: each slot is refilled
// only after a barrier that follows its last reads, and read only after a
// barrier that follows wait_vmcnt for its loads (volatile asm statements keep
// their relative order).
__device__ __forceinline__ void lds_dma16(const uint8_t *gaddr, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gaddr), "{m0}"(lds));
}

// ---- work item -> tile --------------------------------------------------------
struct TileJob {
    int e;             // expert
    int ks;            // K range (split-K index)
    int nks;           // K ranges of the tile (1: not split)
    int KT;            // 32-wide K stages in the range
    int rows;          // valid rows of the tile (<= BM)
    int n0;            // first B row of the tile (first h column in the gated mode)
    int split_j;       // split tiles: index among them (partials in split_ws)
    int mt;            // M tile (tile image block of the A operand and of h)
    int pair;          // up GEMM: the expert's last M tile (at most BM / 2 rows) for n-tiles nt and nt + 1
    long long arow0;   // first A row (expert-ordered row of the tile's first row)
};

// Work items: the items that are not split, then the K ranges of the split
// ones (tail_split).  Each class is dealt to the 8 XCDs in contiguous ranges
// (block L runs on XCD L mod 8): slots 0 .. pf-1 of an XCD take its whole
// items, the next ps slots its split items, which are dispatched last.
//
// The plain list: tile t of W = tile_start[E] * NT, expert-major, then
// blocks of kMBlock M tiles, then n-tile, then M tile.  With g.item_start (the up GEMM, NT even, 256-row
// tiles) an expert whose last M tile holds r <= BM / 2 rows has, per pair of
// n-tiles (2 j, 2 j + 1), the f full M tiles of n-tile 2 j, those of n-tile
// 2 j + 1, then one paired item: its last M tile against both n-tiles (the
// other experts as in the plain list); W = item_start[E].  A paired item runs
// the MFMAs of a full tile, so every workgroup of a round takes about as long
// as the others and the workgroups that share weight tiles stay in step.

// M tiles per block of the plain list's order.
constexpr int kMBlock = 8;

// Items of the work list.
__device__ __forceinline__ int work_items(const GemmArgs &g) {
    return g.item_start ? g.item_start[g.E] : g.tile_start[g.E] * g.n_tiles;
}

// Item -> tile (e, n0, rows, mt, pair); the K range fields are the caller's.
template <int BM, int NB>
__device__ __forceinline__ void decode_item(const GemmArgs &g, int item, TileJob &jb) {
    const int NT = g.n_tiles;
    int lo = 0, hi = g.E - 1;  // largest e whose first item is <= item (a non-empty expert)
    if (g.item_start) {
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (g.item_start[mid] <= item) lo = mid; else hi = mid - 1;
        }
    } else {
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (g.tile_start[mid] * NT <= item) lo = mid; else hi = mid - 1;
        }
    }
    const int e = lo;
    const int c = g.counts[e];
    const int f = c / BM, r = c - f * BM;
    int nt, m, pair = 0;
    if (g.item_start && r > 0 && r <= BM / 2) {
        const int local = item - g.item_start[e];
        const int gs = 2 * f + 1;
        const int j = local / gs, q = local - j * gs;
        if (q < f) { nt = 2 * j; m = q; }
        else if (q < 2 * f) { nt = 2 * j + 1; m = q - f; }
        else { nt = 2 * j; m = f; pair = 1; }
    } else {
        // blocks of kMBlock M tiles: block-major, then n-tile, then M tile,
        // so an expert of many M tiles re-reads neither its rows for every
        // n-tile nor its weights for every M tile (the last block holds the
        // remaining ml tiles)
        const int nte = f + (r > 0 ? 1 : 0);  // = tile_start[e + 1] - tile_start[e]
        const int local = item - (g.item_start ? g.item_start[e] : g.tile_start[e] * NT);
        const int nfb = nte / kMBlock, infull = nfb * kMBlock * NT;
        if (local < infull) {
            const int b = local / (kMBlock * NT), q = local - b * (kMBlock * NT);
            nt = q / kMBlock;
            m = b * kMBlock + (q - nt * kMBlock);
        } else {
            const int ml = nte - nfb * kMBlock, q = local - infull;
            nt = q / ml;
            m = nfb * kMBlock + (q - nt * ml);
        }
    }
    const int m0 = m * BM;
    jb.e = e;
    jb.rows = min(BM, c - m0);
    jb.arow0 = (long long)g.offsets[e] + m0;
    jb.n0 = nt * (NB == 2 ? 128 : 256);
    jb.mt = g.tile_start[e] + m;
    jb.pair = pair;
}

template <int BM, int NB>
__device__ __forceinline__ bool decode_job(const GemmArgs &g, TileJob &jb) {
    const int W = work_items(g);
    const TailSplit ts = tail_split(W, g.ncu, g.ksplit, g.K / 32);
    const int nsi = (W - ts.nfull) * ts.S;  // split items
    const int pf = (ts.nfull + 7) >> 3, ps = (nsi + 7) >> 3;
    const int L = blockIdx.x, x = L & 7, slot = L >> 3;
    int item, ks = 0, nks = 1;
    if (slot < pf) {
        item = x * pf + slot;
        if (item >= ts.nfull) return false;
    } else {
        if (slot - pf >= ps) return false;
        const int q = x * ps + (slot - pf);
        if (q >= nsi) return false;
        item = ts.nfull + q / ts.S;
        ks = q - (q / ts.S) * ts.S;
        nks = ts.S;
    }
    decode_item<BM, NB>(g, item, jb);
    jb.ks = ks;
    jb.nks = nks;
    jb.KT = g.K / 32 / nks;
    jb.split_j = item - ts.nfull;
    return true;
}

// ---- tile images: global -> LDS load addressing ---------------------------------
// The operands of this kernel are stored as tile images, the bytes of each
// LDS ring stage in the order the DMA writes them, so that every load is one
// contiguous, whole-line 1 KB read:
//   A (xp, h): block (M tile mt, K stage s) at ((mt * KTT + s) * BM) * 64 B,
//     BM rows of 64 B (32 bf16 of K);
//   B (packed weights, per expert): block (n block nb of RB rows, stage s) at
//     ((nb * KTT + s) * RB) * BROWB, RB rows of BROWB bytes; RB = 128 for the
//     gated W1 and W3 (a tile takes the same 128 rows of each), else 256;
//     BROWB = 64 (bf16) or 32 (fp8);
// with KTT = K / 32.  Within a row, 16-byte chunk c of K sits at chunk
// position c ^ ((r >> 2) & 3) for 64-B rows and c ^ ((r >> 3) & 1) for
// 32-B rows (r: row in the block), the swizzle the fragment reads expect.
// Load i of wave w covers A rows w * BM / NWAVE + 16 i .. +16 (lane l: 16 B
// at l * 16) and B-tile rows w * 256 / NWAVE + BR i .. +BR, BR = 16 (bf16) or
// 32 (fp8) (gated: tile rows [0, 128) are W1 rows n0.., [128, 256) the same
// W3 rows).  An expert's last M tile also holds rows past its valid ones;
// their products land in rows that are never stored.
// PAIR (a paired item): the first BM / 2 A rows of each image block, and 512
// B-tile rows: those of n-tile nt (rows 0 .. 255 as above), then those of
// n-tile nt + 1.
template <int BM, int NB, int NWAVE, int LA, int LB, int WF8, bool PAIR>
__device__ __forceinline__ void load_plan(const GemmArgs &g, const TileJob &jb, int w, int lane,
                                          const uint8_t *(&gsrc)[LA + LB], uint32_t (&ldst)[LA + LB]) {
    constexpr int ROWB = 64;
    constexpr int BROWB = WF8 ? 32 : 64;  // B bytes per row per stage
    constexpr int BMA = PAIR ? BM / 2 : BM;  // A rows staged
    constexpr int A_IMG = BM * ROWB;         // image block of an M tile and K stage
    constexpr int A_LDS = BMA * ROWB;
    constexpr int BRW = PAIR ? 512 : 256;    // B-tile rows
    constexpr int RB = (NB == 2) ? 128 : 256;
    const long long KTT = g.K / 32;
    const long long s0 = (long long)jb.ks * jb.KT;  // first stage of the K range
    const uint8_t *Ab = (const uint8_t *)g.A + ((long long)jb.mt * KTT + s0) * A_IMG + lane * 16;
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int r = w * (BMA / NWAVE) + 16 * i;
        gsrc[i] = Ab + (long long)r * ROWB;
        ldst[i] = r * ROWB;
    }
    constexpr int BR = WF8 ? 32 : 16;  // B-tile rows per load
    const long long esz = WF8 ? 1 : 2;
#pragma unroll
    for (int i = 0; i < LB; ++i) {
        const int t = w * (BRW / NWAVE) + BR * i;  // first tile row of the load
        const int hf = t >> 8, tt = t & 255;       // n-tile of the pair; row in its 256-row tile
        const int r = (NB == 2) ? (tt & 127) : tt; // row within the n block
        const uint8_t *Bsrc = (NB == 2 && tt >= 128) ? (const uint8_t *)g.B1 : (const uint8_t *)g.B0;
        gsrc[LA + i] = Bsrc + (long long)jb.e * g.b_stride * esz +
                       ((long long)(jb.n0 / RB + hf) * KTT + s0) * RB * BROWB + (long long)r * BROWB + lane * 16;
        ldst[LA + i] = A_LDS + t * BROWB;
    }
}

// B-tile row of fragment block j of a wave whose column group is wn (WN
// B-tile rows per group).  Gated: blocks 2m and 2m + 1 are the W1 and W3 rows
// of h columns wn * WN / 2 + 32 m.
template <int NB, int WN>
__device__ __forceinline__ int b_frag_row(int j, int wn) {
    return (NB == 2) ? ((j & 1) * 128 + wn * (WN / 2) + (j >> 1) * 32) : (wn * WN + j * 32);
}

// Component c (a compile-time constant after unrolling) of a float4.
__device__ __forceinline__ float f4_at(const float4 &v, int c) {
    return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
}

template <int N>
using ic = std::integral_constant<int, N>;

// ---- epilogue ---------------------------------------------------------------------
// The MFMA computes the transposed block (weights are its A operand): lane l
// holds token row l % 32 of the 32-row block and output columns 8 (q / 4) +
// 4 (l / 32) + q % 4, i.e. four consecutive columns per q / 4.  row0: the
// wave's first tile row.  WF8: the accumulators are scaled by the weight
// rows' scales (s0: W1 or W2, s1: W3) before bias and activation.
//
// bf16 outputs (h of both up modes; y of the down GEMM when c_bf16) go to
// put(ml, lc, v0, v1, v2, v3): tile row ml, tile column lc (a multiple of 4),
// four values.  The sink stages the tile in LDS (StagePut, then
// store_staged: h as its tile image, y as whole rows) or, for y rows whose
// N or ldc is not a multiple of 8, stores them directly (DirectPut: 8 bytes
// per lane, 32 rows per store instruction).  fp32 y and the partials of
// split tiles are stored directly.
template <int MODE, int ACT, int IM, int JN, int WN, int WF8, typename Put>
__device__ __forceinline__ void store_tile(const GemmArgs &g, const TileJob &jb, const f32x16_t (&acc)[IM][JN],
                                           int row0, int wn, int lane, Put &&put) {
    const int half = lane >> 5;
    const int r32 = lane & 31;
    const long long sofs = (long long)jb.e * g.s_stride;
    // The per-column vectors of the lane's column groups (weight scales, the
    // bias) are loaded in batches ahead of the accumulator reads that use
    // them: each load placed next to its use would wait out the round trip of
    // the one before it.
    if constexpr (MODE == MODE_GATED_UP) {
        // h pad columns [N, Npad) come out as act(0) * 0 = 0 from the zero weight
        // pad rows, so the whole tile is stored (ldc = Npad).
        constexpr int NG = (JN / 2) * 4;  // column groups of 4 h columns of the lane
        float4 sg[NG], su[NG];
        if constexpr (WF8) {
#pragma unroll
            for (int q = 0; q < NG; ++q) {
                const int lc = wn * (WN / 2) + (q >> 2) * 32 + 8 * (q & 3) + 4 * half;
                sg[q] = *(const float4 *)(g.s0 + sofs + jb.n0 + lc);
                su[q] = *(const float4 *)(g.s1 + sofs + jb.n0 + lc);
            }
        }
#pragma unroll
        for (int m = 0; m < JN / 2; ++m)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int q = m * 4 + g4;
                const int lc = wn * (WN / 2) + m * 32 + 8 * g4 + 4 * half;
#pragma unroll
                for (int i = 0; i < IM; ++i) {
                    const int ml = row0 + i * 32 + r32;
                    float v[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        float gt = acc[i][2 * m][4 * g4 + c], up = acc[i][2 * m + 1][4 * g4 + c];
                        if constexpr (WF8) {
                            gt = gt * f4_at(sg[q], c);
                            up = up * f4_at(su[q], c);
                        }
                        v[c] = act_fast<ACT>(gt) * up;
                    }
                    put(ml, lc, v[0], v[1], v[2], v[3]);
                }
            }
    } else {
        // MODE_STD_UP stores bf16 h (pads are act(b1 pad = 0) of zero rows: 0 for
        // silu, gelu, relu, identity); MODE_DOWN stores y with ldc = N, in bf16
        // (c_bf16) or fp32.  The lane's column blocks in two parts (four with
        // fp8 scales on 256-row tiles, whose accumulators leave fewer
        // registers), each with one batch of vector loads.
        const bool vec4 = (MODE == MODE_STD_UP) || ((g.ldc & 3) == 0);
        const bool yb = (MODE == MODE_STD_UP) || (g.c_bf16 && jb.nks == 1);
        const bool has_bias = g.bias && jb.ks == 0;  // split K: the bias belongs to one partial sum only
        constexpr int JH = ((WF8 || MODE == MODE_STD_UP) && IM == 4) ? 1 : (JN + 1) / 2;  // column blocks per part
        auto part = [&](auto H_, auto DROP_) {
            constexpr int H = decltype(H_)::value;
            constexpr bool DROP = decltype(DROP_)::value;
            constexpr int J0 = H * JH, J1 = (J0 + JH < JN) ? J0 + JH : JN;
            float4 bv[JH * 4], sc[JH * 4];
#pragma unroll
            for (int q = 0; q < (J1 - J0) * 4; ++q) {
                const int n = jb.n0 + wn * WN + (J0 + (q >> 2)) * 32 + 8 * (q & 3) + 4 * half;
                bv[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (has_bias) bv[q] = *(const float4 *)(g.bias + sofs + n);
                if constexpr (WF8) sc[q] = *(const float4 *)(g.s0 + sofs + n);
            }
#pragma unroll
            for (int j = J0; j < J1; ++j)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int q = (j - J0) * 4 + g4;
                    const int lc = wn * WN + j * 32 + 8 * g4 + 4 * half;
                    const int n = jb.n0 + lc;
#pragma unroll
                    for (int i = 0; i < IM; ++i) {
                        const int ml = row0 + i * 32 + r32;
                        float a[4];
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            a[c] = acc[i][j][4 * g4 + c];
                            if constexpr (WF8) a[c] = a[c] * f4_at(sc[q], c);
                            a[c] = a[c] + f4_at(bv[q], c);
                        }
                        if constexpr (MODE == MODE_STD_UP) {
                            float h4[4];
#pragma unroll
                            for (int c = 0; c < 4; ++c) {
                                h4[c] = act_fast<ACT>(a[c]);
                                if constexpr (DROP) h4[c] = dropout_h(g, jb.arow0 + ml, n + c, h4[c]);
                            }
                            put(ml, lc, h4[0], h4[1], h4[2], h4[3]);
                        } else if (yb) {
                            put(ml, lc, a[0], a[1], a[2], a[3]);
                        } else {
                            if (ml >= jb.rows) continue;
                            // fp32 y: K range 0 (or an unsplit tile) writes y; range
                            // r >= 1 its partial block in split_ws (BM x 256, row
                            // stride 256).  bf16 y: every range writes its block.
                            const long long blk = g.c_bf16 ? (long long)jb.split_j * jb.nks + jb.ks
                                                           : (long long)jb.split_j * (jb.nks - 1) + jb.ks - 1;
                            float *crow = (jb.ks == 0 && !g.c_bf16)
                                              ? (float *)g.C + (jb.arow0 + ml) * g.ldc
                                              : g.split_ws + blk * (IM * 64) * 256 + (long long)ml * 256 - jb.n0;
                            if (vec4 && n + 3 < g.N) {
                                *(float4 *)(crow + n) = make_float4(a[0], a[1], a[2], a[3]);
                            } else {
#pragma unroll
                                for (int c = 0; c < 4; ++c)
                                    if (n + c < g.N) crow[n + c] = a[c];
                            }
                        }
                    }
                }
        };
        auto tile = [&](auto DROP_) {
            part(ic<0>{}, DROP_);
            if constexpr (JN > JH) part(ic<1>{}, DROP_);
            if constexpr (JN > 2 * JH) part(ic<2>{}, DROP_);
            if constexpr (JN > 3 * JH) part(ic<3>{}, DROP_);
        };
        if constexpr (MODE == MODE_STD_UP) {
            if (g.drop_p > 0.0f) tile(std::true_type{});
            else tile(std::false_type{});
        } else {
            tile(std::false_type{});
        }
    }
}

// Direct bf16 sink of the down GEMM's y rows (N or ldc not a multiple of 8):
// rows past the tile's valid rows are skipped, columns past N cut.
struct DirectPut {
    const GemmArgs &g;
    const TileJob &jb;
    __device__ __forceinline__ void operator()(int ml, int lc, float v0, float v1, float v2, float v3) const {
        if (ml >= jb.rows) return;
        uint16_t *crow = (uint16_t *)g.C + (jb.arow0 + ml) * g.ldc;
        const int n = jb.n0 + lc;
        if (((g.ldc & 3) == 0) && n + 3 < g.N) {
            *(uint2 *)(crow + n) = pack_bf16x4(v0, v1, v2, v3);
        } else {
            const float v[4] = {v0, v1, v2, v3};
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (n + c < g.N) crow[n + c] = f32_to_bf16(v[c]);
        }
    }
};

// LDS staging of a bf16 output tile: row ml at row_addr(ml), CW bytes (CH
// 16-byte chunks) per row, chunk c of row r kept at chunk c ^ (r mod CH), so
// that both the column-block writes (32 rows, one chunk) and the row reads
// (one row, all chunks) spread over all LDS banks.
template <int CH, typename RowAddr>
struct StagePut {
    RowAddr row_addr;
    __device__ __forceinline__ void operator()(int ml, int lc, float v0, float v1, float v2, float v3) const {
        const int ch = lc >> 3;
        MOE_LDS_AS uint8_t *p = row_addr(ml) + ((ch ^ (ml & (CH - 1))) << 4) + ((lc & 4) << 1);
        const uint2 w = pack_bf16x4(v0, v1, v2, v3);
        *(MOE_LDS_AS u32x2_t *)p = u32x2_t{w.x, w.y};
    }
};

// Stores the staged tile.  Up GEMMs: h goes out as the down GEMM's A tile
// image, in which the tile's CW / 64 K stages of 64-B rows are one contiguous
// region (all BM rows, including rows past the valid ones): thread t writes
// 16-byte units t, t + 256, ..., unit u being chunk position u & 3 of row
// (u >> 2) mod BM of stage block u / (4 BM).  Down GEMM: y rows; thread t
// copies chunk t mod CH of rows t / CH + k (256 / CH), valid rows only and
// the chunks below N (N a multiple of 8).  U LDS reads are in flight before
// their global stores.
template <int MODE, int BM, int CH, typename RowAddr>
__device__ __forceinline__ void store_staged(const GemmArgs &g, const TileJob &jb, RowAddr row_addr) {
    constexpr int U = 8;
    if constexpr (MODE != MODE_DOWN) {
        constexpr int NU = BM * CH;  // 16-byte units of the tile
        const long long KTT = g.ldc / 32;  // h: K of the down GEMM = ldc
        uint8_t *base = (uint8_t *)g.C + ((long long)jb.mt * KTT + jb.n0 / 32) * BM * 64;
#pragma unroll
        for (int u0 = 0; u0 < NU; u0 += 256 * U) {
            u32x4_t v[U];
#pragma unroll
            for (int q = 0; q < U; ++q) {
                const int u = u0 + q * 256 + (int)threadIdx.x;
                const int r = (u >> 2) % BM;
                const int ch = (u / (4 * BM)) * 4 + ((u & 3) ^ ((r >> 2) & 3));  // column chunk in the tile
                v[q] = *(const MOE_LDS_AS u32x4_t *)(row_addr(r) + ((ch ^ (r & (CH - 1))) << 4));
            }
#pragma unroll
            for (int q = 0; q < U; ++q) *(u32x4_t *)(base + (long long)(u0 + q * 256 + threadIdx.x) * 16) = v[q];
        }
    } else {
        constexpr int RPP = 256 / CH;  // rows per pass of the workgroup
        const int ch = threadIdx.x % CH;
        const int rr = threadIdx.x / CH;
        const bool colok = jb.n0 + ch * 8 < g.N;
        uint16_t *cbase = (uint16_t *)g.C + jb.arow0 * g.ldc + jb.n0 + ch * 8;
        for (int p0 = 0; p0 < jb.rows; p0 += RPP * U) {
            u32x4_t v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = min(p0 + u * RPP + rr, BM - 1);
                v[u] = *(const MOE_LDS_AS u32x4_t *)(row_addr(r) + ((ch ^ (r & (CH - 1))) << 4));
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = p0 + u * RPP + rr;
                if (r < jb.rows && colok) *(u32x4_t *)(cbase + (long long)r * g.ldc) = v[u];
            }
        }
    }
}

// A paired item's staged tile (up GEMMs): staging rows hf BM / 2 + r hold row
// r of n-tile nt + hf; each n-tile's rows go to the first BM / 2 rows of its
// h image blocks (units as in store_staged, per n-tile).
template <int MODE, int BM, int CH, typename RowAddr>
__device__ __forceinline__ void store_staged_pair(const GemmArgs &g, const TileJob &jb, RowAddr row_addr) {
    constexpr int U = 8;
    constexpr int BMA = BM / 2;
    constexpr int NUH = BMA * CH;                               // 16-byte units per n-tile
    constexpr int NTW = (MODE == MODE_GATED_UP) ? 128 : 256;    // h columns per n-tile
    const long long KTT = g.ldc / 32;
#pragma unroll
    for (int u0 = 0; u0 < 2 * NUH; u0 += 256 * U) {
        u32x4_t v[U];
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const int u = u0 + q * 256 + (int)threadIdx.x;
            const int hf = u / NUH, up = u - hf * NUH;
            const int r = (up >> 2) % BMA;
            const int ch = (up / (4 * BMA)) * 4 + ((up & 3) ^ ((r >> 2) & 3));
            v[q] = *(const MOE_LDS_AS u32x4_t *)(row_addr(hf * BMA + r) + ((ch ^ (r & (CH - 1))) << 4));
        }
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const int u = u0 + q * 256 + (int)threadIdx.x;
            const int hf = u / NUH, up = u - hf * NUH;
            uint8_t *base = (uint8_t *)g.C + ((long long)jb.mt * KTT + (jb.n0 + hf * NTW) / 32) * BM * 64;
            *(u32x4_t *)(base + (long long)(up / (4 * BMA)) * BM * 64 + (up % (4 * BMA)) * 16) = v[q];
        }
    }
}

// A sink that moves rows by a fixed offset (the paired item's second n-tile).
template <typename Put>
struct RowOffsetPut {
    Put put;
    int off;
    __device__ __forceinline__ void operator()(int ml, int lc, float v0, float v1, float v2, float v3) const {
        put(ml + off, lc, v0, v1, v2, v3);
    }
};

// Prologue: this wave's NL loads of stages 0 .. NS-2 (clamped to the last
// stage), stage s into slot s.
#define MOE_PROLOGUE_LOADS(NS, NL, KT)                                       \
    _Pragma("unroll") for (int s0 = 0; s0 < NS - 1; ++s0) {                  \
        const int kt = min(s0, KT - 1);                                      \
        _Pragma("unroll") for (int i = 0; i < NL; ++i) {                     \
            switch (s0) {                                                    \
            case 0: dma(ic<0>{}, kt, i); break;                              \
            case 1: dma(ic<1>{}, kt, i); break;                              \
            case 2: dma(ic<2>{}, kt, i); break;                              \
            case 3: dma(ic<3>{}, kt, i); break;                              \
            default: dma(ic<4>{}, kt, i); break;                             \
            }                                                                \
        }                                                                    \
    }

// Runs stage(ic<slot>, s) for s = 0 .. KT-1 with slot = s % NS known at
// compile time (the body is unrolled NS times).
#define MOE_STAGE_LOOP(NS, KT)                                                    \
    {                                                                             \
        int st = 0;                                                               \
        for (; st + NS <= KT; st += NS) {                                         \
            stage(ic<0>{}, st);                                                   \
            stage(ic<1>{}, st + 1);                                               \
            stage(ic<2 % NS>{}, st + 2);                                          \
            if constexpr (NS > 3) stage(ic<3 % NS>{}, st + 3);                    \
            if constexpr (NS > 4) stage(ic<4 % NS>{}, st + 4);                    \
            if constexpr (NS > 5) stage(ic<5 % NS>{}, st + 5);                    \
        }                                                                         \
        if (st < KT) stage(ic<0>{}, st);                                          \
        if (st + 1 < KT) stage(ic<1 % NS>{}, st + 1);                             \
        if constexpr (NS > 3) if (st + 2 < KT) stage(ic<2 % NS>{}, st + 2);       \
        if constexpr (NS > 4) if (st + 3 < KT) stage(ic<3 % NS>{}, st + 3);       \
        if constexpr (NS > 5) if (st + 4 < KT) stage(ic<4 % NS>{}, st + 4);       \
    }

// ============================================================================
// 4-wave interleaved kernel, BM = 128 or 256.
// ============================================================================
// OCC: workgroups per CU.  128-row tiles (small experts, weight-bandwidth
// bound, or short K) run two per CU on a shorter ring, so one workgroup's
// prologue and epilogue overlap the other's main loop.
//
// The LDS ring: one array of RING bytes; slot J of a stage size STAGE at J
// STAGE.  The staged epilogue reuses it as rows of CW bytes.
template <int BM, int WF8, int OCC>
struct RingShape {
    static constexpr int STAGE = BM * 64 + 256 * (WF8 ? 32 : 64);
    static constexpr int NS = (OCC == 2) ? (WF8 ? 4 : 3) : ((BM == 256 && !WF8) ? 4 : 6);
    static constexpr int BYTES = NS * STAGE;
};

// One work item.  SPLIT: a K range of a split up-GEMM tile, which stores its
// partial sums (its own instantiation: the branch after the main loop would
// keep registers live through it).  PAIR: a paired item (decode_item): 4
// waves as 2 (n-tile
// of the pair) x 2 (N), each over the item's BM / 2 rows; otherwise 2 (M) x 2
// (N) over the BM rows of one n-tile.
template <int IM, int JN>
__device__ __forceinline__ void store_partial(const GemmArgs &g, const TileJob &jb, const f32x16_t (&acc)[IM][JN]);
template <int MODE, int BM, int ACT, int WF8, int OCC, bool PAIR, int IM, int JN>
__device__ __forceinline__ void tile_epilogue(const GemmArgs &g, const TileJob &jb, const f32x16_t (&acc)[IM][JN],
                                              uint8_t *ring_);

template <int MODE, int BM, int ACT, int WF8, int OCC, bool PAIR, bool SPLIT = false>
__device__ __forceinline__ void tile_body(const GemmArgs &g, const TileJob &jb, uint8_t *ring_) {
    constexpr int NWAVE = 4;
    constexpr int NB = (MODE == MODE_GATED_UP) ? 2 : 1;
    constexpr int ROWB = 64;             // bytes per LDS A row = 32 bf16 of K (one stage)
    constexpr int BROWB = WF8 ? 32 : 64; // bytes per LDS B row
    constexpr int BMA = PAIR ? BM / 2 : BM;  // A rows staged per stage
    constexpr int BRW = PAIR ? 512 : 256;    // B-tile rows per stage
    constexpr int A_BYTES = BMA * ROWB;      // A bytes of a stage in LDS
    constexpr int A_IMG = BM * ROWB;         // A image block stride (one K stage of an M tile)
    constexpr int STAGE = A_BYTES + BRW * BROWB;
    constexpr int RING = RingShape<BM, WF8, OCC>::BYTES;
    // LDS ring slots (<= 144 KB per CU)
    constexpr int NS = PAIR ? RING / STAGE : RingShape<BM, WF8, OCC>::NS;
    static_assert(NS >= 3 && NS <= 6, "ring depth");
    constexpr int WM = BM / 2;           // wave tile rows (2 waves along M; PAIR: the item's BM / 2 rows)
    constexpr int WN = 128;              // wave tile columns (2 waves along N)
    constexpr int IM = WM / 32;          // 32-row blocks per wave
    constexpr int JN = WN / 32;          // 32-column blocks per wave
    constexpr int LA = BMA / (16 * NWAVE);  // A loads (16 rows each) per wave per stage
    constexpr int LB = BRW / ((WF8 ? 32 : 16) * NWAVE);  // B loads per wave per stage
    constexpr int NL = LA + LB;          // 16-byte loads per lane per stage
    constexpr int NL0 = NL / 2;          // of which issued in a stage's first sub-step
    static_assert(NS * STAGE <= RING && RING * OCC <= 160 * 1024, "LDS");
    auto slot = [&](auto J_) -> MOE_LDS_AS uint8_t * {
        constexpr int J = decltype(J_)::value;
        return (MOE_LDS_AS uint8_t *)ring_ + (J < NS ? J : 0) * STAGE;
    };

    const int KT = jb.KT;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = w & 1, wn = w >> 1;

    const uint8_t *gsrc[NL];
    uint32_t ldst[NL];
    load_plan<BM, NB, NWAVE, LA, LB, WF8, PAIR>(g, jb, w, lane, gsrc, ldst);
    // load i of stage kt into ring slot J
    auto dma = [&](auto J_, int kt, int i) {
        const uint32_t l = (uint32_t)(uintptr_t)(slot(J_) + ldst[i]);
        lds_dma16(gsrc[i] + (long long)kt * (i < LA ? A_IMG : (NB == 2 ? 128 : 256) * BROWB),
                  __builtin_amdgcn_readfirstlane(l));
    };

    // ---- fragment addressing (fragment row bases are multiples of 32, so
    // swz(row) = (r32 >> 2) & 3) ------------------------------------------------
    // Lane (r32, half) supplies 8 K values per k16 sub-step kk: K 16 kk + 8 half
    // (bf16 weights, A chunk 2 kk + half) or K 16 half + 8 kk (fp8 weights: A
    // chunk 2 half + kk, and the lane's 16 weight bytes of the stage, K 16 half
    // .. +16, are one B chunk read once per stage).  The MFMA sums over K, so any
    // assignment of K values to (sub-step, lane half) shared by A and B works.
    const int half = lane >> 5;
    const int r32 = lane & 31;
    const int a_frag = ((PAIR ? 0 : wm * WM) + r32) * ROWB;
    int b_frag[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j)
        b_frag[j] = A_BYTES + ((PAIR ? wm * 256 : 0) + b_frag_row<NB, WN>(j, wn) + r32) * BROWB +
                    (WF8 ? ((half ^ ((r32 >> 3) & 1)) << 4) : 0);
    int choff[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
        choff[kk] = ((WF8 ? (half * 2 + kk) : (kk * 2 + half)) ^ ((r32 >> 2) & 3)) << 4;

    f32x16_t acc[IM][JN];
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
        for (int j = 0; j < JN; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

    bf16x8_t fa[2][IM], fb[2][JN];
    u32x4_t braw[JN];  // WF8: this stage's weight bytes (K 16 half .. +16) per column block

    // ---- main loop --------------------------------------------------------------
    // Stage s (32 K columns, two k16 sub-steps) lives in ring slot s % NS and is
    // loaded NS - 1 stages ahead.  Per stage:
    //   sub-step 0: MFMAs of (s, 0) | LDS reads of (s, 1)   | loads of stage s+NS-1, first half
    //   wait until this wave's loads of stage s+1 landed; barrier (every wave's have)
    //   sub-step 1: MFMAs of (s, 1) | LDS reads of (s+1, 0) | loads of stage s+NS-1, second half
    // Stage s+NS-1 goes to the slot of stage s-1, whose last reads (its sub-step
    // 1 fragments) ended before the barrier of stage s-1.  Past the last stage
    // the loads repeat stage KT-1 (in bounds, into a slot nothing reads again),
    // which keeps the vmcnt arithmetic exact: when the barrier of stage s is
    // reached, the loads issued after those of stage s+1 are NS-3 whole stages
    // and the first NL0 loads of stage s+NS-1.
    constexpr int AFTER = (NS - 3) * NL + NL0;
    MOE_PROLOGUE_LOADS(NS, NL, KT)
    wait_vmcnt<(NS - 2) * NL>();  // stage 0 landed
    barrier_lds();

    // The loop of a wave whose first NV 32-row blocks hold rows of the tile:
    // MFMAs and A-fragment reads only for those (NV = 0: the wave only loads
    // and takes part in the barriers).  Accumulators of the other blocks stay
    // 0 and their rows are not stored.
    auto run = [&](auto NV_) {
        constexpr int NV = decltype(NV_)::value;
        constexpr int NMF = NV * JN;
        // WF8: sub-step 0 reads the stage's weight bytes; each sub-step widens
        // its 8 bytes (words 2 kk, 2 kk + 1 of braw) to bf16.
        auto read_frags = [&](auto J_, int kk, bf16x8_t *af, bf16x8_t *bfr) {
            if constexpr (NV > 0) {
                const MOE_LDS_AS uint8_t *sb = slot(J_);
#pragma unroll
                for (int r = 0; r < NV; ++r)
                    af[r] = *(const MOE_LDS_AS bf16x8_t *)(sb + a_frag + r * 32 * ROWB + choff[kk]);
#pragma unroll
                for (int j = 0; j < JN; ++j) {
                    if constexpr (WF8) {
                        if (kk == 0) braw[j] = *(const MOE_LDS_AS u32x4_t *)(sb + b_frag[j]);
                        bfr[j] = widen_fp8x8(braw[j][2 * kk], braw[j][2 * kk + 1]);
                    } else {
                        bfr[j] = *(const MOE_LDS_AS bf16x8_t *)(sb + b_frag[j] + choff[kk]);
                    }
                }
            }
        };
        auto mfmas = [&](const bf16x8_t *af, const bf16x8_t *bfr) {
#pragma unroll
            for (int i = 0; i < NV; ++i)
#pragma unroll
                for (int j = 0; j < JN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
        };
        // One MFMA, then one fragment read of the next sub-step (NRD of them),
        // while both last; then the remaining MFMAs (or reads).
        auto interleave = [&](auto NRD_) {
            constexpr int NRD = decltype(NRD_)::value;
            constexpr int NPAIR = NMF < NRD ? NMF : NRD;
            if constexpr (NMF > 0) {
#pragma unroll
                for (int t = 0; t < NPAIR; ++t) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
                }
                if constexpr (NMF > NPAIR) __builtin_amdgcn_sched_group_barrier(0x008, NMF - NPAIR, 0);
                if constexpr (NRD > NPAIR) __builtin_amdgcn_sched_group_barrier(0x100, NRD - NPAIR, 0);
            }
        };
        read_frags(ic<0>{}, 0, fa[0], fb[0]);
        auto stage = [&](auto J_, int st) {
            constexpr int J = decltype(J_)::value;
            using Jn = ic<(J + 1) % NS>;       // slot of stage s+1
            using Jl = ic<(J + NS - 1) % NS>;  // slot of stage s-1 = s+NS-1
            const int kl = min(st + NS - 1, KT - 1);
            read_frags(J_, 1, fa[1], fb[1]);
#pragma unroll
            for (int t = 0; t < NL0; ++t) dma(Jl{}, kl, t);
            mfmas(fa[0], fb[0]);
            interleave(ic<(NV > 0) ? (WF8 ? NV : NV + JN) : 0>{});
            wait_vmcnt<AFTER>();
            barrier_lds();
            read_frags(Jn{}, 0, fa[0], fb[0]);
#pragma unroll
            for (int t = NL0; t < NL; ++t) dma(Jl{}, kl, t);
            mfmas(fa[1], fb[1]);
            interleave(ic<(NV > 0) ? NV + JN : 0>{});
        };
        MOE_STAGE_LOOP(NS, KT)
    };
    const int nv = min(IM, (max(0, jb.rows - (PAIR ? 0 : wm * WM)) + 31) >> 5);  // wave-uniform
    if (nv == IM) run(ic<IM>{});
    else if (nv == 0) run(ic<0>{});
    else if (nv == 1) run(ic<1>{});
    else if constexpr (IM > 2) {
        if (nv == 2) run(ic<2>{});
        else run(ic<3>{});
    }
    wait_vmcnt<0>();  // no load may still be writing LDS when the workgroup ends
    if constexpr (SPLIT) {
        // a K range of a split up-GEMM tile: its partial sums, for fold_up_kernel
        store_partial<IM, JN>(g, jb, acc);
        return;
    }
    tile_epilogue<MODE, BM, ACT, WF8, OCC, PAIR>(g, jb, acc, ring_);
}

// Partial sums of one K range of a split up-GEMM tile, in fragment order:
// block (split_j S + ks) of split_ws holds BM x 256 floats, thread t's
// accumulator values (i, j, q) at float (((i JN + j) 4 + q / 4) 256 + t) 4 +
// q % 4, so each wave writes and reads whole 1 KB runs.
template <int IM, int JN>
__device__ __forceinline__ void store_partial(const GemmArgs &g, const TileJob &jb, const f32x16_t (&acc)[IM][JN]) {
    float *ws = g.split_ws + ((long long)jb.split_j * jb.nks + jb.ks) * (IM * JN * 16 * 256) + threadIdx.x * 4;
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
        for (int j = 0; j < JN; ++j)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
                *(float4 *)(ws + ((i * JN + j) * 4 + q4) * 1024) =
                    make_float4(acc[i][j][4 * q4], acc[i][j][4 * q4 + 1], acc[i][j][4 * q4 + 2], acc[i][j][4 * q4 + 3]);
}

// The epilogue of a tile whose accumulators are complete.  bf16 outputs are
// staged in the (idle) LDS ring, rows of CW bytes: h as its tile image; y
// rows when y is bf16, the tile not split and N, ldc multiples of 8 (whole
// 16-byte chunks).  A paired item stages the rows of its n-tile nt + wm at
// rows wm BM / 2 ..
template <int MODE, int BM, int ACT, int WF8, int OCC, bool PAIR, int IM, int JN>
__device__ __forceinline__ void tile_epilogue(const GemmArgs &g, const TileJob &jb, const f32x16_t (&acc)[IM][JN],
                                              uint8_t *ring_) {
    constexpr int NB = (MODE == MODE_GATED_UP) ? 2 : 1;
    constexpr int BMA = PAIR ? BM / 2 : BM;
    constexpr int WM = BM / 2;
    constexpr int WN = 128;
    constexpr int RING = RingShape<BM, WF8, OCC>::BYTES;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = w & 1, wn = w >> 1;
    constexpr int CW = (MODE == MODE_GATED_UP ? 128 : 256) * 2;  // output bytes per tile row
    constexpr int CH = CW / 16;
    static_assert(BM * CW <= RING, "LDS staging of the output tile");
    const bool staged = (MODE != MODE_DOWN) || (g.c_bf16 && jb.nks == 1 && ((g.N | g.ldc) & 7) == 0);
    if (staged) {
        auto row_addr = [&](int r) -> MOE_LDS_AS uint8_t * { return (MOE_LDS_AS uint8_t *)ring_ + r * CW; };
        __syncthreads();  // every wave's ring reads and loads are done
        if constexpr (PAIR) {
            TileJob jw = jb;
            jw.n0 = jb.n0 + wm * (NB == 2 ? 128 : 256);
            using SP = StagePut<CH, decltype(row_addr)>;
            store_tile<MODE, ACT, IM, JN, WN, WF8>(g, jw, acc, 0, wn, lane,
                                                   RowOffsetPut<SP>{SP{row_addr}, wm * BMA});
            __syncthreads();
            store_staged_pair<MODE, BM, CH>(g, jb, row_addr);
        } else {
            store_tile<MODE, ACT, IM, JN, WN, WF8>(g, jb, acc, wm * WM, wn, lane,
                                                   StagePut<CH, decltype(row_addr)>{row_addr});
            __syncthreads();
            store_staged<MODE, BM, CH>(g, jb, row_addr);
        }
    } else if constexpr (MODE == MODE_DOWN) {
        store_tile<MODE, ACT, IM, JN, WN, WF8>(g, jb, acc, wm * WM, wn, lane, DirectPut{g, jb});
    }
}

template <int MODE, int BM, int ACT, int WF8, int OCC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void grouped_gemm_bf16_kernel(
    GemmArgs g) {
    __shared__ __attribute__((aligned(1024))) uint8_t ring[RingShape<BM, WF8, OCC>::BYTES];
    TileJob jb;
    if (!decode_job<BM, (MODE == MODE_GATED_UP) ? 2 : 1>(g, jb)) return;
    if constexpr (MODE != MODE_DOWN) {
        if (jb.nks > 1) {
            if constexpr (BM == 256) {
                if (jb.pair) {
                    tile_body<MODE, BM, ACT, WF8, OCC, true, true>(g, jb, ring);
                    return;
                }
            }
            tile_body<MODE, BM, ACT, WF8, OCC, false, true>(g, jb, ring);
            return;
        }
    }
    if constexpr (MODE != MODE_DOWN && BM == 256) {
        if (jb.pair) {
            tile_body<MODE, BM, ACT, WF8, OCC, true>(g, jb, ring);
            return;
        }
    }
    tile_body<MODE, BM, ACT, WF8, OCC, false>(g, jb, ring);
}

// ============================================================================
// Fold of the up GEMM's split tiles (tail_split).  Work unit (j, i, mo) of a
// split tile j: for every thread t of the tile's workgroup, its accumulator
// blocks [i][2 mo], [i][2 mo + 1] (a 32-row block and 64 B-tile columns of its
// wave: one W1 | W3 column pair of the gated mode, two column blocks
// otherwise).  Thread t of a fold workgroup sums those blocks' K-range
// partials in range order (a fixed order, so results are deterministic) and
// runs the tile's epilogue on them (fp8 scales, bias, activation, dropout),
// storing its bf16 h values straight into the h tile image (ImagePut).
// Workgroups stride over the units.
// ============================================================================
// Sink of h values into the h tile image: rows of 64 B per 32-wide K stage
// block of BM rows, chunk c of row r at position c ^ ((r >> 2) & 3) (the
// layout store_staged writes).  base: the image block of the tile's M tile
// and of the stage of column n0.
template <int BM>
struct ImagePut {
    uint8_t *base;
    __device__ __forceinline__ void operator()(int ml, int lc, float v0, float v1, float v2, float v3) const {
        const int p = ((lc >> 3) & 3) ^ ((ml >> 2) & 3);
        uint8_t *a = base + ((long long)(lc >> 5) * BM + ml) * 64 + p * 16 + (lc & 4) * 2;
        *(uint2 *)a = pack_bf16x4(v0, v1, v2, v3);
    }
};

template <int MODE, int BM, int ACT, int WF8>
__global__ __launch_bounds__(256) void fold_up_kernel(GemmArgs g) {
    constexpr int NB = (MODE == MODE_GATED_UP) ? 2 : 1;
    constexpr int IM = BM / 64, JN = 4;  // the accumulator blocks of tile_body's waves
    constexpr int WN = 128;
    constexpr long long BLK = IM * JN * 16 * 256;  // floats per partial block
    const int W = work_items(g);
    const TailSplit ts = tail_split(W, g.ncu, g.ksplit, g.K / 32);
    if (ts.S < 2) return;
    const int nunit = (W - ts.nfull) * IM * 2;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, wm = w & 1, wn = w >> 1;
    const long long KTT = g.ldc / 32;  // h: K of the down GEMM = ldc
    for (int u = blockIdx.x; u < nunit; u += gridDim.x) {
        const int j = u / (IM * 2), i = (u >> 1) % IM, mo = u & 1;
        // every partial of the unit in flight before the work-item decode
        // (a chain of dependent loads) runs
        const float *ws = g.split_ws + (long long)j * ts.S * BLK + ((i * JN + 2 * mo) * 4) * 1024 + t * 4;
        constexpr int RB = 4;  // ranges whose loads are in flight together
        float4 p[RB][8], a[8];
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (r < ts.S) p[r][q] = *(const float4 *)(ws + r * BLK + q * 1024);
        TileJob jb;
        decode_item<BM, NB>(g, ts.nfull + j, jb);
        jb.ks = 0;
        jb.nks = 1;
        jb.KT = g.K / 32;
        jb.split_j = j;
#pragma unroll
        for (int q = 0; q < 8; ++q) a[q] = p[0][q];
        // ranges in order: a = ((p0 + p1) + p2) + ...
#pragma unroll
        for (int r0 = 0; r0 < kUpSplitMax; r0 += RB) {
            if (r0 > 0) {
#pragma unroll
                for (int r = 0; r < RB; ++r)
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        if (r0 + r < ts.S) p[r][q] = *(const float4 *)(ws + (r0 + r) * BLK + q * 1024);
            }
#pragma unroll
            for (int r = (r0 == 0 ? 1 : 0); r < RB; ++r)
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (r0 + r < ts.S) {
                        a[q].x = a[q].x + p[r][q].x; a[q].y = a[q].y + p[r][q].y;
                        a[q].z = a[q].z + p[r][q].z; a[q].w = a[q].w + p[r][q].w;
                    }
        }
        f32x16_t acc[1][2];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            acc[0][q >> 2][4 * (q & 3)] = a[q].x;
            acc[0][q >> 2][4 * (q & 3) + 1] = a[q].y;
            acc[0][q >> 2][4 * (q & 3) + 2] = a[q].z;
            acc[0][q >> 2][4 * (q & 3) + 3] = a[q].w;
        }
        // the columns of these blocks: gated, h columns wn WN / 2 + 32 mo ..;
        // otherwise B-tile columns wn WN + 64 mo ..; a paired item's wave wm
        // holds n-tile nt + wm over the item's rows
        TileJob jw = jb;
        int row0;
        if (jb.pair) {
            jw.n0 += wm * (NB == 2 ? 128 : 256);
            row0 = i * 32;
        } else {
            row0 = wm * (BM / 2) + i * 32;
        }
        jw.n0 += (NB == 2) ? wn * (WN / 2) + 32 * mo : wn * WN + 64 * mo;
        ImagePut<BM> put{(uint8_t *)g.C + ((long long)jw.mt * KTT + jw.n0 / 32) * BM * 64};
        store_tile<MODE, ACT, 1, 2, WN, WF8>(g, jw, acc, row0, 0, lane, put);
    }
}

// ============================================================================
// Fold of the down GEMM's split tiles (tail_split): y += partial 1, then
// partial 2, ... (a fixed order, so results are deterministic).  Block
// (j, q): split tile j, its 16 rows from 16 q; a thread covers 4 columns of
// 4 rows, with all their loads in flight (one batch: no store is followed by
// a load in the same thread).
// ============================================================================
template <int BM>
__global__ __launch_bounds__(256) void fold_split_kernel(GemmArgs g) {
#pragma clang fp contract(off)
    constexpr int bm = BM;
    const int W = work_items(g);
    const TailSplit ts = tail_split(W, g.ncu, g.ksplit, g.K / 32);
    const int j = blockIdx.x;
    if (ts.S < 2 || j >= W - ts.nfull) return;
    TileJob jb;
    decode_item<BM, 1>(g, ts.nfull + j, jb);
    const int rows = jb.rows;
    const long long arow0 = jb.arow0;
    const int n0 = jb.n0;
    const int c4 = (threadIdx.x & 63) * 4;
    const int n = n0 + c4;
    const bool vec4 = (g.ldc & 3) == 0 && n + 3 < g.N;
    const long long pstride = (long long)bm * 256;
    const int r0 = blockIdx.y * 16 + (threadIdx.x >> 6);
    if (g.c_bf16) {
        // y = bf16(((p0 + p1) + p2) + p3), the partials of all ranges
        const float *__restrict__ ws = g.split_ws + (long long)j * ts.S * bm * 256 + c4;
        if (r0 >= rows) return;
        float4 p[4][kDownSplitMax];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = min(r0 + 4 * u, rows - 1);
#pragma unroll
            for (int k = 0; k < kDownSplitMax; ++k)
                if (k < ts.S) p[u][k] = *(const float4 *)(ws + k * pstride + (long long)r * 256);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = r0 + 4 * u;
            if (r >= rows) continue;
            float4 a = p[u][0];
#pragma unroll
            for (int k = 1; k < kDownSplitMax; ++k)
                if (k < ts.S) {
                    a.x = a.x + p[u][k].x; a.y = a.y + p[u][k].y;
                    a.z = a.z + p[u][k].z; a.w = a.w + p[u][k].w;
                }
            uint16_t *__restrict__ yp = (uint16_t *)g.C + (arow0 + r) * g.ldc + n;
            if (vec4) {
                *(uint2 *)yp = pack_bf16x4(a.x, a.y, a.z, a.w);
            } else {
                const float av[4] = {a.x, a.y, a.z, a.w};
                for (int c = 0; c < 4; ++c)
                    if (n + c < g.N) yp[c] = f32_to_bf16(av[c]);
            }
        }
        return;
    }
    const float *__restrict__ ws = g.split_ws + (long long)j * (ts.S - 1) * bm * 256 + c4;
    if (r0 < rows) {
        float4 v[4], p[4][kDownSplitMax - 1];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = min(r0 + 4 * u, rows - 1);
            float *__restrict__ yp = (float *)g.C + (arow0 + r) * g.ldc + n;
            if (vec4) v[u] = *(const float4 *)yp;
#pragma unroll
            for (int k = 0; k < kDownSplitMax - 1; ++k)
                if (k + 1 < ts.S) p[u][k] = *(const float4 *)(ws + k * pstride + (long long)r * 256);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = r0 + 4 * u;
            if (r >= rows) continue;
            float *__restrict__ yp = (float *)g.C + (arow0 + r) * g.ldc + n;
            if (vec4) {
                float4 a = v[u];
#pragma unroll
                for (int k = 0; k < kDownSplitMax - 1; ++k)
                    if (k + 1 < ts.S) {
                        a.x = a.x + p[u][k].x; a.y = a.y + p[u][k].y;
                        a.z = a.z + p[u][k].z; a.w = a.w + p[u][k].w;
                    }
                *(float4 *)yp = a;
            } else {
                for (int c = 0; c < 4; ++c)
                    if (n + c < g.N) {
                        float a = yp[c];
                        for (int k = 1; k < ts.S; ++k) a = a + ws[(k - 1) * pstride + (long long)r * 256 + c];
                        yp[c] = a;
                    }
            }
        }
    }
}

// ============================================================================
// Packed weights -> B tile image.  src: one expert's matrix, Npad rows of Kp
// elements of esz bytes (row-major, as packed); dst: its tile image (RB-row
// blocks, 32-wide K stages, chunk c of a row at c ^ swizzle(row)).  One
// thread per 16-byte unit of the image, written in order.
// ============================================================================
__global__ __launch_bounds__(256) void retile_weights_kernel(const uint8_t *__restrict__ src,
                                                             uint8_t *__restrict__ dst, int Npad, int Kp, int esz,
                                                             int RB) {
    const int upr = 2 * esz;  // 16-byte units per row per stage: 4 (bf16) or 2 (fp8)
    const long long KTT = Kp / 32;
    const long long total = (long long)Npad * Kp * esz / 16;
    for (long long u = blockIdx.x * 256LL + threadIdx.x; u < total; u += (long long)gridDim.x * 256) {
        const long long blk = u / ((long long)RB * upr);
        const int within = (int)(u - blk * RB * upr);
        const int r = within / upr, slot = within - (within / upr) * upr;
        const long long nb = blk / KTT, st = blk - nb * KTT;
        const int c = (upr == 4) ? (slot ^ ((r >> 2) & 3)) : (slot ^ ((r >> 3) & 1));
        const uint8_t *sp = src + (nb * RB + r) * (long long)Kp * esz + st * 32 * esz + c * 16;
        *(u32x4_t *)(dst + u * 16) = *(const u32x4_t *)sp;
    }
}

hipError_t launch_retile_weights(const void *src, void *dst, int Npad, int Kp, int esz, int RB, hipStream_t s) {
    if (Npad % RB != 0 || Kp % 32 != 0 || (esz != 1 && esz != 2)) return hipErrorInvalidValue;
    const long long units = (long long)Npad * Kp * esz / 16;
    const int blocks = (int)std::min<long long>((units + 255) / 256, 8192);
    hipLaunchKernelGGL(retile_weights_kernel, dim3(blocks), dim3(256), 0, s, (const uint8_t *)src, (uint8_t *)dst,
                       Npad, Kp, esz, RB);
    return hipGetLastError();
}

hipError_t launch_fold_split(int bm, const GemmArgs &g, hipStream_t s) {
    if (g.ksplit < 2 || g.ncu < 1 || g.m_tiles_grid <= 0) return hipSuccess;
    if (bm == 256)
        hipLaunchKernelGGL(fold_split_kernel<256>, dim3(g.ncu, 16), dim3(256), 0, s, g);
    else if (bm == 128)
        hipLaunchKernelGGL(fold_split_kernel<128>, dim3(g.ncu, 8), dim3(256), 0, s, g);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int MODE, int BM, int ACT, int WF8>
static hipError_t launch_bf16(const GemmArgs &g, hipStream_t s) {
    // 8 XCDs x (slots for the whole tiles + slots for the split items)
    const long long tiles = (long long)g.m_tiles_grid * g.n_tiles;
    const long long total = 8 * ((tiles + 7) / 8 + (g.ksplit > 1 ? (g.ncu + 7) / 8 : 0));
    // 128-row tiles run two workgroups per CU (the down GEMM's tail split then
    // plans its last round over g.ncu = 2 slots per CU)
    constexpr int OCC = (BM == 128) ? 2 : 1;
    hipLaunchKernelGGL((grouped_gemm_bf16_kernel<MODE, BM, ACT, WF8, OCC>), dim3((unsigned)total), dim3(256), 0, s, g);
    hipError_t e = hipGetLastError();
    // the up GEMM's split tiles (256-row tiles only) are folded in work units
    // over g.ncu workgroups
    if constexpr (MODE != MODE_DOWN && BM == 256) {
        if (e == hipSuccess && g.ksplit > 1) {
            hipLaunchKernelGGL((fold_up_kernel<MODE, BM, ACT, WF8>), dim3((unsigned)g.ncu), dim3(256), 0, s, g);
            e = hipGetLastError();
        }
    }
    return e;
}

template <int MODE, int BM, int WF8>
static hipError_t launch_bf16_act(const GemmArgs &g, hipStream_t s) {
    if constexpr (MODE == MODE_DOWN) {
        return launch_bf16<MODE, BM, MOE_ACT_IDENTITY, WF8>(g, s);
    } else {
        switch (g.act) {
        case MOE_ACT_SILU: return launch_bf16<MODE, BM, MOE_ACT_SILU, WF8>(g, s);
        case MOE_ACT_GELU: return launch_bf16<MODE, BM, MOE_ACT_GELU, WF8>(g, s);
        case MOE_ACT_RELU: return launch_bf16<MODE, BM, MOE_ACT_RELU, WF8>(g, s);
        default: return launch_bf16<MODE, BM, MOE_ACT_IDENTITY, WF8>(g, s);
        }
    }
}

hipError_t launch_grouped_gemm_bf16(int mode, int bm, int wfp8, const GemmArgs &g, hipStream_t s) {
    if (g.m_tiles_grid <= 0 || g.n_tiles <= 0) return hipSuccess;
    // split tiles write partial sums; the up GEMM splits 256-row tiles only
    if (g.ksplit < 1 || (g.ksplit > 1 && (!g.split_ws || g.ncu < 1))) return hipErrorInvalidValue;
    if (g.ksplit > 1 && mode != MODE_DOWN && bm != 256) return hipErrorInvalidValue;
    if (wfp8 && (!g.s0 || (mode == MODE_GATED_UP && !g.s1))) return hipErrorInvalidValue;
#define MOE_BF16_CASE(M, B, F) \
    if (mode == M && bm == B && (wfp8 != 0) == (F != 0)) return launch_bf16_act<M, B, F>(g, s);
    MOE_BF16_CASE(MODE_GATED_UP, 256, 0)
    MOE_BF16_CASE(MODE_STD_UP, 256, 0)
    MOE_BF16_CASE(MODE_DOWN, 256, 0)
    MOE_BF16_CASE(MODE_GATED_UP, 128, 0)
    MOE_BF16_CASE(MODE_STD_UP, 128, 0)
    MOE_BF16_CASE(MODE_DOWN, 128, 0)
    MOE_BF16_CASE(MODE_GATED_UP, 256, 1)
    MOE_BF16_CASE(MODE_DOWN, 256, 1)  // (standard experts with fp8 weights take 128-row tiles)
    MOE_BF16_CASE(MODE_GATED_UP, 128, 1)
    MOE_BF16_CASE(MODE_STD_UP, 128, 1)
    MOE_BF16_CASE(MODE_DOWN, 128, 1)
#undef MOE_BF16_CASE
    return hipErrorInvalidValue;
}

}  // namespace moe
