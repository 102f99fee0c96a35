// moe_gemm_bf16.hip -- the bf16 grouped expert GEMM (the layer's MFMA-bound
// hot spot) for CDNA4: direct global->LDS loads, two LDS stages, 256x256 block
// tiles on v_mfma_f32_32x32x16_bf16 with the expert FFN's elementwise work in
// the epilogue.
//
//   MODE_GATED_UP : h = act(A W1^T) .* (A W3^T)       GatedExpert (src/experts/gated.jl:29-34)
//   MODE_STD_UP   : h = act(A W1^T + b1)              StandardExpert (src/experts/standard.jl:38-47)
//   MODE_DOWN     : y = h W2^T (+ b2)                 both
//
// A is one expert's contiguous segment of rows (the permuted tokens, or h);
// weights are packed [E][Npad][Kpad] bf16, K contiguous.
//
// Work list.  The device-side scan writes tile_start[e] = sum over e' < e of
// ceil(count_e' / BM).  Work item id = (tile_start[e] + m) * ... is ordered
// expert-major, then n-tile, then m-tile, so consecutive items share one
// weight tile.  Workgroups are dealt round-robin to the 8 XCDs, so item ids
// are assigned in contiguous per-XCD ranges: the blocks that share a weight
// tile and walk K in step run behind the same L2.
//
// Block: 256 threads = 4 waves as 2 (M) x 2 (N); each wave owns a
// (BM/2) x 128 sub-tile = (BM/64) x 4 blocks of 32x32 accumulators.  For
// MODE_GATED_UP the 256 B-tile rows are 128 rows of W1 followed by the same
// 128 rows of W3, and each wave's four 32-column blocks are (gate, up) pairs
// for 64 h columns, so the silu-mul pairs sit in the same lane's registers.
//
// LDS: per stage an A tile (BM rows) and a B tile (256 rows) of 64 bf16 =
// 128 B per row; the 16-byte chunks of row r are stored at chunk ^ (r & 7) so
// the fragment reads (32 rows, one chunk) are spread over all banks.  Each
// global_load_lds_dwordx4 writes 1 KB = 8 rows of LDS linearly (lane l ->
// offset 16 l), so the swizzle is applied on the global side: lane l fetches
// logical chunk (l & 7) ^ (l >> 3) of its row.
#include "moe_internal.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
#define MOE_LDS_AS __attribute__((address_space(3)))

__device__ inline float act_apply_bf(int act, float x) {
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

// global_load_lds_dwordx4: lane l copies 16 bytes from base + voff (its own
// offset) to LDS address lds + 16 l.  Issued as inline assembly so that the
// compiler's wait insertion does not treat every later LDS read as dependent
// on it (it cannot tell the two stages apart and would wait for all loads);
// the kernel waits for these loads explicitly with wait_vmcnt.  base and lds
// are wave-uniform.
__device__ __forceinline__ void lds_dma16(const uint8_t *base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}

__device__ __forceinline__ const uint8_t *uniform_ptr(const uint8_t *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const uint8_t *)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ uint32_t lds_addr(const uint8_t *p) {
    return (uint32_t)(uintptr_t)(const MOE_LDS_AS uint8_t *)p;
}

template <int MODE, int BM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void grouped_gemm_bf16_kernel(
    GemmArgs g) {
    constexpr int NB = (MODE == MODE_GATED_UP) ? 2 : 1;
    constexpr int ROWB = 128;            // bytes per LDS row = 64 bf16 of K
    constexpr int A_BYTES = BM * ROWB;
    constexpr int STAGE = A_BYTES + 256 * ROWB;
    constexpr int WM = BM / 2;           // wave tile rows
    constexpr int IM = WM / 32;          // 32-row blocks per wave
    constexpr int LA = BM / 32;          // A loads per wave per stage
    constexpr int NL = LA + 8;           // loads per wave per stage
    __shared__ __attribute__((aligned(1024))) uint8_t buf0[STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t buf1[STAGE];

    // ---- work item -> (expert, n-tile, m-tile) --------------------------------
    const int NT = g.n_tiles;
    const int W = g.tile_start[g.E] * NT;
    const int L = blockIdx.x;
    const int perx = (W + 7) >> 3;
    const int slot = L >> 3;
    if (slot >= perx) return;
    const int id = (L & 7) * perx + slot;
    if (id >= W) return;
    int lo = 0, hi = g.E - 1;  // largest e with tile_start[e] * NT <= id (a non-empty expert)
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (g.tile_start[mid] * NT <= id) lo = mid; else hi = mid - 1;
    }
    const int e = lo;
    const int t0 = g.tile_start[e];
    const int nte = g.tile_start[e + 1] - t0;
    const int local = id - t0 * NT;
    const int nt = local / nte;
    const int m0 = (local - nt * nte) * BM;
    const int rows = min(BM, g.counts[e] - m0);
    const long long arow0 = (long long)g.offsets[e] + m0;
    const int n0 = nt * (NB == 2 ? 128 : 256);  // first B row (h column for the gated mode)

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // ---- per-lane global offsets of this wave's load instructions -----------
    const long long lda_b = g.lda * 2, ldb_b = g.ldb * 2;
    const int lr = lane >> 3;
    const int lch = (lane & 7) ^ lr;  // logical chunk fetched by this lane (row & 7 == lr)
    const uint8_t *Abase = (const uint8_t *)g.A + arow0 * lda_b;
    uint32_t aoff[LA];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int r = w * (BM / 4) + 8 * i + lr;
        aoff[i] = (uint32_t)((long long)min(r, rows - 1) * lda_b) + lch * 16;
    }
    const uint8_t *Bsrc = (NB == 2 && w >= 2) ? (const uint8_t *)g.B1 : (const uint8_t *)g.B0;
    const uint8_t *Bbase = Bsrc + ((long long)e * g.b_stride + (long long)n0 * g.ldb) * 2;  // row n0 of expert e
    uint32_t boff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // gated: waves 0,1 fetch W1 rows [0,128) of the tile, waves 2,3 the same W3 rows
        const int r = ((NB == 2) ? (w & 1) * 64 : w * 64) + 8 * i + lr;
        boff[i] = (uint32_t)((long long)r * ldb_b) + lch * 16;
    }
    const uint32_t a_lds = w * (BM / 4) * ROWB;       // this wave's A rows in a stage
    const uint32_t b_lds = A_BYTES + w * 64 * ROWB;   // this wave's B rows in a stage
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(buf0));
    const uint32_t lds1 = __builtin_amdgcn_readfirstlane(lds_addr(buf1));
    const uint8_t *Au = uniform_ptr(Abase), *Bu = uniform_ptr(Bbase);

    auto issue = [&](int kt, uint32_t lbuf) {
        const long long ko = (long long)kt * ROWB;
#pragma unroll
        for (int i = 0; i < LA; ++i) lds_dma16(Au + ko, aoff[i], lbuf + a_lds + i * 1024);
#pragma unroll
        for (int i = 0; i < 8; ++i) lds_dma16(Bu + ko, boff[i], lbuf + b_lds + i * 1024);
    };

    // ---- fragment addressing --------------------------------------------------
    const int half = lane >> 5;
    const int r32 = lane & 31;
    const int wm = w & 1, wn = w >> 1;
    const int a_frag = (wm * WM + r32) * ROWB;
    int b_frag[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = (NB == 2) ? ((j & 1) * 128 + wn * 64 + (j >> 1) * 32) : (wn * 128 + j * 32);
        b_frag[j] = A_BYTES + (row + r32) * ROWB;
    }
    int choff[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) choff[ks] = ((ks * 2 + half) ^ (r32 & 7)) << 4;

    f32x16_t acc[IM][4];
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

    // Four k16 sub-steps per stage; the fragments of sub-step ks+1 are read
    // from LDS before the MFMAs of sub-step ks are issued.
    auto compute = [&](const uint8_t *buf) {
        bf16x8_t af[2][IM], bfr[2][4];
#pragma unroll
        for (int i = 0; i < IM; ++i) af[0][i] = *(const bf16x8_t *)(buf + a_frag + i * 32 * ROWB + choff[0]);
#pragma unroll
        for (int j = 0; j < 4; ++j) bfr[0][j] = *(const bf16x8_t *)(buf + b_frag[j] + choff[0]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int c = ks & 1;
            if (ks < 3) {
#pragma unroll
                for (int i = 0; i < IM; ++i)
                    af[c ^ 1][i] = *(const bf16x8_t *)(buf + a_frag + i * 32 * ROWB + choff[ks + 1]);
#pragma unroll
                for (int j = 0; j < 4; ++j) bfr[c ^ 1][j] = *(const bf16x8_t *)(buf + b_frag[j] + choff[ks + 1]);
            }
#pragma unroll
            for (int i = 0; i < IM; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[c][i], bfr[c][j], acc[i][j], 0, 0, 0);
        }
    };

    // ---- main loop: stage kt lives in buf[kt & 1] --------------------------------
    const int KT = g.K / 64;
    issue(0, lds0);
    int kt = 0;
    for (; kt + 2 <= KT; kt += 2) {
        issue(kt + 1, lds1);
        wait_vmcnt<NL>();
        barrier_lds();
        compute(buf0);
        barrier_lds();
        if (kt + 2 < KT) {
            issue(kt + 2, lds0);
            wait_vmcnt<NL>();
        } else {
            wait_vmcnt<0>();
        }
        barrier_lds();
        compute(buf1);
        barrier_lds();
    }
    if (kt < KT) {  // odd K-step count: the last stage is in buf0
        wait_vmcnt<0>();
        barrier_lds();
        compute(buf0);
    }

    // ---- epilogue: lane holds column r32 of each 32x32 block, rows
    // 8*(q/4) + 4*half + q%4 ---------------------------------------------------
    const long long sofs = (long long)e * g.s_stride;
    if constexpr (MODE == MODE_GATED_UP) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int n = n0 + wn * 64 + m * 32 + r32;
            if (n >= g.N) continue;
#pragma unroll
            for (int i = 0; i < IM; ++i)
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int ml = wm * WM + i * 32 + 8 * (q >> 2) + 4 * half + (q & 3);
                    if (ml >= rows) continue;
                    const float v = act_apply_bf(g.act, acc[i][2 * m][q]) * acc[i][2 * m + 1][q];
                    ((uint16_t *)g.C)[(arow0 + ml) * g.ldc + n] = f32_to_bf16(v);
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 128 + j * 32 + r32;
            if (n >= g.N) continue;
            const float bias = g.bias ? g.bias[sofs + n] : 0.0f;
#pragma unroll
            for (int i = 0; i < IM; ++i)
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int ml = wm * WM + i * 32 + 8 * (q >> 2) + 4 * half + (q & 3);
                    if (ml >= rows) continue;
                    if constexpr (MODE == MODE_STD_UP) {
                        const float v = act_apply_bf(g.act, acc[i][j][q] + bias);
                        ((uint16_t *)g.C)[(arow0 + ml) * g.ldc + n] = f32_to_bf16(v);
                    } else {
                        ((float *)g.C)[(arow0 + ml) * g.ldc + n] = acc[i][j][q] + bias;
                    }
                }
        }
    }
}

template <int MODE, int BM>
static hipError_t launch_bf16(const GemmArgs &g, hipStream_t s) {
    long long total = (long long)g.m_tiles_grid * g.n_tiles;
    total = (total + 7) / 8 * 8;
    hipLaunchKernelGGL((grouped_gemm_bf16_kernel<MODE, BM>), dim3((unsigned)total), dim3(256), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_grouped_gemm_bf16(int mode, int bm, const GemmArgs &g, hipStream_t s) {
    if (g.m_tiles_grid <= 0 || g.n_tiles <= 0) return hipSuccess;
#define MOE_BF16_CASE(M, B) \
    if (mode == M && bm == B) return launch_bf16<M, B>(g, s);
    MOE_BF16_CASE(MODE_GATED_UP, 256)
    MOE_BF16_CASE(MODE_STD_UP, 256)
    MOE_BF16_CASE(MODE_DOWN, 256)
    MOE_BF16_CASE(MODE_GATED_UP, 128)
    MOE_BF16_CASE(MODE_STD_UP, 128)
    MOE_BF16_CASE(MODE_DOWN, 128)
#undef MOE_BF16_CASE
    return hipErrorInvalidValue;
}

}  // namespace moe
