// moe_api.hip -- the C ABI of libmoe_mi355x.so (declared in moe_mi355x.h):
// handle lifecycle, weight upload/prepack on the device, and the stage
// orchestration of the MoE-layer forward pass on one HIP stream.
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "moe_internal.h"

using namespace moe;

namespace {
thread_local std::string g_create_error;
inline long long round_up(long long v, long long m) { return (v + m - 1) / m * m; }
// Dropout's scale of the kept values, 1 / (1 - p), rounded as Float32
// arithmetic rounds it: 1 - p, then the quotient (NNlib's dropout on a
// Float32 p; src/experts/standard.jl:49-51).
float drop_scale_f32(float p) {
    volatile float q = 1.0f - p;  // one rounding, not fused into the division
    return 1.0f / q;
}
}  // namespace

struct moe_handle {
    moe_config cfg{};
    // E experts; Er router outputs; k routed slots; ns shared slots of
    // SharedExpertGating; lsh shared experts of the layer (num_shared_experts);
    // kt = lsh + ns + k slots per token
    int E = 0, Er = 0, Er_pad = 0, D = 0, H = 0, Dout = 0, k = 0, ns = 0, lsh = 0, kt = 0;
    // slots per token of the current call (the stride of idx / gates / ranks):
    // kt, or the caller's for moe_forward_routed; kl: slots the Switch loss
    // divides by (the router's index rows: kt - lsh, ExpertChoice's capacity)
    int kc = 0, kl = 0;
    bool given = false, given_probs = false;  // the current call routes on the caller's indices
    uint16_t *ec_sel = nullptr;               // ExpertChoiceGating selections [T][E] (slot + 1 <= 512)
    int D_pad = 0, H_pad = 0, Dout_npad = 0;
    int ct = CT_BF16, wt = WT_BF16;
    bool gated = true;
    int device = 0;
    hipStream_t stream = nullptr;
    // Calls on one handle share its workspace and weights.  The last call
    // that enqueued work without waiting for it did so on last_stream
    // (pending).  Calls that complete a layer (moe_forward_async,
    // moe_decode_async, moe_stage_combine_async) record `done` on their
    // stream after their work (done_rec; moe_decode_async through its last
    // kernel's completion signal): a later call on another stream
    // only waits for it, and moe_destroy synchronises on it, so neither
    // touches a caller stream that may be gone by then.  Between the other
    // stage calls nothing is recorded (a marker between two kernels costs
    // ~5 us of GPU time, at every stage boundary): a call on another stream
    // first records `done` on last_stream, which the caller keeps valid
    // until that next call.
    hipEvent_t done = nullptr;
    hipStream_t last_stream = nullptr;
    bool pending = false;
    bool done_rec = false;
    std::mutex mu;
    std::string err;

    // weights
    float *wr = nullptr, *br = nullptr;
    uint16_t *wsplit = nullptr;  // router weight's three bf16 parts as the fused router's fragment image
    // router noise (moe_set_router_noise): scale, seed, training calls so far;
    // with a noise network its weight [D][Er_pad] and the fragment image of
    // the router and noise weights side by side ([W | Wn], 2 Er columns)
    float noise_scale = 0.0f;
    unsigned long long noise_seed = 0, noise_calls = 0;
    float *wn = nullptr, *wrn = nullptr;
    uint16_t *wsplit_n = nullptr;
    bool noise_net = false;  // the noise network is set (its buffers stay allocated once made)
    // StandardExpert dropout in training (moe_set_expert_dropout)
    float drop_p = 0.0f;
    unsigned long long drop_seed = 0, drop_calls = 0;
    int Ep16 = 0, Dp32 = 0;
    bool router_set = false, has_bias = false;
    std::vector<char> expert_set;
    void *w1 = nullptr, *w3 = nullptr, *w2 = nullptr;
    // bf16 kernel handles: the same matrices as B tile images (the packed rows
    // above stay for the decode caller and the readback)
    void *w1t = nullptr, *w3t = nullptr, *w2t = nullptr;
    float *s1 = nullptr, *s3 = nullptr, *s2 = nullptr;
    float *b1 = nullptr, *b2 = nullptr;
    long long w1_stride = 0, w2_stride = 0;  // elements per expert

    // workspace
    // rows_max: expert-ordered positions (rows of xp, h, y); ent_max: entries
    // (t * kt + slot) of the per-slot arrays.  Equal except for
    // ExpertChoiceGating, whose positions are at most E * min(capacity, T).
    int T_max = 0, nblk_max = 0, rows_max = 0, max_tiles = 0;
    long long ent_max = 0;
    long long act_rows = 0;     // rows of xp and h (bf16 kernel: max_tiles * bm, tile images)
    int ld_y = 0;               // row stride of y (elements)
    int bm = kGemmBM;           // GEMM tile rows of this handle's kernels (scan granule)
    bool bf16_gemm = false;     // bf16 weights and activations: the LDS-DMA MFMA kernel
    float *logits = nullptr, *probs = nullptr, *gates = nullptr, *gate_sorted = nullptr;
    float *lse = nullptr;          // [T] per-token logsumexp of the last routing call
    int last_route_T = -1;         // T of the last routing call
    float *logits_in = nullptr;    // [T][Er] the caller's logits (routing from logits)
    int rb = kRtMinBlock;          // tokens per route block of the last routing call
    int ldc = 0;                   // row stride of blk_counts (E rounded up to 4)
    int rpar = 0;                  // parity of the next routing call's totals buffers
    ScanArgs scan{};               // the last routing call's scan (run by its permute)
    bool keep_rows = false;        // the next routing call writes logits / probs to global memory
    int *idx = nullptr, *rank = nullptr, *blk_counts = nullptr;
    double *blk_zh = nullptr;                 // [nblk][2] per route block z-loss / entropy sums
    int *sup_cnt2 = nullptr;                  // [2][nsup_max][ldc] expert counts per super block (two parities)
    unsigned long long *sup_p2 = nullptr;     // [2][nsup_max][ldc] probability sums per super block, fixed point
    int nsup_max = 0;
    int *counts = nullptr, *offsets = nullptr, *cap = nullptr;
    int2 *tiles = nullptr;
    int *num_tiles = nullptr;
    int *tile_start = nullptr;
    int *item_start = nullptr;  // [E+1] the up GEMM's paired work items (up_pairs)
    long long split_cap = 0;    // floats of split_ws
    float *scalars = nullptr;
    int *perm = nullptr, *pos_of = nullptr;
    void *xp = nullptr, *hbuf = nullptr;
    float *y = nullptr;
    float *split_ws = nullptr;  // partial sums of the GEMMs' split tiles / K ranges
    int ncu = 256;              // compute units: workgroup slots of one GEMM round
    void *x_dev = nullptr;
    float *out_dev = nullptr;

    // AuxiliaryFreeLoss state (src/balancing/auxiliary_free.jl:11-20): bias and
    // momentum on the device, the update counter on the host
    bool aux_free = false, aux_use_comp = true;
    float aux_lr = 0.01f, aux_momentum = 0.9f, aux_cw = 0.001f;
    int aux_update_freq = 1;
    long long aux_counter = 0;
    float *aux_bias = nullptr, *aux_mom = nullptr;

    int last_T = -1, last_training = 0, last_x_bf16 = 0;
    std::vector<void *> allocs;
};

static int fail(moe_handle *h, int code, const std::string &msg) {
    if (h) h->err = msg; else g_create_error = msg;
    return code;
}

#define HIP_TRY(h, call)                                                                   \
    do {                                                                                   \
        hipError_t _e = (call);                                                            \
        if (_e != hipSuccess)                                                              \
            return fail((h), MOE_EHIP, std::string(#call) + ": " + hipGetErrorString(_e)); \
    } while (0)

static int dalloc(moe_handle *h, void **p, size_t bytes) {
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        return fail(h, MOE_EOOM, "hipMalloc(" + std::to_string(bytes) + ") failed: " + hipGetErrorString(e));
    }
    h->allocs.push_back(*p);
    return MOE_OK;
}

static void free_all(moe_handle *h) {
    for (void *p : h->allocs) (void)hipFree(p);
    h->allocs.clear();
}

// Stream order between calls on one handle (see moe_handle::done): before a
// call enqueues on s, s waits for the previous call's work when that went to
// another stream.
static int join_stream(moe_handle *h, hipStream_t s) {
    if (h->pending && h->last_stream != s) {
        hipError_t e = hipSuccess;
        if (!h->done_rec) {
            e = hipEventRecord(h->done, h->last_stream);
            if (e != hipSuccess) return fail(h, MOE_EHIP, std::string("hipEventRecord: ") + hipGetErrorString(e));
            h->done_rec = true;
        }
        e = hipStreamWaitEvent(s, h->done, 0);
        if (e != hipSuccess) return fail(h, MOE_EHIP, std::string("hipStreamWaitEvent: ") + hipGetErrorString(e));
    }
    return MOE_OK;
}
// After a call has enqueued its work on s (and not waited for it); a call
// that completes a layer (record) marks its end with `done`.
static int mark_stream(moe_handle *h, hipStream_t s, bool record = false) {
    h->last_stream = s;
    h->pending = true;
    h->done_rec = false;
    if (record) {
        const hipError_t e = hipEventRecord(h->done, s);
        if (e != hipSuccess) return fail(h, MOE_EHIP, std::string("hipEventRecord: ") + hipGetErrorString(e));
        h->done_rec = true;
    }
    return MOE_OK;
}
// After a call that joined and then synchronised its stream: nothing of the
// handle is in flight.
static void settle(moe_handle *h) {
    h->pending = false;
    h->done_rec = false;
}

// ExpertChoiceGating capacity ceil(Int, T * capacity_factor / E) in Float32
// (src/gating/expert_choice.jl:13), saturated at INT_MAX.
static long long expert_choice_capacity(int T, float cf, int E) {
    const float c = ceilf(((float)T * cf) / (float)E);
    return (c >= 2147483647.0f) ? INT_MAX : (long long)c;
}

static int validate_config(const moe_config *c, std::string &why) {
    if (c->num_experts < 1 || c->num_experts > MOE_MAX_EXPERTS) { why = "num_experts out of range [1, MOE_MAX_EXPERTS (512)]"; return 0; }
    if (c->input_dim < 1 || c->hidden_dim < 1 || c->output_dim < 1) { why = "dimensions must be positive"; return 0; }
    if (c->expert_type != MOE_EXPERT_GATED && c->expert_type != MOE_EXPERT_STANDARD) { why = "unknown expert_type"; return 0; }
    if (c->activation < MOE_ACT_GELU || c->activation > MOE_ACT_IDENTITY) { why = "unknown activation"; return 0; }
    if (c->weight_dtype < MOE_F32 || c->weight_dtype > MOE_FP8_E4M3) { why = "unknown weight_dtype"; return 0; }
    if (c->max_tokens < 1) { why = "max_tokens must be >= 1"; return 0; }
    if (c->drop_tokens && !(c->capacity_factor > 0.0f)) { why = "capacity_factor must be > 0"; return 0; }
    const int k = (c->gate_kind == MOE_GATE_SWITCH) ? 1 : c->top_k;
    // the layer's shared experts (forward_with_shared_experts) run with any
    // gate and loss; the router and its gate see the Er = num_experts - lsh
    // routed experts (src/core/moe_layer.jl:47-50, 158-185)
    const int lsh = c->num_shared_experts;
    if (lsh < 0 || lsh >= c->num_experts) { why = "num_shared_experts must be in [0, num_experts)"; return 0; }
    const int Er = c->num_experts - lsh;
    if (c->gate_kind == MOE_GATE_TOPK || c->gate_kind == MOE_GATE_SWITCH || c->gate_kind == MOE_GATE_SOFT) {
        if (k < 1 || k > Er) { why = "top_k must be in [1, num_experts - num_shared_experts]"; return 0; }
        if (lsh + k > MOE_MAX_TOPK) { why = "num_shared_experts + top_k above MOE_MAX_TOPK (16)"; return 0; }
    } else if (c->gate_kind == MOE_GATE_EXPERT_CHOICE) {
        if (!(c->gate_param > 0.0f)) { why = "ExpertChoiceGating capacity_factor (gate_param) must be > 0"; return 0; }
    } else if (c->gate_kind == MOE_GATE_SHARED) {
        const int ns = c->gate_num_shared;
        if (ns < 0 || ns >= Er) { why = "gate_num_shared must be in [0, num_experts - num_shared_experts)"; return 0; }
        if (k < 1 || k > Er - ns) { why = "top_k must be in [1, num_experts - num_shared_experts - num_shared]"; return 0; }
        if (lsh + ns + k > MOE_MAX_TOPK) { why = "num_shared_experts + num_shared + top_k above MOE_MAX_TOPK (16)"; return 0; }
    } else {
        why = "unknown gate_kind";
        return 0;
    }
    const int slots = (c->gate_kind == MOE_GATE_EXPERT_CHOICE)
                          ? lsh + (int)std::min<long long>(Er, expert_choice_capacity(c->max_tokens, c->gate_param, Er))
                          : k + lsh + (c->gate_kind == MOE_GATE_SHARED ? c->gate_num_shared : 0);
    const long long rows = (long long)c->max_tokens * slots;
    if (rows > INT_MAX / 2) { why = "max_tokens * slots too large"; return 0; }
    return 1;
}

// ============================================================================
// Weight packing kernels (run once per upload).
// ============================================================================
namespace {

// Source element (o, i) of an (out N, in K) matrix as fp32 (fp8 dequantised by
// the per-output-channel scale).
template <int SRC>
__device__ inline float src_elem(const void *src, long long off, const float *scales, int o) {
    if (SRC == MOE_F32) return ((const float *)src)[off];
    if (SRC == MOE_BF16) return bf16_to_f32(((const uint16_t *)src)[off]);
    return fp8e4m3_to_f32(((const uint8_t *)src)[off]) * scales[o];
}

// src (any layout / dtype) -> fp32 [N][K] row-major (K contiguous).
template <int SRC>
__global__ void to_f32_rows_kernel(const void *src, int layout, int N, int K, const float *scales,
                                   float *dst) {
    __shared__ float tile[32][33];
    const int tx = threadIdx.x, ty = threadIdx.y;  // 32 x 8
    const int o0 = blockIdx.x * 32, i0 = blockIdx.y * 32;
    if (layout == MOE_LAYOUT_FLUX_OUT_IN) {  // memory [K][N]
        for (int j = ty; j < 32; j += 8) {
            const int i = i0 + j, o = o0 + tx;
            if (i < K && o < N) tile[j][tx] = src_elem<SRC>(src, (long long)i * N + o, scales, o);
        }
        __syncthreads();
        for (int j = ty; j < 32; j += 8) {
            const int o = o0 + j, i = i0 + tx;
            if (i < K && o < N) dst[(long long)o * K + i] = tile[tx][j];
        }
    } else {  // memory [N][K]
        for (int j = ty; j < 32; j += 8) {
            const int o = o0 + j, i = i0 + tx;
            if (i < K && o < N) dst[(long long)o * K + i] = src_elem<SRC>(src, (long long)o * K + i, scales, o);
        }
    }
}

__device__ inline uint8_t f32_to_fp8e4m3_dev(float v) {
    const uint8_t sign = (__float_as_uint(v) >> 24) & 0x80u;
    const float a = fabsf(v);
    if (!(a < 448.0f)) return sign | 0x7e;  // saturate (and NaN) to max finite
    if (a < 0.015625f) {
        int m = (int)rintf(a * 512.0f);
        return m >= 8 ? (uint8_t)(sign | 0x08) : (uint8_t)(sign | m);
    }
    int ex;
    const float fr = frexpf(a, &ex);
    int e = ex - 1;
    int m = (int)rintf((2.0f * fr - 1.0f) * 8.0f);
    if (m == 8) { m = 0; ++e; }
    if (e > 8 || (e == 8 && m > 6)) return sign | 0x7e;
    return sign | (uint8_t)(((e + 7) << 3) | m);
}

// fp32 [N][K] -> packed [Npad][Kpad] of DST (row o of this expert), one block
// per row.  fp8 rows get scale = max|w| / 448 (1 for an all-zero row).
template <int DST>
__global__ __launch_bounds__(256) void pack_rows_kernel(const float *src, int K, int Kpad, void *dst,
                                                        float *scales) {
    const int o = blockIdx.x;
    const float *row = src + (long long)o * K;
    float inv = 1.0f;
    if (DST == WT_FP8) {
        __shared__ float red[256];
        float m = 0.0f;
        for (int i = threadIdx.x; i < K; i += 256) m = fmaxf(m, fabsf(row[i]));
        red[threadIdx.x] = m;
        __syncthreads();
        for (int s = 128; s > 0; s >>= 1) {
            if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
            __syncthreads();
        }
        const float amax = red[0];
        const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
        if (threadIdx.x == 0) scales[o] = sc;
        inv = sc;
    }
    for (int i = threadIdx.x; i < Kpad; i += 256) {
        const float v = (i < K) ? row[i] : 0.0f;
        if (DST == WT_F32) ((float *)dst)[(long long)o * Kpad + i] = v;
        else if (DST == WT_BF16) ((uint16_t *)dst)[(long long)o * Kpad + i] = f32_to_bf16(v);
        else ((uint8_t *)dst)[(long long)o * Kpad + i] = f32_to_fp8e4m3_dev(v / inv);
    }
}

// fp8 source kept bit-exact when the packed type is fp8 too.
__global__ void fp8_rows_kernel(const uint8_t *src, int layout, int N, int K, int Kpad, uint8_t *dst) {
    const long long total = (long long)N * Kpad;
    for (long long t = blockIdx.x * (long long)blockDim.x + threadIdx.x; t < total;
         t += (long long)gridDim.x * blockDim.x) {
        const int o = (int)(t / Kpad), i = (int)(t % Kpad);
        uint8_t v = 0;
        if (i < K) v = (layout == MOE_LAYOUT_FLUX_OUT_IN) ? src[(long long)i * N + o] : src[(long long)o * K + i];
        dst[t] = v;
    }
}

// rows [n][D] of fp32/bf16 -> compute type with row stride ld (pads
// untouched); bm > 0: bf16 rows of one expert starting at M tile 0 of the
// bf16 kernel's A tile image (row r: row r mod bm of tile r / bm, ld / 32 K
// stages of 64 B, chunk q of a stage at q ^ ((row >> 2) & 3))
__global__ void convert_rows_kernel(const void *src, int src_bf16, int n, int D, int ct, void *dst, int ld, int bm) {
    const long long total = (long long)n * D;
    for (long long t = blockIdx.x * (long long)blockDim.x + threadIdx.x; t < total;
         t += (long long)gridDim.x * blockDim.x) {
        const long long r = t / D, c = t % D;
        const float v = src_bf16 ? bf16_to_f32(((const uint16_t *)src)[t]) : ((const float *)src)[t];
        if (ct == CT_F32) {
            ((float *)dst)[r * ld + c] = v;
        } else if (bm > 0) {
            const long long mt = r / bm, lr = r % bm, st = c / 32;
            const long long q = ((c % 32) / 8) ^ ((lr >> 2) & 3);
            ((uint16_t *)dst)[((mt * (ld / 32) + st) * bm + lr) * 32 + q * 8 + c % 8] = f32_to_bf16(v);
        } else {
            ((uint16_t *)dst)[r * ld + c] = f32_to_bf16(v);
        }
    }
}

// ---- convert_to_moe expert initialisation (src/llama2/conversion.jl:277-331) ----


// Expert e's matrix m (0 = w1, 1 = w2, 2 = w3) from the dense one, rows
// [N][K] fp32 (K = the matrix's input features), per create_single_expert:
// COPY: the dense rows; PERTURB: w .+ randn .* noise_scale; SPLIT: only the
// hidden units [lo, hi) of expert e, lo = e H / E, hi = min((e + 1) H / E,
// H) (w1 / w3 rows, w2 columns), zero elsewhere; RANDOM: randn .* sigma.
__global__ void init_expert_kernel(const float *__restrict__ src, int N, int K, int strategy, int m, int e, int E,
                                   int H, float noise_scale, float sigma, unsigned long long seed,
                                   float *__restrict__ dst) {
#pragma clang fp contract(off)
    const long long total = (long long)N * K;
    const int lo = (int)(((long long)e * H) / E);
    const int hi = min((int)(((long long)(e + 1) * H) / E), H);
    const unsigned long long stream = (unsigned long long)e * 3 + m;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        float v = src ? src[i] : 0.0f;
        if (strategy == MOE_INIT_PERTURB) {
            v = v + init_normal(seed, stream, (unsigned long long)i) * noise_scale;
        } else if (strategy == MOE_INIT_RANDOM) {
            v = init_normal(seed, stream, (unsigned long long)i) * sigma;
        } else if (strategy == MOE_INIT_SPLIT) {
            const int hu = (m == 1) ? (int)(i % K) : (int)(i / K);  // the hidden unit of this element
            if (hu < lo || hu >= hi) v = 0.0f;
        }
        dst[i] = v;
    }
}

// Packed [Npad][Kpad] rows of expert weights back to an (N out, K in) matrix
// in the caller's layout and the packed dtype (bytes per element esz).
__global__ void unpack_rows_kernel(const uint8_t *__restrict__ src, int esz, int N, int K, int Kpad, int layout,
                                   uint8_t *__restrict__ dst) {
    const long long total = (long long)N * K;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const int o = (int)(i / K), k = (int)(i % K);
        const long long d = (layout == MOE_LAYOUT_FLUX_OUT_IN) ? (long long)k * N + o : i;
        const long long sidx = (long long)o * Kpad + k;
        for (int b = 0; b < esz; ++b) dst[d * esz + b] = src[sidx * esz + b];
    }
}

}  // namespace

static bool is_device_ptr(const void *p) {
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice;
}

// Make a device copy of `bytes` at p unless p already is device memory.
static int stage_to_device(moe_handle *h, const void *p, size_t bytes, const void **dptr, void **owned) {
    *owned = nullptr;
    if (is_device_ptr(p)) {
        *dptr = p;
        return MOE_OK;
    }
    void *d = nullptr;
    hipError_t e = hipMalloc(&d, bytes);
    if (e != hipSuccess) return fail(h, MOE_EOOM, std::string("staging allocation failed: ") + hipGetErrorString(e));
    e = hipMemcpy(d, p, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return fail(h, MOE_EHIP, std::string("staging copy failed: ") + hipGetErrorString(e));
    }
    *dptr = d;
    *owned = d;
    return MOE_OK;
}

// fp32 rows [N][K] (device) -> the packed dtype of the handle, [N][Kpad]
// (fp8: per-row scales), on the handle's stream.
static hipError_t pack_f32_rows(moe_handle *h, const float *tmp, int N, int K, int Kpad, void *dst, float *scales) {
    if (h->wt == WT_F32)
        hipLaunchKernelGGL(pack_rows_kernel<WT_F32>, dim3(N), dim3(256), 0, h->stream, tmp, K, Kpad, dst, scales);
    else if (h->wt == WT_BF16)
        hipLaunchKernelGGL(pack_rows_kernel<WT_BF16>, dim3(N), dim3(256), 0, h->stream, tmp, K, Kpad, dst, scales);
    else
        hipLaunchKernelGGL(pack_rows_kernel<WT_FP8>, dim3(N), dim3(256), 0, h->stream, tmp, K, Kpad, dst, scales);
    return hipGetLastError();
}

// Source matrix (any layout / dtype, host or device) -> fp32 rows [N][K] in
// a new device buffer *out (the caller frees it).
static int load_f32_rows(moe_handle *h, int layout, int src_dtype, const void *src, const float *src_scales, int N,
                         int K, float **out) {
    *out = nullptr;
    const size_t esz = src_dtype == MOE_F32 ? 4 : (src_dtype == MOE_BF16 ? 2 : 1);
    const void *dsrc = nullptr, *dsc = nullptr;
    void *own_src = nullptr, *own_sc = nullptr;
    int r = stage_to_device(h, src, esz * (size_t)N * K, &dsrc, &own_src);
    if (r != MOE_OK) return r;
    if (src_dtype == MOE_FP8_E4M3) {
        r = stage_to_device(h, src_scales, sizeof(float) * (size_t)N, &dsc, &own_sc);
        if (r != MOE_OK) {
            if (own_src) (void)hipFree(own_src);
            return r;
        }
    }
    float *tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, sizeof(float) * (size_t)N * K);
    if (e == hipSuccess) {
        dim3 grid((N + 31) / 32, (K + 31) / 32), block(32, 8);
        if (src_dtype == MOE_F32)
            hipLaunchKernelGGL(to_f32_rows_kernel<MOE_F32>, grid, block, 0, h->stream, dsrc, layout, N, K,
                               (const float *)dsc, tmp);
        else if (src_dtype == MOE_BF16)
            hipLaunchKernelGGL(to_f32_rows_kernel<MOE_BF16>, grid, block, 0, h->stream, dsrc, layout, N, K,
                               (const float *)dsc, tmp);
        else
            hipLaunchKernelGGL(to_f32_rows_kernel<MOE_FP8_E4M3>, grid, block, 0, h->stream, dsrc, layout, N, K,
                               (const float *)dsc, tmp);
        e = hipGetLastError();
        hipError_t e2 = hipStreamSynchronize(h->stream);
        if (e == hipSuccess) e = e2;
    }
    if (own_src) (void)hipFree(own_src);
    if (own_sc) (void)hipFree(own_sc);
    if (e != hipSuccess) {
        if (tmp) (void)hipFree(tmp);
        return fail(h, MOE_EHIP, std::string("weight load failed: ") + hipGetErrorString(e));
    }
    *out = tmp;
    return MOE_OK;
}

// Pack one (N out, K in) matrix of expert e into dst [Npad][Kpad] (+ scales).
static int pack_matrix(moe_handle *h, int layout, int src_dtype, const void *src, const float *src_scales,
                       int N, int K, int Kpad, void *dst_expert, float *dst_scales) {
    const size_t esz = src_dtype == MOE_F32 ? 4 : (src_dtype == MOE_BF16 ? 2 : 1);
    const void *dsrc = nullptr;
    void *own_src = nullptr, *own_sc = nullptr;
    const void *dsc = nullptr;
    int r = stage_to_device(h, src, esz * (size_t)N * K, &dsrc, &own_src);
    if (r != MOE_OK) return r;
    if (src_dtype == MOE_FP8_E4M3) {
        r = stage_to_device(h, src_scales, sizeof(float) * (size_t)N, &dsc, &own_sc);
        if (r != MOE_OK) { if (own_src) (void)hipFree(own_src); return r; }
    }
    hipError_t e = hipSuccess;
    if (src_dtype == MOE_FP8_E4M3 && h->wt == WT_FP8) {
        hipLaunchKernelGGL(fp8_rows_kernel, dim3(1024), dim3(256), 0, h->stream, (const uint8_t *)dsrc, layout, N,
                           K, Kpad, (uint8_t *)dst_expert);
        e = hipGetLastError();
        if (e == hipSuccess)
            e = hipMemcpyAsync(dst_scales, dsc, sizeof(float) * N, hipMemcpyDeviceToDevice, h->stream);
    } else {
        float *tmp = nullptr;
        e = hipMalloc(&tmp, sizeof(float) * (size_t)N * K);
        if (e == hipSuccess) {
            dim3 grid((N + 31) / 32, (K + 31) / 32), block(32, 8);
            if (src_dtype == MOE_F32)
                hipLaunchKernelGGL(to_f32_rows_kernel<MOE_F32>, grid, block, 0, h->stream, dsrc, layout, N, K,
                                   (const float *)dsc, tmp);
            else if (src_dtype == MOE_BF16)
                hipLaunchKernelGGL(to_f32_rows_kernel<MOE_BF16>, grid, block, 0, h->stream, dsrc, layout, N, K,
                                   (const float *)dsc, tmp);
            else
                hipLaunchKernelGGL(to_f32_rows_kernel<MOE_FP8_E4M3>, grid, block, 0, h->stream, dsrc, layout, N, K,
                                   (const float *)dsc, tmp);
            e = hipGetLastError();
            if (e == hipSuccess) e = pack_f32_rows(h, tmp, N, K, Kpad, dst_expert, dst_scales);
            hipError_t e2 = hipStreamSynchronize(h->stream);
            if (e == hipSuccess) e = e2;
            (void)hipFree(tmp);
        }
    }
    hipError_t e3 = hipStreamSynchronize(h->stream);
    if (e == hipSuccess) e = e3;
    if (own_src) (void)hipFree(own_src);
    if (own_sc) (void)hipFree(own_sc);
    if (e != hipSuccess) return fail(h, MOE_EHIP, std::string("weight packing failed: ") + hipGetErrorString(e));
    return MOE_OK;
}

// ============================================================================
// Forward orchestration
// ============================================================================
static int check_ready(moe_handle *h) {
    if (!h->router_set) return fail(h, MOE_ENOTREADY, "router weights not set (moe_set_router)");
    for (int e = 0; e < h->E; ++e)
        if (!h->expert_set[e]) return fail(h, MOE_ENOTREADY, "expert " + std::to_string(e) + " has no weights");
    return MOE_OK;
}

static int m_tiles_for(const moe_handle *h, int T) {
    long long mt = (long long)T * h->kc / h->bm + h->E;
    if (mt > h->max_tiles) mt = h->max_tiles;
    return (int)mt;
}

enum { PERMUTE_NONE = 0, PERMUTE_INDEX = 1, PERMUTE_ROWS = 2 };

// The capacity constraint runs in forward_standard only
// (src/core/moe_layer.jl:142-147), not in forward_with_shared_experts.
static bool drop_active(const moe_handle *h) { return h->cfg.drop_tokens && h->lsh == 0; }
// AuxiliaryFreeLoss bias / momentum length: the router's experts, or, with
// shared experts of the layer, all num_experts: update_bias! then receives
// the gate's ids shifted by num_shared_experts (src/core/moe_layer.jl:172,
// 182), up to num_experts, and indexes the bias with them
static int aux_free_len(const moe_handle *h) { return h->lsh > 0 ? h->E : h->Er; }

static int run_permute(moe_handle *h, const void *x_dev, int x_bf16, int T, int training, int mode, hipStream_t s) {
    PermuteArgs pa{};
    pa.x = x_dev; pa.x_bf16 = x_bf16; pa.T = T; pa.D = h->D; pa.ld_xp = h->D_pad; pa.kt = h->kc; pa.E = h->E;
    pa.ct = h->ct; pa.idx = h->idx; pa.gates = h->gates; pa.rank = h->rank; pa.rb = h->rb; pa.s = h->scan;
    pa.renorm = (training && drop_active(h)) ? 1 : 0;
    pa.perm = h->perm; pa.pos_of = h->pos_of; pa.gate_sorted = h->gate_sorted; pa.xp = h->xp;
    pa.tiled = h->bf16_gemm ? 1 : 0; pa.bm = h->bm; pa.ktt = h->D_pad / 32;
    pa.copy_rows = mode == PERMUTE_ROWS ? 1 : 0;
    HIP_TRY(h, launch_permute(pa, s));
    return MOE_OK;
}

// logits -> gating -> scan -> permute (mode PERMUTE_*).  A forward
// (compute_logits) with an AuxiliaryFreeLoss gates on logits + its bias
// (src/core/moe_layer.jl:137-140) in a second route pass and, when training,
// counts one compute_loss call for the bias update (auxiliary_free.jl:36-40).
// Workgroup slots of the bf16 GEMMs (their tail split plans its last round
// over them): 128-row tiles run two workgroups per CU.
static int gemm_slots(const moe_handle *h) { return h->bm == 128 ? 2 * h->ncu : h->ncu; }

// n-tiles of the up GEMM
static int up_ntiles(const moe_handle *h) {
    return h->bf16_gemm ? h->H_pad / (h->gated ? 128 : 256) : h->H_pad / kGemmBN;
}
// The bf16 up GEMM on 256-row tiles with an even n-tile count pairs an
// expert's last M tile of at most 128 rows with two n-tiles (item_start).
static bool up_pairs(const moe_handle *h) { return h->bf16_gemm && h->bm == 256 && up_ntiles(h) % 2 == 0; }

static int run_routing(moe_handle *h, const void *x_dev, int x_bf16, int T, int training, bool compute_logits,
                       int permute_mode, float *loss_dev, hipStream_t s) {
    const bool aux = compute_logits && h->aux_free && !h->given;
    // forward_standard gates on logits .+ bias (src/core/moe_layer.jl:137-140);
    // forward_with_shared_experts gates on the plain logits and only hands the
    // (shifted) ids to the loss (:168-182)
    const bool aux_gate = aux && h->lsh == 0;
    const bool ec = h->cfg.gate_kind == MOE_GATE_EXPERT_CHOICE && !h->given;
    bool aux_update = false;
    if (aux && training) {
        ++h->aux_counter;
        aux_update = h->aux_counter % h->aux_update_freq == 0;
    }
    RtArgs A{};
    RouteArgs &ra = A.r;
    if (compute_logits) {
        RouterArgs &rg = A.g;
        rg.x = x_dev; rg.x_bf16 = x_bf16; rg.T = T; rg.D = h->D; rg.Er = h->Er; rg.Ep = h->Ep16; rg.Dp = h->Dp32;
        rg.ws = h->wsplit;
        ra.bias = h->has_bias ? h->br : nullptr;
        if (training && h->noise_scale > 0.0f) {
            // router noise (src/core/router.jl:32-41), one stream of the
            // generator per training call
            A.noise_scale = h->noise_scale;
            A.noise_seed = h->noise_seed;
            A.noise_call = h->noise_calls++;
            if (h->noise_net) {
                A.noise_net = 1;
                rg.Er = 2 * h->Er;
                rg.ws = h->wsplit_n;
            }
        }
    } else {
        ra.part = h->logits_in;  // the caller's logits
        ra.bias = nullptr;
    }
    ra.logits = h->logits; ra.T = T; ra.Er = h->Er; ra.E = h->Er; ra.Eh = h->E;
    ra.gate_kind = h->cfg.gate_kind; ra.lsh = h->lsh;
    ra.k = h->k; ra.ns = h->ns; ra.kt = h->kc; ra.probs = h->probs; ra.idx = h->idx; ra.gates = h->gates;
    ra.soft_lambda = h->cfg.gate_param; ra.given = h->given; ra.given_probs = h->given_probs;
    // the call's super-block totals (parity rpar); the router zeroes the
    // other parity's for the next call.  rpar flips once the router kernel
    // is launched: a call that fails before that leaves the next one on the
    // same (still clear) parity.
    const int par = h->rpar;
    ra.rank = h->rank; ra.blk_counts = h->blk_counts; ra.ldc = h->ldc; ra.blk_zh = h->blk_zh;
    ra.lse = h->lse;
    h->last_route_T = T;
    ra.nsup_max = h->nsup_max;
    ra.sup_cnt = h->sup_cnt2 + (size_t)par * h->nsup_max * h->ldc;
    ra.clr_sup = h->sup_cnt2 + (size_t)(par ^ 1) * h->nsup_max * h->ldc;
    ra.sup_p = h->sup_p2 + (size_t)par * h->nsup_max * h->ldc;
    ra.clr_supp = h->sup_p2 + (size_t)(par ^ 1) * h->nsup_max * h->ldc;
    ScanArgs sa{};
    sa.blk_counts = h->blk_counts; sa.ldc = h->ldc; sa.blk_zh = h->blk_zh;
    sa.sup_cnt = ra.sup_cnt; sa.sup_p = ra.sup_p;
    sa.T = T; sa.E = h->E; sa.kt = h->kc;
    sa.training = training; sa.drop = drop_active(h); sa.z_enabled = h->cfg.z_loss_weight > 0.0f;
    sa.Np = h->Er; sa.lsh = h->lsh; sa.kl = h->kl; sa.ec_empty = (ec && h->lsh > 0) ? 1 : 0;
    sa.capacity_factor = h->cfg.capacity_factor; sa.alpha = h->cfg.balance_alpha; sa.beta = h->cfg.z_loss_weight;
    sa.bm = h->bm; sa.tile_start = h->tile_start; sa.counts = h->counts; sa.offsets = h->offsets;
    sa.item_start = up_pairs(h) ? h->item_start : nullptr; sa.pair_nt = up_ntiles(h);
    sa.cap_out = h->cap; sa.tiles = h->tiles; sa.num_tiles = h->num_tiles; sa.scalars = h->scalars;
    sa.loss_out = loss_dev;
    sa.aux_free = aux; sa.aux_use_comp = h->aux_use_comp; sa.aux_update = aux_update;
    sa.aux_cw = h->aux_cw; sa.aux_lr = h->aux_lr; sa.aux_momentum = h->aux_momentum;
    sa.aux_bias = h->aux_bias; sa.aux_mom = h->aux_mom;
    // logits / probs rows in global memory: for the caller, and for the
    // ExpertChoiceGating kernels that read them
    A.store_rows = (h->keep_rows || ec || !compute_logits) ? 1 : 0;
    h->keep_rows = false;
    if (aux_gate) {
        // probabilities pass on the logits, gating pass on logits + the loss's bias
        A.npass = 2;
        A.aux_bias = h->aux_bias;
        ra.out_mask = ROUTE_OUT_PROBS | ROUTE_OUT_GATING;
    } else {
        A.npass = 1;
        ra.out_mask = ec ? ROUTE_OUT_PROBS : (ROUTE_OUT_PROBS | ROUTE_OUT_GATING);
    }
    A.ncu = h->ncu;
    {
        const hipError_t e = launch_router(A, &h->rb, s);
        if (e != hipSuccess) {
            // whether the kernel ran is unknown (a launch error may come from
            // earlier work): clear both parities' totals so that no later
            // call adds onto stale counts
            (void)hipMemsetAsync(h->sup_cnt2, 0, sizeof(int) * 2 * (size_t)h->nsup_max * h->ldc, s);
            (void)hipMemsetAsync(h->sup_p2, 0, sizeof(unsigned long long) * 2 * (size_t)h->nsup_max * h->ldc, s);
            return fail(h, MOE_EHIP, std::string("launch_router: ") + hipGetErrorString(e));
        }
    }
    h->rpar = par ^ 1;
    if (ec) {
        // the experts' choices give the slots, the stable ranks and the
        // per-block histogram
        HIP_TRY(h, launch_expert_choice(h->logits, h->probs, T, h->Er, h->lsh, h->kl, h->kc, h->ec_sel, h->idx,
                                        h->gates, h->rank, h->blk_counts, h->ldc, ra.sup_cnt, h->rb, s));
    }
    // the scan runs in the permute kernel (its workgroups are the route blocks)
    sa.nblk = (T + h->rb - 1) / h->rb;
    sa.nsup = (sa.nblk + kSuper - 1) / kSuper;
    h->scan = sa;
    if (permute_mode != PERMUTE_NONE) return run_permute(h, x_dev, x_bf16, T, training, permute_mode, s);
    return MOE_OK;
}

static GemmArgs up_args(moe_handle *h, int mt_grid, bool training) {
    GemmArgs g{};
    if (training && !h->gated && h->drop_p > 0.0f) {
        // Dropout(p) on h in training (src/experts/standard.jl:49-51), one
        // stream of the generator per call
        g.drop_p = h->drop_p;
        // 1 / (1 - p) in Float32 arithmetic, as NNlib's dropout computes it
        // for the Float32 p of StandardExpert's Dropout (two fp32 roundings)
        g.drop_scale = drop_scale_f32(h->drop_p);
        g.drop_seed = h->drop_seed;
        g.drop_call = h->drop_calls++;
    }
    g.A = h->xp; g.lda = h->D_pad;
    g.B0 = h->bf16_gemm ? h->w1t : h->w1;
    g.B1 = h->gated ? (h->bf16_gemm ? h->w3t : h->w3) : nullptr;
    g.b_stride = h->w1_stride; g.ldb = h->D_pad;
    g.s0 = h->s1; g.s1 = h->s3; g.bias = h->gated ? nullptr : h->b1; g.s_stride = h->H_pad;
    g.N = h->H; g.K = h->D_pad; g.C = h->hbuf; g.ldc = h->H_pad;
    g.tiles = h->tiles; g.num_tiles = h->num_tiles; g.counts = h->counts; g.offsets = h->offsets;
    g.tile_start = h->tile_start; g.E = h->E;
    g.item_start = up_pairs(h) ? h->item_start : nullptr;
    // bf16 kernel on 256-row tiles (one workgroup per CU, whose last round
    // would leave most CUs idle for a whole tile): the tail split of that
    // round, folded by fold_up_kernel
    g.ksplit = (h->bf16_gemm && h->split_ws && h->bm == 256) ? kUpSplitMax : 1;
    g.ncu = h->bf16_gemm ? gemm_slots(h) : h->ncu; g.split_ws = h->split_ws; g.split_cap = h->split_cap;
    g.m_tiles_grid = mt_grid; g.act = h->cfg.activation;
    // bf16 kernel: 128 h columns (gated, W1 and W3 rows) or 256 rows per tile
    g.n_tiles = up_ntiles(h);
    return g;
}

// The most K ranges a tile of the bf16 down GEMM may be split into: the
// tiles of the last, partial round of ncu workgroups are split (tail_split),
// and fold_split_kernel adds their partials to y in range order.
static int down_ksplit(const moe_handle *h) { return h->bf16_gemm ? kDownSplitMax : 1; }


static GemmArgs down_args(moe_handle *h, int mt_grid, int ksplit, bool y_f32) {
    GemmArgs g{};
    g.A = h->hbuf; g.lda = h->H_pad;
    g.B0 = h->bf16_gemm ? h->w2t : h->w2; g.B1 = nullptr;
    g.b_stride = h->w2_stride; g.ldb = h->H_pad;
    g.s0 = h->s2; g.s1 = nullptr; g.bias = h->gated ? nullptr : h->b2; g.s_stride = h->Dout_npad;
    g.N = h->Dout; g.K = h->H_pad; g.C = h->y; g.ldc = h->ld_y;
    g.c_bf16 = (h->bf16_gemm && !y_f32) ? 1 : 0;  // the bf16-kernel paths keep y in bf16
    g.ksplit = ksplit; g.ncu = h->bf16_gemm ? gemm_slots(h) : h->ncu;
    g.split_ws = h->split_ws; g.split_cap = h->split_cap;
    g.tiles = h->tiles; g.num_tiles = h->num_tiles; g.counts = h->counts; g.offsets = h->offsets;
    g.tile_start = h->tile_start; g.E = h->E;
    g.m_tiles_grid = mt_grid; g.act = h->cfg.activation;
    g.n_tiles = h->bf16_gemm ? h->Dout_npad / 256 : h->Dout_npad / kGemmBN;
    return g;
}

// The expert up GEMM (W1/W3 or W1 + activation) and the down GEMM (W2) over
// mt_grid M tiles: the LDS-DMA kernel for bf16 and fp8 weights (bf16
// activations), the register-staged fp32 kernel for fp32 weights.
static hipError_t launch_up(moe_handle *h, int mt_grid, hipStream_t s, bool training = false) {
    const int mode = h->gated ? MODE_GATED_UP : MODE_STD_UP;
    const GemmArgs g = up_args(h, mt_grid, training);
    if (h->bf16_gemm) return launch_grouped_gemm_bf16(mode, h->bm, h->wt == WT_FP8, g, s);
    return launch_grouped_gemm_f32(mode, g, s);
}

// y_f32: write y in fp32 also on the bf16-kernel path (moe_expert_forward
// hands y back as fp32); the layer paths keep it in bf16 there.
static hipError_t launch_down(moe_handle *h, int mt_grid, hipStream_t s, int ksplit, bool y_f32 = false) {
    if (h->bf16_gemm) {
        const GemmArgs g = down_args(h, mt_grid, ksplit, y_f32);
        hipError_t e = launch_grouped_gemm_bf16(MODE_DOWN, h->bm, h->wt == WT_FP8, g, s);
        if (e == hipSuccess && ksplit > 1) e = launch_fold_split(h->bm, g, s);
        return e;
    }
    return launch_grouped_gemm_f32(MODE_DOWN, down_args(h, mt_grid, 1, true), s);
}

static int run_experts(moe_handle *h, int T, int training, hipStream_t s) {
    const int mt = m_tiles_for(h, T);
    HIP_TRY(h, launch_up(h, mt, s, training != 0));
    HIP_TRY(h, launch_down(h, mt, s, down_ksplit(h)));
    return MOE_OK;
}

static int run_combine(moe_handle *h, int T, float *out_dev, hipStream_t s) {
    CombineArgs c{};
    c.y = h->y; c.ld_y = h->ld_y; c.y_bf16 = h->bf16_gemm ? 1 : 0;
    c.idx = h->idx; c.pos_of = h->pos_of; c.gates = h->gates;
    c.T = T; c.D = h->Dout; c.kt = h->kc; c.lsh = h->lsh; c.out = out_dev;
    HIP_TRY(h, launch_combine(c, s));
    return MOE_OK;
}

// Slots of a call routed by the handle's own gate: kt per token, and the
// Switch loss's index rows (ExpertChoiceGating: its capacity
// ceil(Int, T * capacity_factor / E) in Float32, expert_choice.jl:13).
static int begin_call(moe_handle *h, int T) {
    h->given = false;
    h->given_probs = false;
    h->kc = h->kt;
    h->kl = h->kt - h->lsh;
    if (h->cfg.gate_kind == MOE_GATE_EXPERT_CHOICE) {
        // the call's min(capacity, E) <= kt = min(capacity at max_tokens, E)
        // slots are filled, the rest stay empty; the Switch loss counts all
        // capacity rows of the reference's (capacity, T) index matrix
        h->kl = (int)expert_choice_capacity(T, h->cfg.gate_param, h->Er);
    }
    return MOE_OK;
}

static int forward_locked(moe_handle *h, const void *x_dev, int x_dtype, int T, int training, float *out_dev,
                          float *loss_dev, hipStream_t s) {
    int r = check_ready(h);
    if (r != MOE_OK) return r;
    if (x_dtype != MOE_F32 && x_dtype != MOE_BF16) return fail(h, MOE_EINVAL, "x_dtype must be F32 or BF16");
    if (T < 1 || T > h->T_max) return fail(h, MOE_EINVAL, "T must be in [1, max_tokens]");
    if (!x_dev || !out_dev) return fail(h, MOE_EINVAL, "null buffer");
    if (!h->given) {
        r = begin_call(h, T);
        if (r != MOE_OK) return r;
    }
    const int xb = x_dtype == MOE_BF16;
    r = run_routing(h, x_dev, xb, T, training, true, PERMUTE_ROWS, loss_dev, s);
    if (r != MOE_OK) return r;
    r = run_experts(h, T, training, s);
    if (r != MOE_OK) return r;
    r = run_combine(h, T, out_dev, s);
    if (r != MOE_OK) return r;
    h->last_T = T;
    h->last_training = training;
    h->last_x_bf16 = xb;
    return MOE_OK;
}

static int ensure_io_buffers(moe_handle *h) {
    if (!h->x_dev) {
        int r = dalloc(h, &h->x_dev, sizeof(float) * (size_t)h->T_max * h->D);
        if (r != MOE_OK) return r;
    }
    if (!h->out_dev) {
        int r = dalloc(h, (void **)&h->out_dev, sizeof(float) * (size_t)h->T_max * h->Dout);
        if (r != MOE_OK) return r;
    }
    return MOE_OK;
}

// ============================================================================
// C ABI
// ============================================================================
extern "C" {

int moe_abi_version(void) { return MOE_ABI_VERSION; }

const char *moe_last_error(const moe_handle *h) { return h ? h->err.c_str() : g_create_error.c_str(); }

int moe_router_outputs(const moe_handle *h) { return h ? h->Er : -1; }
int moe_slots_per_token(const moe_handle *h) { return h ? h->kt : -1; }

int moe_create(const moe_config *cfg, moe_handle **out) {
    if (!cfg || !out) return fail(nullptr, MOE_EINVAL, "null argument");
    *out = nullptr;
    std::string why;
    if (!validate_config(cfg, why)) return fail(nullptr, MOE_EINVAL, why);
    moe_handle *h = new moe_handle();
    h->cfg = *cfg;
    h->E = cfg->num_experts;
    h->lsh = cfg->num_shared_experts;
    h->Er = cfg->num_experts - h->lsh;
    h->Er_pad = (int)round_up(h->Er, 8);
    h->D = cfg->input_dim;
    h->H = cfg->hidden_dim;
    h->Dout = cfg->output_dim;
    h->k = (cfg->gate_kind == MOE_GATE_SWITCH || cfg->gate_kind == MOE_GATE_EXPERT_CHOICE) ? 1 : cfg->top_k;
    h->ns = (cfg->gate_kind == MOE_GATE_SHARED) ? cfg->gate_num_shared : 0;
    h->kt = (cfg->gate_kind == MOE_GATE_EXPERT_CHOICE)
                ? h->lsh + (int)std::min<long long>(h->Er, expert_choice_capacity(cfg->max_tokens, cfg->gate_param, h->Er))
                : h->lsh + h->ns + h->k;
    h->kc = h->kt;
    h->kl = h->kt - h->lsh;
    h->D_pad = (int)round_up(h->D, kKPad);
    // N of the up GEMM, K of the down GEMM: a whole number of up-GEMM tiles
    h->H_pad = (int)round_up(h->H, cfg->expert_type == MOE_EXPERT_GATED ? kNPadGated : kNPad);
    h->Dout_npad = (int)round_up(h->Dout, kNPad);
    h->ct = (cfg->weight_dtype == MOE_F32) ? CT_F32 : CT_BF16;
    h->wt = (cfg->weight_dtype == MOE_F32) ? WT_F32 : (cfg->weight_dtype == MOE_BF16 ? WT_BF16 : WT_FP8);
    h->gated = cfg->expert_type == MOE_EXPERT_GATED;
    h->expert_set.assign(h->E, 0);
    (void)hipGetDevice(&h->device);
    {
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, h->device) == hipSuccess && cu > 0)
            h->ncu = cu;
    }

    auto cleanup = [&](int code) {
        g_create_error = h->err;
        free_all(h);
        if (h->done) (void)hipEventDestroy(h->done);
        if (h->stream) (void)hipStreamDestroy(h->stream);
        delete h;
        return code;
    };
    if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess) {
        h->err = "hipStreamCreate failed";
        return cleanup(MOE_EHIP);
    }
    // ordering between streams of this device only: no system-scope fence
    // (a cache write-back each time it is recorded)
    if (hipEventCreateWithFlags(&h->done, hipEventDisableTiming | hipEventDisableSystemFence) != hipSuccess) {
        h->err = "hipEventCreate failed";
        return cleanup(MOE_EHIP);
    }
    int r = MOE_OK;
    auto A = [&](void **p, size_t bytes) {
        if (r == MOE_OK) r = dalloc(h, p, bytes);
    };
    const size_t wsz = (h->wt == WT_F32) ? 4 : (h->wt == WT_BF16 ? 2 : 1);
    const size_t asz = (h->ct == CT_F32) ? 4 : 2;
    h->w1_stride = (long long)h->H_pad * h->D_pad;
    h->w2_stride = (long long)h->Dout_npad * h->H_pad;
    const size_t wr_bytes = sizeof(float) * (size_t)h->D * h->Er_pad;
    A((void **)&h->wr, wr_bytes);
    A((void **)&h->br, sizeof(float) * (size_t)h->Er_pad);
    h->Ep16 = (int)round_up(h->Er, 16);
    h->Dp32 = (int)round_up(h->D, 32);
    A((void **)&h->wsplit, sizeof(uint16_t) * 3 * (size_t)h->Ep16 * h->Dp32);
    A(&h->w1, wsz * (size_t)h->E * h->w1_stride);
    if (h->gated) A(&h->w3, wsz * (size_t)h->E * h->w1_stride);
    A(&h->w2, wsz * (size_t)h->E * h->w2_stride);
    if (h->wt == WT_FP8) {
        A((void **)&h->s1, sizeof(float) * (size_t)h->E * h->H_pad);
        if (h->gated) A((void **)&h->s3, sizeof(float) * (size_t)h->E * h->H_pad);
        A((void **)&h->s2, sizeof(float) * (size_t)h->E * h->Dout_npad);
    }
    if (!h->gated) {
        A((void **)&h->b1, sizeof(float) * (size_t)h->E * h->H_pad);
        A((void **)&h->b2, sizeof(float) * (size_t)h->E * h->Dout_npad);
    }
    h->T_max = cfg->max_tokens;
    h->nblk_max = (h->T_max + kRtMinBlock - 1) / kRtMinBlock;
    h->ent_max = (long long)h->T_max * h->kt;
    h->rows_max = h->T_max * h->kt;
    if (cfg->gate_kind == MOE_GATE_EXPERT_CHOICE) {
        // each routed expert takes at most min(capacity, T) tokens; every
        // token holds the lsh shared experts
        const long long cmax = std::min<long long>(
            expert_choice_capacity(h->T_max, cfg->gate_param, h->Er), h->T_max);
        h->rows_max = (int)std::min<long long>(h->rows_max, (long long)h->T_max * h->lsh + (long long)h->Er * cmax);
    }
    h->bf16_gemm = h->ct == CT_BF16 && (h->wt == WT_BF16 || h->wt == WT_FP8);
    // 256-row tiles for a few large experts (at most 16, averaging at least 384
    // rows at max_tokens); 128-row tiles, two workgroups per CU, for many or
    // small ones (fine-grained MoE layers: skewed counts, short K), and for
    // standard experts with fp8 weights (on 256-row tiles their up GEMM's
    // accumulators, fp8 stage bytes and epilogue scales exceed the registers)
    const bool fp8_std = h->wt == WT_FP8 && !h->gated;
    h->bm = (h->bf16_gemm && !fp8_std && h->E <= 16 && (long long)h->rows_max >= 384LL * h->E) ? 256 : kGemmBM;
    h->max_tiles = h->rows_max / h->bm + h->E + 1;
    // bf16 kernel: xp and h are A tile images of up to max_tiles M tiles
    h->act_rows = h->bf16_gemm ? (long long)h->max_tiles * h->bm : h->rows_max;
    if (h->bf16_gemm) {
        A(&h->w1t, wsz * (size_t)h->E * h->w1_stride);
        if (h->gated) A(&h->w3t, wsz * (size_t)h->E * h->w1_stride);
        A(&h->w2t, wsz * (size_t)h->E * h->w2_stride);
    }
    const size_t T = (size_t)h->T_max, E = (size_t)h->E, nent = (size_t)h->ent_max;
    A((void **)&h->logits, sizeof(float) * T * h->Er);
    A((void **)&h->logits_in, sizeof(float) * T * h->Er);
    A((void **)&h->probs, sizeof(float) * T * h->Er);
    A((void **)&h->lse, sizeof(float) * T);
    A((void **)&h->idx, sizeof(int) * nent);
    A((void **)&h->gates, sizeof(float) * nent);
    A((void **)&h->rank, sizeof(int) * nent);
    h->ldc = (int)((E + 3) / 4 * 4);
    A((void **)&h->blk_counts, sizeof(int) * (size_t)h->nblk_max * h->ldc);
    A((void **)&h->blk_zh, sizeof(double) * (size_t)h->nblk_max * 2);
    h->nsup_max = (h->nblk_max + kSuper - 1) / kSuper;
    A((void **)&h->sup_cnt2, sizeof(int) * 2 * (size_t)h->nsup_max * h->ldc);
    A((void **)&h->sup_p2, sizeof(unsigned long long) * 2 * (size_t)h->nsup_max * h->ldc);
    A((void **)&h->counts, sizeof(int) * E);
    A((void **)&h->offsets, sizeof(int) * (E + 1));
    A((void **)&h->cap, sizeof(int));
    A((void **)&h->tiles, sizeof(int2) * (size_t)h->max_tiles);
    A((void **)&h->num_tiles, sizeof(int));
    A((void **)&h->tile_start, sizeof(int) * (E + 1));
    A((void **)&h->item_start, sizeof(int) * (E + 1));
    A((void **)&h->scalars, sizeof(float) * 8);
    if (cfg->gate_kind == MOE_GATE_EXPERT_CHOICE) A((void **)&h->ec_sel, sizeof(uint16_t) * T * E);
    A((void **)&h->aux_bias, sizeof(float) * aux_free_len(h));
    A((void **)&h->aux_mom, sizeof(float) * aux_free_len(h));
    A((void **)&h->perm, sizeof(int) * nent);
    A((void **)&h->pos_of, sizeof(int) * nent);
    A((void **)&h->gate_sorted, sizeof(float) * (size_t)h->rows_max);
    A(&h->xp, asz * (size_t)h->act_rows * h->D_pad);
    A(&h->hbuf, asz * (size_t)h->act_rows * h->H_pad);
    // bf16 kernel: y rows padded by 128 B (bf16) past a multiple of 64
    // elements, so that a tile's rows (a power-of-two stride apart otherwise)
    // spread over the HBM channels
    h->ld_y = h->bf16_gemm ? (int)round_up(h->Dout, 64) + 64 : h->Dout;
    A((void **)&h->y, sizeof(float) * (size_t)h->rows_max * h->ld_y);
    // tail split: at most gemm_slots partial blocks of BM x 256 floats
    // (rem * S <= slots) for either GEMM; the fp32 kernel's K split of small
    // tile grids: about two workgroups per CU of NB x 128 x 128 floats
    h->split_cap = h->bf16_gemm ? (long long)gemm_slots(h) * h->bm * 256 : 2LL * h->ncu * kGemmBM * kGemmBN;
    A((void **)&h->split_ws, sizeof(float) * (size_t)h->split_cap);
    if (r != MOE_OK) return cleanup(r);
    // Pads of the packed weights and of the activation rows must read as 0.
    hipError_t ze = hipSuccess;
    auto Z = [&](void *p, size_t bytes) {
        if (ze == hipSuccess && p) ze = hipMemsetAsync(p, 0, bytes, h->stream);
    };
    Z(h->wr, wr_bytes);
    Z(h->br, sizeof(float) * (size_t)h->Er_pad);
    Z(h->w1, wsz * (size_t)h->E * h->w1_stride);
    Z(h->w3, wsz * (size_t)h->E * h->w1_stride);
    Z(h->w2, wsz * (size_t)h->E * h->w2_stride);
    Z(h->w1t, wsz * (size_t)h->E * h->w1_stride);
    Z(h->w3t, wsz * (size_t)h->E * h->w1_stride);
    Z(h->w2t, wsz * (size_t)h->E * h->w2_stride);
    Z(h->s1, sizeof(float) * (size_t)h->E * h->H_pad);
    Z(h->s3, sizeof(float) * (size_t)h->E * h->H_pad);
    Z(h->s2, sizeof(float) * (size_t)h->E * h->Dout_npad);
    Z(h->b1, sizeof(float) * (size_t)h->E * h->H_pad);
    Z(h->b2, sizeof(float) * (size_t)h->E * h->Dout_npad);
    Z(h->sup_cnt2, sizeof(int) * 2 * (size_t)h->nsup_max * h->ldc);
    Z(h->sup_p2, sizeof(unsigned long long) * 2 * (size_t)h->nsup_max * h->ldc);
    Z(h->aux_bias, sizeof(float) * aux_free_len(h));
    Z(h->aux_mom, sizeof(float) * aux_free_len(h));
    Z(h->xp, asz * (size_t)h->act_rows * h->D_pad);
    Z(h->hbuf, asz * (size_t)h->act_rows * h->H_pad);
    if (ze == hipSuccess) ze = hipStreamSynchronize(h->stream);
    if (ze != hipSuccess) {
        h->err = std::string("initialising device memory failed: ") + hipGetErrorString(ze);
        return cleanup(MOE_EHIP);
    }
    *out = h;
    return MOE_OK;
}

int moe_destroy(moe_handle *h) {
    if (!h) return MOE_OK;
    {
        std::lock_guard<std::mutex> lk(h->mu);
        // the handle's last work: up to `done` when a layer-completing call
        // recorded it; after a bare stage call, everything on the device (its
        // stream is not used here: it may be gone, e.g. from a finalizer)
        if (h->pending) {
            if (h->done_rec) (void)hipEventSynchronize(h->done);
            else (void)hipDeviceSynchronize();
        }
        if (h->stream) (void)hipStreamSynchronize(h->stream);
        free_all(h);
        if (h->done) (void)hipEventDestroy(h->done);
        if (h->stream) (void)hipStreamDestroy(h->stream);
        h->stream = nullptr;
    }
    delete h;
    return MOE_OK;
}

static hipError_t build_noise_image(moe_handle *h);

int moe_router_lse(moe_handle *h, int32_t T, float *lse) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (!lse) return fail(h, MOE_EINVAL, "null lse");
    if (T != h->last_route_T || T < 1) return fail(h, MOE_EINVAL, "T must be the last routing call's token count");
    hipStream_t s = h->stream;
    int r = join_stream(h, s);
    if (r != MOE_OK) return r;
    HIP_TRY(h, hipMemcpyAsync(lse, h->lse, sizeof(float) * (size_t)T, hipMemcpyDeviceToHost, s));
    HIP_TRY(h, hipStreamSynchronize(s));
    settle(h);
    return MOE_OK;
}

int moe_set_expert_dropout(moe_handle *h, float p, uint64_t seed) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (h->gated) return fail(h, MOE_EUNSUPPORTED, "dropout: StandardExpert only (GatedExpert has none)");
    if (!(p >= 0.0f && p < 1.0f)) return fail(h, MOE_EINVAL, "dropout p must be in [0, 1)");
    h->drop_p = p;
    h->drop_seed = seed;
    h->drop_calls = 0;
    return MOE_OK;
}

int moe_set_router(moe_handle *h, const float *weight, const float *bias) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (!weight) return fail(h, MOE_EINVAL, "null router weight");
    const bool dev_w = is_device_ptr(weight);
    const bool dev_b = bias && is_device_ptr(bias);
    // device sources may still be in flight on another stream (this handle's
    // stream does not order with the caller's): wait for the whole device
    if (dev_w || dev_b) HIP_TRY(h, hipDeviceSynchronize());
    int r = join_stream(h, h->stream);
    if (r != MOE_OK) return r;
    // memory [D][Er] -> [D][Er_pad]
    HIP_TRY(h, hipMemcpy2DAsync(h->wr, sizeof(float) * h->Er_pad, weight, sizeof(float) * h->Er,
                                sizeof(float) * h->Er, h->D, dev_w ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                h->stream));
    if (bias)
        HIP_TRY(h, hipMemcpyAsync(h->br, bias, sizeof(float) * h->Er, dev_b ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                  h->stream));
    HIP_TRY(h, launch_router_split(h->wr, h->D, h->Er, h->Er_pad, h->Dp32, h->wsplit, h->stream));
    if (h->noise_net) HIP_TRY(h, build_noise_image(h));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    settle(h);
    h->has_bias = bias != nullptr;
    h->router_set = true;
    return MOE_OK;
}

// [W | Wn] ([D][2 Er], rows padded to a multiple of 8) and its fragment image
static hipError_t build_noise_image(moe_handle *h) {
    const int Er2 = 2 * h->Er, Er2_pad = (int)round_up(Er2, 8);
    hipError_t e = hipMemcpy2DAsync(h->wrn, sizeof(float) * Er2_pad, h->wr, sizeof(float) * h->Er_pad,
                                    sizeof(float) * h->Er, h->D, hipMemcpyDeviceToDevice, h->stream);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(h->wrn + h->Er, sizeof(float) * Er2_pad, h->wn, sizeof(float) * h->Er_pad,
                             sizeof(float) * h->Er, h->D, hipMemcpyDeviceToDevice, h->stream);
    if (e == hipSuccess) e = launch_router_split(h->wrn, h->D, Er2, Er2_pad, h->Dp32, h->wsplit_n, h->stream);
    return e;
}

int moe_set_router_noise(moe_handle *h, float noise_scale, const float *noise_weight, uint64_t seed) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (!(noise_scale >= 0.0f) || !std::isfinite(noise_scale)) return fail(h, MOE_EINVAL, "noise_scale must be >= 0");
    if (noise_weight && 2 * h->Er > MOE_MAX_EXPERTS)
        return fail(h, MOE_EUNSUPPORTED, "a noise network needs 2 * router rows <= MOE_MAX_EXPERTS");
    if (noise_weight && h->cfg.gate_kind != MOE_GATE_TOPK && h->cfg.gate_kind != MOE_GATE_SWITCH &&
        h->cfg.gate_kind != MOE_GATE_SHARED && h->cfg.gate_kind != MOE_GATE_SOFT)
        return fail(h, MOE_EUNSUPPORTED, "router noise: the gate's logits come from the router GEMM only");
    const bool dev_w = noise_weight && is_device_ptr(noise_weight);
    if (dev_w) HIP_TRY(h, hipDeviceSynchronize());
    int r = join_stream(h, h->stream);
    if (r != MOE_OK) return r;
    if (noise_weight) {
        if (!h->wn) {
            const int Er2_pad = (int)round_up(2 * h->Er, 8);
            r = dalloc(h, (void **)&h->wn, sizeof(float) * (size_t)h->D * h->Er_pad);
            if (r == MOE_OK) r = dalloc(h, (void **)&h->wrn, sizeof(float) * (size_t)h->D * Er2_pad);
            if (r == MOE_OK)
                r = dalloc(h, (void **)&h->wsplit_n,
                           sizeof(uint16_t) * 3 * round_up(2 * h->Er, 16) * (size_t)h->Dp32);
            if (r != MOE_OK) return r;
            HIP_TRY(h, hipMemsetAsync(h->wn, 0, sizeof(float) * (size_t)h->D * h->Er_pad, h->stream));
        }
        HIP_TRY(h, hipMemcpy2DAsync(h->wn, sizeof(float) * h->Er_pad, noise_weight, sizeof(float) * h->Er,
                                    sizeof(float) * h->Er, h->D,
                                    dev_w ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, h->stream));
        HIP_TRY(h, build_noise_image(h));
    }
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    settle(h);
    h->noise_net = noise_weight != nullptr;
    h->noise_scale = noise_scale;
    h->noise_seed = seed;
    h->noise_calls = 0;
    return MOE_OK;
}

// The bf16 kernel's B tile images of expert x's packed matrices (W1 / W3 in
// 128-row blocks when gated, else 256; W2 in 256-row blocks), on the handle's
// stream after the packing.
static hipError_t retile_expert(moe_handle *h, int x) {
    if (!h->bf16_gemm) return hipSuccess;
    const size_t esz = (h->wt == WT_FP8) ? 1 : 2;
    const size_t o1 = esz * (size_t)x * h->w1_stride, o2 = esz * (size_t)x * h->w2_stride;
    const int rb1 = h->gated ? kNPadGated : kNPad;
    hipError_t e = launch_retile_weights((uint8_t *)h->w1 + o1, (uint8_t *)h->w1t + o1, h->H_pad, h->D_pad, (int)esz,
                                         rb1, h->stream);
    if (e == hipSuccess && h->gated)
        e = launch_retile_weights((uint8_t *)h->w3 + o1, (uint8_t *)h->w3t + o1, h->H_pad, h->D_pad, (int)esz, rb1,
                                  h->stream);
    if (e == hipSuccess)
        e = launch_retile_weights((uint8_t *)h->w2 + o2, (uint8_t *)h->w2t + o2, h->Dout_npad, h->H_pad, (int)esz,
                                  kNPad, h->stream);
    return e;
}

int moe_set_expert(moe_handle *h, int32_t expert, int32_t layout, int32_t src_dtype, const void *w1, const void *w2,
                   const void *w3, const float *b1, const float *b2, const float *s1, const float *s2,
                   const float *s3) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (expert < 0 || expert >= h->E) return fail(h, MOE_EINVAL, "expert index out of range");
    if (layout != MOE_LAYOUT_FLUX_OUT_IN && layout != MOE_LAYOUT_LLAMA_IN_OUT) return fail(h, MOE_EINVAL, "bad layout");
    if (src_dtype < MOE_F32 || src_dtype > MOE_FP8_E4M3) return fail(h, MOE_EINVAL, "bad src_dtype");
    if (!w1 || !w2 || (h->gated && !w3)) return fail(h, MOE_EINVAL, "missing expert weight matrix");
    if (src_dtype == MOE_FP8_E4M3 && (!s1 || !s2 || (h->gated && !s3)))
        return fail(h, MOE_EINVAL, "fp8 weights need per-output-channel scales");
    // device sources may still be in flight on another stream (this handle's
    // stream does not order with the caller's): wait for the whole device
    {
        const void *srcs[8] = {w1, w2, w3, b1, b2, s1, s2, s3};
        bool any_dev = false;
        for (const void *p : srcs)
            if (p && is_device_ptr(p)) any_dev = true;
        if (any_dev) HIP_TRY(h, hipDeviceSynchronize());
    }
    int r = join_stream(h, h->stream);
    if (r != MOE_OK) return r;
    const size_t wsz = (h->wt == WT_F32) ? 4 : (h->wt == WT_BF16 ? 2 : 1);
    uint8_t *w1d = (uint8_t *)h->w1 + wsz * (size_t)expert * h->w1_stride;
    uint8_t *w2d = (uint8_t *)h->w2 + wsz * (size_t)expert * h->w2_stride;
    float *s1d = h->s1 ? h->s1 + (size_t)expert * h->H_pad : nullptr;
    float *s2d = h->s2 ? h->s2 + (size_t)expert * h->Dout_npad : nullptr;
    r = pack_matrix(h, layout, src_dtype, w1, s1, h->H, h->D, h->D_pad, w1d, s1d);
    if (r != MOE_OK) return r;
    if (h->gated) {
        uint8_t *w3d = (uint8_t *)h->w3 + wsz * (size_t)expert * h->w1_stride;
        float *s3d = h->s3 ? h->s3 + (size_t)expert * h->H_pad : nullptr;
        r = pack_matrix(h, layout, src_dtype, w3, s3, h->H, h->D, h->D_pad, w3d, s3d);
        if (r != MOE_OK) return r;
    }
    r = pack_matrix(h, layout, src_dtype, w2, s2, h->Dout, h->H, h->H_pad, w2d, s2d);
    if (r != MOE_OK) return r;
    HIP_TRY(h, retile_expert(h, expert));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    settle(h);
    if (!h->gated) {
        if (b1)
            HIP_TRY(h, hipMemcpy(h->b1 + (size_t)expert * h->H_pad, b1, sizeof(float) * h->H,
                                 is_device_ptr(b1) ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice));
        if (b2)
            HIP_TRY(h, hipMemcpy(h->b2 + (size_t)expert * h->Dout_npad, b2, sizeof(float) * h->Dout,
                                 is_device_ptr(b2) ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice));
    }
    h->expert_set[expert] = 1;
    return MOE_OK;
}

int moe_init_experts_from_dense(moe_handle *h, int32_t layout, int32_t src_dtype, const void *w1, const void *w2,
                                const void *w3, const float *s1, const float *s2, const float *s3, int32_t strategy,
                                float noise_scale, uint64_t seed) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (!h->gated) return fail(h, MOE_EUNSUPPORTED, "expert initialisation from a dense FFN: gated experts only");
    if (layout != MOE_LAYOUT_FLUX_OUT_IN && layout != MOE_LAYOUT_LLAMA_IN_OUT) return fail(h, MOE_EINVAL, "bad layout");
    if (src_dtype < MOE_F32 || src_dtype > MOE_FP8_E4M3) return fail(h, MOE_EINVAL, "bad src_dtype");
    if (strategy < MOE_INIT_COPY || strategy > MOE_INIT_RANDOM)
        return fail(h, MOE_EINVAL, "unknown initialisation strategy (ArgumentError)");
    const bool need_src = strategy != MOE_INIT_RANDOM;
    if (need_src && (!w1 || !w2 || !w3)) return fail(h, MOE_EINVAL, "missing dense FFN matrix");
    if (need_src && src_dtype == MOE_FP8_E4M3 && (!s1 || !s2 || !s3))
        return fail(h, MOE_EINVAL, "fp8 weights need per-output-channel scales");
    {
        const void *srcs[6] = {w1, w2, w3, s1, s2, s3};
        bool any_dev = false;
        for (const void *p : srcs)
            if (p && is_device_ptr(p)) any_dev = true;
        if (any_dev) HIP_TRY(h, hipDeviceSynchronize());
    }
    int r = join_stream(h, h->stream);
    if (r != MOE_OK) return r;
    // the three dense matrices as fp32 rows: w1 / w3 (H, D), w2 (Dout, H)
    const int Ns[3] = {h->H, h->Dout, h->H}, Ks[3] = {h->D, h->H, h->D}, Kp[3] = {h->D_pad, h->H_pad, h->D_pad};
    const void *ws[3] = {w1, w2, w3};
    const float *ss[3] = {s1, s2, s3};
    float *dense[3] = {nullptr, nullptr, nullptr};
    float *tmp = nullptr;
    size_t most = 0;
    for (int m = 0; m < 3; ++m) {
        most = std::max(most, (size_t)Ns[m] * Ks[m]);
        if (need_src && r == MOE_OK) r = load_f32_rows(h, layout, src_dtype, ws[m], ss[m], Ns[m], Ks[m], &dense[m]);
    }
    hipError_t e = hipSuccess;
    if (r == MOE_OK) e = hipMalloc(&tmp, sizeof(float) * most);
    const size_t wsz = (h->wt == WT_F32) ? 4 : (h->wt == WT_BF16 ? 2 : 1);
    // Random init: sigma = sqrt(2f0 / dim) in Float32 (conversion.jl:306-310)
    const float sigma = sqrtf(2.0f / (float)h->D);
    for (int x = 0; x < h->E && r == MOE_OK && e == hipSuccess; ++x) {
        for (int m = 0; m < 3 && e == hipSuccess; ++m) {
            const long long total = (long long)Ns[m] * Ks[m];
            const int blocks = (int)std::min<long long>((total + 255) / 256, 4096);
            hipLaunchKernelGGL(init_expert_kernel, dim3(blocks), dim3(256), 0, h->stream, dense[m], Ns[m], Ks[m],
                               strategy, m, x, h->E, h->H, noise_scale, sigma, (unsigned long long)seed, tmp);
            e = hipGetLastError();
            void *base = (m == 0) ? h->w1 : (m == 1 ? h->w2 : h->w3);
            const long long stride = (m == 1) ? h->w2_stride : h->w1_stride;
            float *sc = nullptr;
            if (h->wt == WT_FP8) {
                float *sb = (m == 0) ? h->s1 : (m == 1 ? h->s2 : h->s3);
                sc = sb + (size_t)x * (m == 1 ? h->Dout_npad : h->H_pad);
            }
            if (e == hipSuccess)
                e = pack_f32_rows(h, tmp, Ns[m], Ks[m], Kp[m], (uint8_t *)base + wsz * (size_t)x * stride, sc);
            // tmp is reused by the next matrix: the stream orders the kernels
        }
        if (e == hipSuccess) e = retile_expert(h, x);
        if (e == hipSuccess) h->expert_set[x] = 1;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
    if (e == hipSuccess) settle(h);
    for (float *d : dense)
        if (d) (void)hipFree(d);
    if (tmp) (void)hipFree(tmp);
    if (r != MOE_OK) return r;
    if (e != hipSuccess) return fail(h, MOE_EHIP, std::string("expert initialisation failed: ") + hipGetErrorString(e));
    return MOE_OK;
}

int moe_get_expert(moe_handle *h, int32_t expert, int32_t layout, void *w1, void *w2, void *w3, float *s1, float *s2,
                   float *s3) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (expert < 0 || expert >= h->E) return fail(h, MOE_EINVAL, "expert index out of range");
    if (!h->expert_set[expert]) return fail(h, MOE_ENOTREADY, "expert has no weights");
    if (layout != MOE_LAYOUT_FLUX_OUT_IN && layout != MOE_LAYOUT_LLAMA_IN_OUT) return fail(h, MOE_EINVAL, "bad layout");
    const int esz = (h->wt == WT_F32) ? 4 : (h->wt == WT_BF16 ? 2 : 1);
    const int Ns[3] = {h->H, h->Dout, h->H}, Ks[3] = {h->D, h->H, h->D}, Kp[3] = {h->D_pad, h->H_pad, h->D_pad};
    void *outs[3] = {w1, w2, h->gated ? w3 : nullptr};
    float *souts[3] = {s1, s2, h->gated ? s3 : nullptr};
    const size_t most = (size_t)std::max((size_t)h->H * h->D, (size_t)h->Dout * h->H) * esz;
    int r = join_stream(h, h->stream);
    if (r != MOE_OK) return r;
    uint8_t *tmp = nullptr;
    HIP_TRY(h, hipMalloc(&tmp, most));
    hipError_t e = hipSuccess;
    for (int m = 0; m < 3 && e == hipSuccess; ++m) {
        if (!outs[m] && !souts[m]) continue;
        const void *base = (m == 0) ? h->w1 : (m == 1 ? h->w2 : h->w3);
        const long long stride = (m == 1) ? h->w2_stride : h->w1_stride;
        if (outs[m]) {
            const long long total = (long long)Ns[m] * Ks[m];
            const int blocks = (int)std::min<long long>((total + 255) / 256, 4096);
            hipLaunchKernelGGL(unpack_rows_kernel, dim3(blocks), dim3(256), 0, h->stream,
                               (const uint8_t *)base + (size_t)esz * expert * stride, esz, Ns[m], Ks[m], Kp[m], layout,
                               tmp);
            e = hipGetLastError();
            if (e == hipSuccess)
                e = hipMemcpyAsync(outs[m], tmp, (size_t)esz * total, hipMemcpyDeviceToHost, h->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
        }
        if (souts[m] && h->wt == WT_FP8 && e == hipSuccess) {
            const float *sb = (m == 0) ? h->s1 : (m == 1 ? h->s2 : h->s3);
            e = hipMemcpy(souts[m], sb + (size_t)expert * (m == 1 ? h->Dout_npad : h->H_pad), sizeof(float) * Ns[m],
                          hipMemcpyDeviceToHost);
        }
    }
    (void)hipFree(tmp);
    if (e != hipSuccess) return fail(h, MOE_EHIP, std::string("expert readback failed: ") + hipGetErrorString(e));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    settle(h);
    return MOE_OK;
}

int moe_set_aux_free(moe_handle *h, int32_t enable, const float *bias, const float *bias_momentum,
                     float learning_rate, float momentum, int32_t update_freq, int64_t update_counter,
                     int32_t use_complementary_loss, float complementary_weight) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (!enable) {
        h->aux_free = false;
        return MOE_OK;
    }
    if (update_freq < 1) return fail(h, MOE_EINVAL, "update_freq must be >= 1");
    if (update_counter < 0) return fail(h, MOE_EINVAL, "update_counter must be >= 0");
    hipStream_t s = h->stream;
    int r = join_stream(h, s);
    if (r != MOE_OK) return r;
    const size_t bytes = sizeof(float) * aux_free_len(h);
    if (bias) HIP_TRY(h, hipMemcpyAsync(h->aux_bias, bias, bytes, hipMemcpyHostToDevice, s));
    else HIP_TRY(h, hipMemsetAsync(h->aux_bias, 0, bytes, s));
    if (bias_momentum) HIP_TRY(h, hipMemcpyAsync(h->aux_mom, bias_momentum, bytes, hipMemcpyHostToDevice, s));
    else HIP_TRY(h, hipMemsetAsync(h->aux_mom, 0, bytes, s));
    HIP_TRY(h, hipStreamSynchronize(s));
    settle(h);
    h->aux_free = true;
    h->aux_lr = learning_rate;
    h->aux_momentum = momentum;
    h->aux_update_freq = update_freq;
    h->aux_counter = update_counter;
    h->aux_use_comp = use_complementary_loss != 0;
    h->aux_cw = complementary_weight;
    return MOE_OK;
}

int moe_get_aux_free(moe_handle *h, float *bias, float *bias_momentum, int64_t *update_counter) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    hipStream_t s = h->stream;
    int r = join_stream(h, s);
    if (r != MOE_OK) return r;
    const size_t bytes = sizeof(float) * aux_free_len(h);
    if (bias) HIP_TRY(h, hipMemcpyAsync(bias, h->aux_bias, bytes, hipMemcpyDeviceToHost, s));
    if (bias_momentum) HIP_TRY(h, hipMemcpyAsync(bias_momentum, h->aux_mom, bytes, hipMemcpyDeviceToHost, s));
    HIP_TRY(h, hipStreamSynchronize(s));
    settle(h);
    if (update_counter) *update_counter = h->aux_counter;
    return MOE_OK;
}

int moe_compute_gates(moe_handle *h, const float *logits, int32_t T, int32_t *indices, float *gates, float *probs) {
    return moe_route_from_logits(h, logits, T, 0, indices, gates, probs, nullptr, nullptr, nullptr);
}

int moe_route_from_logits(moe_handle *h, const float *logits, int32_t T, int32_t training, int32_t *indices,
                          float *gates, float *probs, int32_t *counts, int32_t *offsets, int32_t *perm) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (T < 0 || T > h->T_max) return fail(h, MOE_EINVAL, "T must be in [0, max_tokens]");
    if (T > 0 && !logits) return fail(h, MOE_EINVAL, "null logits");
    if (T == 0) {
        if (counts) memset(counts, 0, sizeof(int32_t) * h->E);
        if (offsets) memset(offsets, 0, sizeof(int32_t) * (h->E + 1));
        return MOE_OK;
    }
    hipStream_t s = h->stream;
    h->last_T = -1;  // routing state no longer matches a forward call
    int r = begin_call(h, T);
    if (r != MOE_OK) return r;
    r = join_stream(h, s);
    if (r != MOE_OK) return r;
    HIP_TRY(h, hipMemcpyAsync(h->logits_in, logits, sizeof(float) * (size_t)T * h->Er, hipMemcpyHostToDevice, s));
    r = run_routing(h, nullptr, 0, T, training, false, PERMUTE_INDEX, nullptr, s);
    if (r != MOE_OK) return r;
    const size_t nk = (size_t)T * h->kc;
    if (indices) HIP_TRY(h, hipMemcpyAsync(indices, h->idx, sizeof(int) * nk, hipMemcpyDeviceToHost, s));
    if (gates) HIP_TRY(h, hipMemcpyAsync(gates, h->gates, sizeof(float) * nk, hipMemcpyDeviceToHost, s));
    if (probs) HIP_TRY(h, hipMemcpyAsync(probs, h->probs, sizeof(float) * (size_t)T * h->Er, hipMemcpyDeviceToHost, s));
    if (counts) HIP_TRY(h, hipMemcpyAsync(counts, h->counts, sizeof(int) * h->E, hipMemcpyDeviceToHost, s));
    if (offsets) HIP_TRY(h, hipMemcpyAsync(offsets, h->offsets, sizeof(int) * (h->E + 1), hipMemcpyDeviceToHost, s));
    if (perm) HIP_TRY(h, hipMemcpyAsync(perm, h->perm, sizeof(int) * nk, hipMemcpyDeviceToHost, s));
    HIP_TRY(h, hipStreamSynchronize(s));
    settle(h);
    return MOE_OK;
}

static int forward_host_locked(moe_handle *h, const void *x, int32_t x_dtype, int32_t T, int32_t training,
                               float *out, float *loss, moe_forward_aux *aux);

int moe_forward(moe_handle *h, const void *x, int32_t x_dtype, int32_t T, int32_t training, float *out, float *loss,
                moe_forward_aux *aux) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    h->given = false;
    return forward_host_locked(h, x, x_dtype, T, training, out, loss, aux);
}

int moe_forward_routed(moe_handle *h, const void *x, int32_t x_dtype, int32_t T, int32_t training,
                       const int32_t *indices, const float *gates, int32_t kd, const float *probs, float *out,
                       float *loss, moe_forward_aux *aux) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (T < 0 || T > h->T_max) return fail(h, MOE_EINVAL, "T must be in [0, max_tokens]");
    if (kd < 1 || kd > MOE_MAX_TOPK) return fail(h, MOE_EINVAL, "slots per token must be in [1, MOE_MAX_TOPK]");
    if ((long long)T * kd > h->rows_max) return fail(h, MOE_EINVAL, "T * slots exceeds the handle's max_tokens * slots");
    if (h->lsh > 0) return fail(h, MOE_EUNSUPPORTED, "routed forward with num_shared_experts > 0");
    if (h->aux_free) return fail(h, MOE_EUNSUPPORTED, "routed forward with an AuxiliaryFreeLoss");
    if (T > 0 && (!indices || !gates)) return fail(h, MOE_EINVAL, "null indices or gates");
    // an expert listed twice for one token would be computed twice in the
    // reference; the bucketing here assumes distinct ids per token
    for (int t = 0; t < T; ++t)
        for (int i = 0; i < kd; ++i) {
            const int e = indices[(size_t)t * kd + i];
            if (e < 1 || e > h->E) continue;
            for (int j = i + 1; j < kd; ++j)
                if (indices[(size_t)t * kd + j] == e)
                    return fail(h, MOE_EUNSUPPORTED, "an expert id repeated within one token's slots");
        }
    h->given = true;
    h->given_probs = probs != nullptr;
    h->kc = kd;
    h->kl = kd;
    hipStream_t s = h->stream;
    int jr = join_stream(h, s);
    if (jr != MOE_OK) return jr;
    if (T > 0) {
        HIP_TRY(h, hipMemcpyAsync(h->idx, indices, sizeof(int) * (size_t)T * kd, hipMemcpyHostToDevice, s));
        HIP_TRY(h, hipMemcpyAsync(h->gates, gates, sizeof(float) * (size_t)T * kd, hipMemcpyHostToDevice, s));
        if (probs)
            HIP_TRY(h, hipMemcpyAsync(h->probs, probs, sizeof(float) * (size_t)T * h->Er, hipMemcpyHostToDevice, s));
    }
    const int r = forward_host_locked(h, x, x_dtype, T, training, out, loss, aux);
    h->given = false;
    h->kc = h->kt;
    h->kl = h->kt - h->lsh;
    h->last_T = -1;  // the stage entry points replay the handle's own gate only
    return r;
}

static int forward_host_locked(moe_handle *h, const void *x, int32_t x_dtype, int32_t T, int32_t training,
                               float *out, float *loss, moe_forward_aux *aux) {
    if (T < 0 || T > h->T_max) return fail(h, MOE_EINVAL, "T must be in [0, max_tokens]");
    if (T == 0) {
        // empty batch: zero-size output; loss 0 (inference) or NaN (means over no tokens)
        if (loss) *loss = training ? NAN : 0.0f;
        if (aux) {
            if (aux->counts) memset(aux->counts, 0, sizeof(int32_t) * h->E);
            if (aux->offsets) memset(aux->offsets, 0, sizeof(int32_t) * (h->E + 1));
            if (aux->mean_entropy) *aux->mean_entropy = NAN;
            if (aux->switch_loss) *aux->switch_loss = training ? NAN : 0.0f;
            if (aux->z_loss) *aux->z_loss = training ? NAN : 0.0f;
        }
        return MOE_OK;
    }
    if (!x || !out) return fail(h, MOE_EINVAL, "null x or out");
    int r = ensure_io_buffers(h);
    if (r != MOE_OK) return r;
    hipStream_t s = h->stream;
    r = join_stream(h, s);
    if (r != MOE_OK) return r;
    const size_t xbytes = (x_dtype == MOE_BF16 ? 2 : 4) * (size_t)T * h->D;
    HIP_TRY(h, hipMemcpyAsync(h->x_dev, x, xbytes, hipMemcpyHostToDevice, s));
    h->keep_rows = aux && (aux->logits || aux->probs);
    r = forward_locked(h, h->x_dev, x_dtype, T, training, h->out_dev, nullptr, s);
    if (r != MOE_OK) return r;
    HIP_TRY(h, hipMemcpyAsync(out, h->out_dev, sizeof(float) * (size_t)T * h->Dout, hipMemcpyDeviceToHost, s));
    float sc[4] = {0, 0, 0, 0};
    HIP_TRY(h, hipMemcpyAsync(sc, h->scalars, sizeof(float) * 4, hipMemcpyDeviceToHost, s));
    const size_t nk = (size_t)T * h->kc;
    if (aux) {
        if (aux->logits) HIP_TRY(h, hipMemcpyAsync(aux->logits, h->logits, sizeof(float) * (size_t)T * h->Er, hipMemcpyDeviceToHost, s));
        if (aux->probs) HIP_TRY(h, hipMemcpyAsync(aux->probs, h->probs, sizeof(float) * (size_t)T * h->Er, hipMemcpyDeviceToHost, s));
        if (aux->indices) HIP_TRY(h, hipMemcpyAsync(aux->indices, h->idx, sizeof(int) * nk, hipMemcpyDeviceToHost, s));
        if (aux->gates) HIP_TRY(h, hipMemcpyAsync(aux->gates, h->gates, sizeof(float) * nk, hipMemcpyDeviceToHost, s));
        if (aux->counts) HIP_TRY(h, hipMemcpyAsync(aux->counts, h->counts, sizeof(int) * h->E, hipMemcpyDeviceToHost, s));
        if (aux->offsets) HIP_TRY(h, hipMemcpyAsync(aux->offsets, h->offsets, sizeof(int) * (h->E + 1), hipMemcpyDeviceToHost, s));
        if (aux->perm) HIP_TRY(h, hipMemcpyAsync(aux->perm, h->perm, sizeof(int) * nk, hipMemcpyDeviceToHost, s));
    }
    HIP_TRY(h, hipStreamSynchronize(s));
    settle(h);
    if (loss) *loss = sc[2];
    if (aux) {
        if (aux->switch_loss) *aux->switch_loss = sc[0];
        if (aux->z_loss) *aux->z_loss = sc[1];
        if (aux->mean_entropy) *aux->mean_entropy = sc[3];
    }
    return MOE_OK;
}

int moe_expert_forward(moe_handle *h, int32_t expert, const float *x, int32_t n, float *y) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    if (expert < 0 || expert >= h->E) return fail(h, MOE_EINVAL, "expert index out of range");
    if (!h->expert_set[expert]) return fail(h, MOE_ENOTREADY, "expert has no weights");
    if (n < 0 || n > h->rows_max) return fail(h, MOE_EINVAL, "n must be in [0, max_tokens * slots]");
    if (n == 0) return MOE_OK;
    if (!x || !y) return fail(h, MOE_EINVAL, "null buffer");
    hipStream_t s = h->stream;
    int r = join_stream(h, s);
    if (r != MOE_OK) return r;
    // single segment: counts[expert] = n, all others 0
    std::vector<int> cnt(h->E, 0), off(h->E + 1, 0);
    cnt[expert] = n;
    for (int e = 0; e < h->E; ++e) off[e + 1] = off[e] + cnt[e];
    const int nt = (n + h->bm - 1) / h->bm;
    std::vector<int2> tl(nt);
    for (int i = 0; i < nt; ++i) tl[i] = make_int2(expert, i * h->bm);
    std::vector<int> ts(h->E + 1, 0);
    for (int e = 0; e <= h->E; ++e) ts[e] = e > expert ? nt : 0;
    // the up GEMM's work items (the device scan's rule): a last M tile of at
    // most bm/2 rows covers two n-tiles in one item
    std::vector<int> is(h->E + 1, 0);
    if (up_pairs(h)) {
        const int pnt = up_ntiles(h), f = n / h->bm, rr = n % h->bm;
        const int items = (rr > 0 && 2 * rr <= h->bm) ? pnt * f + pnt / 2 : pnt * nt;
        for (int e = 0; e <= h->E; ++e) is[e] = e > expert ? items : 0;
    }
    void *xs = nullptr;
    HIP_TRY(h, hipMalloc(&xs, sizeof(float) * (size_t)n * h->D));
    hipError_t e = hipMemcpyAsync(xs, x, sizeof(float) * (size_t)n * h->D, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(h->counts, cnt.data(), sizeof(int) * h->E, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(h->offsets, off.data(), sizeof(int) * (h->E + 1), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(h->tiles, tl.data(), sizeof(int2) * nt, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(h->num_tiles, &nt, sizeof(int), hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(h->tile_start, ts.data(), sizeof(int) * (h->E + 1), hipMemcpyHostToDevice, s);
    if (e == hipSuccess && up_pairs(h))
        e = hipMemcpyAsync(h->item_start, is.data(), sizeof(int) * (h->E + 1), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(convert_rows_kernel, dim3(1024), dim3(256), 0, s, (const void *)xs, 0, n, h->D, h->ct,
                           h->xp, h->D_pad, h->bf16_gemm ? h->bm : 0);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = launch_up(h, nt, s);
    if (e == hipSuccess) e = launch_down(h, nt, s, 1, true);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(y, sizeof(float) * h->Dout, h->y, sizeof(float) * (size_t)h->ld_y,
                             sizeof(float) * h->Dout, n, hipMemcpyDeviceToHost, s);
    hipError_t e2 = hipStreamSynchronize(s);
    if (e == hipSuccess) e = e2;
    if (e == hipSuccess) settle(h);
    (void)hipFree(xs);
    h->last_T = -1;  // routing state no longer matches a forward call
    if (e != hipSuccess) return fail(h, MOE_EHIP, std::string("expert forward failed: ") + hipGetErrorString(e));
    return MOE_OK;
}

// ---- decode (moe_ffn_forward!, src/llama2/inference.jl:58-121) -------------
static int decode_check(moe_handle *h, int n) {
    int r = check_ready(h);
    if (r != MOE_OK) return r;
    if (!h->gated) return fail(h, MOE_EUNSUPPORTED, "decode path: gated experts only (gated_expert_forward!)");
    // gated_expert_forward! applies silu inline whatever the layer's config says
    // (src/llama2/inference.jl:160); a layer configured with another activation
    // would compute something else through layer(x) than through this path
    if (h->cfg.activation != MOE_ACT_SILU)
        return fail(h, MOE_EUNSUPPORTED, "decode path: silu experts only (gated_expert_forward! applies silu)");
    if (h->cfg.gate_kind != MOE_GATE_TOPK && h->cfg.gate_kind != MOE_GATE_SWITCH)
        return fail(h, MOE_EUNSUPPORTED, "decode path: TopKGating or SwitchGating only");
    if ((h->D & 3) != 0) return fail(h, MOE_EUNSUPPORTED, "decode path: input_dim must be a multiple of 4");
    // h of the n * k slots is kept as fp32 rows in the expert workspace
    const long long cap = (long long)h->rows_max * h->H_pad * (h->ct == CT_F32 ? 4 : 2) / (4LL * h->H_pad * h->kt);
    if (n < 1 || n > h->T_max || n > cap)
        return fail(h, MOE_EINVAL, "n must be in [1, max_tokens] (bf16 / fp8 handles: [1, max_tokens / 2])");
    return MOE_OK;
}

static int decode_locked(moe_handle *h, const float *x_dev, int n, float *out_dev, hipStream_t s,
                         hipEvent_t done = nullptr) {
    DecodeArgs a{};
    a.x = x_dev; a.D = h->D; a.n = n; a.kt = h->kt; a.k = h->k; a.E = h->Er; a.lsh = h->lsh;
    a.wr = h->wr; a.Er_pad = h->Er_pad; a.br = h->has_bias ? h->br : nullptr;
    a.logits = h->logits; a.probs = h->probs; a.idx = h->idx; a.gates = h->gates;
    a.wt = h->wt; a.w1 = h->w1; a.w3 = h->w3; a.w2 = h->w2;
    a.w1_stride = h->w1_stride; a.w2_stride = h->w2_stride;
    a.Dpad = h->D_pad; a.H = h->H; a.Hpad = h->H_pad; a.Dout = h->Dout;
    a.s1 = h->s1; a.s3 = h->s3; a.s2 = h->s2; a.Dout_npad = h->Dout_npad;
    a.h = (float *)h->hbuf; a.out = out_dev;
    HIP_TRY(h, launch_decode_ffn(a, h->ncu, s, done));
    h->last_T = -1;  // the routing buffers no longer describe a layer forward
    return MOE_OK;
}

int moe_decode(moe_handle *h, const float *xb, int32_t n, float *out, float *logits, int32_t *indices, float *gates) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    int r = decode_check(h, n);
    if (r != MOE_OK) return r;
    if (!xb || !out) return fail(h, MOE_EINVAL, "null xb or out");
    r = ensure_io_buffers(h);
    if (r != MOE_OK) return r;
    hipStream_t s = h->stream;
    r = join_stream(h, s);
    if (r != MOE_OK) return r;
    HIP_TRY(h, hipMemcpyAsync(h->x_dev, xb, sizeof(float) * (size_t)n * h->D, hipMemcpyHostToDevice, s));
    r = decode_locked(h, (const float *)h->x_dev, n, h->out_dev, s);
    if (r != MOE_OK) return r;
    HIP_TRY(h, hipMemcpyAsync(out, h->out_dev, sizeof(float) * (size_t)n * h->Dout, hipMemcpyDeviceToHost, s));
    if (logits) HIP_TRY(h, hipMemcpyAsync(logits, h->logits, sizeof(float) * (size_t)n * h->Er, hipMemcpyDeviceToHost, s));
    if (indices) HIP_TRY(h, hipMemcpyAsync(indices, h->idx, sizeof(int) * (size_t)n * h->kt, hipMemcpyDeviceToHost, s));
    if (gates) HIP_TRY(h, hipMemcpyAsync(gates, h->gates, sizeof(float) * (size_t)n * h->kt, hipMemcpyDeviceToHost, s));
    HIP_TRY(h, hipStreamSynchronize(s));
    settle(h);
    return MOE_OK;
}

int moe_decode_async(moe_handle *h, const float *xb_dev, int32_t n, float *out_dev, void *stream) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    int r = decode_check(h, n);
    if (r != MOE_OK) return r;
    if (!xb_dev || !out_dev) return fail(h, MOE_EINVAL, "null buffer");
    if ((uintptr_t)xb_dev & 15) return fail(h, MOE_EINVAL, "xb_dev must be 16-byte aligned");
    hipStream_t s = stream ? (hipStream_t)stream : h->stream;
    r = join_stream(h, s);
    if (r == MOE_OK) r = decode_locked(h, xb_dev, n, out_dev, s, h->done);
    if (r == MOE_OK) {
        mark_stream(h, s);
        h->done_rec = true;  // recorded by the last kernel's completion
    }
    return r;
}

int moe_forward_async(moe_handle *h, const void *x_dev, int32_t x_dtype, int32_t T, int32_t training, float *out_dev,
                      float *loss_dev, void *stream) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    hipStream_t s = stream ? (hipStream_t)stream : h->stream;
    int r = join_stream(h, s);
    if (r == MOE_OK) r = forward_locked(h, x_dev, x_dtype, T, training, out_dev, loss_dev, s);
    if (r == MOE_OK) r = mark_stream(h, s, true);
    return r;
}

static int stage_check(moe_handle *h, int T) {
    if (h->last_T != T) return fail(h, MOE_EINVAL, "stage call must follow a moe_forward_async with the same T");
    return MOE_OK;
}

int moe_stage_router_async(moe_handle *h, const void *x_dev, int32_t x_dtype, int32_t T, int32_t training,
                           void *stream) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    int r = stage_check(h, T);
    if (r != MOE_OK) return r;
    hipStream_t s = stream ? (hipStream_t)stream : h->stream;
    h->last_training = training;
    r = join_stream(h, s);
    if (r == MOE_OK) r = run_routing(h, x_dev, x_dtype == MOE_BF16, T, training, true, PERMUTE_NONE, nullptr, s);
    if (r == MOE_OK) r = mark_stream(h, s);
    return r;
}

int moe_stage_permute_async(moe_handle *h, const void *x_dev, int32_t x_dtype, int32_t T, void *stream) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    int r = stage_check(h, T);
    if (r != MOE_OK) return r;
    hipStream_t s = stream ? (hipStream_t)stream : h->stream;
    r = join_stream(h, s);
    if (r == MOE_OK) r = run_permute(h, x_dev, x_dtype == MOE_BF16, T, h->last_training, PERMUTE_ROWS, s);
    if (r == MOE_OK) r = mark_stream(h, s);
    return r;
}

int moe_stage_expert_up_async(moe_handle *h, int32_t T, void *stream) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    int r = stage_check(h, T);
    if (r != MOE_OK) return r;
    hipStream_t s = stream ? (hipStream_t)stream : h->stream;
    r = join_stream(h, s);
    if (r != MOE_OK) return r;
    HIP_TRY(h, launch_up(h, m_tiles_for(h, T), s, h->last_training != 0));
    return mark_stream(h, s);
}

int moe_stage_expert_down_async(moe_handle *h, int32_t T, void *stream) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    int r = stage_check(h, T);
    if (r != MOE_OK) return r;
    hipStream_t s = stream ? (hipStream_t)stream : h->stream;
    r = join_stream(h, s);
    if (r != MOE_OK) return r;
    HIP_TRY(h, launch_down(h, m_tiles_for(h, T), s, down_ksplit(h)));
    return mark_stream(h, s);
}

int moe_stage_combine_async(moe_handle *h, int32_t T, float *out_dev, void *stream) {
    if (!h) return fail(nullptr, MOE_EINVAL, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    int r = stage_check(h, T);
    if (r != MOE_OK) return r;
    if (!out_dev) return fail(h, MOE_EINVAL, "null out");
    hipStream_t s = stream ? (hipStream_t)stream : h->stream;
    r = join_stream(h, s);
    if (r == MOE_OK) r = run_combine(h, T, out_dev, s);
    if (r == MOE_OK) r = mark_stream(h, s, true);
    return r;
}

int moe_switch_loss(const int32_t *indices, int32_t T, int32_t k, const float *probs, int32_t E, float alpha,
                    float *loss) {
    if (!loss || T < 0 || k < 1 || E < 1) return fail(nullptr, MOE_EINVAL, "bad switch-loss arguments");
    if (E > MOE_MAX_EXPERTS) return fail(nullptr, MOE_EINVAL, "switch loss: E above MOE_MAX_EXPERTS (512)");
    if ((long long)T * k > INT_MAX) return fail(nullptr, MOE_EINVAL, "switch loss: T * k too large");
    if (T > 0 && (!indices || !probs)) return fail(nullptr, MOE_EINVAL, "null indices or probs");
    if (T == 0) { *loss = NAN; return MOE_OK; }
    const size_t ni = (size_t)T * k, np_ = (size_t)T * E;
    // one allocation: the partials (8-byte aligned first), indices, probs, the loss
    const size_t pb = switch_loss_scratch_bytes(T, E);
    void *buf = nullptr;
    const size_t bytes = pb + sizeof(int) * ni + sizeof(float) * np_ + 16;
    if (hipMalloc(&buf, bytes) != hipSuccess) return fail(nullptr, MOE_EOOM, "hipMalloc failed");
    int *di = (int *)((uint8_t *)buf + pb);
    float *dp = (float *)(di + ni);
    float *dout = dp + np_;
    hipError_t e = hipMemcpy(di, indices, sizeof(int) * ni, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dp, probs, sizeof(float) * np_, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_switch_loss(di, T, k, dp, E, alpha, buf, dout, nullptr);
    if (e == hipSuccess) e = hipMemcpy(loss, dout, sizeof(float), hipMemcpyDeviceToHost);
    (void)hipFree(buf);
    if (e != hipSuccess) return fail(nullptr, MOE_EHIP, std::string("switch loss failed: ") + hipGetErrorString(e));
    return MOE_OK;
}

// ---- the allocation-free Switch loss -------------------------------------------
// The largest partials launch_switch_loss writes: kSwitchLossMaxBlocks rows of
// MOE_MAX_EXPERTS doubles and ints (384 KiB).
constexpr size_t kSwitchLossScratchBytes =
    (size_t)kSwitchLossMaxBlocks * MOE_MAX_EXPERTS * (sizeof(double) + sizeof(int));
static_assert(kSwitchLossScratchBytes == MOE_SWITCH_LOSS_SCRATCH_BYTES, "header and library agree");

// File-scope device array of those partials.  Each GPU the library runs on
// holds its own copy until the process ends.  In host code its name is a
// host-side stand-in, never an address: the device address of a GPU's copy
// comes from hipGetSymbolAddress, looked up once per device (the first call
// on it) and kept in scratch_dev.
static __device__ __align__(256) uint8_t scratch[kSwitchLossScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *scratch_dev[kMaxDevices] = {};

// The device address of the current device's scratch array.
static int current_scratch(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(nullptr, MOE_EHIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(nullptr, MOE_EINVAL, "device ordinal above 63");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!scratch_dev[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(nullptr, MOE_EHIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        scratch_dev[dev] = p;
    }
    *out = scratch_dev[dev];
    return MOE_OK;
}

int moe_switch_loss_noalloc(const int32_t *indices_dev, int32_t T, int32_t k, const float *probs_dev, int32_t E,
                            float alpha, float *loss_dev, void *stream) {
    if (!loss_dev || T < 0 || k < 1 || E < 1) return fail(nullptr, MOE_EINVAL, "bad switch-loss arguments");
    if (E > MOE_MAX_EXPERTS)
        return fail(nullptr, MOE_EINVAL,
                    "moe_switch_loss_noalloc: E above MOE_MAX_EXPERTS (512), the limit of its scratch array");
    if ((long long)T * k > INT_MAX) return fail(nullptr, MOE_EINVAL, "switch loss: T * k too large");
    if (T > 0 && (!indices_dev || !probs_dev)) return fail(nullptr, MOE_EINVAL, "null indices or probs");
    if (switch_loss_scratch_bytes(T, E) > kSwitchLossScratchBytes)
        return fail(nullptr, MOE_EINVAL, "moe_switch_loss_noalloc: partials exceed the scratch array");
    void *ws = nullptr;
    const int r = current_scratch(&ws);
    if (r != MOE_OK) return r;
    // T = 0 runs too: the partials are zeros and the loss the NaN of a mean
    // over no tokens, as moe_switch_loss returns
    const hipError_t e = launch_switch_loss(indices_dev, T, k, probs_dev, E, alpha, ws, loss_dev, (hipStream_t)stream);
    if (e != hipSuccess) return fail(nullptr, MOE_EHIP, std::string("switch loss failed: ") + hipGetErrorString(e));
    return MOE_OK;
}

int moe_z_loss(const float *logits, int32_t T, int32_t E, float beta, float *loss) {
    if (!loss || T < 0 || E < 1) return fail(nullptr, MOE_EINVAL, "bad z-loss arguments");
    if (T > 0 && !logits) return fail(nullptr, MOE_EINVAL, "null logits");
    if (T == 0) { *loss = NAN; return MOE_OK; }
    void *buf = nullptr;
    const size_t n = (size_t)T * E;
    if (hipMalloc(&buf, sizeof(float) * (n + 4)) != hipSuccess) return fail(nullptr, MOE_EOOM, "hipMalloc failed");
    float *dl = (float *)buf;
    float *dout = dl + n;
    hipError_t e = hipMemcpy(dl, logits, sizeof(float) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_z_loss(dl, T, E, beta, dout, nullptr);
    if (e == hipSuccess) e = hipMemcpy(loss, dout, sizeof(float), hipMemcpyDeviceToHost);
    (void)hipFree(buf);
    if (e != hipSuccess) return fail(nullptr, MOE_EHIP, std::string("z loss failed: ") + hipGetErrorString(e));
    return MOE_OK;
}

int moe_aux_free_update_bias(const int32_t *indices, int64_t n, int32_t E, float learning_rate, float momentum,
                             float *bias, float *bias_momentum) {
    if (n < 0 || E < 1 || E > MOE_MAX_EXPERTS || !bias || !bias_momentum || (n > 0 && !indices))
        return fail(nullptr, MOE_EINVAL, "bad update_bias! arguments");
    for (int64_t i = 0; i < n; ++i)
        if (indices[i] > E) return fail(nullptr, MOE_EINVAL, "expert id above num_experts (BoundsError in update_bias!)");
    int *di = nullptr;
    float *db = nullptr;
    hipError_t e = hipMalloc(&di, sizeof(int) * (size_t)(n > 0 ? n : 1));
    if (e == hipSuccess) e = hipMalloc(&db, sizeof(float) * 2 * (size_t)E);
    if (e == hipSuccess && n > 0) e = hipMemcpy(di, indices, sizeof(int) * (size_t)n, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(db, bias, sizeof(float) * E, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(db + E, bias_momentum, sizeof(float) * E, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_aux_free_update(di, n, E, learning_rate, momentum, db, db + E, nullptr);
    if (e == hipSuccess) e = hipMemcpy(bias, db, sizeof(float) * E, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(bias_momentum, db + E, sizeof(float) * E, hipMemcpyDeviceToHost);
    (void)hipFree(di);
    (void)hipFree(db);
    if (e != hipSuccess) return fail(nullptr, MOE_EHIP, std::string("update_bias! failed: ") + hipGetErrorString(e));
    return MOE_OK;
}

int moe_read_counts(moe_handle *h, int32_t *counts) {
    if (!h || !counts) return fail(h, MOE_EINVAL, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    int r = join_stream(h, h->stream);
    if (r != MOE_OK) return r;
    HIP_TRY(h, hipMemcpyAsync(counts, h->counts, sizeof(int) * h->E, hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    settle(h);
    return MOE_OK;
}

}  // extern "C"
