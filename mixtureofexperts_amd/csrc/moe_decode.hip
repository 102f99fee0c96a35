// moe_decode.hip -- the decode caller of the MoE FFN (moe_ffn_forward!,
// src/llama2/inference.jl:58-121): one token at a time (or n independent
// tokens), its k selected gated experts as matrix-vector products, combined
// in slot order.  Weight-bandwidth bound: every selected expert's three
// matrices are read once per token.
//
//   decode_up_kernel   : h_s = silu(W1_e xb) .* (W3_e xb) for slot s (expert e),
//                        silu(g) = g * (1 / (1 + exp(-g)))   (inference.jl:154-167)
//   decode_down_kernel : out = ((0 + g_1 y_1) + g_2 y_2) + ...,  y_s = W2_e h_s
//                                                             (inference.jl:83-104)
//
// The weights are the handle's packed [E][Npad][Kpad] rows (K contiguous), fp32,
// bf16 or fp8-e4m3 with per-row scales.  A wave computes one row's dot product:
// lane l takes elements 4 l, 4 l + 256, ... and the 64 partial sums are added
// by a fixed butterfly, so results are deterministic.
#include "moe_internal.h"

namespace moe {

// 4 consecutive weights of row `row` (element offset `o`, a multiple of 4) as fp32
template <int WT>
__device__ __forceinline__ float4 load_w4(const void *w, long long o) {
    if constexpr (WT == WT_F32) {
        return *(const float4 *)((const float *)w + o);
    } else if constexpr (WT == WT_BF16) {
        const uint2 q = *(const uint2 *)((const uint16_t *)w + o);
        return make_float4(__uint_as_float(q.x << 16), __uint_as_float(q.x & 0xffff0000u), __uint_as_float(q.y << 16),
                           __uint_as_float(q.y & 0xffff0000u));
    } else {
        const uint32_t q = *(const uint32_t *)((const uint8_t *)w + o);
        return make_float4(fp8e4m3_to_f32((uint8_t)q), fp8e4m3_to_f32((uint8_t)(q >> 8)),
                           fp8e4m3_to_f32((uint8_t)(q >> 16)), fp8e4m3_to_f32((uint8_t)(q >> 24)));
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o);
    return v;
}

// dot(W row starting at element `row0`, v[0..n)), n a multiple of 4; v fp32
template <int WT>
__device__ __forceinline__ float dot_row(const void *w, long long row0, const float *v, int n, int lane) {
    float acc = 0.0f;
    for (int i = lane * 4; i < n; i += 256) {
        const float4 a = load_w4<WT>(w, row0 + i);
        const float4 b = *(const float4 *)(v + i);
        acc = acc + a.x * b.x;
        acc = acc + a.y * b.y;
        acc = acc + a.z * b.z;
        acc = acc + a.w * b.w;
    }
    return wave_sum(acc);
}

// Block (token * kt + slot, row group): 4 waves, one h row each, over all
// Hpad rows (pad rows have zero weights, so their h is 0 and the down
// products may run over Hpad).
template <int WT>
__global__ __launch_bounds__(256) void decode_up_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int ts = blockIdx.x;  // token * kt + slot
    const int t = ts / a.kt;
    const int j = blockIdx.y * 4 + w;
    if (j >= a.Hpad) return;
    const int e = a.idx[ts] - 1;
    float hv = 0.0f;
    if (e >= 0 && e < a.E) {
        const float *x = a.x + (long long)t * a.D;
        const long long r = (long long)e * a.w1_stride + (long long)j * a.Dpad;
        float gt = dot_row<WT>(a.w1, r, x, a.D, lane);
        float up = dot_row<WT>(a.w3, r, x, a.D, lane);
        if (WT == WT_FP8) {
            gt = gt * a.s1[(long long)e * a.Hpad + j];
            up = up * a.s3[(long long)e * a.Hpad + j];
        }
        hv = (gt * (1.0f / (1.0f + expf(-gt)))) * up;
    }
    if (lane == 0) a.h[(long long)ts * a.Hpad + j] = hv;
}

// Block (token, row group): 4 waves, one output row each; the slots' products
// are combined in slot order on a zero start.
template <int WT>
__global__ __launch_bounds__(256) void decode_down_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = blockIdx.x;
    const int i = blockIdx.y * 4 + w;
    if (i >= a.Dout) return;
    float acc = 0.0f;
    for (int s = 0; s < a.kt; ++s) {
        const int ts = t * a.kt + s;
        const int e = a.idx[ts] - 1;
        if (e < 0 || e >= a.E) continue;
        float y = dot_row<WT>(a.w2, (long long)e * a.w2_stride + (long long)i * a.Hpad, a.h + (long long)ts * a.Hpad,
                              a.Hpad, lane);
        if (WT == WT_FP8) y = y * a.s2[(long long)e * a.Dout_npad + i];
        acc = acc + a.gates[ts] * y;
    }
    if (lane == 0) a.out[(long long)t * a.Dout + i] = acc;
}

template <int WT>
static hipError_t launch_decode_wt(const DecodeArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(decode_up_kernel<WT>, dim3(a.n * a.kt, (a.Hpad + 3) / 4), dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(decode_down_kernel<WT>, dim3(a.n, (a.Dout + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_decode_ffn(const DecodeArgs &a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    // rows are read 4 elements at a time: the padded strides are multiples of 64
    if ((a.D & 3) || (a.Dpad & 3) || (a.Hpad & 3) || a.D > a.Dpad || a.H > a.Hpad) return hipErrorInvalidValue;
    switch (a.wt) {
    case WT_F32: return launch_decode_wt<WT_F32>(a, s);
    case WT_BF16: return launch_decode_wt<WT_BF16>(a, s);
    default: return launch_decode_wt<WT_FP8>(a, s);
    }
}

}  // namespace moe
