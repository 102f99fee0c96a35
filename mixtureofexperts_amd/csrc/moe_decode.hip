// moe_decode.hip -- the decode caller of the MoE FFN (moe_ffn_forward!,
// src/llama2/inference.jl:58-121): one token at a time (or n independent
// tokens), its k selected gated experts as matrix-vector products, combined
// in slot order, and the layer's shared experts (process_shared_experts!,
// :184-216) averaged and blended 0.5 / 0.5 with them.  Weight-bandwidth bound: every selected expert's three
// matrices are read once per token; two kernels per call.
//
//   decode_up_kernel   : the token's routing (logits = W' xb + b, softmax,
//                        top-k, gates; inference.jl:62-66), recomputed by every
//                        block from the L2-resident router, then for the
//                        block's share of the (slot, row) units
//                        h_s = silu(W1_e xb) .* (W3_e xb),
//                        silu(g) = g * (1 / (1 + exp(-g)))   (inference.jl:154-167)
//   decode_down_kernel : out = ((0 + g_1 y_1) + g_2 y_2) + ...,  y_s = W2_e h_s
//                                                             (inference.jl:83-104)
//
// The weights are the handle's packed [E][Npad][Kpad] rows (K contiguous), fp32,
// bf16 or fp8-e4m3 with per-row scales.  A wave computes whole dot products:
// lane l takes the 4-element chunks l, l + 64, ... of the row, in that order,
// and the 64 partial sums are added by a fixed butterfly, so every result is
// deterministic.  All of a batch's loads are issued before its products
// (clamped addresses, out-of-row chunks selected to zero).
#include <hip/hip_ext.h>

#include "moe_internal.h"

namespace moe {

// 4 consecutive weights (element offset `o`, a multiple of 4) as fp32
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

__device__ __forceinline__ float readlane_f(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over each 16-lane row in a fixed order, every lane of the row ending
// with the same bits: pairs (quad_perm 1,0,3,2), quads (quad_perm 2,3,0,1),
// 8-lane halves (row_half_mirror), rows (row_mirror); additions commute
// exactly, so partner lanes hold identical values after every step.
__device__ __forceinline__ float row16_sum(float v) {
    v = v + dpp_f<0xb1>(v);
    v = v + dpp_f<0x4e>(v);
    v = v + dpp_f<0x141>(v);
    v = v + dpp_f<0x140>(v);
    return v;
}

// Wave sum (all 64 lanes active), uniform result: row sums, then the four rows
// in row order.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return ((readlane_f(v, 0) + readlane_f(v, 16)) + readlane_f(v, 32)) + readlane_f(v, 48);
}

__device__ __forceinline__ float4 zero_unless(bool v, float4 a) {
    return v ? a : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

__device__ __forceinline__ float dot4_acc(float acc, float4 a, float4 b) {
#pragma clang fp contract(off)
    acc = acc + a.x * b.x;
    acc = acc + a.y * b.y;
    acc = acc + a.z * b.z;
    acc = acc + a.w * b.w;
    return acc;
}

// ---- routing of one token by a 256-thread block --------------------------------
struct DecodeRouteLds {
    __attribute__((aligned(16))) float part[4][MOE_MAX_EXPERTS];  // per-wave logit partials
};

// The routed slots' experts of one token (0-based), 16 bits each: slot j in
// bits [16 (j % 4), +16) of word j / 4 (wave-uniform; k <= 16).
struct DecodeSel {
    unsigned long long w[4] = {0ull, 0ull, 0ull, 0ull};
    __device__ __forceinline__ void set(int j, int e) {
        const unsigned long long v = (unsigned long long)e << (16 * (j & 3));
        if (j < 4) w[0] |= v;
        else if (j < 8) w[1] |= v;
        else if (j < 12) w[2] |= v;
        else w[3] |= v;
    }
    __device__ __forceinline__ int get(int j) const {
        const unsigned long long v = j < 4 ? w[0] : (j < 8 ? w[1] : (j < 12 ? w[2] : w[3]));
        return (int)((v >> (16 * (j & 3))) & 0xffffu);
    }
};

// compute_gates of token t from the wave partials in L (see decode_route_block);
// E > 64: lane l holds experts l, l + 64, ..., l + 64 (NH - 1) (E <= 64:
// decode_gates64).  The per-expert passes walk part h = 0 .. NH - 1, then its
// lanes, i.e. the experts in ascending order; every register array is read
// with compile-time indices only (a part picked at run time would be a
// private-memory array).
template <int NH>
__device__ __forceinline__ DecodeSel decode_gates(const DecodeArgs &a, int t, bool write,
                                                           const DecodeRouteLds &L, float &gate) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, E = a.E;
    float lg[NH], ev[NH], pv[NH];
    uint32_t key[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int e = lane + 64 * h;
        const int ec = min(e, a.Er_pad - 1);
        float v = ((L.part[0][ec] + L.part[1][ec]) + L.part[2][ec]) + L.part[3][ec];
        if (a.br) v = v + a.br[min(e, E - 1)];
        lg[h] = v;
    }
    float m = -INFINITY;                                // max, NaN ignored
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int nh = min(64, E - 64 * h);             // experts of part h (<= 0: none)
        for (int i0 = 0; i0 < nh; i0 += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = readlane_f(lg[h], min(i0 + u, nh - 1));
#pragma unroll
            for (int u = 0; u < 8; ++u) m = (i0 + u < nh) ? fmaxf(m, v[u]) : m;
        }
    }
#pragma unroll
    for (int h = 0; h < NH; ++h)
        ev[h] = (m == INFINITY) ? ((lg[h] == INFINITY) ? 1.0f : 0.0f) : (float)exp((double)(lg[h] - m));
    float s = 0.0f;                                     // expert order
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int nh = min(64, E - 64 * h);
        for (int i0 = 0; i0 < nh; i0 += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = readlane_f(ev[h], min(i0 + u, nh - 1));
#pragma unroll
            for (int u = 0; u < 8; ++u) s = (i0 + u < nh) ? s + v[u] : s;
        }
    }
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        pv[h] = ev[h] / s;
        key[h] = (lane + 64 * h < E) ? isless_key(pv[h]) : 0u;
    }
    int rank[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) rank[h] = 0;
#pragma unroll
    for (int h2 = 0; h2 < NH; ++h2) {
        const int nh = min(64, E - 64 * h2);
        for (int i0 = 0; i0 < nh; i0 += 8) {
            uint32_t kv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) kv[u] = (uint32_t)__builtin_amdgcn_readlane((int)key[h2], min(i0 + u, nh - 1));
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = 64 * h2 + i0 + u;
#pragma unroll
                for (int h = 0; h < NH; ++h) {
                    const int e = lane + 64 * h;
                    rank[h] += (i0 + u < nh && (kv[u] > key[h] || (kv[u] == key[h] && i < e))) ? 1 : 0;
                }
            }
        }
    }
    float ssum = 0.0f, myp = 0.0f;
    int mye = 0;
    DecodeSel packed;
    for (int j = 0; j < a.k; ++j) {
        // the expert of rank j: the first part whose ballot holds it
        int e = 0;
        bool found = false;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const unsigned long long b = __ballot(lane + 64 * h < E && rank[h] == j);
            e = (!found && b) ? 64 * h + __builtin_ctzll(b) : e;
            found = found || b;
        }
        float pj = 0.0f;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const float c = readlane_f(pv[h], e & 63);
            pj = ((e >> 6) == h) ? c : pj;
        }
        ssum = (j == 0) ? pj : ssum + pj;  // slot order
        packed.set(j, e);
        if (lane == j) {
            myp = pj;
            mye = e;
        }
    }
    gate = lane < a.k ? myp / ssum : 0.0f;
    if (write) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const int e = lane + 64 * h;
            if (e < E) {
                a.logits[(long long)t * E + e] = lg[h];
                a.probs[(long long)t * E + e] = pv[h];
            }
        }
        // slots: the shared experts 1..lsh, then the routed ones shifted by lsh
        if (lane < a.lsh) {
            a.idx[(long long)t * a.kt + lane] = lane + 1;
            a.gates[(long long)t * a.kt + lane] = 1.0f / (float)a.lsh;
        }
        if (lane < a.k) {
            a.idx[(long long)t * a.kt + a.lsh + lane] = a.lsh + mye + 1;
            a.gates[(long long)t * a.kt + a.lsh + lane] = gate;
        }
    }
    return packed;
}

// Wave maximum of v (unsigned or float compare), uniform: within each 16-lane
// row by DPP steps, then the row results (rows past the first only when
// `rows4`).  Maxima are exact, so the order of the steps does not matter.
__device__ __forceinline__ uint32_t wave_umax(uint32_t v, bool rows4) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false));
    uint32_t r = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    if (rows4) {
        r = max(r, (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
        r = max(r, (uint32_t)__builtin_amdgcn_readlane((int)v, 32));
        r = max(r, (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
    }
    return r;
}
__device__ __forceinline__ float wave_fmax(float v, bool rows4) {  // v never NaN
    v = fmaxf(v, dpp_f<0xb1>(v));
    v = fmaxf(v, dpp_f<0x4e>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    float r = readlane_f(v, 0);
    if (rows4) r = fmaxf(fmaxf(r, readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
    return r;
}

// compute_gates for E <= 64, lane e holding expert e: the same recipe and
// results as decode_gates, in fewer dependent steps.  The max (NaN ignored:
// NaN lanes enter as -Inf, so all-NaN logits give -Inf as there) is a DPP
// reduction; the sum runs in expert order over 8-lane groups, lanes past E
// adding exact zeros; the k slots are k rounds of "largest isless key, lowest
// expert among equal keys", the partialsortperm order that decode_gates
// derives from ranks.
__device__ __forceinline__ DecodeSel decode_gates64(const DecodeArgs &a, int t, bool write,
                                                             const DecodeRouteLds &L, float &gate) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, E = a.E;
    const bool valid = lane < E, rows4 = E > 16;
    const int ec = min(lane, a.Er_pad - 1);
    float lg = ((L.part[0][ec] + L.part[1][ec]) + L.part[2][ec]) + L.part[3][ec];
    if (a.br) lg = lg + a.br[min(lane, E - 1)];
    const float m = wave_fmax(valid && !__builtin_isnan(lg) ? lg : -INFINITY, rows4);
    float ev = (m == INFINITY) ? ((lg == INFINITY) ? 1.0f : 0.0f) : (float)exp((double)(lg - m));
    ev = valid ? ev : 0.0f;
    float s = 0.0f;  // expert order: s + 0 == s for the lanes past E (s >= 0 or NaN)
    for (int i0 = 0; i0 < E; i0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = readlane_f(ev, i0 + u);
#pragma unroll
        for (int u = 0; u < 8; ++u) s = s + v[u];
    }
    const float p = ev / s;
    uint32_t key = valid ? isless_key(p) : 0u;  // every float's key is > 0
    float ssum = 0.0f, myp = 0.0f;
    int mye = 0;
    DecodeSel packed;
    for (int j = 0; j < a.k; ++j) {
        const uint32_t mk = wave_umax(key, rows4);
        const int e = __builtin_ctzll(__ballot(valid && key == mk));
        const float pj = readlane_f(p, e);
        ssum = (j == 0) ? pj : ssum + pj;  // slot order
        packed.set(j, e);
        if (lane == e) key = 0u;  // taken
        if (lane == j) {
            myp = pj;
            mye = e;
        }
    }
    gate = lane < a.k ? myp / ssum : 0.0f;
    if (write) {
        if (valid) {
            a.logits[(long long)t * E + lane] = lg;
            a.probs[(long long)t * E + lane] = p;
        }
        if (lane < a.lsh) {
            a.idx[(long long)t * a.kt + lane] = lane + 1;
            a.gates[(long long)t * a.kt + lane] = 1.0f / (float)a.lsh;
        }
        if (lane < a.k) {
            a.idx[(long long)t * a.kt + a.lsh + lane] = a.lsh + mye + 1;
            a.gates[(long long)t * a.kt + a.lsh + lane] = gate;
        }
    }
    return packed;
}

// Logits: lane (q, c) = q C + c of wave w sums x[d] W[d][4q..4q+3] over the
// chunk g = w C + c of D in d order (one float4 per router row, 4 rows in
// flight); the C chunks of a wave are added by a fixed tree (DPP steps within
// 16-lane rows, then lane xor 16 and 32), the 4 wave sums in wave order, then
// the bias.  Every wave then evaluates compute_gates on its own copy (identical
// results, no second barrier) with the recipe of the layer's routing kernel:
// m = max (NaN ignored), e_i = (float)exp((double)(l_i - m)) (a +Inf maximum
// gives 1 at the +Inf logits, 0 elsewhere), the sum in expert order, p_i = e_i
// / sum; top-k by the isless key descending, lower index first among equal
// keys (partialsortperm(p, 1:k, rev=true)): the rank of expert i is the number
// of experts before it in that order; the gates are p of the slots over their
// sum in slot order.  Lane l holds experts l, l + 64, l + 128, ... < E.
// Returns the 0-based experts of the routed slots (uniform), and in `gate`
// of lane j < k that slot's gate; `write` (wave 0 of
// one block per token) stores logits, probs, indices, gates.
__device__ __forceinline__ DecodeSel decode_route_block(const DecodeArgs &a, int t, bool write, DecodeRouteLds &L,
                                                 float &gate) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int E = a.E, Q = a.Er_pad >> 2;               // router row: Q float4 (Er_pad % 8 == 0)
    int QP = 1;
    while (QP < Q) QP <<= 1;                            // Q <= MOE_MAX_EXPERTS / 4
    const int C = QP >= 64 ? 1 : 64 / QP;               // chunks per wave
    const int NQ = QP > 64 ? QP / 64 : 1;               // float4 columns per lane (lane, lane + 64, ...)
    const int CH = (a.D + 4 * C - 1) / (4 * C);
    const float *x = a.x + (long long)t * a.D;
    const float4 *wr4 = (const float4 *)a.wr;
    for (int qi = 0; qi < NQ; ++qi) {
        const int q = C == 1 ? lane + 64 * qi : lane / C, c = C == 1 ? 0 : lane - q * C;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        {
            const int d0 = (w * C + c) * CH, d1 = min(a.D, d0 + CH);
            const int qq = min(q, Q - 1);
            for (int d = d0; d < d1; d += 4) {
                float xv[4];
                float4 wv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int dd = min(d + u, d1 - 1);
                    xv[u] = x[dd];
                    wv[u] = wr4[(long long)dd * Q + qq];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (d + u < d1) {
                        acc.x = acc.x + xv[u] * wv[u].x;
                        acc.y = acc.y + xv[u] * wv[u].y;
                        acc.z = acc.z + xv[u] * wv[u].z;
                        acc.w = acc.w + xv[u] * wv[u].w;
                    }
            }
        }
        // groups of C contiguous lanes: every lane of a group ends with the same sum
        if (C >= 2) {
            acc.x = acc.x + dpp_f<0xb1>(acc.x); acc.y = acc.y + dpp_f<0xb1>(acc.y);
            acc.z = acc.z + dpp_f<0xb1>(acc.z); acc.w = acc.w + dpp_f<0xb1>(acc.w);
        }
        if (C >= 4) {
            acc.x = acc.x + dpp_f<0x4e>(acc.x); acc.y = acc.y + dpp_f<0x4e>(acc.y);
            acc.z = acc.z + dpp_f<0x4e>(acc.z); acc.w = acc.w + dpp_f<0x4e>(acc.w);
        }
        if (C >= 8) {
            acc.x = acc.x + dpp_f<0x141>(acc.x); acc.y = acc.y + dpp_f<0x141>(acc.y);
            acc.z = acc.z + dpp_f<0x141>(acc.z); acc.w = acc.w + dpp_f<0x141>(acc.w);
        }
        if (C >= 16) {
            acc.x = acc.x + dpp_f<0x140>(acc.x); acc.y = acc.y + dpp_f<0x140>(acc.y);
            acc.z = acc.z + dpp_f<0x140>(acc.z); acc.w = acc.w + dpp_f<0x140>(acc.w);
        }
        for (int o = 16; o < C; o <<= 1) {
            acc.x = acc.x + __shfl_xor(acc.x, o); acc.y = acc.y + __shfl_xor(acc.y, o);
            acc.z = acc.z + __shfl_xor(acc.z, o); acc.w = acc.w + __shfl_xor(acc.w, o);
        }
        if (c == 0 && q < Q) *(float4 *)&L.part[w][4 * q] = acc;
    }
    __syncthreads();

    if (E > 256) return decode_gates<8>(a, t, write, L, gate);
    if (E > 128) return decode_gates<4>(a, t, write, L, gate);
    return E > 64 ? decode_gates<2>(a, t, write, L, gate) : decode_gates64(a, t, write, L, gate);
}

// ---- up: the waves of token t take units u = (slot, row j) two at a time,
// wave v of the token (v = y * 4 + wave of its block y) the units u0 = 2 v,
// stepping 2 nv.  A unit is the pair of dot products (W1_e row j) . x and
// (W3_e row j) . x over all Hpad rows (pad rows have zero weights, so their h
// is 0 and the down products may run over Hpad).
template <int WT>
__device__ __forceinline__ void decode_up_units(const DecodeArgs &a, int t, int v, int nv, const DecodeSel &sel) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int units = a.kt * a.Hpad;
    const int nch = a.D >> 2;  // 4-element chunks per row
    const float4 *x4 = (const float4 *)(a.x + (long long)t * a.D);
    for (int u0 = 2 * v; u0 < units; u0 += 2 * nv) {
        const bool two = u0 + 1 < units;
        const int u1 = two ? u0 + 1 : u0;
        const int s0 = u0 / a.Hpad, j0 = u0 - s0 * a.Hpad;
        const int s1 = u1 / a.Hpad, j1 = u1 - s1 * a.Hpad;
        // expert of a slot: shared s < lsh, else routed lsh + (slot s - lsh's pick)
        const int e0 = s0 < a.lsh ? s0 : a.lsh + sel.get(s0 - a.lsh);
        const int e1 = s1 < a.lsh ? s1 : a.lsh + sel.get(s1 - a.lsh);
        const bool ok0 = e0 >= 0 && e0 < a.E + a.lsh, ok1 = e1 >= 0 && e1 < a.E + a.lsh;
        const long long r0 = (long long)(ok0 ? e0 : 0) * a.w1_stride + (long long)j0 * a.Dpad;
        const long long r1 = (long long)(ok1 ? e1 : 0) * a.w1_stride + (long long)j1 * a.Dpad;
        float g0 = 0.0f, q0 = 0.0f, g1 = 0.0f, q1 = 0.0f;
        for (int c0 = 0; c0 < nch; c0 += 128) {
            const int c = c0 + lane;
            const bool va = c < nch, vb = c + 64 < nch;
            const int ca = min(c, nch - 1), cb = min(c + 64, nch - 1);
            const float4 xa = x4[ca], xb = x4[cb];
            const float4 ga0 = load_w4<WT>(a.w1, r0 + 4 * ca), gb0 = load_w4<WT>(a.w1, r0 + 4 * cb);
            const float4 ua0 = load_w4<WT>(a.w3, r0 + 4 * ca), ub0 = load_w4<WT>(a.w3, r0 + 4 * cb);
            const float4 ga1 = load_w4<WT>(a.w1, r1 + 4 * ca), gb1 = load_w4<WT>(a.w1, r1 + 4 * cb);
            const float4 ua1 = load_w4<WT>(a.w3, r1 + 4 * ca), ub1 = load_w4<WT>(a.w3, r1 + 4 * cb);
            const float4 xa_ = zero_unless(va, xa), xb_ = zero_unless(vb, xb);
            g0 = dot4_acc(g0, zero_unless(va, ga0), xa_);
            q0 = dot4_acc(q0, zero_unless(va, ua0), xa_);
            g1 = dot4_acc(g1, zero_unless(va, ga1), xa_);
            q1 = dot4_acc(q1, zero_unless(va, ua1), xa_);
            g0 = dot4_acc(g0, zero_unless(vb, gb0), xb_);
            q0 = dot4_acc(q0, zero_unless(vb, ub0), xb_);
            g1 = dot4_acc(g1, zero_unless(vb, gb1), xb_);
            q1 = dot4_acc(q1, zero_unless(vb, ub1), xb_);
        }
        g0 = wave_sum(g0);
        q0 = wave_sum(q0);
        g1 = wave_sum(g1);
        q1 = wave_sum(q1);
        if (lane == 0) {
            if (WT == WT_FP8) {
                if (ok0) {
                    g0 = g0 * a.s1[(long long)e0 * a.Hpad + j0];
                    q0 = q0 * a.s3[(long long)e0 * a.Hpad + j0];
                }
                if (ok1) {
                    g1 = g1 * a.s1[(long long)e1 * a.Hpad + j1];
                    q1 = q1 * a.s3[(long long)e1 * a.Hpad + j1];
                }
            }
            const long long hb = (long long)t * a.kt * a.Hpad;
            a.h[hb + u0] = ok0 ? (g0 * (1.0f / (1.0f + expf(-g0)))) * q0 : 0.0f;
            if (two) a.h[hb + u1] = ok1 ? (g1 * (1.0f / (1.0f + expf(-g1)))) * q1 : 0.0f;
        }
    }
}

// block (token t, y) routes t, then runs its waves' units
template <int WT>
__global__ __launch_bounds__(256) void decode_up_kernel(DecodeArgs a) {
    __shared__ DecodeRouteLds L;
    const int w = threadIdx.x >> 6;
    float gate;
    const DecodeSel sel = decode_route_block(a, blockIdx.x, blockIdx.y == 0 && w == 0, L, gate);
    decode_up_units<WT>(a, blockIdx.x, blockIdx.y * 4 + w, gridDim.y * 4, sel);
}

// ---- down: one wave per output row i of token t; slots two at a time, U
// chunks per lane and slot in flight (one batch covers rows of up to 256 U
// elements); the first batch's h loads do not depend on the routing and are
// issued before the slot's expert is read.  The slots' products are combined
// in slot order on a zero start.
template <int WT, int U>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 2))) void decode_down_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x;
    const int t = blockIdx.x, i = blockIdx.y;
    const int nch = a.Hpad >> 2;
    const float sw = a.lsh > 0 ? 1.0f / (float)a.lsh : 0.0f;  // shared_weight (inference.jl:201)
    float acc = 0.0f, sh = 0.0f;
    int s0 = 0;
    do {  // kt >= 1
        const bool two = s0 + 1 < a.kt;
        const int ts0 = t * a.kt + s0, ts1 = two ? ts0 + 1 : ts0;
        const float4 *h0 = (const float4 *)(a.h + (long long)ts0 * a.Hpad);
        const float4 *h1 = (const float4 *)(a.h + (long long)ts1 * a.Hpad);
        float4 ha[U], hb[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = min(u * 64 + lane, nch - 1);
            ha[u] = h0[c];
            hb[u] = h1[c];
        }
        __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the wait for idx
        const int e0 = a.idx[ts0] - 1, e1 = a.idx[ts1] - 1;
        const bool ok0 = e0 >= 0 && e0 < a.E + a.lsh, ok1 = two && e1 >= 0 && e1 < a.E + a.lsh;
        const long long r0 = (long long)(ok0 ? e0 : 0) * a.w2_stride + (long long)i * a.Hpad;
        const long long r1 = (long long)(ok1 ? e1 : 0) * a.w2_stride + (long long)i * a.Hpad;
        float y0 = 0.0f, y1 = 0.0f;
        for (int c0 = 0; c0 < nch; c0 += 64 * U) {
            float4 wa[U], wb[U];
            if (c0 > 0) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int c = min(c0 + u * 64 + lane, nch - 1);
                    ha[u] = h0[c];
                    hb[u] = h1[c];
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = min(c0 + u * 64 + lane, nch - 1);
                wa[u] = load_w4<WT>(a.w2, r0 + 4 * c);
                wb[u] = load_w4<WT>(a.w2, r1 + 4 * c);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const bool v = c0 + u * 64 + lane < nch;
                y0 = dot4_acc(y0, zero_unless(v, wa[u]), zero_unless(v, ha[u]));
                y1 = dot4_acc(y1, zero_unless(v, wb[u]), zero_unless(v, hb[u]));
            }
        }
        y0 = wave_sum(y0);
        y1 = wave_sum(y1);
        if (WT == WT_FP8) {
            if (ok0) y0 = y0 * a.s2[(long long)e0 * a.Dout_npad + i];
            if (ok1) y1 = y1 * a.s2[(long long)e1 * a.Dout_npad + i];
        }
        // routed slots: xb2 += gate * y in slot order (inference.jl:94-104);
        // shared slots: shared_output += shared_weight * y in order (:196-205)
        if (ok0) {
            if (s0 < a.lsh) sh = sh + sw * y0;
            else acc = acc + a.gates[ts0] * y0;
        }
        if (ok1) {
            if (s0 + 1 < a.lsh) sh = sh + sw * y1;
            else acc = acc + a.gates[ts1] * y1;
        }
        s0 += 2;
    } while (s0 < a.kt);
    // xb2 = 0.5 * shared + 0.5 * xb2 (:208-215)
    if (a.lsh > 0) acc = 0.5f * sh + 0.5f * acc;
    if (lane == 0) a.out[(long long)t * a.Dout + i] = acc;
}

template <int WT>
static hipError_t launch_decode_wt(const DecodeArgs &a, int ncu, hipStream_t s, hipEvent_t done) {
    const int tasks = (a.kt * a.Hpad + 1) / 2;                  // unit pairs per token
    const int gy = max(1, min((tasks + 3) / 4, max(1, 4 * ncu / a.n)));
    hipLaunchKernelGGL(decode_up_kernel<WT>, dim3(a.n, gy), dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // `done` is recorded by the down kernel's own completion (no marker packet
    // after it: that costs about 1 us of GPU time per call)
    const dim3 grid(a.n, a.Dout), block(64);
    if (a.Hpad <= 1024) hipExtLaunchKernelGGL((decode_down_kernel<WT, 4>), grid, block, 0, s, nullptr, done, 0, a);
    else hipExtLaunchKernelGGL((decode_down_kernel<WT, 8>), grid, block, 0, s, nullptr, done, 0, a);
    return hipGetLastError();
}

hipError_t launch_decode_ffn(const DecodeArgs &a, int ncu, hipStream_t s, hipEvent_t done) {
    if (a.n <= 0) return hipSuccess;
    if (a.E < 1 || a.E + a.lsh > MOE_MAX_EXPERTS || a.k < 1 || a.k > a.E || a.lsh < 0 || a.kt != a.k + a.lsh ||
        a.kt > MOE_MAX_TOPK)
        return hipErrorInvalidValue;
    // rows are read 4 elements at a time
    if (a.D < 4 || (a.D & 3) || (a.Dpad & 3) || (a.Hpad & 3) || a.D > a.Dpad || a.H > a.Hpad) return hipErrorInvalidValue;
    if (((uintptr_t)a.x & 15) || ((uintptr_t)a.h & 15)) return hipErrorInvalidValue;
    switch (a.wt) {
    case WT_F32: return launch_decode_wt<WT_F32>(a, ncu, s, done);
    case WT_BF16: return launch_decode_wt<WT_BF16>(a, ncu, s, done);
    default: return launch_decode_wt<WT_FP8>(a, ncu, s, done);
    }
}

}  // namespace moe
