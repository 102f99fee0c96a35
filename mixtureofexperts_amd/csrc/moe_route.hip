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
#include <climits>

#include "moe_internal.h"

namespace moe {

// ============================================================================
// Router logits: logits[t][e] = sum_d x[t][d] * W[d][e] (+ bias[e]), fp32.
// W is the Flux weight memory [D][Er_pad] (experts contiguous per feature).
// A block of 4 waves handles 16 tokens (4 per wave); each lane walks the
// feature axis 4 at a time, experts in chunks of 8.
// ============================================================================
template <int XBF16>
__global__ __launch_bounds__(256) void router_logits_kernel(const void *__restrict__ xv, int T,
                                                            int D, int Er, int Er_pad,
                                                            const float *__restrict__ w,
                                                            const float *__restrict__ bias,
                                                            float *__restrict__ logits) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 16 + wave * 4;
    if (t0 >= T) return;
    for (int e0 = 0; e0 < Er; e0 += 8) {
        float acc[4][8];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[j][c] = 0.0f;
        for (int d0 = lane * 4; d0 < D; d0 += 256) {
            float xv4[4][4];
            const int nd = min(4, D - d0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = min(t0 + j, T - 1);
                if (XBF16) {
                    const uint16_t *xr = (const uint16_t *)xv + (long long)t * D + d0;
                    if (nd == 4 && (D & 3) == 0) {
                        uint2 p = *(const uint2 *)xr;
                        xv4[j][0] = bf16_to_f32((uint16_t)(p.x & 0xffff));
                        xv4[j][1] = bf16_to_f32((uint16_t)(p.x >> 16));
                        xv4[j][2] = bf16_to_f32((uint16_t)(p.y & 0xffff));
                        xv4[j][3] = bf16_to_f32((uint16_t)(p.y >> 16));
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) xv4[j][i] = (i < nd) ? bf16_to_f32(xr[i]) : 0.0f;
                    }
                } else {
                    const float *xr = (const float *)xv + (long long)t * D + d0;
                    if (nd == 4 && (D & 3) == 0) {
                        float4 p = *(const float4 *)xr;
                        xv4[j][0] = p.x; xv4[j][1] = p.y; xv4[j][2] = p.z; xv4[j][3] = p.w;
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) xv4[j][i] = (i < nd) ? xr[i] : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (i < nd) {
                    const float4 *wr = (const float4 *)(w + (long long)(d0 + i) * Er_pad + e0);
                    float4 wa = wr[0], wb = wr[1];
                    float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int c = 0; c < 8; ++c) acc[j][c] = __builtin_fmaf(xv4[j][i], wv[c], acc[j][c]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                float v = acc[j][c];
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
                acc[j][c] = v;
            }
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = t0 + j;
                if (t < T) {
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const int e = e0 + c;
                        if (e < Er) logits[(long long)t * Er + e] = acc[j][c] + (bias ? bias[e] : 0.0f);
                    }
                }
            }
        }
    }
}

hipError_t launch_router_logits(const void *x, int x_bf16, int T, int D, int Er, int Er_pad,
                                const float *wr, const float *bias, float *logits, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    dim3 grid((T + 15) / 16), block(256);
    if (x_bf16)
        hipLaunchKernelGGL(router_logits_kernel<1>, grid, block, 0, s, x, T, D, Er, Er_pad, wr, bias, logits);
    else
        hipLaunchKernelGGL(router_logits_kernel<0>, grid, block, 0, s, x, T, D, Er, Er_pad, wr, bias, logits);
    return hipGetLastError();
}

// ============================================================================
// Gating.  One thread per token, 256 tokens per block.
// ============================================================================

// NNlib.softmax over l[0..n) into p (global), recipe:
//   m = max (NaN ignored); e = (float)exp((double)(l - m)) (NNlib's branch for
//   m == +Inf: e = l == +Inf); s = sequential fp32 sum; p = e / s.
// Returns s and m so the caller can form logsumexp.
__device__ inline void softmax_row(const float *__restrict__ l, int n, float *__restrict__ p,
                                   float &m_out, float &s_out) {
#pragma clang fp contract(off)
    float m = -INFINITY;
    for (int i = 0; i < n; ++i) {
        const float v = l[i];
        if (v > m) m = v;
    }
    float s = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float v = l[i];
        float e;
        if (m == INFINITY)
            e = (v == INFINITY) ? 1.0f : 0.0f;
        else
            e = (float)exp((double)(v - m));
        p[i] = e;
        s = s + e;
    }
    for (int i = 0; i < n; ++i) p[i] = p[i] / s;
    m_out = m;
    s_out = s;
}

// Top-k by the isless key, descending, lower index first on ties; then the
// gates p_sel ./ sum(p_sel) with the sum in slot order.
__device__ inline void topk_row(const float *__restrict__ p, int n, int k, int *sel, float *g) {
#pragma clang fp contract(off)
    uint64_t taken0 = 0, taken1 = 0;
    for (int j = 0; j < k; ++j) {
        int best = -1;
        uint32_t bk = 0;
        for (int i = 0; i < n; ++i) {
            const bool taken = (i < 64) ? ((taken0 >> i) & 1ull) : ((taken1 >> (i - 64)) & 1ull);
            if (taken) continue;
            const uint32_t key = isless_key(p[i]);
            if (best < 0 || key > bk) { best = i; bk = key; }
        }
        if (best < 64) taken0 |= 1ull << best; else taken1 |= 1ull << (best - 64);
        sel[j] = best;
    }
    float s = p[sel[0]];
    for (int j = 1; j < k; ++j) s = s + p[sel[j]];
    for (int j = 0; j < k; ++j) g[j] = p[sel[j]] / s;
}

__global__ __launch_bounds__(kRouteBlock) void route_kernel(RouteArgs a) {
#pragma clang fp contract(off)
    __shared__ int wcnt[kRouteBlock / 64][MOE_MAX_EXPERTS];
    __shared__ double red[2][kRouteBlock];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int t = blockIdx.x * kRouteBlock + tid;
    const bool valid = t < a.T;

    for (int i = tid; i < (kRouteBlock / 64) * MOE_MAX_EXPERTS; i += kRouteBlock) (&wcnt[0][0])[i] = 0;

    int ex[MOE_MAX_TOPK];     // 1-based expert ids of this token's slots
    double zterm = 0.0, hterm = 0.0;
#pragma unroll
    for (int j = 0; j < MOE_MAX_TOPK; ++j) ex[j] = 0;

    if (valid) {
        const float *l = a.logits + (long long)t * a.Er;
        float *p = a.probs + (long long)t * a.E;
        int sel[MOE_MAX_TOPK];
        float g[MOE_MAX_TOPK];
        float m, s;
        if (a.gate_kind == MOE_GATE_SHARED) {
            const int ns = a.ns, Eall = a.E;
            softmax_row(l + ns, Eall - ns, p + ns, m, s);
            topk_row(p + ns, Eall - ns, a.k, sel, g);
            const int tk = a.kt;
            const double gscale = 1.0 - (double)ns / (double)tk;
            const double pscale = 1.0 - (double)ns / (double)Eall;
            const float gshared = 1.0f / (float)tk;
            const float pshared = 1.0f / (float)Eall;
            for (int j = 0; j < ns; ++j) {
                ex[j] = j + 1;
                a.gates[(long long)t * tk + j] = gshared;
            }
            for (int j = 0; j < a.k; ++j) {
                ex[ns + j] = sel[j] + ns + 1;
                a.gates[(long long)t * tk + ns + j] = (float)((double)g[j] * gscale);
            }
            for (int i = 0; i < ns; ++i) p[i] = pshared;
            for (int i = ns; i < Eall; ++i) p[i] = (float)((double)p[i] * pscale);
            // z-loss runs over every router row (src/core/moe_layer.jl:117-121)
            float mz = -INFINITY;
            for (int i = 0; i < a.Er; ++i) if (l[i] > mz) mz = l[i];
            float sz = 0.0f;
            for (int i = 0; i < a.Er; ++i) sz = sz + (float)exp((double)(l[i] - mz));
            m = mz;
            s = sz;
        } else {
            softmax_row(l, a.E, p, m, s);
            topk_row(p, a.E, a.k, sel, g);
            for (int j = 0; j < a.k; ++j) {
                ex[j] = sel[j] + 1;
                a.gates[(long long)t * a.kt + j] = g[j];
            }
        }
        for (int j = 0; j < a.kt; ++j) a.idx[(long long)t * a.kt + j] = ex[j];
        // logsumexp (src/balancing/losses.jl:111-114) from the same exp recipe
        const float lse = m + (float)log((double)s);
        zterm = (double)(lse * lse);
        // entropy of update_stats! in Float64
        double hs = 0.0;
        for (int i = 0; i < a.E; ++i) {
            const double pv = (double)p[i];
            hs = hs + pv * log(pv + 1e-8);
        }
        hterm = -hs;
    }
    __syncthreads();

    // ---- stable rank of each entry among the block's entries of its expert ----
    int r[MOE_MAX_TOPK];
    unsigned done = 0;
#pragma unroll
    for (int j = 0; j < MOE_MAX_TOPK; ++j) {
        r[j] = 0;
        if (j >= a.kt || ex[j] <= 0) done |= 1u << j;
    }
    const unsigned all = (1u << MOE_MAX_TOPK) - 1u;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    while (true) {
        const bool has = done != all;
        const uint64_t act = __ballot(has);
        if (act == 0) break;
        const int leader = __ffsll((unsigned long long)act) - 1;
        int mine = 0;
        if (has) {
            const int j0 = __ffs(~done & all) - 1;
            mine = ex[j0];
        }
        const int estar = __shfl(mine, leader);
        int js = -1;
#pragma unroll
        for (int j = 0; j < MOE_MAX_TOPK; ++j)
            if (!((done >> j) & 1u) && ex[j] == estar) js = j;
        const uint64_t mm = __ballot(js >= 0);
        if (js >= 0) {
#pragma unroll
            for (int j = 0; j < MOE_MAX_TOPK; ++j)
                if (j == js) r[j] = __popcll(mm & lt_mask);
            done |= 1u << js;
        }
        if (lane == leader) wcnt[wave][estar - 1] = __popcll(mm);
    }
    __syncthreads();
    if (valid) {
#pragma unroll
        for (int j = 0; j < MOE_MAX_TOPK; ++j) {
            if (j < a.kt) {
                int base = 0;
                if (ex[j] > 0)
                    for (int w = 0; w < wave; ++w) base += wcnt[w][ex[j] - 1];
                a.rank[(long long)t * a.kt + j] = base + r[j];
            }
        }
    }
    const int nb = blockIdx.x;
    for (int e = tid; e < a.E; e += kRouteBlock) {
        int c = 0;
        for (int w = 0; w < kRouteBlock / 64; ++w) c += wcnt[w][e];
        a.blk_counts[(long long)nb * a.E + e] = c;
        // per-expert probability sums (Switch loss P_e) in fp64, token order
        double ps = 0.0;
        const int tend = min(kRouteBlock, a.T - nb * kRouteBlock);
        for (int i = 0; i < tend; ++i) ps += (double)a.probs[(long long)(nb * kRouteBlock + i) * a.E + e];
        a.blk_stats[(long long)nb * (a.E + 2) + e] = ps;
    }
    red[0][tid] = zterm;
    red[1][tid] = hterm;
    __syncthreads();
    for (int st = kRouteBlock / 2; st > 0; st >>= 1) {
        if (tid < st) {
            red[0][tid] += red[0][tid + st];
            red[1][tid] += red[1][tid + st];
        }
        __syncthreads();
    }
    if (tid == 0) {
        a.blk_stats[(long long)nb * (a.E + 2) + a.E] = red[0][0];
        a.blk_stats[(long long)nb * (a.E + 2) + a.E + 1] = red[1][0];
    }
}

hipError_t launch_route(const RouteArgs &a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    const int nblk = (a.T + kRouteBlock - 1) / kRouteBlock;
    hipLaunchKernelGGL(route_kernel, dim3(nblk), dim3(kRouteBlock), 0, s, a);
    return hipGetLastError();
}

// ============================================================================
// Scan: one block.  Per-expert totals, capacity clamp, offsets, per-block rank
// bases, the (expert, m0) GEMM tile list and the loss scalars.
// ============================================================================
__global__ __launch_bounds__(256) void scan_kernel(ScanArgs a) {
#pragma clang fp contract(off)
    __shared__ int cnt[MOE_MAX_EXPERTS];
    __shared__ int off[MOE_MAX_EXPERTS + 1];
    __shared__ int tstart[MOE_MAX_EXPERTS + 1];
    __shared__ double psum[MOE_MAX_EXPERTS];
    __shared__ int cap_s;
    const int tid = threadIdx.x;
    if (tid == 0) {
        int cap = INT_MAX;
        if (a.training && a.drop) {
            // capacity = ceil(Int, capacity_factor * batch_size / num_experts), Float32
            const float c = ceilf((a.capacity_factor * (float)a.T) / (float)a.E);
            cap = (c >= 2147483647.0f) ? INT_MAX : (int)c;
        }
        cap_s = cap;
        a.cap_out[0] = cap;
    }
    __syncthreads();
    for (int e = tid; e < a.E; e += blockDim.x) {
        int run = 0;
        double ps = 0.0;
        for (int b = 0; b < a.nblk; ++b) {
            a.rank_base[(long long)b * a.E + e] = run;
            run += a.blk_counts[(long long)b * a.E + e];
            ps += a.blk_stats[(long long)b * (a.E + 2) + e];
        }
        cnt[e] = min(run, cap_s);
        psum[e] = ps;
    }
    __syncthreads();
    if (tid == 0) {
        int o = 0, ts = 0;
        for (int e = 0; e < a.E; ++e) {
            off[e] = o;
            tstart[e] = ts;
            o += cnt[e];
            ts += (cnt[e] + a.bm - 1) / a.bm;
        }
        off[a.E] = o;
        tstart[a.E] = ts;
        a.num_tiles[0] = ts;

        // losses (src/balancing/losses.jl:15-36, 103-114)
        double zs = 0.0, hs = 0.0;
        for (int b = 0; b < a.nblk; ++b) {
            zs += a.blk_stats[(long long)b * (a.E + 2) + a.E];
            hs += a.blk_stats[(long long)b * (a.E + 2) + a.E + 1];
        }
        const float total = (float)((long long)a.T * a.kt);
        float s = 0.0f;
        for (int e = 0; e < a.E; ++e) {
            float f = (float)cnt[e];
            if (a.T * a.kt > 0) f = f / total;
            const float P = (float)psum[e] / (float)a.T;
            const float fp = f * P;
            s = (e == 0) ? fp : s + fp;
        }
        const float sw = (a.alpha * (float)a.E) * s;
        const float z = a.beta * ((float)zs / (float)a.T);
        float loss = 0.0f;
        if (a.training) loss = a.z_enabled ? sw + z : sw;
        a.scalars[0] = a.training ? sw : 0.0f;
        a.scalars[1] = (a.training && a.z_enabled) ? z : 0.0f;
        a.scalars[2] = loss;
        a.scalars[3] = (float)(hs / (double)a.T);
        if (a.loss_out) a.loss_out[0] = loss;
    }
    __syncthreads();
    for (int e = tid; e <= a.E; e += blockDim.x) {
        a.offsets[e] = off[e];
        a.tile_start[e] = tstart[e];
    }
    for (int e = tid; e < a.E; e += blockDim.x) {
        a.counts[e] = cnt[e];
        const int nt = tstart[e + 1] - tstart[e];
        for (int i = 0; i < nt; ++i) a.tiles[tstart[e] + i] = make_int2(e, i * a.bm);
    }
}

hipError_t launch_scan(const ScanArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(256), 0, s, a);
    return hipGetLastError();
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
    int e = 0, pos = -1;
    float g = 0.0f;
    if (lane < a.kt) {
        const long long ent = (long long)t * a.kt + lane;
        e = a.idx[ent];
        g = a.gates[ent];
        if (e > 0 && e <= a.E) {
            const int rk = a.rank_base[(long long)blk * a.E + (e - 1)] + a.rank[ent];
            if (rk < cap) {
                pos = a.offsets[e - 1] + rk;
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
    for (int j = 0; j < a.kt; ++j) {
        const int p = __shfl(pos, j);
        if (p < 0) continue;
        if (a.ct == CT_BF16) {
            uint16_t *dst = (uint16_t *)a.xp + (long long)p * a.ld_xp;
            if (a.x_bf16) {
                const uint16_t *src = (const uint16_t *)a.x + (long long)t * a.D;
                if ((a.D & 7) == 0) {
                    for (int d = lane * 8; d < a.D; d += 512)
                        *(uint4 *)(dst + d) = *(const uint4 *)(src + d);
                } else {
                    for (int d = lane; d < a.D; d += 64) dst[d] = src[d];
                }
            } else {
                const float *src = (const float *)a.x + (long long)t * a.D;
                for (int d = lane; d < a.D; d += 64) dst[d] = f32_to_bf16(src[d]);
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

hipError_t launch_permute(const PermuteArgs &a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    hipLaunchKernelGGL(permute_kernel, dim3((a.T + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ============================================================================
// Combine: one wave per token.  out[t] = sum over the token's entries in
// ascending expert order of gate * y, as separate fp32 multiply and add on a
// zero start (src/core/moe_layer.jl:132, 205-217).  No atomics.
// ============================================================================
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
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
    // y row of an entry: the sum, in split order, of the down GEMM's K-range partials
    if ((a.D & 3) == 0 && (a.ld_y & 3) == 0) {
        for (int d = lane * 4; d < a.D; d += 256) {
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            for (int i = 0; i < n; ++i) {
                const float *yr = a.y + (long long)pp[i] * a.ld_y + d;
                float4 v = *(const float4 *)yr;
                for (int sp = 1; sp < a.nsplit; ++sp) {
                    const float4 u = *(const float4 *)(yr + sp * a.split_stride);
                    v.x = v.x + u.x; v.y = v.y + u.y; v.z = v.z + u.z; v.w = v.w + u.w;
                }
                const float g = gg[i];
                acc.x = acc.x + g * v.x;
                acc.y = acc.y + g * v.y;
                acc.z = acc.z + g * v.z;
                acc.w = acc.w + g * v.w;
            }
            *(float4 *)(o + d) = acc;
        }
    } else {
        for (int d = lane; d < a.D; d += 64) {
            float acc = 0.0f;
            for (int i = 0; i < n; ++i) {
                const float *yr = a.y + (long long)pp[i] * a.ld_y + d;
                float v = yr[0];
                for (int sp = 1; sp < a.nsplit; ++sp) v = v + yr[sp * a.split_stride];
                acc = acc + gg[i] * v;
            }
            o[d] = acc;
        }
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
// compute_loss(::SwitchTransformerLoss, indices, probs): one block.
__global__ __launch_bounds__(256) void switch_loss_kernel(const int *idx, int T, int k, const float *probs, int E,
                                                          float alpha, int *cnt_ws, float *out) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += 256) cnt_ws[e] = 0;
    __syncthreads();
    for (long long i = tid; i < (long long)T * k; i += 256) {
        const int e = idx[i];
        if (e > 0 && e <= E) atomicAdd(&cnt_ws[e - 1], 1);
    }
    __syncthreads();
    if (tid == 0) {
        const float total = (float)((long long)T * k);
        float s = 0.0f;
        for (int e = 0; e < E; ++e) {
            double ps = 0.0;
            for (int t = 0; t < T; ++t) ps += (double)probs[(long long)t * E + e];
            float f = (float)cnt_ws[e];
            if ((long long)T * k > 0) f = f / total;
            const float P = (float)ps / (float)T;
            const float fp = f * P;
            s = (e == 0) ? fp : s + fp;
        }
        out[0] = (alpha * (float)E) * s;
    }
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
        const float lse = m + (float)log((double)s);
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

hipError_t launch_switch_loss(const int *idx, int T, int k, const float *probs, int E, float alpha, int *cnt_ws,
                              float *out, hipStream_t s) {
    hipLaunchKernelGGL(switch_loss_kernel, dim3(1), dim3(256), 0, s, idx, T, k, probs, E, alpha, cnt_ws, out);
    return hipGetLastError();
}

hipError_t launch_z_loss(const float *logits, int T, int E, float beta, float *out, hipStream_t s) {
    hipLaunchKernelGGL(z_loss_kernel, dim3(1), dim3(256), 0, s, logits, T, E, beta, out);
    return hipGetLastError();
}

}  // namespace moe
