// route_wide.hip — routing and dispatch of layers wider than the fast
// routing kernels take (more than 256 experts or top-k above 16), built
// with fp32 denormal flushing like the other routing kernels.  The same
// recipe, in general form:
//   logits     one FMA chain per (token, expert), k ascending from +0,
//              skipping x == 0 (src/matrix.c:381-400), then + bias;
//   finish     softmax_rows (src/matrix.c:529-586) with 8 lanes per token,
//              lane l the AVX2 accumulator lane l (elements 8b + l, b
//              ascending), the hsum256 tree, the scalar E % 8 tail; top-k
//              as src/transformer.c:317-337 (k rounds of argmax over the
//              experts not yet chosen, strict '>', best_e = 0 when nothing
//              beats -1), gate weights p * (1 / sum of the chosen p);
//   dispatch   the stable counting sort by expert (perm, counts, offsets,
//              the m-tile schedule) over chunks of 2048 assignments: chunk
//              histograms, a column scan per expert, and in-order placement
//              by one wave per chunk.
// These run only where the fast kernels' LDS and register tables end, so
// they favour plainness over speed.
#include <climits>

#include "moe_internal.h"
#include "moe_math.h"
#include "route_rows.h"

namespace moe {
namespace {

constexpr int kWlE = 64, kWlT = 32, kWlK = 256;   // logits tile: experts, tokens, k slice
constexpr int kWideChunk = 2048;                  // dispatch chunk (assignments)

// Workgroup (expert block blockIdx.x, token block blockIdx.y): lane = expert,
// wave w = tokens 8w .. 8w + 7 of the block; x rows pass through LDS one
// 256-wide k slice at a time and are read as wave-wide broadcasts.
__global__ __launch_bounds__(256) void wide_logits_kernel(RouteArgs a) {
    __shared__ float xs[kWlT][kWlK];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e = blockIdx.x * kWlE + lane;
    const int t0 = blockIdx.y * kWlT;
    const bool ev = e < a.E;
    const float *wcol = a.wr + (ev ? e : 0);
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    for (int k0 = 0; k0 < a.d; k0 += kWlK) {
        const int kc = min(kWlK, a.d - k0);
        __syncthreads();
        for (int i = threadIdx.x; i < kWlT * kWlK; i += 256) {
            const int tt = i / kWlK, kk = i - tt * kWlK, t = t0 + tt;
            xs[tt][kk] = (t < a.T && kk < kc) ? a.x[(size_t)t * a.d + k0 + kk] : 0.0f;
        }
        __syncthreads();
        for (int kk = 0; kk < kc; ++kk) {
            const float w = wcol[(size_t)(k0 + kk) * a.E];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float xv = xs[8 * wave + j][kk];
                acc[j] = xv != 0.0f ? fmaf(xv, w, acc[j]) : acc[j];
            }
        }
    }
    if (!ev) return;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int t = t0 + 8 * wave + j;
        if (t < a.T) a.probs[(size_t)t * a.E + e] = a.bias ? acc[j] + a.bias[e] : acc[j];
    }
}

// Dynamic LDS of the finish: per token its row [E], chosen bits [ceil(E/32)]
// and chosen experts [k].
size_t wide_finish_lds(int E, int k) {
    return sizeof(float) * 8 * ((size_t)E + (E + 31) / 32 + k);
}

// One wave = 8 tokens, 8 lanes each (lane l of token ct: threadIdx.x = 8 ct + l).
__global__ __launch_bounds__(64) void wide_finish_kernel(RouteArgs a) {
    extern __shared__ float wsm[];
    const int E = a.E, k = a.k, nw = (E + 31) / 32;
    const int ct = threadIdx.x >> 3, l = threadIdx.x & 7;
    const int t = blockIdx.x * 8 + ct;
    const bool tv = t < a.T;
    float *row = wsm + (size_t)ct * E;
    unsigned *chosen = reinterpret_cast<unsigned *>(wsm + (size_t)8 * E) + (size_t)ct * nw;
    int *sel = reinterpret_cast<int *>(wsm + (size_t)8 * (E + nw)) + (size_t)ct * k;
    const float *src = a.probs + (size_t)(tv ? t : 0) * E;
    for (int e = l; e < E; e += 8) row[e] = src[e];
    for (int w = l; w < nw; w += 8) chosen[w] = 0u;
    __syncthreads();

    const int nb = E >> 3, tail = E - 8 * nb;
    float m = -1e38f;
    for (int b = 0; b < nb; ++b) m = fmaxf(m, row[8 * b + l]);
    m = fmaxf(m, xor8f<4>(m));
    m = fmaxf(m, xor8f<2>(m));
    m = fmaxf(m, xor8f<1>(m));
    for (int j = 8 * nb; j < E; ++j) {
        const float v = row[j];
        if (v > m) m = v;
    }
    float vs = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const float ex = exp_poly(row[8 * b + l] - m);
        row[8 * b + l] = ex;
        vs = vs + ex;
    }
    vs = vs + xor8f<4>(vs);   // v_l + v_(l+4)
    vs = vs + xor8f<1>(vs);   // (v0+v4) + (v1+v5) and (v2+v6) + (v3+v7)
    vs = vs + xor8f<2>(vs);   // the two halves
    float tex = 0.0f;
    for (int j = 8 * nb; j < E; ++j) {
        const float ex = glibc_expf(row[j] - m);
        vs = vs + ex;
        if (j - 8 * nb == l) tex = ex;
    }
    const float inv = 1.0f / vs;
    for (int b = 0; b < nb; ++b) row[8 * b + l] = ftz_f(row[8 * b + l] * inv);
    if (l < tail) row[8 * nb + l] = ftz_f(tex * inv);
    __syncthreads();
    if (tv && a.probs)
        for (int e = l; e < E; e += 8) a.probs[(size_t)t * E + e] = row[e];

    float s = 0.0f;
    for (int ki = 0; ki < k; ++ki) {
        float best = -1.0f;
        int be = INT_MAX;
        for (int e = l; e < E; e += 8) {
            const float p = row[e];
            if (!((chosen[e >> 5] >> (e & 31)) & 1u) && p > best) { best = p; be = e; }
        }
        auto merge = [&](float ob, int oe) {
            if (ob > best || (ob == best && oe < be)) { best = ob; be = oe; }
        };
        merge(xor8f<4>(best), xor8<4>(be));
        merge(xor8f<2>(best), xor8<2>(be));
        merge(xor8f<1>(best), xor8<1>(be));
        float p = best;
        if (be == INT_MAX) {   // nothing beat -1: the reference keeps best_e = 0
            be = 0;
            p = row[0];
        }
        s = s + p;
        if (l == 0) {
            chosen[be >> 5] |= 1u << (be & 31);
            sel[ki] = be;
        }
        __syncthreads();
    }
    const float inv_s = (s > 1e-9f) ? 1.0f / s : 0.0f;
    if (!tv) return;
    for (int ki = l; ki < k; ki += 8) {
        const int e = sel[ki];
        a.ids[(size_t)t * k + ki] = e;
        if (a.gw) a.gw[(size_t)t * k + ki] = ftz_f(row[e] * inv_s);
    }
}

// Chunk c's count of each expert: ccount[c][e].
__global__ __launch_bounds__(256) void wide_hist_kernel(DispatchArgs d, int *ccount) {
    extern __shared__ int hist[];
    for (int e = threadIdx.x; e < d.E; e += 256) hist[e] = 0;
    __syncthreads();
    const size_t a0 = (size_t)blockIdx.x * kWideChunk;
    for (int i = threadIdx.x; i < kWideChunk; i += 256) {
        const size_t a = a0 + i;
        if (a < (size_t)d.n) atomicAdd(&hist[min(max(d.ids[a], 0), d.E - 1)], 1);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < d.E; e += 256) ccount[(size_t)blockIdx.x * d.E + e] = hist[e];
}

// Per expert: ccount[c][e] becomes the count in chunks before c; counts[e]
// the total.
__global__ __launch_bounds__(256) void wide_colscan_kernel(DispatchArgs d, int *ccount, int nchunk) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= d.E) return;
    int run = 0;
    for (int c = 0; c < nchunk; ++c) {
        const int v = ccount[(size_t)c * d.E + e];
        ccount[(size_t)c * d.E + e] = run;
        run += v;
    }
    d.counts[e] = run;
}

// One workgroup: offsets (exclusive scan of counts), the m-tile prefix
// tile_off and the expert of every m-tile.  Thread i takes experts
// 4i .. 4i + 3 (E <= 4096).
__global__ __launch_bounds__(1024) void wide_offsets_kernel(DispatchArgs d) {
    __shared__ int2 sc[1024];
    const int i = threadIdx.x;
    int c[4], tl[4];
    int2 own = make_int2(0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * i + j;
        c[j] = e < d.E ? d.counts[e] : 0;
        tl[j] = (c[j] + d.bm - 1) / d.bm;
        own.x += c[j];
        own.y += tl[j];
    }
    sc[i] = own;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {   // inclusive scan (Hillis-Steele)
        const int2 v = i >= off ? sc[i - off] : make_int2(0, 0);
        __syncthreads();
        sc[i] = make_int2(sc[i].x + v.x, sc[i].y + v.y);
        __syncthreads();
    }
    int2 base = i > 0 ? sc[i - 1] : make_int2(0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * i + j;
        if (e < d.E) {
            d.offsets[e] = base.x;
            d.tile_off[e] = base.y;
            if (d.tile_expert)
                for (int q = 0; q < tl[j]; ++q) d.tile_expert[base.y + q] = e;
        }
        base.x += c[j];
        base.y += tl[j];
    }
    if (i == 1023) {
        d.offsets[d.E] = sc[1023].x;
        d.tile_off[d.E] = sc[1023].y;
    }
}

// One wave per chunk places its assignments in order: run[e] starts at
// offsets[e] + the count in earlier chunks; each group of 64 ranks a lane
// among the earlier lanes of its expert, and the group's last lane of an
// expert advances run[e].
__global__ __launch_bounds__(64) void wide_place_kernel(DispatchArgs d, const int *ccount) {
    extern __shared__ int run[];
    const int lane = threadIdx.x;
    for (int e = lane; e < d.E; e += 64)
        run[e] = d.offsets[e] + ccount[(size_t)blockIdx.x * d.E + e];
    __syncthreads();
    const size_t a0 = (size_t)blockIdx.x * kWideChunk;
    for (int g = 0; g < kWideChunk; g += 64) {
        const size_t a = a0 + g + lane;
        const bool valid = a < (size_t)d.n;
        const int e = valid ? min(max(d.ids[a], 0), d.E - 1) : -1;
        int rank = 0, after = 0;
        for (int j = 0; j < 64; ++j) {
            const int ej = __shfl(e, j);
            if (ej == e) {
                rank += j < lane;
                after += j > lane;
            }
        }
        if (valid) {
            d.perm[run[e] + rank] = (int)a;
        }
        __syncthreads();
        if (valid && after == 0) run[e] += rank + 1;
        __syncthreads();
    }
}

}  // namespace

size_t wide_dispatch_ints(size_t n, int E) {
    return ((n + kWideChunk - 1) / kWideChunk) * (size_t)E;
}

bool route_wide_ok(int E, int k) {
    return E >= 1 && E <= kWideMaxExperts && k >= 1 && k <= E && k <= kWideMaxTopK &&
           wide_finish_lds(E, k) <= 160 * 1024;
}

hipError_t launch_route_wide(const RouteArgs &a, const DispatchArgs &da, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    if (!route_wide_ok(a.E, a.k) || !a.probs || !a.ids) return hipErrorInvalidValue;
    if (a.rms_w) {
        hipError_t e = launch_rms_norm(a.x_raw, a.rms_w, a.rms_eps, a.T, a.d, a.xn_out, s);
        if (e != hipSuccess) return e;
    }
    const size_t lds = wide_finish_lds(a.E, a.k);
    static size_t attr = 0;
    if (lds > attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&wide_finish_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr = lds;
    }
    hipLaunchKernelGGL(wide_logits_kernel, dim3((unsigned)((a.E + kWlE - 1) / kWlE), (unsigned)((a.T + kWlT - 1) / kWlT)),
                       dim3(256), 0, s, a);
    hipLaunchKernelGGL(wide_finish_kernel, dim3((unsigned)((a.T + 7) / 8)), dim3(64), lds, s, a);
    if (a.no_dispatch) return hipGetLastError();
    if (!da.wide || !da.counts || !da.offsets || !da.tile_off || !da.perm || da.n <= 0)
        return hipErrorInvalidValue;
    const int nchunk = (int)((da.n + kWideChunk - 1) / kWideChunk);
    const size_t elds = sizeof(int) * (size_t)da.E;
    hipLaunchKernelGGL(wide_hist_kernel, dim3((unsigned)nchunk), dim3(256), elds, s, da, da.wide);
    hipLaunchKernelGGL(wide_colscan_kernel, dim3((unsigned)((da.E + 255) / 256)), dim3(256), 0, s, da,
                       da.wide, nchunk);
    hipLaunchKernelGGL(wide_offsets_kernel, dim3(1), dim3(1024), 0, s, da);
    hipLaunchKernelGGL(wide_place_kernel, dim3((unsigned)nchunk), dim3(64), elds, s, da,
                       (const int *)da.wide);
    return hipGetLastError();
}

}  // namespace moe
