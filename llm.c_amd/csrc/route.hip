// route.hip — router logits, softmax, top-k gating and the stable expert
// dispatch for gfx950.
//
// Bit-exactness contract (reference paths relative to the reference root):
//  * logits: one fused-multiply-add chain per (token, expert), k ascending
//    from +0.0f, skipping x == 0 — the AVX2+FMA mat_mul (src/matrix.c:381-400
//    with axpy_avx2fma :278-303).  Register-blocked VALU FMAs keep every
//    accumulator its own ascending chain, so blocking changes no bit.
//  * softmax: softmax_rows (src/matrix.c:529-586): 8-lane blocks through the
//    exp_avx2 polynomial (:82-116) with lane sums folded in hsum256 order
//    (include/simd.h:110-121), glibc expf on the E % 8 tail, 1/sum times each.
//  * top-k: src/transformer.c:317-337 (strict '>', best = -1, ties -> lowest
//    expert, renormalised gate weights).
//  * The reference executables run with FTZ/DAZ (-ffast-math startup code);
//    this file is built with fp32 denormal flushing and the explicit flushes
//    below mirror that.
//  * dispatch: stable counting sort of the (token, slot) assignments by expert
//    through per-wave LDS histograms, an exclusive scan and ballot ranks.
#include "moe_internal.h"
#include "moe_math.h"

namespace moe {
namespace {

// Softmax of one row in place (src/matrix.c:529-586, AVX2+FMA build, with
// the tail division compiled as a multiply by 1/sum).
__device__ inline void softmax_row(float *row, int E) {
    int nb = E >> 3;
    float lane_max[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) lane_max[l] = -1e38f;
    for (int b = 0; b < nb; ++b)
#pragma unroll
        for (int l = 0; l < 8; ++l) lane_max[l] = fmaxf(lane_max[l], row[8 * b + l]);
    float mx = lane_max[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) mx = fmaxf(mx, lane_max[l]);
    for (int j = nb * 8; j < E; ++j) if (row[j] > mx) mx = row[j];

    float vs[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) vs[l] = 0.0f;
    for (int b = 0; b < nb; ++b)
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            float ex = exp_poly(row[8 * b + l] - mx);
            row[8 * b + l] = ex;
            vs[l] = vs[l] + ex;
        }
    float sum = ((vs[0] + vs[4]) + (vs[1] + vs[5])) + ((vs[2] + vs[6]) + (vs[3] + vs[7]));
    for (int j = nb * 8; j < E; ++j) {
        float ex = glibc_expf(row[j] - mx);
        row[j] = ex;
        sum = sum + ex;
    }
    float inv = 1.0f / sum;
    for (int j = 0; j < E; ++j) row[j] = ftz_f(row[j] * inv);
}

constexpr int kRouteTM = 32;   // tokens per workgroup
constexpr int kRouteKT = 32;   // K slice staged per step

// One workgroup: 32 tokens x all experts.  Thread (tx, ty) owns tokens
// ty + 16 i (i < 2) and experts tx + 16 j (j < RE).
template <int RE>
__global__ __launch_bounds__(256) void router_kernel(RouteArgs a) {
    constexpr int EP = 16 * RE;
    __shared__ float xs[kRouteKT][kRouteTM + 1];
    __shared__ float ws[kRouteKT][EP];
    __shared__ float lg[kRouteTM][EP + 1];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int t0 = blockIdx.x * kRouteTM;
    const int T = a.T, d = a.d, E = a.E;

    float acc[2][RE];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < RE; ++j) acc[i][j] = 0.0f;

    for (int k0 = 0; k0 < d; k0 += kRouteKT) {
        // x tile, transposed into xs[k][token]; out-of-range reads as 0,
        // which the zero-skip turns into "no update" (exact padding).
        for (int idx = tid; idx < kRouteTM * kRouteKT; idx += 256) {
            int r = idx / kRouteKT, c = idx % kRouteKT;
            float v = 0.0f;
            int t = t0 + r, kk = k0 + c;
            if (t < T && kk < d) v = a.x[(size_t)t * d + kk];
            uint32_t u = __float_as_uint(v);
            if ((u & 0x7f800000u) == 0u) v = 0.0f;     // DAZ
            xs[c][r] = v;
        }
        for (int idx = tid; idx < kRouteKT * EP; idx += 256) {
            int r = idx / EP, c = idx % EP;
            float v = 0.0f;
            int kk = k0 + r;
            if (kk < d && c < E) v = a.wr[(size_t)kk * E + c];
            ws[r][c] = ftz_f(v);
        }
        __syncthreads();
#pragma unroll 4
        for (int kk = 0; kk < kRouteKT; ++kk) {
            float xv0 = xs[kk][ty];
            float xv1 = xs[kk][ty + 16];
#pragma unroll
            for (int j = 0; j < RE; ++j) {
                float wv = ws[kk][tx + 16 * j];
                acc[0][j] = (xv0 != 0.0f) ? fmaf(xv0, wv, acc[0][j]) : acc[0][j];
                acc[1][j] = (xv1 != 0.0f) ? fmaf(xv1, wv, acc[1][j]) : acc[1][j];
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < RE; ++j) {
            int e = tx + 16 * j;
            if (e < E) {
                float v = acc[i][j];
                if (a.bias) v = v + a.bias[e];
                lg[ty + 16 * i][e] = v;
            }
        }
    __syncthreads();

    // One thread per token: softmax, top-k, gate weights.
    if (tid < kRouteTM && t0 + tid < T) {
        const int t = t0 + tid;
        float *row = &lg[tid][0];
        softmax_row(row, E);
        int ids[kMaxTopK];
        const int k = a.k;
        for (int ki = 0; ki < k; ++ki) {
            float best = -1.0f;
            int best_e = 0;
            for (int e = 0; e < E; ++e) {
                bool already = false;
                for (int kj = 0; kj < ki; ++kj)
                    if (ids[kj] == e) { already = true; break; }
                if (!already && row[e] > best) { best = row[e]; best_e = e; }
            }
            ids[ki] = best_e;
        }
        float s = 0.0f;
        for (int ki = 0; ki < k; ++ki) s = s + row[ids[ki]];
        float inv = (s > 1e-9f) ? 1.0f / s : 0.0f;
        for (int ki = 0; ki < k; ++ki) {
            if (a.ids) a.ids[(size_t)t * k + ki] = ids[ki];
            if (a.gw) a.gw[(size_t)t * k + ki] = ftz_f(row[ids[ki]] * inv);
        }
    }
    __syncthreads();
    if (a.probs) {
        for (int idx = tid; idx < kRouteTM * E; idx += 256) {
            int r = idx / E, e = idx % E;
            if (t0 + r < T) a.probs[(size_t)(t0 + r) * E + e] = lg[r][e];
        }
    }
}

// ---------------------------------------------------------------------------
// Dispatch: one workgroup of 16 waves.  Wave w owns the contiguous run
// [w*chunk, (w+1)*chunk) of the flattened assignments a = t*k + slot.
//   pass 1: per-wave expert histograms in LDS;
//   scan:   counts, offsets (exclusive), per-(wave, expert) bases in
//           expert-major, wave-minor order;
//   pass 2: each wave walks its run in order; a lane's rank among earlier
//           lanes with the same expert comes from bit-sliced ballots.
// The result is the stable counting sort: pos(a) = offsets[e] + #{a' < a
// with the same expert}.
// ---------------------------------------------------------------------------
constexpr int kDispWaves = 16;

__global__ __launch_bounds__(1024) void dispatch_kernel(DispatchArgs a) {
    __shared__ int hist[kDispWaves][kMaxExperts];
    __shared__ int offs[kMaxExperts + 1];
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int E = a.E, n = a.n;
    for (int i = tid; i < kDispWaves * kMaxExperts; i += 1024) (&hist[0][0])[i] = 0;
    __syncthreads();

    const int chunk = ((n + kDispWaves * 64 - 1) / (kDispWaves * 64)) * 64;
    const int beg = w * chunk;
    const int end = min(n, beg + chunk);
    for (int i = beg + lane; i < end; i += 64) atomicAdd(&hist[w][a.ids[i]], 1);
    __syncthreads();

    if (tid < E) {
        int c = 0;
        for (int ww = 0; ww < kDispWaves; ++ww) c += hist[ww][tid];
        a.counts[tid] = c;
        offs[tid + 1] = c;
    }
    __syncthreads();
    if (tid == 0) {
        offs[0] = 0;
        int tiles = 0;
        a.tile_off[0] = 0;
        for (int e = 0; e < E; ++e) {
            int c = offs[e + 1];
            offs[e + 1] = offs[e] + c;
            tiles += (c + a.bm - 1) / a.bm;
            a.tile_off[e + 1] = tiles;
        }
        for (int e = 0; e <= E; ++e) a.offsets[e] = offs[e];
    }
    __syncthreads();
    if (tid < E) {
        int base = offs[tid];
        for (int ww = 0; ww < kDispWaves; ++ww) {
            int c = hist[ww][tid];
            hist[ww][tid] = base;
            base += c;
        }
    }
    __syncthreads();

    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int i0 = beg; i0 < end; i0 += 64) {
        const int i = i0 + lane;
        const bool valid = i < end;
        const int e = valid ? a.ids[i] : 0;
        uint64_t peers = __ballot(valid);
        for (int b = 0; b < nbits; ++b) {
            uint64_t m = __ballot(valid && ((e >> b) & 1));
            peers &= ((e >> b) & 1) ? m : ~m;
        }
        int base = 0;
        if (valid) base = hist[w][e];
        const int rank = __popcll(peers & below);
        if (valid) a.perm[base + rank] = i;
        // The highest lane of each peer group advances that expert's base.
        const bool last = valid && ((peers >> lane) >> 1) == 0ull;
        __builtin_amdgcn_wave_barrier();
        if (last) hist[w][e] = base + rank + 1;
        __builtin_amdgcn_wave_barrier();
    }
}

__global__ __launch_bounds__(256) void eval_exp_kernel(int which, const float *x, float *y,
                                                      size_t n) {
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        y[i] = which == 0 ? exp_poly(x[i]) : glibc_expf(x[i]);
}

}  // namespace

hipError_t launch_eval_exp(int which, const float *x, float *y, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    unsigned blocks = (unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    hipLaunchKernelGGL(eval_exp_kernel, dim3(blocks), dim3(256), 0, s, which, x, y, n);
    return hipGetLastError();
}

hipError_t launch_route(const RouteArgs &a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    dim3 grid((a.T + kRouteTM - 1) / kRouteTM);
    if (a.E <= 16)       hipLaunchKernelGGL(router_kernel<1>, grid, dim3(256), 0, s, a);
    else if (a.E <= 32)  hipLaunchKernelGGL(router_kernel<2>, grid, dim3(256), 0, s, a);
    else if (a.E <= 64)  hipLaunchKernelGGL(router_kernel<4>, grid, dim3(256), 0, s, a);
    else if (a.E <= 128) hipLaunchKernelGGL(router_kernel<8>, grid, dim3(256), 0, s, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_dispatch(const DispatchArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace moe
