// decode_tiny.hip — expert products of decode steps with a few routed rows
// (a KV-cache step of up to four sequences at top-2: at most kTinySlots = 8
// assignments with the routing inside, kTinyLaunchSlots = 4 after a router
// launch), on gfx950.
//
// With T * k <= 8 only a few experts hold rows, and the item kernels (one
// workgroup per 128 features of every expert) would leave most CUs idle:
// two experts' items take 32 of the 256 CUs, so one sequence's step read
// its 25 MB of weights at ~0.8 TB/s.  Here the work is cut per used expert
// into 16-feature groups, one workgroup each (the two used experts of a
// one-token step give 2 x F/16 = 256 workgroups at F = 2048): a workgroup
// reads the group's gate and up rows (2 x 16 x d floats) and its 16 columns
// of W_down (d x 16), 96 KB at d = 512, all loads in flight at once (non-
// temporal: 31.7 -> 29.85 us per layer at four sequences).  (After
// a router launch, eight assignments, about seven experts, ran faster on
// the fused kernel's items; with the routing inside, on these groups.)
//   gate/up  thread t: packed row t / 8 (gate rows 0-15, up rows 16-31 of
//            the group), k chunk t % 8 (d / 8 long, k ascending), one dot
//            per slot of the expert; the chunks' sums added by a fixed
//            xor tree; SwiGLU per (slot, feature) through LDS;
//   down     thread t: output columns t, t + 256, ...: the 16 features'
//            products added in feature order;
// and the group's partial output of every slot goes to Yp[g][slot][d]
// (g = feature group), which the combine adds in group order (fixed, so
// the bits do not depend on the schedule).  Weights are read from the packed
// unit layout (gemm.hip): element (row 16 nb + j, k = 16 qb + 4 h + s) of a
// matrix with K columns sits at ((nb * K / 16) + qb) * 256 + h * 64 + j * 4 + s.
//
// ROUTE: every workgroup first routes the step's T <= 8 tokens itself (no
// router launch, no ids read back): the rows (rms-normalised in place when
// the FFN norm runs here) stay in LDS and feed the dots; lane (r, c) of wave
// w runs token c's chain for expert 4 w + r, k ascending, with the router
// row in VGPRs reaching the lanes by DPP, and eight lanes per token finish
// (softmax, top-k, renormalisation) — the row-block router's chains and
// finish (route_rows.h), so probabilities and experts are the same bits.
// Workgroup t writes token t's ids, gate weights and probabilities after
// its products.  Wave 0 finds the used experts and the workgroup's slots
// with ballots (lane i: assignment i's expert).
#include <algorithm>
#include <climits>
#include <utility>

#include "moe_internal.h"
#include "moe_math.h"
#include "route_rows.h"

namespace moe {
namespace {

constexpr int kTinyThreads = 256;

// Weights are read once per step: non-temporal (streaming) loads.
__device__ inline float4 ld_weights4(const float *p) {
    typedef float fx4 __attribute__((ext_vector_type(4)));
    const fx4 v = __builtin_nontemporal_load(reinterpret_cast<const fx4 *>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
}

// f(integral_constant<int, S>) for S in the sequence, in order.
template <class Fn, int... S>
__device__ inline void tiny_static_for(std::integer_sequence<int, S...>, Fn &&f) {
    (f(std::integral_constant<int, S>{}), ...);
}

// The routing of the step's T <= kTinySlots tokens (E <= 16, d = KC): rows
// to xs (normalised in place with ra.rms_w), then the chains and the finish
// of eight token rows (rows past T repeat row T - 1; nothing reads them).
// isel / psel: [8][k], invs [8].
template <int KC>
__device__ inline void tiny_route(const RouteArgs &ra, float (*xs)[KC + 4], float *lg, int *isel,
                                  float *psel, float *invs) {
    constexpr int WV4 = KC / 64, NS = KC / 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int T = ra.T, E = ra.E, k = ra.k;
    const float *src = ra.rms_w ? ra.x_raw : ra.x;
    for (int i = tid; i < T * (KC / 4); i += kTinyThreads) {
        const int t = i / (KC / 4), c4 = i - t * (KC / 4);
        *reinterpret_cast<float4 *>(&xs[t][4 * c4]) =
            *reinterpret_cast<const float4 *>(src + (size_t)t * KC + 4 * c4);
    }
    // Lane (r, c): k = 64 b + 4 c .. 64 b + 4 c + 3 of expert 4 wave + r.
    const int r = lane >> 4, c = lane & 15;
    const int ej = min(4 * wave + r, E - 1);
    float4 w4[WV4];
    const float *wrow = ra.wrT + (size_t)ej * KC + 4 * c;
#pragma unroll
    for (int b = 0; b < WV4; ++b) w4[b] = *reinterpret_cast<const float4 *>(wrow + 64 * b);
    const float bv = ra.bias ? ra.bias[ej] : 0.0f;
    __syncthreads();
    if (ra.rms_w) {
        // (rms_row16 holds a whole row in registers first, so in place is safe)
        for (int rr = tid >> 4; rr < T; rr += kTinyThreads / 16) {
            float *xr = &xs[rr][0];
            rms_row16([&](int i) { return xr[i]; }, ra.rms_w, KC / 16, ra.rms_eps, ra.rms_rcp,
                      nullptr, false, xr, false);
        }
        __syncthreads();
    }
    if (4 * wave < E) {
        float acc = 0.0f;
        const float *xrow = &xs[min(c, T - 1)][0];
        auto xread = [&](float (&xv)[16], int sl) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = *reinterpret_cast<const float4 *>(xrow + 16 * sl + 4 * q);
                xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
            }
        };
        float xa[16], xb[16];
        xread(xa, 0);
        tiny_static_for(std::make_integer_sequence<int, NS / 2>{}, [&](auto sc) {
            constexpr int SL = 2 * decltype(sc)::value;
            xread(xb, SL + 1);
            chain16_dpp4<SL % 4>(acc, w4[SL / 4], xa);
            if constexpr (SL + 2 < NS) xread(xa, SL + 2);
            chain16_dpp4<(SL + 1) % 4>(acc, w4[(SL + 1) / 4], xb);
        });
        if (c < 8 && 4 * wave + r < E) lg[c * (E + 1) + 4 * wave + r] = ra.bias ? acc + bv : acc;
    }
    __syncthreads();
    if (tid < 64) {
        const int ct = tid >> 3, l = tid & 7;
        const float inv = finish_token8<2>(ra, lg + ct * (E + 1), l, isel + ct * k, psel + ct * k);
        if (l == 0) invs[ct] = inv;
    }
    __syncthreads();
}

// Token t's routing results (ids, gate weights, probabilities, normalised
// rows when the caller takes them), from workgroup t: after its products,
// so that no barrier waits for these stores.
template <int KC>
__device__ inline void tiny_route_results(const RouteArgs &ra, float (*xs)[KC + 4],
                                          const float *lg, const int *isel, const float *psel,
                                          const float *invs) {
    const int tid = threadIdx.x;
    const int T = ra.T, E = ra.E, k = ra.k;
    for (int ct = blockIdx.x; ct < T; ct += gridDim.x) {
        if (tid < k) {
            const int i = ct * k + tid;
            if (ra.ids) ra.ids[i] = isel[i];
            if (ra.gw) ra.gw[i] = ftz_f(psel[i] * invs[ct]);
        }
        if (ra.probs)
            for (int ex = tid; ex < E; ex += kTinyThreads) ra.probs[ct * E + ex] = lg[ct * (E + 1) + ex];
        if (ra.rms_w && ra.xn_out)
            for (int c4 = tid; c4 < KC / 4; c4 += kTinyThreads)
                *reinterpret_cast<float4 *>(ra.xn_out + (size_t)ct * KC + 4 * c4) =
                    *reinterpret_cast<const float4 *>(&xs[ct][4 * c4]);
    }
}

// Workgroup b: used expert b / (F / 16) (the ascending list of the experts
// the ids name), feature group b % (F / 16).  KCH = d / 8.  ROUTE: the ids
// come from the routing above, the rows from LDS.
template <int KCH, bool ROUTE>
__global__ __launch_bounds__(kTinyThreads) void decode_tiny_kernel(DecodeArgs a, RouteArgs ra) {
    constexpr int KQ = KCH / 16;              // 16-wide k units per chunk
    constexpr int NCO = 8 * KCH / kTinyThreads;   // output columns per thread (d / 256)
    constexpr int KC = 8 * KCH;
    __shared__ int slot[kTinySlots];
    __shared__ int e_s, ns_s;
    __shared__ float gu[kTinySlots][32];
    __shared__ float hh[kTinySlots][16];
    __shared__ __align__(16) float xs[ROUTE ? kTinySlots : 1][KC + 4];
    __shared__ float lg[ROUTE ? 8 * 17 : 1];
    __shared__ int isel[ROUTE ? 8 * kTinySlots : 1];
    __shared__ float psel[ROUTE ? 8 * kTinySlots : 1], invs[8];
    const int tid = threadIdx.x;
    const int n = a.nslots, d = a.d, F = a.F;
    const int nfg = F / 16;
    const int ub = blockIdx.x / nfg, fg = blockIdx.x - ub * nfg;
    if constexpr (ROUTE) tiny_route<KC>(ra, xs, lg, isel, psel, invs);
    // Wave 0, lane i < n holding assignment i's expert: the distinct experts
    // in ascending order (rank of each first occurrence among them), this
    // workgroup's expert (rank ub) and its slots in slot order.
    if (tid < 64) {
        int id = INT_MAX;
        if (tid < n) {
            if constexpr (ROUTE) id = isel[tid];
            else                 id = a.ids[tid];
        }
        // (every shuffle runs in all 64 lanes: a lane reading an inactive
        // lane would get 0)
        bool first = tid < n;
#pragma unroll
        for (int j = 0; j < kTinySlots; ++j) {
            const int idj = __shfl(id, j);
            if (j < tid && idj == id) first = false;
        }
        const unsigned long long fm = __ballot(first);
        int rank = 0;
#pragma unroll
        for (int j = 0; j < kTinySlots; ++j) {
            const int idj = __shfl(id, j);
            if (((fm >> j) & 1ull) && idj < id) ++rank;
        }
        const int nu = __popcll(fm);
        const unsigned long long mine = __ballot(first && rank == ub);
        const int src = __ffsll((long long)mine) - 1;
        const int idm = __shfl(id, src < 0 ? 0 : src);
        const int eb = ub < nu && src >= 0 && idm >= 0 && idm < a.E ? idm : -1;
        const unsigned long long match = __ballot(tid < n && id == eb);
        if ((match >> tid) & 1ull) slot[__popcll(match & ((1ull << tid) - 1))] = tid;
        if (tid == 0) {
            e_s = eb;
            ns_s = __popcll(match);
        }
    }
    __syncthreads();
    if (e_s < 0) {
        if constexpr (ROUTE) tiny_route_results<KC>(ra, xs, lg, isel, psel, invs);
        return;
    }
    const int e = e_s, ns = ns_s;
    const int f0 = 16 * fg;

    // Gate/up: packed row of thread t (gate features f0 .. f0 + 15 at packed
    // rows 64 (f0 / 32) + f0 % 32 + j, their up rows 32 further).
    const int r = tid >> 3, c = tid & 7;
    const int prow = 64 * (f0 / 32) + (f0 % 32) + (r < 16 ? r : 16 + r);
    const float *wg = a.w + (size_t)e * 2 * F * d + ((size_t)(prow >> 4) * (d / 16)) * 256 +
                      (prow & 15) * 4;
    float4 w[KQ][4];
#pragma unroll
    for (int q = 0; q < KQ; ++q)
#pragma unroll
        for (int h = 0; h < 4; ++h)
            w[q][h] = ld_weights4(wg + (size_t)(c * KQ + q) * 256 + h * 64);
    // Down: columns o = tid + 256 i of W_down's features f0 .. f0 + 15.
    float4 wd[NCO][4];
    const float *wdb = a.w2 + (size_t)e * d * F + (f0 / 16) * 256;
#pragma unroll
    for (int i = 0; i < NCO; ++i) {
        const int o = tid + kTinyThreads * i;
        const float *p = wdb + ((size_t)(o >> 4) * (F / 16)) * 256 + (o & 15) * 4;
#pragma unroll
        for (int h = 0; h < 4; ++h) wd[i][h] = ld_weights4(p + h * 64);
    }

    // Dots of the chunk for every slot of the expert (k ascending), then the
    // eight chunks added by a fixed xor tree.
    for (int s = 0; s < ns; ++s) {
        const int t = slot[s] / a.topk;
        const float *xr = (ROUTE ? &xs[t][0] : a.x + (size_t)t * d) + c * KCH;
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < KQ; ++q)
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const float4 xv = *reinterpret_cast<const float4 *>(xr + 16 * q + 4 * h);
                acc = fmaf(xv.x, w[q][h].x, acc);
                acc = fmaf(xv.y, w[q][h].y, acc);
                acc = fmaf(xv.z, w[q][h].z, acc);
                acc = fmaf(xv.w, w[q][h].w, acc);
            }
        acc += __shfl_xor(acc, 4, 8);
        acc += __shfl_xor(acc, 2, 8);
        acc += __shfl_xor(acc, 1, 8);
        if (c == 0) gu[s][r] = acc;
    }
    __syncthreads();
    if (tid < 16 * ns) {
        const int s = tid >> 4, f = tid & 15;
        hh[s][f] = swiglu_fast(gu[s][f], gu[s][16 + f]);
    }
    __syncthreads();
    for (int s = 0; s < ns; ++s) {
        float *yp = a.out + ((size_t)fg * n + slot[s]) * d;
#pragma unroll
        for (int i = 0; i < NCO; ++i) {
            float y = 0.0f;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                y = fmaf(hh[s][4 * h], wd[i][h].x, y);
                y = fmaf(hh[s][4 * h + 1], wd[i][h].y, y);
                y = fmaf(hh[s][4 * h + 2], wd[i][h].z, y);
                y = fmaf(hh[s][4 * h + 3], wd[i][h].w, y);
            }
            yp[tid + kTinyThreads * i] = y;
        }
    }
    if constexpr (ROUTE) tiny_route_results<KC>(ra, xs, lg, isel, psel, invs);
}

}  // namespace

bool decode_tiny_ok(int n, int d, int F, int E) {
    return n >= 1 && n <= kTinySlots && E >= 1 && (d == 256 || d == 512 || d == 1024) &&
           F % 32 == 0 && F / 16 <= kTinyMaxGroups;
}

bool decode_tiny_routed_ok(int T, int d, int F, int E, int k) {
    return T >= 1 && k >= 1 && k <= E && E <= 16 && (d == 256 || d == 512) &&
           decode_tiny_ok(T * k, d, F, E);
}

hipError_t launch_decode_tiny(const DecodeArgs &a, const RouteArgs *ra, hipStream_t s) {
    if (!decode_tiny_ok(a.nslots, a.d, a.F, a.E) || !a.w2) return hipErrorInvalidValue;
    if (ra && (!decode_tiny_routed_ok(ra->T, a.d, a.F, a.E, ra->k) || ra->d != a.d ||
               ra->E != a.E || ra->k != a.topk || a.nslots != ra->T * ra->k || !ra->wrT ||
               (ra->rms_w && !ra->x_raw)))
        return hipErrorInvalidValue;
    const int groups = a.F / 16;
    const dim3 grid((unsigned)(std::min(a.E, a.nslots) * groups));
    const RouteArgs none{};
    if (ra) {
        if (a.d == 256) hipLaunchKernelGGL((decode_tiny_kernel<32, true>), grid, dim3(kTinyThreads), 0, s, a, *ra);
        else            hipLaunchKernelGGL((decode_tiny_kernel<64, true>), grid, dim3(kTinyThreads), 0, s, a, *ra);
        return hipGetLastError();
    }
    switch (a.d) {
        case 256:  hipLaunchKernelGGL((decode_tiny_kernel<32, false>), grid, dim3(kTinyThreads), 0, s, a, none); break;
        case 512:  hipLaunchKernelGGL((decode_tiny_kernel<64, false>), grid, dim3(kTinyThreads), 0, s, a, none); break;
        default:   hipLaunchKernelGGL((decode_tiny_kernel<128, false>), grid, dim3(kTinyThreads), 0, s, a, none); break;
    }
    return hipGetLastError();
}

}  // namespace moe
