// decode_tiny.hip — expert products of decode steps with a few routed rows
// (a KV-cache step of one or two sequences at top-2: at most kTinySlots = 4
// assignments), on gfx950.
//
// With T * k <= 4 only a few experts hold rows, and the item kernels (one
// workgroup per 128 features of every expert) would leave most CUs idle:
// two experts' items take 32 of the 256 CUs, so one sequence's step read
// its 25 MB of weights at ~0.8 TB/s.  Here the work is cut per used expert
// into 16-feature groups, one workgroup each (the two used experts of a
// one-token step give 2 x F/16 = 256 workgroups at F = 2048): a workgroup
// reads the group's gate and up rows (2 x 16 x d floats) and its 16 columns
// of W_down (d x 16), 96 KB at d = 512, all loads in flight at once.  (At
// eight assignments, about seven experts, the fused kernel's items read the
// weights faster than these groups do, so those steps stay with it.)
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
#include <algorithm>
#include <climits>

#include "moe_internal.h"
#include "moe_math.h"

namespace moe {
namespace {

constexpr int kTinyThreads = 256;

// Workgroup b: used expert b / (F / 16) (the ascending list of the experts
// the ids name), feature group b % (F / 16).  KCH = d / 8.
template <int KCH>
__global__ __launch_bounds__(kTinyThreads) void decode_tiny_kernel(DecodeArgs a) {
    constexpr int KQ = KCH / 16;              // 16-wide k units per chunk
    constexpr int NCO = 8 * KCH / kTinyThreads;   // output columns per thread (d / 256)
    __shared__ int uexp[kTinySlots], slot[kTinySlots];
    __shared__ int nu_s, ns_s;
    __shared__ float gu[kTinySlots][32];
    __shared__ float hh[kTinySlots][16];
    const int tid = threadIdx.x;
    const int n = a.nslots, d = a.d, F = a.F;
    const int nfg = F / 16;
    const int ub = blockIdx.x / nfg, fg = blockIdx.x - ub * nfg;
    if (tid == 0) {
        // Distinct experts in ascending order, then the expert of this
        // workgroup's slots in slot order (n <= kTinySlots).
        int ids[kTinySlots], nu = 0;
        for (int i = 0; i < n; ++i) ids[i] = a.ids[i];
        int last = -1;
        for (;;) {
            int next = INT_MAX;
            for (int i = 0; i < n; ++i)
                if (ids[i] > last && ids[i] < next) next = ids[i];
            if (next == INT_MAX) break;
            uexp[nu++] = next;
            last = next;
        }
        nu_s = nu;
        int ns = 0;
        if (ub < nu)
            for (int i = 0; i < n; ++i)
                if (ids[i] == uexp[ub]) slot[ns++] = i;
        ns_s = ns;
    }
    __syncthreads();
    if (ub >= nu_s) return;
    const int e = uexp[ub], ns = ns_s;
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
            w[q][h] = *reinterpret_cast<const float4 *>(wg + (size_t)(c * KQ + q) * 256 + h * 64);
    // Down: columns o = tid + 256 i of W_down's features f0 .. f0 + 15.
    float4 wd[NCO][4];
    const float *wdb = a.w2 + (size_t)e * d * F + (f0 / 16) * 256;
#pragma unroll
    for (int i = 0; i < NCO; ++i) {
        const int o = tid + kTinyThreads * i;
        const float *p = wdb + ((size_t)(o >> 4) * (F / 16)) * 256 + (o & 15) * 4;
#pragma unroll
        for (int h = 0; h < 4; ++h) wd[i][h] = *reinterpret_cast<const float4 *>(p + h * 64);
    }

    // Dots of the chunk for every slot of the expert (k ascending), then the
    // eight chunks added by a fixed xor tree.
    for (int s = 0; s < ns; ++s) {
        const float *xr = a.x + (size_t)(slot[s] / a.topk) * d + c * KCH;
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
}

}  // namespace

bool decode_tiny_ok(int n, int d, int F, int E) {
    return n >= 1 && n <= kTinySlots && E >= 1 && (d == 256 || d == 512 || d == 1024) &&
           F % 32 == 0 && F / 16 <= kTinyMaxGroups;
}

hipError_t launch_decode_tiny(const DecodeArgs &a, hipStream_t s) {
    if (!decode_tiny_ok(a.nslots, a.d, a.F, a.E) || !a.w2) return hipErrorInvalidValue;
    const int groups = a.F / 16;
    const dim3 grid((unsigned)(std::min(a.E, a.nslots) * groups));
    switch (a.d) {
        case 256:  hipLaunchKernelGGL(decode_tiny_kernel<32>, grid, dim3(kTinyThreads), 0, s, a); break;
        case 512:  hipLaunchKernelGGL(decode_tiny_kernel<64>, grid, dim3(kTinyThreads), 0, s, a); break;
        default:   hipLaunchKernelGGL(decode_tiny_kernel<128>, grid, dim3(kTinyThreads), 0, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace moe
