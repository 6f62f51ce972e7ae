// decode.hip — bandwidth-bound expert products for few rows per expert (the
// KV-cache decode step: a handful of tokens per expert), on gfx950.
//
// Both kernels stream each routed expert's packed weights exactly once per
// 32-row pass and feed them to v_mfma_f32_16x16x4f32 straight from
// registers: a lane holds a 16-byte piece of one weight row (K contiguous),
// the MFMA's k-row h (lane/16) takes the piece's 4 elements in turn, and the
// activations come from LDS as 128-bit reads with the same k mapping.
// Weights are in the unit layout (16 x 16 tiles in MFMA operand order, see
// gemm.hip): a K step of 16 is one contiguous 1 KB unit per wave.
//   gate/up: grid = E x (F/64); wave w of a workgroup owns features
//            64*fb + 16w .. +15 and both their gate and up rows, so the SwiGLU
//            epilogue is lane-local and writes H [n x F] at the assignment
//            index a = t*k + slot.
//   down:    grid = E x (d/64) x S; split s covers F/S of the reduction and
//            writes its partial product to Yp[s] at the assignment index;
//            the combine adds the S partials in fixed order.
// Each workgroup finds its expert's assignments itself (a ballot scan of the
// router's expert ids into an ascending list in LDS), after it has issued its
// first weight loads, which depend on nothing the router computes.
#include "moe_internal.h"
#include "moe_math.h"

namespace moe {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 32;        // rows per pass (two 16-row MFMA blocks)
constexpr int kChunk = 512;      // K elements staged per LDS fill
constexpr int kLd = kChunk + 4;  // padded LDS row

constexpr int kUnit = 256;      // floats per 16 x 16 unit = one K step of 16

__device__ inline floatx4 mfma16(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Ascending list of the assignments a < n with ids[a] == e, built by the
// workgroup's four waves with ballots, and (tok != nullptr) the token a / topk
// of each; returns the list length.  Every thread calls this, with id0 =
// ids[threadIdx.x] (or -1 past n) loaded by the caller before its first
// weight loads so that waiting for it does not wait for them; wcnt is 4 ints
// of LDS.
__device__ inline void slot_chunk(int i, int n, int e, int id, int topk, int *list, int *tok,
                                  int *wcnt, int &total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const bool hit = i < n && id == e;
    const uint64_t m = __ballot(hit);
    if (lane == 0) wcnt[wave] = __popcll(m);
    __syncthreads();
    int off = total;
    for (int w = 0; w < wave; ++w) off += wcnt[w];
    if (hit) {
        const int at = off + __popcll(m & below);
        list[at] = i;
        if (tok) tok[at] = i / topk;
    }
    total += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
    __syncthreads();
}

__device__ int expert_slots(const int *ids, int n, int e, int id0, int topk, int *list, int *tok,
                            int *wcnt) {
    int total = 0;
    slot_chunk(threadIdx.x, n, e, id0, topk, list, tok, wcnt, total);
    for (int base = 256; base < n; base += 256) {
        const int i = base + threadIdx.x;
        slot_chunk(i, n, e, ids[min(i, n - 1)], topk, list, tok, wcnt, total);
    }
    return total;
}

// Staging of rows rowlist[pos0 .. pos0 + rows) of src, columns [k0, k0 + kc),
// into LDS rows of stride kLd by global-to-LDS DMA (no registers): wave w
// copies rows w, w + 4, ... as two 1 KB pieces each (64 lanes x 16 bytes),
// columns clamped to the source row.  Columns past kc and rows past rows are
// never read.
__device__ inline void stage_lds(float *xs, const float *src, int ld, const int *rowlist,
                                 int pos0, int rows, int k0, int kc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int r = wave; r < rows; r += 4) {
        const float *srow = src + (size_t)rowlist[pos0 + r] * ld;
#pragma unroll
        for (int p = 0; p < kChunk / 256; ++p)
            if (256 * p < kc)
                __builtin_amdgcn_global_load_lds(srow + min(k0 + 256 * p + 4 * lane, ld - 4),
                                                 xs + r * kLd + 256 * p, 16, 0, 0);
    }
}

// s_waitcnt with only the vector-memory count limited (expcnt and lgkmcnt at
// their maxima).
#define WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | 0x0F70)

// Streams NB weight rows (NB = 2: gate and up of the lane's feature, NB = 1:
// one down row) over nq 16-wide K steps against RB 16-row activation blocks
// in LDS.  The stream is cut into groups of kU = 8/NB steps held in two
// register sets; the loads of group g + 2 are issued as soon as group g's
// MFMAs are done, so one to two groups (8 to 16 16-byte loads per lane) stay
// in flight.
template <int NB> struct Unroll { static constexpr int kU = 8 / NB; };

template <int NB>
using WGroup = floatx4[Unroll<NB>::kU][NB];

// Loads steps q .. q + kU - 1 of the stream, each clamped to step last (so
// a short chunk never reads past its weights).
template <int NB>
__device__ inline void wload(const float *const (&pb)[2], int q, int last, WGroup<NB> &w) {
#pragma unroll
    for (int u = 0; u < Unroll<NB>::kU; ++u)
#pragma unroll
        for (int b = 0; b < NB; ++b)
            w[u][b] = *reinterpret_cast<const floatx4 *>(pb[b] + kUnit * min(q + u, last));
}

// Issues the loads of groups 0 and 1 of a chunk of nq steps, unconditionally
// (wait counts stay exact); groups the chunk lacks are never used.
template <int NB>
__device__ inline void gemv_prime(const float *p0, const float *p1, int nq, WGroup<NB> &wa,
                                  WGroup<NB> &wb) {
    constexpr int kU = Unroll<NB>::kU;
    const float *const pb[2] = {p0, p1};
    wload<NB>(pb, 0, nq - 1, wa);
    wload<NB>(pb, kU, nq - 1, wb);
}

template <int NB, int RB>
__device__ inline void gemv_group(const float *as, int q, const WGroup<NB> &w,
                                  floatx4 (&acc)[2][NB]) {
#pragma unroll
    for (int u = 0; u < Unroll<NB>::kU; ++u) {
        floatx4 a0 = *reinterpret_cast<const floatx4 *>(as + 16 * (q + u));
        floatx4 a1;
        if (RB == 2) a1 = *reinterpret_cast<const floatx4 *>(as + 16 * kLd + 16 * (q + u));
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                acc[0][b] = mfma16(a0[s], w[u][b][s], acc[0][b]);
                if (RB == 2) acc[1][b] = mfma16(a1[s], w[u][b][s], acc[1][b]);
            }
    }
}

// wa / wb must hold groups 0 / 1 (gemv_prime).
template <int NB, int RB>
__device__ inline void gemv_loop(const float *p0, const float *p1, const float *as, int nq,
                                 floatx4 (&acc)[2][NB], WGroup<NB> &wa, WGroup<NB> &wb) {
    constexpr int kU = Unroll<NB>::kU;
    const float *const pb[2] = {p0, p1};
    const int ng = nq / kU;
    int g = 0;
    // Steady state with unconditional loads (exact wait counts).
    // (Scheduling barriers keep each group's loads right after the MFMAs
    // that free its registers.)
    for (; g + 4 <= ng; g += 2) {
        gemv_group<NB, RB>(as, kU * g, wa, acc);
        __builtin_amdgcn_sched_barrier(0);
        wload<NB>(pb, kU * (g + 2), nq - 1, wa);
        __builtin_amdgcn_sched_barrier(0);
        gemv_group<NB, RB>(as, kU * (g + 1), wb, acc);
        __builtin_amdgcn_sched_barrier(0);
        wload<NB>(pb, kU * (g + 3), nq - 1, wb);
        __builtin_amdgcn_sched_barrier(0);
    }
    const int left = ng - g;   // 0 .. 3 groups, the first two already loaded
    if (left == 3) {
        gemv_group<NB, RB>(as, kU * g, wa, acc);
        wload<NB>(pb, kU * (g + 2), nq - 1, wa);
        gemv_group<NB, RB>(as, kU * (g + 1), wb, acc);
        gemv_group<NB, RB>(as, kU * (g + 2), wa, acc);
    } else if (left == 2) {
        gemv_group<NB, RB>(as, kU * g, wa, acc);
        gemv_group<NB, RB>(as, kU * (g + 1), wb, acc);
    } else if (left == 1) {
        gemv_group<NB, RB>(as, kU * g, wa, acc);
    }
    for (int q = kU * ng; q < nq; ++q) {
        floatx4 w[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) w[b] = *reinterpret_cast<const floatx4 *>(pb[b] + kUnit * q);
        floatx4 a0 = *reinterpret_cast<const floatx4 *>(as + 16 * q);
        floatx4 a1;
        if (RB == 2) a1 = *reinterpret_cast<const floatx4 *>(as + 16 * kLd + 16 * q);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                acc[0][b] = mfma16(a0[s], w[b][s], acc[0][b]);
                if (RB == 2) acc[1][b] = mfma16(a1[s], w[b][s], acc[1][b]);
            }
    }
}

__global__ __launch_bounds__(256) void decode_gateup_kernel(DecodeArgs a) {
    extern __shared__ __align__(16) float xs[];     // [kRows][kLd], slot list, token list
    __shared__ int wcnt[4];
    int *list = reinterpret_cast<int *>(xs + kRows * kLd);
    int *tok = list + a.nslots;
    const int nfb = a.F / 64;
    const int e = blockIdx.x / nfb, fb = blockIdx.x % nfb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, h = lane >> 4;
    const int f = fb * 64 + wave * 16 + j;
    // Gate rows of this wave's 16 features form unit row nbg; up rows are
    // 32 packed rows (2 unit rows) further.
    const int nbg = 8 * fb + 4 * (wave >> 1) + (wave & 1);
    const float *pg = a.w + (size_t)e * 2 * a.F * a.d + (size_t)nbg * (a.d / 16) * kUnit + 4 * lane;
    const float *pu = pg + (size_t)2 * (a.d / 16) * kUnit;

    const int id0 = (int)threadIdx.x < a.nslots ? a.ids[threadIdx.x] : -1;
    WGroup<2> wa, wb;
    gemv_prime<2>(pg, pu, min(kChunk, a.d) / 16, wa, wb);
    const int cnt = expert_slots(a.ids, a.nslots, e, id0, a.topk, list, tok, wcnt);
    if (cnt == 0) return;
    for (int r0 = 0; r0 < cnt; r0 += kRows) {
        const int rows = min(kRows, cnt - r0);
        floatx4 acc[2][2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int g = 0; g < 2; ++g) acc[b][g] = floatx4{0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < a.d; k0 += kChunk) {
            const int kc = min(kChunk, a.d - k0);
            __syncthreads();   // every wave is done with the previous rows
            stage_lds(xs, a.x, a.d, tok, r0, rows, k0, kc);
            if (r0 > 0 || k0 > 0) {
                gemv_prime<2>(pg + 16 * k0, pu + 16 * k0, kc / 16, wa, wb);
                WAIT_VMCNT(4 * Unroll<2>::kU);   // the rows, not the weights behind them
            } else {
                WAIT_VMCNT(0);
            }
            __syncthreads();
            const float *as = xs + j * kLd + 4 * h;
            if (rows > 16) gemv_loop<2, 2>(pg + 16 * k0, pu + 16 * k0, as, kc / 16, acc, wa, wb);
            else           gemv_loop<2, 1>(pg + 16 * k0, pu + 16 * k0, as, kc / 16, acc, wa, wb);
        }
        // 16x16 accumulator: lane holds rows 4*(lane/16) + r, column lane%16.
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = b * 16 + 4 * h + r;
                if (row < rows)
                    a.out[(size_t)list[r0 + row] * a.F + f] =
                        swiglu_fast(acc[b][0][r], acc[b][1][r]);
            }
    }
}

__global__ __launch_bounds__(256) void decode_down_kernel(DecodeArgs a) {
    extern __shared__ __align__(16) float hs[];     // [kRows][kLd], then the slot list
    __shared__ int wcnt[4];
    int *list = reinterpret_cast<int *>(hs + kRows * kLd);
    const int ncb = a.d / 64;
    const int S = a.ksplit;
    const int e = blockIdx.x / (ncb * S);
    const int rem = blockIdx.x % (ncb * S);
    const int cb = rem / S, sp = rem % S;
    const int kspan = a.F / S, kbeg = sp * kspan;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, h = lane >> 4;
    const int col = cb * 64 + wave * 16 + j;
    const float *pw = a.w + (size_t)e * a.d * a.F +
                      ((size_t)(cb * 4 + wave) * (a.F / 16) + kbeg / 16) * kUnit + 4 * lane;
    const size_t nslots = (size_t)a.nslots;

    const int id0 = (int)threadIdx.x < a.nslots ? a.ids[threadIdx.x] : -1;
    WGroup<1> wa, wb;
    gemv_prime<1>(pw, nullptr, min(kChunk, kspan) / 16, wa, wb);
    const int cnt = expert_slots(a.ids, a.nslots, e, id0, a.topk, list, nullptr, wcnt);
    if (cnt == 0) return;
    for (int r0 = 0; r0 < cnt; r0 += kRows) {
        const int rows = min(kRows, cnt - r0);
        floatx4 acc[2][1] = {{floatx4{0.f, 0.f, 0.f, 0.f}}, {floatx4{0.f, 0.f, 0.f, 0.f}}};
        for (int k0 = 0; k0 < kspan; k0 += kChunk) {
            const int kc = min(kChunk, kspan - k0);
            __syncthreads();   // every wave is done with the previous rows
            stage_lds(hs, a.x, a.F, list, r0, rows, kbeg + k0, kc);
            if (r0 > 0 || k0 > 0) {
                gemv_prime<1>(pw + 16 * k0, nullptr, kc / 16, wa, wb);
                WAIT_VMCNT(2 * Unroll<1>::kU);   // the rows, not the weights behind them
            } else {
                WAIT_VMCNT(0);
            }
            __syncthreads();
            const float *as = hs + j * kLd + 4 * h;
            if (rows > 16) gemv_loop<1, 2>(pw + 16 * k0, nullptr, as, kc / 16, acc, wa, wb);
            else           gemv_loop<1, 1>(pw + 16 * k0, nullptr, as, kc / 16, acc, wa, wb);
        }
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = b * 16 + 4 * h + r;
                if (row < rows) {
                    const size_t slot = (size_t)list[r0 + row];
                    a.out[((size_t)sp * nslots + slot) * a.d + col] = acc[b][0][r];
                }
            }
    }

}

hipError_t set_lds(const void *kernel, size_t bytes, bool *done) {
    if (*done) return hipSuccess;
    hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)bytes);
    if (e == hipSuccess) *done = true;
    return e;
}

}  // namespace

constexpr size_t kDecodeMaxLds = (size_t)kRows * kLd * sizeof(float) + 2 * sizeof(int) * kDecodeMaxSlots;

int decode_ksplit(int d, int F, int E) {
    int S = 1;
    while ((long)E * (d / 64) * S < 512 && F % (S * 2 * 32) == 0 && F / (S * 2) >= 256) S *= 2;
    return S;
}

// Dynamic LDS: the staged rows, a slot list and a token list of up to n
// entries each.
size_t decode_lds(const DecodeArgs &a) {
    return (size_t)kRows * kLd * sizeof(float) + 2 * sizeof(int) * (size_t)a.nslots;
}

hipError_t launch_decode_gateup(const DecodeArgs &a, hipStream_t s) {
    const size_t lds = decode_lds(a);
    static bool attr = false;
    hipError_t e = set_lds(reinterpret_cast<const void *>(&decode_gateup_kernel), kDecodeMaxLds, &attr);
    if (e != hipSuccess) return e;
    dim3 grid((unsigned)(a.E * (a.F / 64)));
    hipLaunchKernelGGL(decode_gateup_kernel, grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_decode_down(const DecodeArgs &a, hipStream_t s) {
    const size_t lds = decode_lds(a);
    static bool attr = false;
    hipError_t e = set_lds(reinterpret_cast<const void *>(&decode_down_kernel), kDecodeMaxLds, &attr);
    if (e != hipSuccess) return e;
    dim3 grid((unsigned)(a.E * (a.d / 64) * a.ksplit));
    hipLaunchKernelGGL(decode_down_kernel, grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

}  // namespace moe
