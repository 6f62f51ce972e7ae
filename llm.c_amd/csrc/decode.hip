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
// workgroup's four waves with ballots; returns its length.  Every thread
// calls this; wcnt is 4 ints of LDS.
__device__ int expert_slots(const int *ids, int n, int e, int *list, int *wcnt) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int total = 0;
    for (int base = 0; base < n; base += 256) {
        const int i = base + threadIdx.x;
        const bool hit = i < n && ids[i] == e;
        const uint64_t m = __ballot(hit);
        if (lane == 0) wcnt[wave] = __popcll(m);
        __syncthreads();
        int off = total;
        for (int w = 0; w < wave; ++w) off += wcnt[w];
        if (hit) list[off + __popcll(m & below)] = i;
        total += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
        __syncthreads();
    }
    return total;
}

// Staging of rows list[pos0 .. pos0 + rows) / div of src, columns
// [k0, k0 + kc), into LDS, split so the caller can issue weight loads
// between the global reads and the LDS writes.
constexpr int kStageMax = kRows * kChunk / 4 / 256;   // float4s per thread

__device__ inline void stage_load(floatx4 (&v)[kStageMax], const float *src, int ld,
                                  const int *list, int div, int pos0, int rows, int k0, int kc) {
    const int q4 = kc >> 2;
#pragma unroll
    for (int i = 0; i < kStageMax; ++i) {
        const int q = threadIdx.x + 256 * i;
        const int r = q / q4, c4 = q % q4;
        v[i] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (r < rows) {
            const size_t row = (size_t)(list[pos0 + r] / div);
            v[i] = *reinterpret_cast<const floatx4 *>(src + row * ld + k0 + 4 * c4);
        }
    }
}

__device__ inline void stage_store(const floatx4 (&v)[kStageMax], float *xs, int kc) {
    const int q4 = kc >> 2;
#pragma unroll
    for (int i = 0; i < kStageMax; ++i) {
        const int q = threadIdx.x + 256 * i;
        const int r = q / q4, c4 = q % q4;
        if (r < kRows) *reinterpret_cast<floatx4 *>(xs + r * kLd + 4 * c4) = v[i];
    }
}

// Streams NB weight rows (NB = 2: gate and up of the lane's feature, NB = 1:
// one down row) over nq 16-wide K steps against RB 16-row activation blocks
// in LDS.  Loads run one group of kU = 8/NB steps ahead of the MFMAs that use
// them, so each wave keeps up to 16 16-byte loads per lane in flight.
template <int NB> struct Unroll { static constexpr int kU = 8 / NB; };

template <int NB>
__device__ inline void gemv_first(const float *p0, const float *p1, int nq,
                                  floatx4 (&cur)[Unroll<NB>::kU][NB]) {
    constexpr int kU = Unroll<NB>::kU;
    const float *pb[2] = {p0, p1};
    if (nq < kU) return;
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int b = 0; b < NB; ++b) cur[u][b] = *reinterpret_cast<const floatx4 *>(pb[b] + kUnit * u);
}

// cur must hold the first kU steps (gemv_first) when nq >= kU.
template <int NB, int RB>
__device__ inline void gemv_loop(const float *p0, const float *p1, const float *as, int nq,
                                 floatx4 (&acc)[2][NB], floatx4 (&cur)[Unroll<NB>::kU][NB]) {
    constexpr int kU = Unroll<NB>::kU;
    const float *pb[2] = {p0, p1};
    floatx4 nxt[kU][NB];
    int q = 0;
    const int ng = nq / kU;
    for (int g = 0; g < ng; ++g, q += kU) {
        if (g + 1 < ng) {
#pragma unroll
            for (int u = 0; u < kU; ++u)
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    nxt[u][b] = *reinterpret_cast<const floatx4 *>(pb[b] + kUnit * (q + kU + u));
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            floatx4 a0 = *reinterpret_cast<const floatx4 *>(as + 16 * (q + u));
            floatx4 a1;
            if (RB == 2) a1 = *reinterpret_cast<const floatx4 *>(as + 16 * kLd + 16 * (q + u));
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    acc[0][b] = mfma16(a0[s], cur[u][b][s], acc[0][b]);
                    if (RB == 2) acc[1][b] = mfma16(a1[s], cur[u][b][s], acc[1][b]);
                }
        }
        if (g + 1 < ng) {
#pragma unroll
            for (int u = 0; u < kU; ++u)
#pragma unroll
                for (int b = 0; b < NB; ++b) cur[u][b] = nxt[u][b];
        }
    }
    for (; q < nq; ++q) {
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
    extern __shared__ __align__(16) float xs[];     // [kRows][kLd], then the slot list
    __shared__ int wcnt[4];
    int *list = reinterpret_cast<int *>(xs + kRows * kLd);
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

    floatx4 cur[Unroll<2>::kU][2];
    gemv_first<2>(pg, pu, min(kChunk, a.d) / 16, cur);
    const int cnt = expert_slots(a.ids, a.nslots, e, list, wcnt);
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
            floatx4 stg[kStageMax];
            stage_load(stg, a.x, a.d, list, a.topk, r0, rows, k0, kc);
            if (r0 > 0 || k0 > 0) gemv_first<2>(pg + 16 * k0, pu + 16 * k0, kc / 16, cur);
            __syncthreads();
            stage_store(stg, xs, kc);
            __syncthreads();
            const float *as = xs + j * kLd + 4 * h;
            if (rows > 16) gemv_loop<2, 2>(pg + 16 * k0, pu + 16 * k0, as, kc / 16, acc, cur);
            else           gemv_loop<2, 1>(pg + 16 * k0, pu + 16 * k0, as, kc / 16, acc, cur);
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

    floatx4 cur[Unroll<1>::kU][1];
    gemv_first<1>(pw, nullptr, min(kChunk, kspan) / 16, cur);
    const int cnt = expert_slots(a.ids, a.nslots, e, list, wcnt);
    if (cnt == 0) return;
    for (int r0 = 0; r0 < cnt; r0 += kRows) {
        const int rows = min(kRows, cnt - r0);
        floatx4 acc[2][1] = {{floatx4{0.f, 0.f, 0.f, 0.f}}, {floatx4{0.f, 0.f, 0.f, 0.f}}};
        for (int k0 = 0; k0 < kspan; k0 += kChunk) {
            const int kc = min(kChunk, kspan - k0);
            floatx4 stg[kStageMax];
            stage_load(stg, a.x, a.F, list, 1, r0, rows, kbeg + k0, kc);
            if (r0 > 0 || k0 > 0) gemv_first<1>(pw + 16 * k0, nullptr, kc / 16, cur);
            __syncthreads();
            stage_store(stg, hs, kc);
            __syncthreads();
            const float *as = hs + j * kLd + 4 * h;
            if (rows > 16) gemv_loop<1, 2>(pw + 16 * k0, nullptr, as, kc / 16, acc, cur);
            else           gemv_loop<1, 1>(pw + 16 * k0, nullptr, as, kc / 16, acc, cur);
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

constexpr size_t kDecodeMaxLds = (size_t)kRows * kLd * sizeof(float) + sizeof(int) * kDecodeMaxSlots;

int decode_ksplit(int d, int F, int E) {
    int S = 1;
    while ((long)E * (d / 64) * S < 512 && F % (S * 2 * 32) == 0 && F / (S * 2) >= 256) S *= 2;
    return S;
}

// Dynamic LDS: the staged rows and a slot list of up to n entries.
size_t decode_lds(const DecodeArgs &a) {
    return (size_t)kRows * kLd * sizeof(float) + sizeof(int) * (size_t)a.nslots;
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
