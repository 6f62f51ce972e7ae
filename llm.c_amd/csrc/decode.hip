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
#include "decode_gemv.h"

namespace moe {
namespace {

// grid = E x (F/(16*NW)): one gate/up item of NW waves per workgroup (NW =
// 8: one workgroup per CU, two waves per SIMD).  The fused items store their
// split-K partials write-through (coherent stores): none are left dirty in an
// XCD's L2 when the launch ends, and the combine launch reads them from
// memory either way.
template <bool FUSED, int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void decode_gateup_kernel(DecodeArgs a) {
    extern __shared__ __align__(16) float xs[];     // [kRows][kLd], slot list, token list
    __shared__ int wcnt[NW];
    const int nfb = a.F / (16 * NW);
    int e, fb;
    item_of(blockIdx.x, a.E, nfb, e, fb);
    gateup_item<FUSED, NW, FUSED>(a, e, fb, xs, wcnt);
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
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const unsigned lo = 16u * lane;   // the lane's column of each weight unit
    const int j = lane & 15, h = lane >> 4;
    const int col = cb * 64 + wave * 16 + j;
    const WSrc ws = wsrc(a.w + (size_t)e * a.d * a.F, (size_t)a.d * a.F, lo);
    const int ow = kUnitBytes * ((cb * 4 + wave) * (a.F / 16) + kbeg / 16);
    const size_t nslots = (size_t)a.nslots;

    const int id0 = (int)threadIdx.x < a.nslots ? a.ids[threadIdx.x] : -1;
    WGroup<1> wa, wb;
    const int cnt = expert_slots(a.ids, a.nslots, e, id0, a.topk, list, nullptr, wcnt);
    if (cnt == 0) return;
    for (int r0 = 0; r0 < cnt; r0 += kRows) {
        const int rows = min(kRows, cnt - r0);
        floatx4 acc[2][1] = {{floatx4{0.f, 0.f, 0.f, 0.f}}, {floatx4{0.f, 0.f, 0.f, 0.f}}};
        for (int k0 = 0; k0 < kspan; k0 += kChunk) {
            const int kc = min(kChunk, kspan - k0);
            __syncthreads();   // every wave is done with the previous rows
            stage_lds(hs, a.x, a.F, list, r0, rows, kbeg + k0, kc);
            __builtin_amdgcn_sched_barrier(0);   // (the counted wait takes the DMA as issued first)
            gemv_prime<1>(ws, ow + 64 * k0, 0, kc / 16, wa, wb);
            WAIT_VMCNT(2 * Unroll<1>::kU);   // the rows, not the weights behind them
            __builtin_amdgcn_s_barrier();   // (a fence here would wait for the weights too)
            dma_landed(hs);
            const float *as0 = hs + j * kLd + 4 * h, *as1 = as0 + 16 * kLd;
            if (rows > 16) gemv_loop<1, 2>(ws, ow + 64 * k0, 0, as0, as1, kc / 16, acc, wa, wb);
            else           gemv_loop<1, 1>(ws, ow + 64 * k0, 0, as0, as1, kc / 16, acc, wa, wb);
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

int decode_fused_waves(int d, int F) { return d % 128 == 0 && F % 128 == 0 ? 8 : 4; }

hipError_t launch_decode_gateup(const DecodeArgs &a, hipStream_t s) {
    const size_t lds = decode_lds(a);
    static bool attr = false, attr_f4 = false, attr_f8 = false;
    if (a.w2 && decode_fused_waves(a.d, a.F) == 8) {
        hipError_t e = set_lds(reinterpret_cast<const void *>(&decode_gateup_kernel<true, 8>),
                               kDecodeMaxLds, &attr_f8);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((decode_gateup_kernel<true, 8>), dim3((unsigned)(a.E * (a.F / 128))),
                           dim3(512), lds, s, a);
    } else if (a.w2) {
        hipError_t e = set_lds(reinterpret_cast<const void *>(&decode_gateup_kernel<true, 4>),
                               kDecodeMaxLds, &attr_f4);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((decode_gateup_kernel<true, 4>), dim3((unsigned)(a.E * (a.F / 64))),
                           dim3(256), lds, s, a);
    } else {
        hipError_t e = set_lds(reinterpret_cast<const void *>(&decode_gateup_kernel<false, 4>),
                               kDecodeMaxLds, &attr);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((decode_gateup_kernel<false, 4>), dim3((unsigned)(a.E * (a.F / 64))),
                           dim3(256), lds, s, a);
    }
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
