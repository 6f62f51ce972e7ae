// decode_routed.hip — the fused decode kernel with the routing inside, for
// a KV-cache decode step of up to 64 tokens over up to 16 experts, on
// gfx950.  Its own translation unit, so that the shared item code keeps the
// register allocation it has in decode.hip.
#include <utility>

#include "decode_gemv.h"
#include "route_rows.h"

namespace moe {
namespace {

// ---------------------------------------------------------------------------
// Routed fused kernel: the router inside the fused gate/up + down kernel, for
// a decode step of T <= 64 tokens, E <= 16 experts and d = KC (256 or 512).
// Every workgroup routes all T tokens itself (the row-block router's chains
// and finish, route_rows.h, so probabilities and experts are the same bits),
// with the token rows resident in LDS, which then feed its item's products
// directly: no rows are staged and no router launch precedes the kernel.
// Order of the loads: the rows (DMA) and router rows, a wait for them, the
// item's first weight group (streaming under the routing), and the second
// group once the chains are done.  At the end workgroup b also writes ids,
// gate weights and probabilities of tokens b, b + grid, ... (and, when the
// caller takes them, their normalised rows).
//
// LDS: rows [T][KC + 4]; the H block, whose start holds the rms weights
// until the rows are normalised; the routing results (logits, then
// probabilities, chosen experts and their probabilities, renormalisation
// factors), kept to the end, where they are written out; the slot and
// token lists.
constexpr int kRoutedMaxT = 64;
constexpr int kRoutedHBlock = kRows * hld<8>();   // floats

// Floats of routing results for E experts and top-k.
__host__ __device__ constexpr int routed_results(int E, int k) {
    return kRoutedMaxT * (E + 1) + 2 * kRoutedMaxT * k + kRoutedMaxT;
}

// f(integral_constant<int, S>) for S in the sequence, in order.
template <class F, int... S>
__device__ inline void static_for(std::integer_sequence<int, S...>, F &&f) {
    (f(std::integral_constant<int, S>{}), ...);
}

template <int KC, int RE>
__global__ __launch_bounds__(512, 1) void decode_routed_kernel(DecodeArgs a, RouteArgs ra) {
    constexpr int NW = 8, LD = KC + 4, WV4 = KC / 64, NS = KC / 16;
    extern __shared__ __align__(16) float smem[];
    __shared__ int wcnt[NW];
    const int T = ra.T, E = ra.E, k = ra.k, n = a.nslots;
    float *xs = smem;                                   // [T][LD]
    float *hs = xs + (size_t)T * LD;                    // H block
    float *rw_l = hs;                                   // [KC] rms weights, until normalised
    float *lg = hs + kRoutedHBlock;                     // [64][E + 1] logits, then probabilities
    float *psel = lg + kRoutedMaxT * (E + 1);           // [64 * k]
    int *isel = reinterpret_cast<int *>(psel + kRoutedMaxT * k);   // [64 * k]
    float *invs = reinterpret_cast<float *>(isel + kRoutedMaxT * k);   // [64]
    int *list = reinterpret_cast<int *>(lg + routed_results(E, k));
    int *tok = list + n;

    const int nfb = a.F / (16 * NW);
    int e, fb;
    item_of(blockIdx.x, a.E, nfb, e, fb);
    const ItemGeo<NW> g = item_geo<true, NW>(a, e, fb);
    const int tid = threadIdx.x, lane = g.lane, wave = g.wave;

    // Rows (raw when normalising) and rms weights to LDS.
    const float *src = ra.rms_w ? ra.x_raw : ra.x;
    for (int r = wave; r < T; r += NW)
#pragma unroll
        for (int p = 0; p < KC / 256; ++p)
            __builtin_amdgcn_global_load_lds(src + (size_t)r * KC + 256 * p + 4 * lane,
                                             xs + r * LD + 256 * p, 16, 0, 0);
    if (ra.rms_w && wave == 0)
#pragma unroll
        for (int p = 0; p < KC / 256; ++p)
            __builtin_amdgcn_global_load_lds(ra.rms_w + 256 * p + 4 * lane, rw_l + 256 * p, 16, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    // Router rows: waves 2 tb and 2 tb + 1 run token block tb; lane (r, c)
    // the chains of token 16 tb + c with experts 4 (half RE + j) + r.
    const int tb = wave >> 1, half = wave & 1, r = lane >> 4, c = lane & 15;
    float4 w4[RE][WV4];
    float bv[RE];
#pragma unroll
    for (int j = 0; j < RE; ++j) {
        const int ej = min(4 * (half * RE + j) + r, E - 1);
        const float *wrow = ra.wrT + (size_t)ej * KC + 4 * c;
#pragma unroll
        for (int b = 0; b < WV4; ++b) w4[j][b] = *reinterpret_cast<const float4 *>(wrow + 64 * b);
        bv[j] = *(ra.bias ? ra.bias + ej : ra.wrT + ej);   // (a load either way: no branch)
    }
    __builtin_amdgcn_sched_barrier(0);
    WGroup<2> wa, wb;
    constexpr int ng = NS / Unroll<2>::kU;
    const int g0 = g.rot_of(NS);
    const int ob[2] = {g.og, g.ou};
    __builtin_amdgcn_sched_barrier(0);
    WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
    dma_landed(xs);
    // The first weight group goes out once the rows are in (issued earlier,
    // it slows their arrival more than it gains).
    __builtin_amdgcn_sched_barrier(0);
    wload<2>(g.gs, ob, group_step<2>(0, g0, ng), NS - 1, wa);
    __builtin_amdgcn_sched_barrier(0);
    if (ra.rms_w) {
        // (rms_row16 holds a whole row in registers first, so in place is safe)
        for (int rr = tid >> 4; rr < T; rr += 64 * NW / 16) {
            float *xr = xs + rr * LD;
            rms_row16([&](int i) { return xr[i]; }, rw_l, KC / 16, ra.rms_eps, ra.rms_rcp,
                      nullptr, false, xr, false);
        }
        __syncthreads();
    }

    // The chains, k ascending; x of the next 16 steps is read while the FMAs
    // of these run.  Every wave runs them (rows past T repeat row T - 1), so
    // that no branch splits the register state the weight stream shares.
    float acc[RE];
#pragma unroll
    for (int j = 0; j < RE; ++j) acc[j] = 0.0f;
    {
        const float *xrow = xs + min(16 * tb + c, T - 1) * LD;
        auto xread = [&](float (&xv)[16], int sl) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = *reinterpret_cast<const float4 *>(xrow + 16 * sl + 4 * q);
                xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
            }
        };
        auto chains = [&](const float (&xv)[16], auto slc) {
            constexpr int SL = decltype(slc)::value;
            if constexpr (RE == 2)
                chain16x2_dpp4<SL % 4>(acc[0], acc[1], w4[0][SL / 4], w4[1][SL / 4], xv);
            else
#pragma unroll
                for (int j = 0; j < RE; ++j) chain16_dpp4<SL % 4>(acc[j], w4[j][SL / 4], xv);
        };
        float xa[16], xb[16];
        xread(xa, 0);
        static_for(std::make_integer_sequence<int, NS / 2>{}, [&](auto sc) {
            constexpr int SL = 2 * decltype(sc)::value;
            xread(xb, SL + 1);
            chains(xa, std::integral_constant<int, SL>{});
            if constexpr (SL + 2 < NS) xread(xa, SL + 2);
            chains(xb, std::integral_constant<int, SL + 1>{});
        });
    }
    // The second weight group once the chains are done (issued during the
    // chains, it blocks them while the memory queues are full; issued after
    // the finish below, the layer took 0.85 us longer).
    __builtin_amdgcn_sched_barrier(0);
    wload<2>(g.gs, ob, group_step<2>(1, g0, ng), NS - 1, wb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < RE; ++j) {
        const int ej = 4 * (half * RE + j) + r;
        if (ej < E) lg[(16 * tb + c) * (E + 1) + ej] = ra.bias ? acc[j] + bv[j] : acc[j];
    }
    __syncthreads();
    {
        // (tokens past T finish rows that nothing reads)
        const int ct = tid >> 3, l = tid & 7;
        const float inv = finish_token8<(8 * RE + 7) / 8>(ra, lg + ct * (E + 1), l, isel + ct * k,
                                                          psel + ct * k);
        if (l == 0) invs[ct] = inv;
    }
    __syncthreads();

    // The item: its slots from the experts just chosen, then the products
    // with the rows read in place (row j of a 16-row block: token tok[r0 + j]).
    const int id0 = tid < n ? isel[tid] : -1;
    const int cnt = expert_slots<NW>(isel, n, e, id0, a.topk, list, tok, wcnt);
    for (int r0 = 0; r0 < cnt; r0 += kRows) {
        const int rows = min(kRows, cnt - r0);
        floatx4 acc2[2][2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int q = 0; q < 2; ++q) acc2[b][q] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (r0 > 0) gemv_prime<2>(g.gs, g.og, g.ou, NS, wa, wb, g0);
        const float *as0 = xs + tok[r0 + min(g.j, rows - 1)] * LD + 4 * g.h;
        const float *as1 = xs + tok[r0 + min(16 + g.j, rows - 1)] * LD + 4 * g.h;
        if (rows > 16) gemv_loop<2, 2, true, NW>(g.gs, g.og, g.ou, as0, as1, NS, acc2, wa, wb, g.dh, g0);
        else           gemv_loop<2, 1, true, NW>(g.gs, g.og, g.ou, as0, as1, NS, acc2, wa, wb, g.dh, g0);
        fused_down_pass<NW, true>(a, g, fb, acc2, rows, list, r0, hs, wa, wb);
    }

    // The routing results (and the normalised rows, when wanted), token t
    // by workgroup t (every workgroup holds them all), last, so that no
    // stores of varying count sit among the weight loads whose completion
    // the loops count, and no one workgroup's end waits on all of them.
    for (int ct = blockIdx.x; ct < T; ct += gridDim.x) {
        if (tid < k) {
            const int i = ct * k + tid;
            if (ra.ids) ra.ids[i] = isel[i];
            if (ra.gw) ra.gw[i] = ftz_f(psel[i] * invs[ct]);
        }
        if (ra.probs)
            for (int ex = tid; ex < E; ex += 64 * NW) ra.probs[ct * E + ex] = lg[ct * (E + 1) + ex];
        if (ra.rms_w && ra.xn_out)
            for (int c4 = tid; c4 < KC / 4; c4 += 64 * NW)
                *reinterpret_cast<float4 *>(ra.xn_out + (size_t)ct * KC + 4 * c4) =
                    *reinterpret_cast<const float4 *>(xs + ct * LD + 4 * c4);
    }
}

// Dynamic LDS of the routed kernel: rows, H block, routing results, slot
// and token lists.
size_t decode_routed_lds(int T, int d, int E, int k) {
    return sizeof(float) * ((size_t)T * (d + 4) + kRoutedHBlock + routed_results(E, k)) +
           2 * sizeof(int) * (size_t)T * k;
}
constexpr size_t kRoutedMaxLds = 160 * 1024;   // LDS of a gfx950 workgroup

template <int KC, int RE>
hipError_t launch_routed(const DecodeArgs &a, const RouteArgs &ra, size_t lds, hipStream_t s) {
    static size_t attr = 0;
    if (lds > attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&decode_routed_kernel<KC, RE>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr = lds;
    }
    hipLaunchKernelGGL((decode_routed_kernel<KC, RE>), dim3((unsigned)(a.E * (a.F / 128))),
                       dim3(512), lds, s, a, ra);
    return hipGetLastError();
}

}  // namespace

bool decode_routed_ok(int T, int d, int F, int E, int k) {
    return T >= 1 && T <= kRoutedMaxT && E >= 1 && E <= 16 && k >= 1 && k <= E &&
           (d == 256 || d == 512) && F % 128 == 0 &&
           decode_routed_lds(T, d, E, k) <= kRoutedMaxLds;
}

hipError_t launch_decode_routed(const DecodeArgs &a, const RouteArgs &ra, hipStream_t s) {
    if (!decode_routed_ok(ra.T, a.d, a.F, a.E, ra.k) || ra.d != a.d || ra.E != a.E ||
        a.nslots != ra.T * ra.k || !ra.wrT || !a.w2 || (ra.rms_w && !ra.x_raw))
        return hipErrorInvalidValue;
    const size_t lds = decode_routed_lds(ra.T, a.d, a.E, ra.k);
    if (a.d == 512) return a.E <= 8 ? launch_routed<512, 1>(a, ra, lds, s) : launch_routed<512, 2>(a, ra, lds, s);
    return a.E <= 8 ? launch_routed<256, 1>(a, ra, lds, s) : launch_routed<256, 2>(a, ra, lds, s);
}

}  // namespace moe
