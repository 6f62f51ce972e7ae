// layer.hip — one launch per decode MoE layer: routing and the fused
// gate/up + split-K down expert items in a single persistent grid.
//
// Workgroups 0 .. TB-1 first route one 16-token block each (the row-block
// router, route_rows.h) and publish the expert ids with device-scope atomic
// stores followed by one counter increment per block.  Every other
// workgroup starts on an expert item: once the router blocks hold their
// inputs (a second counter) it issues its first weight loads, which depend
// on nothing the router computes, and only then waits for the routing
// counter, so HBM streams expert weights while the router computes.  Items past the first round are taken from a device-scope counter.
// The grid never exceeds what is co-resident (occupancy query), waits are
// bounded (they raise an error flag instead of hanging), and the last
// workgroup to finish resets the counters for the next launch.  The
// weighted combine of the split-K partials stays a separate launch.
#include <algorithm>

#include "moe_internal.h"
#include "moe_math.h"
#include "route_rows.h"
#include "decode_gemv.h"

namespace moe {
namespace {

template <int KC>
constexpr size_t layer_lds_bytes(int nslots) {
    return sizeof(float) * (RowsSmem<KC>::kFloats > kRows * kLd ? RowsSmem<KC>::kFloats
                                                                 : kRows * kLd) +
           2 * sizeof(int) * (size_t)nslots;
}

template <int RE, int KC, bool SKIP>
__global__ __launch_bounds__(256, 2) void decode_layer_kernel(LayerArgs la) {
    extern __shared__ __align__(16) float smem[];
    __shared__ int wcnt[4];
    __shared__ int s_item;
    const int tid = threadIdx.x;
    const int G = gridDim.x;
    const int TB = (la.r.T + 15) / 16;
    const int nfb = la.g.F / 64;
    const int items = la.g.E * nfb;
    int item = (int)blockIdx.x - TB;   // static first item; router blocks take theirs later
    if ((int)blockIdx.x < TB) {
        route_rows_block<4, RE, KC, SKIP, true>(la.r, blockIdx.x, smem, la.sync + 3);
        WAIT_VMCNT(0);   // this thread's expert-id stores are performed
        __syncthreads();
        if (tid == 0)
            __hip_atomic_fetch_add(&la.sync[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    bool first = true;
    for (;;) {
        if (item < 0) {
            if (tid == 0)
                s_item = (G - TB) + __hip_atomic_fetch_add(&la.sync[1], 1, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            item = s_item;
            __syncthreads();
        }
        if (item >= items) break;
        // The first item's weight loads wait until the router blocks have
        // their inputs (their loads would queue behind the weight stream).
        if (first && (int)blockIdx.x >= TB) wait_count(la.sync + 3, TB, la.err);
        gateup_item<true, true>(la.g, item / nfb, item % nfb, smem, wcnt,
                                first ? la.sync : nullptr, TB, la.err);
        first = false;
        item = -1;
    }
    // The last workgroup out resets the counters (every other one is past
    // its last use of them).
    __syncthreads();
    if (tid == 0 &&
        __hip_atomic_fetch_add(&la.sync[2], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1) {
        __hip_atomic_store(&la.sync[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&la.sync[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&la.sync[2], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&la.sync[3], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

struct LayerLaunch {
    bool init = false;
    int blocks_per_cu = 0;
};

// The router's loads compete with the item workgroups' weight stream, so it
// stages x in as few chunks as its LDS allows (one for d = 512).
template <int RE, int KC, bool SKIP>
hipError_t launch_layer_re(const LayerArgs &la, hipStream_t s) {
    const void *fn = reinterpret_cast<const void *>(&decode_layer_kernel<RE, KC, SKIP>);
    const size_t lds_max = layer_lds_bytes<KC>(kDecodeMaxSlots);
    const size_t lds = layer_lds_bytes<KC>(la.g.nslots);
    static LayerLaunch L;
    if (!L.init) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_max);
        if (e != hipSuccess) return e;
        L.init = true;
    }
    int per_cu = 0, dev = 0, cus = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, lds);
    if (e == hipSuccess) e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    const int TB = (la.r.T + 15) / 16;
    const int items = la.g.E * (la.g.F / 64);
    const int G = std::min(per_cu * cus, TB + items);
    if (G <= TB) return hipErrorInvalidConfiguration;   // every router block must be resident with room for items
    hipLaunchKernelGGL((decode_layer_kernel<RE, KC, SKIP>), dim3(G), dim3(256), lds, s, la);
    return hipGetLastError();
}

template <int RE, bool SKIP>
hipError_t launch_layer_kc(const LayerArgs &la, hipStream_t s) {
    if constexpr (RE <= 2 && !SKIP) {
        if (la.r.d % 512 == 0) return launch_layer_re<RE, 512, SKIP>(la, s);
    }
    return launch_layer_re<RE, 128, SKIP>(la, s);
}

}  // namespace

bool decode_layer_supported(int d, int E) { return d % 128 == 0 && E <= 64; }

hipError_t launch_decode_layer(const LayerArgs &la, hipStream_t s) {
    if (!decode_layer_supported(la.r.d, la.r.E)) return hipErrorInvalidValue;
    const bool skip = la.r.wr_nonfinite != 0;
    if (la.r.E <= 16) return skip ? launch_layer_kc<1, true>(la, s) : launch_layer_kc<1, false>(la, s);
    if (la.r.E <= 32) return skip ? launch_layer_kc<2, true>(la, s) : launch_layer_kc<2, false>(la, s);
    return skip ? launch_layer_kc<4, true>(la, s) : launch_layer_kc<4, false>(la, s);
}

}  // namespace moe
