// handoff.h — data handed between workgroups of one launch (device code).
#pragma once
#include <hip/hip_runtime.h>

namespace moe {
namespace {

// Data handed between workgroups of one launch is written with
// device-scope relaxed atomic stores, which are coherent across the XCDs'
// separate L2s, and read with loads of the same (sc1) cache policy.  The
// writer waits for its stores, passes a barrier and then bumps a counter;
// the reader loads only after seeing the count.  (A device-scope fence per
// workgroup instead writes back and invalidates the XCD's L2 each time,
// which serialises the workgroups.)
__device__ inline void cstore(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void cstore4(float *p, float4 v) {
    cstore(p, v.x); cstore(p + 1, v.y); cstore(p + 2, v.z); cstore(p + 3, v.w);
}
// Reader side: buffer loads with the sc1 cache policy from a workgroup-
// uniform base at per-lane offsets (under 2 GiB).  Unlike atomic loads they
// carry no ordering among themselves, so a batch is in flight together.
constexpr int kCachePolicySc1 = 16;
struct CRead {
    __amdgpu_buffer_rsrc_t r;
    __device__ explicit CRead(const float *base)
        : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, 0x7FFFFFFF,
                                              0x00020000)) {}
    __device__ float operator()(size_t idx) const {
        return __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)(idx * 4), 0, kCachePolicySc1));
    }
    __device__ float4 f4(size_t idx) const {   // idx a multiple of 4
        return __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(idx * 4), 0, kCachePolicySc1));
    }
};
// Plain loads, for data written by an earlier launch.
struct PRead {
    const float *p;
    __device__ explicit PRead(const float *base) : p(base) {}
    __device__ float operator()(size_t idx) const { return p[idx]; }
    __device__ float4 f4(size_t idx) const { return *reinterpret_cast<const float4 *>(p + idx); }
};

// Every thread's stores are performed, then the workgroup passes a barrier.
__device__ inline void publish() {
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
}

}  // namespace
}  // namespace moe
