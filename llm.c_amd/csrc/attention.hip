// attention.hip — the attention half of the KV-cache decode step
// (src/inference.c:252-308) for B sequences at once, each at its own
// position, on gfx950.
//
//   proj_kernel<QKV>  q, k, v = xn . W_Q, W_K, W_V as the reference's matvec
//                     (:174-182): per output one FMA chain over the input
//                     index, ascending, zero inputs skipped.  Epilogue: RoPE
//                     at the sequence's position from the caller's tables
//                     (:187-203) on q and k, k and v written into the caches.
//   attn_chunk_kernel one workgroup per (sequence, kv head, 256 positions):
//                     scores of the kv head's query heads in the reference's
//                     vec_dot order (:133-155) times 1/sqrt(hd), exp against
//                     the chunk maximum, then the V sum with lane = dimension
//                     as FMAs in position order.  Bound by the K/V reads.
//   attn_merge_kernel the chunks of a head: o = sum_c e^(m_c - M) o_c /
//                     sum_c e^(m_c - M) l_c.
//   proj_kernel<WO>   x += o . W_O (matvec, then the element add of :306).
// The reference normalises the scores before the V sum and sums the
// exponentials sequentially over all positions; chunking reorders those
// sums, so outputs match within the layer tolerance, not bit for bit.
#include "moe_internal.h"
#include "moe_math.h"

namespace moe {
namespace {

constexpr int kChunkPos = 256;   // positions per attention workgroup

// Four outputs (columns n .. n+3 of one matrix) of two rows b, b+1: the
// reference matvec's chain for each.  in: [B x M] rows, w: [M x N].
__device__ inline void chain4x2(const float *in0, const float *in1, const float *w, int M, int N,
                                int n, float (&o0)[4], float (&o1)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) o0[c] = o1[c] = 0.0f;
    for (int i = 0; i < M; ++i) {
        const float4 wv = *reinterpret_cast<const float4 *>(w + (size_t)i * N + n);
        const float a = in0[i], b = in1[i];
        if (a != 0.0f) {
            o0[0] = fmaf(a, wv.x, o0[0]); o0[1] = fmaf(a, wv.y, o0[1]);
            o0[2] = fmaf(a, wv.z, o0[2]); o0[3] = fmaf(a, wv.w, o0[3]);
        }
        if (b != 0.0f) {
            o1[0] = fmaf(b, wv.x, o1[0]); o1[1] = fmaf(b, wv.y, o1[1]);
            o1[2] = fmaf(b, wv.z, o1[2]); o1[3] = fmaf(b, wv.w, o1[3]);
        }
    }
}

// RoPE on the pair (v0, v1) = columns 2i, 2i + 1 of a head (:196-199).
__device__ inline void rope_pair(float &v0, float &v1, float c, float s) {
    const float a = v0, b = v1;
    v0 = a * c - b * s;
    v1 = a * s + b * c;
}

// One thread: rows 2r, 2r + 1 and four columns.  QKV: columns [0, qd) of
// W_Q, then [qd, qd + kd) of W_K and [qd + kd, qd + 2kd) of W_V.
template <bool QKV>
__global__ __launch_bounds__(256) void proj_kernel(AttnArgs a, const float *in, int M) {
    const int ncol = QKV ? a.qd + 2 * a.kd : a.d;
    const int nq = ncol / 4;
    const int gid = blockIdx.x * 256 + threadIdx.x;
    const int r = gid / nq, n = 4 * (gid % nq);
    const int b0 = 2 * r, b1 = min(2 * r + 1, a.B - 1);
    if (b0 >= a.B) return;
    const float *w;
    int col, N;
    if (!QKV)               { w = a.wo; col = n; N = a.d; }
    else if (n < a.qd)      { w = a.wq; col = n; N = a.qd; }
    else if (n < a.qd + a.kd) { w = a.wk; col = n - a.qd; N = a.kd; }
    else                    { w = a.wv; col = n - a.qd - a.kd; N = a.kd; }
    float o[2][4];
    chain4x2(in + (size_t)b0 * M, in + (size_t)b1 * M, w, M, N, col, o[0], o[1]);
    for (int rr = 0; rr < 2; ++rr) {
        const int b = rr ? b1 : b0;
        if (rr && b1 == b0) break;
        const int p = a.pos[b];
        if (p < 0 || p >= a.max_seq) continue;   // (no such position: the row is left out)
        if (!QKV) {
            float4 *xp = reinterpret_cast<float4 *>(a.x + (size_t)b * a.d + col);
            float4 v = *xp;
            v.x = v.x + o[rr][0]; v.y = v.y + o[rr][1]; v.z = v.z + o[rr][2]; v.w = v.w + o[rr][3];
            *xp = v;
            continue;
        }
        const int half = a.hd / 2;
        if (n < a.qd + a.kd) {   // q or k: RoPE at p on both pairs
            const int i0 = (col % a.hd) / 2;
            const float *cr = a.cos_t + (size_t)p * half, *sr = a.sin_t + (size_t)p * half;
            rope_pair(o[rr][0], o[rr][1], cr[i0], sr[i0]);
            rope_pair(o[rr][2], o[rr][3], cr[i0 + 1], sr[i0 + 1]);
        }
        const float4 v = make_float4(o[rr][0], o[rr][1], o[rr][2], o[rr][3]);
        if (n < a.qd)
            *reinterpret_cast<float4 *>(a.q + (size_t)b * a.qd + col) = v;
        else
            *reinterpret_cast<float4 *>((n < a.qd + a.kd ? a.kc : a.vc) +
                                        ((size_t)b * a.max_seq + p) * a.kd + col) = v;
    }
}

// Workgroup (b, kv head, chunk c): positions j in [256c, min(256c + 256,
// pos + 1)).  Phase 1, lane = position: the scores of the kv head's gqa
// query heads in vec_dot's order.  Phase 2: per head the chunk maximum m,
// p_j = exp(s_j - m), l = sum p_j.  Phase 3, lane = dimension, wave = head
// (heads past 4 in turns): o = sum_j p_j V[j] as FMAs in position order.
// The partial (m, l, o[hd]) goes to part[(b, head, c)].
__global__ __launch_bounds__(256) void attn_chunk_kernel(AttnArgs a) {
    __shared__ float q_s[8][64];          // gqa <= 8 heads, hd <= 64
    __shared__ float sc[8][kChunkPos];
    __shared__ float red[8][4];
    const int nchunk = (a.max_seq + kChunkPos - 1) / kChunkPos;
    const int c = blockIdx.x % nchunk;
    const int kvh = (blockIdx.x / nchunk) % a.nkv;
    const int b = blockIdx.x / (nchunk * a.nkv);
    const int gqa = a.nh / a.nkv, hd = a.hd;
    const int pb = a.pos[b];
    const int p = pb >= 0 && pb < a.max_seq ? pb : -1;   // (out of range: attends nothing)
    const int j0 = c * kChunkPos, j1 = min(j0 + kChunkPos, p + 1);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float *part = a.part + ((size_t)(b * a.nh + kvh * gqa) * nchunk + c) * (hd + 2);
    const size_t head_stride = (size_t)nchunk * (hd + 2);
    if (j0 >= j1) {   // past the sequence: an empty partial
        if (tid < gqa) {
            part[tid * head_stride] = -INFINITY;
            part[tid * head_stride + 1] = 0.0f;
        }
        return;
    }
    for (int i = tid; i < gqa * hd; i += 256)
        q_s[i / hd][i % hd] = a.q[(size_t)b * a.qd + (size_t)(kvh * gqa) * hd + i];
    __syncthreads();
    const float *K = a.kc + (size_t)b * a.max_seq * a.kd + kvh * hd;
    const float *V = a.vc + (size_t)b * a.max_seq * a.kd + kvh * hd;
    const int j = j0 + tid;
    if (j < j1) {
        const float *kr = K + (size_t)j * a.kd;
        for (int h = 0; h < gqa; ++h) {
            float v0[8], v1[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) v0[l] = v1[l] = 0.0f;
            int i = 0;
            for (; i + 16 <= hd; i += 16)
#pragma unroll
                for (int l = 0; l < 8; ++l) {
                    v0[l] = fmaf(q_s[h][i + l], kr[i + l], v0[l]);
                    v1[l] = fmaf(q_s[h][i + 8 + l], kr[i + 8 + l], v1[l]);
                }
#pragma unroll
            for (int l = 0; l < 8; ++l) v0[l] = v0[l] + v1[l];
            for (; i + 8 <= hd; i += 8)
#pragma unroll
                for (int l = 0; l < 8; ++l) v0[l] = fmaf(q_s[h][i + l], kr[i + l], v0[l]);
            float r = ((v0[0] + v0[4]) + (v0[1] + v0[5])) + ((v0[2] + v0[6]) + (v0[3] + v0[7]));
            for (; i < hd; ++i) r = fmaf(q_s[h][i], kr[i], r);
            sc[h][tid] = r * a.scale;
        }
    }
    __syncthreads();
    // Per head: chunk maximum, then exponentials and their sum.
    const int n = j1 - j0;
    for (int h = 0; h < gqa; ++h) {
        float m = -INFINITY;
        for (int t = tid; t < n; t += 256) m = fmaxf(m, sc[h][t]);
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        if (lane == 0) red[h][wave] = m;
    }
    __syncthreads();
    for (int h = 0; h < gqa; ++h) {
        const float m = fmaxf(fmaxf(red[h][0], red[h][1]), fmaxf(red[h][2], red[h][3]));
        float l = 0.0f;
        for (int t = tid; t < n; t += 256) {
            const float e = expf(sc[h][t] - m);
            sc[h][t] = e;
            l += e;
        }
        for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off);
        __syncthreads();   // every wave has read red[h] before it is reused
        if (lane == 0) red[h][wave] = l;
        if (tid == 0) part[h * head_stride] = m;
    }
    __syncthreads();
    for (int h = wave; h < gqa; h += 4) {
        if (lane < hd) {
            float o = 0.0f;
            for (int t = 0; t < n; ++t) o = fmaf(sc[h][t], V[(size_t)(j0 + t) * a.kd + lane], o);
            part[h * head_stride + 2 + lane] = o;
        }
        if (lane == 0)
            part[h * head_stride + 1] = (red[h][0] + red[h][1]) + (red[h][2] + red[h][3]);
    }
}

// One thread per (b, head, dimension): merge the chunks into o[b][head][dim].
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a) {
    const int nchunk = (a.max_seq + kChunkPos - 1) / kChunkPos;
    const int gid = blockIdx.x * 256 + threadIdx.x;
    if (gid >= a.B * a.qd) return;
    const int b = gid / a.qd, h = (gid % a.qd) / a.hd, t = gid % a.hd;
    const float *part = a.part + (size_t)(b * a.nh + h) * nchunk * (a.hd + 2);
    const int p = a.pos[b];
    if (p < 0 || p >= a.max_seq) {   // no such position: a zero attention output
        a.o[gid] = 0.0f;
        return;
    }
    const int nc = (p + kChunkPos) / kChunkPos;   // chunks holding positions <= pos
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, part[c * (a.hd + 2)]);
    float L = 0.0f, O = 0.0f;
    for (int c = 0; c < nc; ++c) {
        const float *pc = part + c * (a.hd + 2);
        const float f = expf(pc[0] - M);
        L = fmaf(f, pc[1], L);
        O = fmaf(f, pc[2 + t], O);
    }
    a.o[gid] = O / L;
}

}  // namespace

size_t attn_part_floats(int B, int nh, int hd, int max_seq) {
    return (size_t)B * nh * ((max_seq + kChunkPos - 1) / kChunkPos) * (hd + 2);
}

hipError_t launch_attn_decode(const AttnArgs &a, hipStream_t s) {
    if (a.B <= 0) return hipSuccess;
    const int gqa = a.nh / a.nkv;
    if (a.hd > 64 || a.hd % 8 || gqa > 8 || a.nh % a.nkv || a.d % 4 || a.qd % 4)
        return hipErrorInvalidValue;
    const int rows2 = (a.B + 1) / 2;
    const int qkv_threads = rows2 * (a.qd + 2 * a.kd) / 4;
    hipLaunchKernelGGL(proj_kernel<true>, dim3((unsigned)((qkv_threads + 255) / 256)), dim3(256),
                       0, s, a, a.xn, a.d);
    const int nchunk = (a.max_seq + kChunkPos - 1) / kChunkPos;
    hipLaunchKernelGGL(attn_chunk_kernel, dim3((unsigned)(a.B * a.nkv * nchunk)), dim3(256), 0, s,
                       a);
    hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)((a.B * a.qd + 255) / 256)), dim3(256),
                       0, s, a);
    const int wo_threads = rows2 * a.d / 4;
    hipLaunchKernelGGL(proj_kernel<false>, dim3((unsigned)((wo_threads + 255) / 256)), dim3(256),
                       0, s, a, a.o, a.qd);
    return hipGetLastError();
}

}  // namespace moe
