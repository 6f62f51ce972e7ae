// attention.hip — the attention half of the KV-cache decode step
// (src/inference.c:252-308) for B sequences at once, each at its own
// position, on gfx950:  x += W_O . Attn(RoPE(W_Q xn), RoPE(W_K xn), W_V xn)
// with xn = rms_norm(x) and the new k, v rows appended to the caches.
//
// Three roles, run as one launch (attn_fused_kernel, head_dim 16/32/64 with
// 2/4/8 query heads per kv head) or as separate launches:
//   QKV tile      q, k, v as a split-K tiled product: 32 x 32 output tiles,
//                 128-long reduction slices per workgroup (32 per wave,
//                 summed through LDS).  rms_norm's row scale 1/rms (:48-60)
//                 is taken out of the reduction: tiles multiply x * w_rms,
//                 each slice also sums its x^2, and the tile's last slice
//                 to finish adds the slices, scales by 1/sqrt(ss/d + eps),
//                 applies RoPE at the sequence's position from the caller's
//                 tables (:187-203) to q and k, and writes q and the cache
//                 rows at pos.
//   chunk         one workgroup per (sequence, kv head, 128 positions)
//                 streams that K and V once for the kv head's query heads:
//                 scores times 1/sqrt(hd), exp against the chunk maximum,
//                 the V sum; the last chunk of a (sequence, kv head) merges
//                 the chunk partials (m, l, o) into o.  Bound by the K/V
//                 reads.  In the fused launch the cache rows before pos are
//                 requested at once, before the QKV tiles are done; only q
//                 and the new row wait for them.
//   W_O tile      x += o . W_O with the same tiles; the tile's last slice
//                 adds the slices into x (the element add of :306).
// Roles hand data to each other within a launch through device-scope
// coherent stores and loads and counters (see the helpers below); in the
// fused launch later roles wait, boundedly, for earlier ones, which sit at
// lower workgroup indices and so are dispatched first.
// Sequences whose position lies outside [0, max_seq) are left untouched.
// Reductions run in a fixed order, so results are deterministic, but the
// order differs from the reference's sequential sums (and the reference
// normalises x before the products): outputs match within the layer
// tolerance, not bit for bit.
#include <type_traits>

#include "handoff.h"
#include "moe_internal.h"
#include "moe_math.h"

namespace moe {
namespace {

constexpr int kChunkPos = 128;   // positions per attention workgroup
constexpr int kTile = 32;        // rows and columns of a projection tile
constexpr int kSliceK = 128;     // reduction length per projection workgroup

// RoPE on the pair (v0, v1) = columns 2i, 2i + 1 of a head (:196-199).
__device__ inline void rope_pair(float &v0, float &v1, float c, float s) {
    const float a = v0, b = v1;
    v0 = a * c - b * s;
    v1 = a * s + b * c;
}

__device__ inline float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ inline float comp(const float4 &v, int j) {
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

// Readiness of a count in the one-launch sublayer: kFlagCopies flags, one
// per 128-byte line, all set by the workgroup that completes the count;
// waiters each poll one copy, so polling is spread over many addresses.
constexpr int kFlagCopies = 64, kFlagStride = 32;   // ints
// sync layout: [0] QKV tiles done, [1] merges done, [2] workgroups out, then
// the two flag sets.
constexpr int kSyncQkvFlags = kFlagStride;
constexpr int kSyncMergeFlags = kSyncQkvFlags + kFlagCopies * kFlagStride;
// After publish(), one bump of *ctr; the bump that makes it `expect` sets
// the flags.
__device__ inline void signal(int *ctr, int expect, int *flags) {
    publish();
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == expect - 1)
        for (int i = 0; i < kFlagCopies; ++i)
            __hip_atomic_store(flags + i * kFlagStride, 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}
// True in every thread of the workgroup that arrives last of `expect` at
// *cnt (after publishing its stores); that one also resets the counter.
__device__ inline bool arrive_last(int *cnt, int expect, int *flag) {
    publish();
    if (threadIdx.x == 0) {
        const bool last =
            __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == expect - 1;
        if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = last;
    }
    __syncthreads();
    return *flag;
}
// Thread 0 waits (bounded; past the bound it raises *err and goes on, so
// every wave ends) until its copy of the flags is set; then the workgroup
// passes a barrier.
__device__ inline void wait_flag(const int *flags, int *err) {
    if (threadIdx.x == 0) {
        const int *f = flags + (blockIdx.x % kFlagCopies) * kFlagStride;
        int spins = 0;
        while (__hip_atomic_load(const_cast<int *>(f), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) == 0) {
            if (++spins > kSpinLimit) {
                __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(8);
        }
    }
    __syncthreads();
}

__host__ __device__ inline int slices(int M) { return (M + kSliceK - 1) / kSliceK; }
__host__ __device__ inline int tiles(int n) { return (n + kTile - 1) / kTile; }

// ---------------------------------------------------------------------------
// Projection tiles.
struct ProjSmem {
    union {
        struct {
            float4 xs[kTile][kSliceK / 4 + 1];   // X rows of the slice (padded)
            float4 ws[kSliceK][kTile / 4];       // W rows of the slice
        };
        float4 red[4][kTile][kTile / 4];         // per-wave partial tiles, after the products
    };
    int flag;
};

// Tile (tx, ty) and reduction slice z of Y = X . W for X [B x M], W [M x N]:
// QKV: X = x scaled by w_rms, W = [W_Q | W_K | W_V]; WO: X = o, W = W_O.
// Threads load row tid / 8 of X and rows tid / 8 + 32i of W; wave w takes
// slice rows 32w .. 32w + 31, lane (rq, cq) = (lane / 8, lane % 8) rows
// 4rq .. 4rq + 3 and columns 4cq .. 4cq + 3 of the tile.  FUSED: part of the
// one-launch sublayer (WO waits for the merges; QKV's outputs are written
// coherently and counted).
template <bool QKV, bool FUSED>
__device__ void proj_tile(const AttnArgs &a, int tx, int ty, int z, int ntx, int S, ProjSmem &sm) {
    const int M = QKV ? a.d : a.qd, N = QKV ? a.qd + 2 * a.kd : a.d;
    const int r0 = ty * kTile, c0 = tx * kTile, k0 = z * kSliceK;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    float4 wv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = tid + 256 * i, k = k0 + (idx >> 3), col = c0 + 4 * (idx & 7);
        const float *src = nullptr;
        if (k < M && col < N) {
            if (!QKV)                     src = a.wo + (size_t)k * a.d + col;
            else if (col < a.qd)          src = a.wq + (size_t)k * a.qd + col;
            else if (col < a.qd + a.kd)   src = a.wk + (size_t)k * a.kd + (col - a.qd);
            else                          src = a.wv + (size_t)k * a.kd + (col - a.qd - a.kd);
        }
        wv[i] = src ? *reinterpret_cast<const float4 *>(src) : zero;
    }
    if (FUSED && !QKV) wait_flag(a.sync + kSyncMergeFlags, a.err);   // every merge is done
    const int xr = tid >> 3, xrow = r0 + xr;
    float4 xv[4];
    {
        const float *X = QKV ? a.x : a.o;
        const size_t rb = (size_t)(xrow < a.B ? xrow : 0) * M;
        const CRead cx(X);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = k0 + 4 * ((tid & 7) + 8 * i);
            const bool in = xrow < a.B && k < M;
            if (FUSED && !QKV) xv[i] = cx.f4(in ? rb + k : 0);
            else               xv[i] = in ? *reinterpret_cast<const float4 *>(X + rb + k) : zero;
            if (!in) xv[i] = zero;
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int kq = (tid & 7) + 8 * i, k = k0 + 4 * kq;
        float4 v = xv[i];
        if (QKV && k < M) {
            ss = fmaf(v.x, v.x, ss); ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss); ss = fmaf(v.w, v.w, ss);
            const float4 w = *reinterpret_cast<const float4 *>(a.rms_w + k);
            v = make_float4(v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w);
        }
        sm.xs[xr][kq] = v;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = tid + 256 * i;
        sm.ws[idx >> 3][idx & 7] = wv[i];
    }
    if (QKV) {
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        if ((tid & 7) == 0 && xrow < a.B) cstore(a.sspart + (size_t)z * a.B + xrow, ss);
    }
    __syncthreads();

    const int rq = lane >> 3, cq = lane & 7;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[i][c] = 0.0f;
#pragma unroll
    for (int s = 0; s < kSliceK / 16; ++s) {
        const int kq = wave * (kSliceK / 16) + s;
        float4 xa[4], wb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xa[i] = sm.xs[4 * rq + i][kq];
#pragma unroll
        for (int j = 0; j < 4; ++j) wb[j] = sm.ws[4 * kq + j][cq];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float xij = comp(xa[i], j);
                acc[i][0] = fmaf(xij, wb[j].x, acc[i][0]);
                acc[i][1] = fmaf(xij, wb[j].y, acc[i][1]);
                acc[i][2] = fmaf(xij, wb[j].z, acc[i][2]);
                acc[i][3] = fmaf(xij, wb[j].w, acc[i][3]);
            }
    }
    __syncthreads();   // (red overlays xs and ws)
#pragma unroll
    for (int i = 0; i < 4; ++i)
        sm.red[wave][4 * rq + i][cq] = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    __syncthreads();
    const int orow = r0 + (tid >> 3), ocol = c0 + 4 * (tid & 7);
    const bool owned = orow < a.B && ocol < N;
    if (owned) {
        const int r = tid >> 3, c = tid & 7;
        const float4 v = add4(add4(sm.red[0][r][c], sm.red[1][r][c]),
                              add4(sm.red[2][r][c], sm.red[3][r][c]));
        cstore4(a.gpart + ((size_t)z * a.B + orow) * N + ocol, v);
    }

    // The last slice of this tile to finish adds the slices and writes out;
    // what that epilogue needs besides the slices is fetched before arriving.
    const int p = owned ? a.pos[orow] : -1;
    const bool live = owned && p >= 0 && p < a.max_seq;
    const int col = ocol < a.qd ? ocol : ocol < a.qd + a.kd ? ocol - a.qd : ocol - a.qd - a.kd;
    const bool rope = QKV && live && ocol < a.qd + a.kd;
    float4 cs = zero;   // (cos, sin) of the column's two RoPE pairs
    if (rope) {
        const int half = a.hd / 2, i0 = (col % a.hd) / 2;
        const float *cr = a.cos_t + (size_t)p * half + i0, *sr = a.sin_t + (size_t)p * half + i0;
        cs = make_float4(cr[0], sr[0], cr[1], sr[1]);
    }
    float4 xo = zero;
    if (!QKV && live) xo = *reinterpret_cast<const float4 *>(a.x + (size_t)orow * a.d + ocol);

    if (!arrive_last((QKV ? a.cnt_qkv : a.cnt_wo) + ty * ntx + tx, S, &sm.flag)) return;
    if (live) {
        const CRead gp(a.gpart), sp(a.sspart);
        float4 y = zero;
        float sq = 0.0f;
        for (int z0 = 0; z0 < S; z0 += 4) {
            float4 v[4];
            float q2[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int zz = z0 + u < S ? z0 + u : 0;
                v[u] = gp.f4(((size_t)zz * a.B + orow) * N + ocol);
                q2[u] = QKV ? sp((size_t)zz * a.B + orow) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (z0 + u < S) {
                    y = add4(y, v[u]);
                    sq += q2[u];
                }
        }
        if (!QKV) {
            *reinterpret_cast<float4 *>(a.x + (size_t)orow * a.d + ocol) = add4(xo, y);
        } else {
            const float inv = 1.0f / sqrtf(sq / (float)M + a.eps);
            y = make_float4(y.x * inv, y.y * inv, y.z * inv, y.w * inv);
            if (rope) {   // q or k: RoPE at p on both pairs
                rope_pair(y.x, y.y, cs.x, cs.y);
                rope_pair(y.z, y.w, cs.z, cs.w);
            }
            float *dst = ocol < a.qd ? a.q + (size_t)orow * a.qd
                                     : (ocol < a.qd + a.kd ? a.kc : a.vc) +
                                           ((size_t)orow * a.max_seq + p) * a.kd;
            if (FUSED) cstore4(dst + col, y);
            else       *reinterpret_cast<float4 *>(dst + col) = y;
        }
    }
    if (FUSED && QKV) signal(a.sync, a.nqkv_tiles, a.sync + kSyncQkvFlags);   // q, k, v are out
}

// Projection tiles without a split reduction: one 1024-thread workgroup per
// 16 x 16 output tile (tile column blockIdx.x, row blockIdx.y).  The X rows
// and W columns of a 512-long reduction chunk are staged in LDS: thread t
// loads float4 t % 128 of X rows t / 128 and 8 + t / 128, and float4s t and
// t + 1024 of the W block.  Wave w takes chunk rows 32w .. 32w + 31, lane
// (rr, cq) = (lane / 4, lane % 4) row rr and columns 4cq .. 4cq + 3; the
// sixteen waves' sums are added through LDS in wave order.  QKV: row r's
// sum of x^2 is each thread's k-ordered share, summed over its wave and
// then over the row's two waves; the epilogue (1/rms, RoPE, q and the cache
// rows) as in proj_tile.  WO: x += the products.  One global round trip.
constexpr int kPT = 16, kPK = 512;
struct Proj16Smem {
    union {
        struct {
            float4 xs[kPT][kPK / 4 + 1];
            float4 ws[kPK][kPT / 4];
        };
        float4 red[16][kPT][kPT / 4];
    };
    float ssw[2][16];
};

template <bool QKV>
__global__ __launch_bounds__(1024) void proj16_kernel(AttnArgs a) {
    __shared__ Proj16Smem sm;
    const int M = QKV ? a.d : a.qd, N = QKV ? a.qd + 2 * a.kd : a.d;
    const float *X = QKV ? a.x : a.o;
    const int r0 = blockIdx.y * kPT, c0 = blockIdx.x * kPT;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    // Epilogue threads (tid < 64: row tid / 4, columns 4 (tid % 4) ..) fetch
    // what they need besides the products up front.
    const int orow = r0 + (tid >> 2), ocol = c0 + 4 * (tid & 3);
    const bool owned = tid < 64 && orow < a.B && ocol < N;
    const int p = owned ? a.pos[orow] : -1;
    const bool live = owned && p >= 0 && p < a.max_seq;
    const int col = ocol < a.qd ? ocol : ocol < a.qd + a.kd ? ocol - a.qd : ocol - a.qd - a.kd;
    const bool rope = QKV && live && ocol < a.qd + a.kd;
    float4 cs = zero, xo = zero;
    if (rope) {
        const int half = a.hd / 2, i0 = (col % a.hd) / 2;
        const float *cr = a.cos_t + (size_t)p * half + i0, *sr = a.sin_t + (size_t)p * half + i0;
        cs = make_float4(cr[0], sr[0], cr[1], sr[1]);
    }
    if (!QKV && live) xo = *reinterpret_cast<const float4 *>(a.x + (size_t)orow * a.d + ocol);

    const int rr = lane >> 2, cq = lane & 3;
    const int xq = tid % (kPK / 4), xr0 = tid / (kPK / 4);   // X float4 and first row
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float ss[2] = {0.0f, 0.0f};
    for (int k0 = 0; k0 < M; k0 += kPK) {
        const int k = k0 + 4 * xq;
        float4 xv[2], wv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = r0 + xr0 + 8 * i;
            xv[i] = row < a.B && k < M ? *reinterpret_cast<const float4 *>(X + (size_t)row * M + k)
                                       : zero;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 1024 * i, kk = k0 + idx / (kPT / 4), cc = c0 + 4 * (idx % (kPT / 4));
            const float *src = nullptr;
            const float *wp = QKV ? a.wqkv_p : a.wo_p;
            if (kk < M && cc < N) {
                if (wp)                      src = wp + ((size_t)(cc >> 4) * M + kk) * 16 + (cc & 15);
                else if (!QKV)               src = a.wo + (size_t)kk * a.d + cc;
                else if (cc < a.qd)          src = a.wq + (size_t)kk * a.qd + cc;
                else if (cc < a.qd + a.kd)   src = a.wk + (size_t)kk * a.kd + (cc - a.qd);
                else                         src = a.wv + (size_t)kk * a.kd + (cc - a.qd - a.kd);
            }
            wv[i] = src ? *reinterpret_cast<const float4 *>(src) : zero;
        }
        float4 wr = zero;
        if (QKV && k < M) wr = *reinterpret_cast<const float4 *>(a.rms_w + k);
        if (k0 > 0) __syncthreads();   // the previous chunk's products are done
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float4 v = xv[i];
            if (QKV) {
                ss[i] = fmaf(v.x, v.x, ss[i]); ss[i] = fmaf(v.y, v.y, ss[i]);
                ss[i] = fmaf(v.z, v.z, ss[i]); ss[i] = fmaf(v.w, v.w, ss[i]);
                v = make_float4(v.x * wr.x, v.y * wr.y, v.z * wr.z, v.w * wr.w);
            }
            sm.xs[xr0 + 8 * i][xq] = v;
            const int idx = tid + 1024 * i;
            sm.ws[idx / (kPT / 4)][idx % (kPT / 4)] = wv[i];
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int kq = wave * 8 + s;
            const float4 xa = sm.xs[rr][kq];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 wb = sm.ws[4 * kq + j][cq];
                const float xj = comp(xa, j);
                acc[0] = fmaf(xj, wb.x, acc[0]);
                acc[1] = fmaf(xj, wb.y, acc[1]);
                acc[2] = fmaf(xj, wb.z, acc[2]);
                acc[3] = fmaf(xj, wb.w, acc[3]);
            }
        }
    }
    if (QKV) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            for (int off = 32; off >= 1; off >>= 1) ss[i] += __shfl_xor(ss[i], off);
        if (lane == 0) {
            sm.ssw[0][wave] = ss[0];   // row wave / 2
            sm.ssw[1][wave] = ss[1];   // row 8 + wave / 2
        }
    }
    __syncthreads();   // (red overlays xs and ws)
    sm.red[wave][rr][cq] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    __syncthreads();
    if (!live) return;
    float4 y = zero;
    for (int w = 0; w < 16; ++w) y = add4(y, sm.red[w][tid >> 2][tid & 3]);
    if (!QKV) {
        *reinterpret_cast<float4 *>(a.x + (size_t)orow * a.d + ocol) = add4(xo, y);
        return;
    }
    const int r = tid >> 2, h = r >> 3, rw = 2 * (r & 7);
    const float sq = sm.ssw[h][rw] + sm.ssw[h][rw + 1];
    const float inv = 1.0f / sqrtf(sq / (float)M + a.eps);
    y = make_float4(y.x * inv, y.y * inv, y.z * inv, y.w * inv);
    if (rope) {
        rope_pair(y.x, y.y, cs.x, cs.y);
        rope_pair(y.z, y.w, cs.z, cs.w);
    }
    float *dst = ocol < a.qd ? a.q + (size_t)orow * a.qd
                             : (ocol < a.qd + a.kd ? a.kc : a.vc) +
                                   ((size_t)orow * a.max_seq + p) * a.kd;
    *reinterpret_cast<float4 *>(dst + col) = y;
}

// Merged output of one head at dimension dim from its chunk partials at
// float index ph + c * (hd + 2) = (m_c, l_c, o_c[hd]), c < nc:
// o = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c with M = max_c m_c,
// taken eight chunks at a time (online: the running sums are rescaled when
// the maximum grows).  Loads past nc read chunk 0 and are masked, so every
// batch's loads are in flight together.
template <class RD>
__device__ inline float merge_head(const RD &rd, size_t ph, int nc, int hd, int dim) {
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += 8) {
        float m[8], l[8], o[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const size_t pc = ph + (size_t)(c0 + u < nc ? c0 + u : 0) * (hd + 2);
            m[u] = rd(pc);
            l[u] = rd(pc + 1);
            o[u] = rd(pc + 2 + dim);
        }
        float Mn = M;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (c0 + u < nc) Mn = fmaxf(Mn, m[u]);
        const float f0 = expf(M - Mn);
        L *= f0;
        O *= f0;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (c0 + u < nc) {
                const float f = expf(m[u] - Mn);
                L = fmaf(f, l[u], L);
                O = fmaf(f, o[u], O);
            }
        M = Mn;
    }
    return O / L;
}

// ---------------------------------------------------------------------------
// Attention chunks.

// Lane pairing of reduce-scatter step `bit` within groups of 16 lanes: the
// partner of a lane has the other value of that lane-index bit.
template <int BIT> __device__ inline float dpp_partner(float v) {
    constexpr int ctrl = BIT == 8 ? 0x140      // row_mirror: i <-> 15 - i
                       : BIT == 4 ? 0x141      // row_half_mirror: i <-> 7 - i (in 8)
                       : BIT == 2 ? 0x1B       // quad_perm [3,2,1,0]
                                  : 0xB1;      // quad_perm [1,0,3,2]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true));
}

// Reduce-scatter of CNT values over groups of L lanes: afterwards lane r of
// a group holds, in v[0 .. CNT/L), the group sums of values r*CNT/L onward.
template <int L, int CNT> __device__ inline void reduce_scatter(float (&v)[CNT], int lane) {
    if constexpr (L > 1) {
        constexpr int H = CNT / 2;
        const bool up = lane & (L / 2);
#pragma unroll
        for (int k = 0; k < H; ++k) {
            const float send = up ? v[k] : v[k + H];
            const float keep = up ? v[k + H] : v[k];
            v[k] = keep + dpp_partner<L / 2>(send);
        }
        float w[H];
#pragma unroll
        for (int k = 0; k < H; ++k) w[k] = v[k];
        reduce_scatter<L / 2, H>(w, lane);
#pragma unroll
        for (int k = 0; k < H; ++k) v[k] = w[k];
    }
}

template <int HD, int G> struct ChunkSmem {
    static constexpr int L = HD / 4, R = 256 / L;
    float sc[G][kChunkPos];
    float4 red[R][G][L];
    int flag;
};

// Chunk c of (sequence b, kv head kvh) for head_dim HD and G query heads
// per kv head: rows j0 + row, row < n = min(128, pos + 1 - j0), of K and V
// are loaded at once as float4s (thread: column quad t % L, rows i * R +
// t / L, L = HD / 4 lanes per row, R = 256 / L rows per load).  Scores:
// per-thread partial dot products of the four columns, summed over the
// row's L lanes by reduce_scatter, times 1/sqrt(hd).  One wave per head
// takes the chunk maximum m, p = exp(s - m) and l = sum p; the V sum uses
// the V registers, then LDS across the R row groups.  The partial (m, l,
// o[HD]) goes out coherently; the last of the pos / 128 + 1 chunks with
// positions merges them into o.  FUSED: q and the row at pos come from the
// QKV tiles of the same launch (waited for, read coherently); the merge is
// counted, and a sequence without a valid position counts once (chunk 0).
template <int HD, int G, bool FUSED>
__device__ void chunk(const AttnArgs &a, int bid, ChunkSmem<HD, G> &sm) {
    constexpr int L = HD / 4, R = 256 / L, NI = kChunkPos / R, CNT = NI * G, PER = CNT / L;
    static_assert(PER >= 1 && CNT % L == 0, "chunk layout");
    const int nchunk = (a.max_seq + kChunkPos - 1) / kChunkPos;
    // Chunk index slowest: the first workgroups to run hold full chunks,
    // the (often short) last chunks of the sequences come at the end.
    const int pairs = a.B * a.nkv;
    const int c = bid / pairs;
    const int kvh = bid % a.nkv;
    const int b = (bid % pairs) / a.nkv;
    const int pb = a.pos[b];
    const int p = pb >= 0 && pb < a.max_seq ? pb : -1;   // (out of range: attends nothing)
    const int j0 = c * kChunkPos, n = min(kChunkPos, p + 1 - j0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cq = tid % L, rg = tid / L;
    if (n <= 0) {   // past the sequence (the merge reads chunks 0 .. pos / 128)
        if (FUSED && p < 0 && c == 0) signal(a.sync + 1, a.B * a.nkv, a.sync + kSyncMergeFlags);
        return;
    }
    float *part = a.part + ((size_t)(b * a.nh + kvh * G) * nchunk + c) * (HD + 2);
    const size_t head_stride = (size_t)nchunk * (HD + 2);
    const int prow = FUSED ? p - j0 : -1;   // the new row (in this chunk if < 128)
    const size_t base = ((size_t)b * a.max_seq + j0) * a.kd + kvh * HD + 4 * cq;
    float4 kv[NI], vv[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = i * R + rg;
        const bool in = row < n && row != prow;
        const size_t off = base + (size_t)(in ? row : 0) * a.kd;
        kv[i] = in ? *reinterpret_cast<const float4 *>(a.kc + off) : make_float4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = i * R + rg;
        const bool in = row < n && row != prow;
        const size_t off = base + (size_t)(in ? row : 0) * a.kd;
        vv[i] = in ? *reinterpret_cast<const float4 *>(a.vc + off) : make_float4(0, 0, 0, 0);
    }
    float4 q[G];
    if (FUSED) {
        wait_flag(a.sync + kSyncQkvFlags, a.err);   // q and the new k, v rows are out
        const CRead qr(a.q + (size_t)b * a.qd + kvh * G * HD);
#pragma unroll
        for (int h = 0; h < G; ++h) q[h] = qr.f4(h * HD + 4 * cq);
        if (prow < kChunkPos) {
            const size_t rowoff = ((size_t)b * a.max_seq + p) * a.kd + kvh * HD;
            const CRead kr(a.kc + rowoff), vr(a.vc + rowoff);
#pragma unroll
            for (int i = 0; i < NI; ++i)
                if (i * R + rg == prow) {
                    kv[i] = kr.f4(4 * cq);
                    vv[i] = vr.f4(4 * cq);
                }
        }
    } else {
#pragma unroll
        for (int h = 0; h < G; ++h)
            q[h] = *reinterpret_cast<const float4 *>(a.q + (size_t)b * a.qd + (kvh * G + h) * HD +
                                                     4 * cq);
    }
    float v[CNT];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float s = q[h].x * kv[i].x;
            s = fmaf(q[h].y, kv[i].y, s);
            s = fmaf(q[h].z, kv[i].z, s);
            v[i * G + h] = fmaf(q[h].w, kv[i].w, s);
        }
    reduce_scatter<L, CNT>(v, lane);
    const int r = lane % L;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int idx = r * PER + k, i = idx / G, h = idx % G;
        sm.sc[h][i * R + rg] = v[k] * a.scale;
    }
    __syncthreads();
    for (int h = wave; h < G; h += 4) {
        float m = -INFINITY;
        for (int t = lane; t < n; t += 64) m = fmaxf(m, sm.sc[h][t]);
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float l = 0.0f;
        for (int t = lane; t < kChunkPos; t += 64) {
            const float e = t < n ? expf(sm.sc[h][t] - m) : 0.0f;
            sm.sc[h][t] = e;
            l += e;
        }
        for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) {
            cstore(part + h * head_stride, m);
            cstore(part + h * head_stride + 1, l);
        }
    }
    __syncthreads();
    float4 o[G];
#pragma unroll
    for (int h = 0; h < G; ++h) o[h] = make_float4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = i * R + rg;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float e = sm.sc[h][row];
            o[h].x = fmaf(e, vv[i].x, o[h].x);
            o[h].y = fmaf(e, vv[i].y, o[h].y);
            o[h].z = fmaf(e, vv[i].z, o[h].z);
            o[h].w = fmaf(e, vv[i].w, o[h].w);
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) sm.red[rg][h][cq] = o[h];
    __syncthreads();
    for (int t = tid; t < G * HD; t += 256) {
        const int h = t / HD, dim = t % HD;
        const float *rp = reinterpret_cast<const float *>(&sm.red[0][h][0]) + dim;
        float acc = 0.0f;
        for (int g = 0; g < R; ++g) acc += rp[(size_t)g * G * HD];
        cstore(part + h * head_stride + 2 + dim, acc);
    }
    // The chunks holding positions 0 .. pos number pos / 128 + 1; the last
    // of them to finish merges the partials of this kv head's query heads.
    const int nc = p / kChunkPos + 1;
    if (!arrive_last(a.cnt_merge + b * a.nkv + kvh, nc, &sm.flag)) return;
    const size_t ph0 = (size_t)(b * a.nh + kvh * G) * nchunk * (HD + 2);
    const CRead rd(a.part + ph0);
    float *ob = a.o + (size_t)b * a.qd + kvh * G * HD;
    for (int t = tid; t < G * HD; t += 256) {
        const float ov = merge_head(rd, (size_t)(t / HD) * head_stride, nc, HD, t % HD);
        if (FUSED) cstore(ob + t, ov);
        else       ob[t] = ov;
    }
    if (FUSED) signal(a.sync + 1, a.B * a.nkv, a.sync + kSyncMergeFlags);
}

// ---------------------------------------------------------------------------
// Kernels.

// The whole sublayer in one launch: workgroups [0, nq) QKV tiles, [nq,
// nq + nc) chunks, the rest W_O tiles.  The last workgroup to exit resets
// the launch's counters.
template <int HD, int G>
__global__ __launch_bounds__(256) void attn_fused_kernel(AttnArgs a, int nq, int nc) {
    __shared__ union Smem {
        ProjSmem p;
        ChunkSmem<HD, G> c;
    } sm;
    const int bid = blockIdx.x;
    if (bid < nq) {
        const int S = slices(a.d), ntx = tiles(a.qd + 2 * a.kd), t = bid / S;
        proj_tile<true, true>(a, t % ntx, t / ntx, bid % S, ntx, S, sm.p);
    } else if (bid < nq + nc) {
        chunk<HD, G, true>(a, bid - nq, sm.c);
    } else {
        const int r = bid - nq - nc, S = slices(a.qd), ntx = tiles(a.d), t = r / S;
        proj_tile<false, true>(a, t % ntx, t / ntx, r % S, ntx, S, sm.p);
    }
    __syncthreads();
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(a.sync + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            (int)gridDim.x - 1) {
        for (int i = 0; i < 3; ++i)
            __hip_atomic_store(a.sync + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int i = 0; i < kFlagCopies; ++i) {
            __hip_atomic_store(a.sync + kSyncQkvFlags + i * kFlagStride, 0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.sync + kSyncMergeFlags + i * kFlagStride, 0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <bool QKV>
__global__ __launch_bounds__(256) void proj_tile_kernel(AttnArgs a) {
    __shared__ ProjSmem sm;
    proj_tile<QKV, false>(a, blockIdx.x, blockIdx.y, blockIdx.z, gridDim.x, gridDim.z, sm);
}

template <int HD, int G>
__global__ __launch_bounds__(256) void attn_chunk_fast_kernel(AttnArgs a) {
    __shared__ ChunkSmem<HD, G> sm;
    chunk<HD, G, false>(a, blockIdx.x, sm);
}

// Generic head shapes.  Workgroup (b, kv head, chunk c): positions j in
// [128c, min(128c + 128, pos + 1)).  Phase 1, lane = position: the scores of the kv head's gqa
// query heads in vec_dot's order.  Phase 2: per head the chunk maximum m,
// p_j = exp(s_j - m), l = sum p_j.  Phase 3, lane = dimension, wave = head
// (heads past 4 in turns): o = sum_j p_j V[j] as FMAs in position order.
// The partial (m, l, o[hd]) goes to part[(b, head, c)].
__global__ __launch_bounds__(256) void attn_chunk_kernel(AttnArgs a) {
    __shared__ float q_s[8][64];          // gqa <= 8 heads, hd <= 64
    __shared__ float sc[8][kChunkPos];
    __shared__ float red[8][4];
    const int nchunk = (a.max_seq + kChunkPos - 1) / kChunkPos;
    const int pairs = a.B * a.nkv;
    const int c = blockIdx.x / pairs;
    const int kvh = blockIdx.x % a.nkv;
    const int b = (blockIdx.x % pairs) / a.nkv;
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

// Generic path: one thread per (b, head, dimension) merges the chunks.
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a) {
    const int nchunk = (a.max_seq + kChunkPos - 1) / kChunkPos;
    const int gid = blockIdx.x * 256 + threadIdx.x;
    if (gid >= a.B * a.qd) return;
    const int b = gid / a.qd, h = (gid % a.qd) / a.hd, t = gid % a.hd;
    const int p = a.pos[b];
    if (p < 0 || p >= a.max_seq) return;   // (the row is left out downstream)
    a.o[gid] = merge_head(PRead(a.part), (size_t)(b * a.nh + h) * nchunk * (a.hd + 2),
                          p / kChunkPos + 1, a.hd, t);
}

// Head shapes with a fast chunk kernel (and the one-launch sublayer).
template <class F> bool with_fast_shape(int hd, int g, F &&f) {
#define MOE_ATTN_SHAPE(HD_, G_)                                     \
    if (hd == HD_ && g == G_) {                                     \
        f(std::integral_constant<int, HD_>{}, std::integral_constant<int, G_>{}); \
        return true;                                                \
    }
    MOE_ATTN_SHAPE(64, 2) MOE_ATTN_SHAPE(64, 4) MOE_ATTN_SHAPE(64, 8)
    MOE_ATTN_SHAPE(32, 2) MOE_ATTN_SHAPE(32, 4) MOE_ATTN_SHAPE(32, 8)
    MOE_ATTN_SHAPE(16, 2) MOE_ATTN_SHAPE(16, 4) MOE_ATTN_SHAPE(16, 8)
#undef MOE_ATTN_SHAPE
    return false;
}

}  // namespace

size_t attn_part_floats(int B, int nh, int hd, int max_seq) {
    return (size_t)B * nh * ((max_seq + kChunkPos - 1) / kChunkPos) * (hd + 2);
}

size_t attn_gpart_floats(int B, int d, int qd, int kd) {
    const size_t qkv = (size_t)slices(d) * (qd + 2 * kd), wo = (size_t)slices(qd) * d;
    return (size_t)B * (qkv > wo ? qkv : wo);
}

size_t attn_sspart_floats(int B, int d) { return (size_t)slices(d) * B; }

int attn_sync_ints() { return kSyncMergeFlags + kFlagCopies * kFlagStride; }

AttnCounters attn_counters(int B, int d, int qd, int kd, int nkv) {
    AttnCounters c;
    c.qkv = tiles(qd + 2 * kd) * tiles(B);
    c.wo = tiles(d) * tiles(B);
    c.merge = B * nkv;
    return c;
}

bool attn_fused_supported(int hd, int nh, int nkv) {
    return nkv > 0 && nh % nkv == 0 && with_fast_shape(hd, nh / nkv, [](auto, auto) {});
}

namespace {
__global__ __launch_bounds__(256) void pack_cols16_kernel(const float *src, float *dst, int K,
                                                          int N, int col0) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;   // float4 of dst
    if (i >= (size_t)K * N / 4) return;
    const int t = (int)(i / ((size_t)K * 4)), rem = (int)(i % ((size_t)K * 4));
    const int k = rem >> 2, c = 16 * t + 4 * (rem & 3);
    *reinterpret_cast<float4 *>(dst + ((size_t)(col0 / 16 + t) * K + k) * 16 + 4 * (rem & 3)) =
        *reinterpret_cast<const float4 *>(src + (size_t)k * N + c);
}
}  // namespace

hipError_t launch_pack_cols16(const float *src, float *dst, int K, int N, int col0,
                              hipStream_t s) {
    if (K <= 0 || N <= 0 || N % 16 || col0 % 16) return hipErrorInvalidValue;
    const size_t n4 = (size_t)K * N / 4;
    hipLaunchKernelGGL(pack_cols16_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                       src, dst, K, N, col0);
    return hipGetLastError();
}

hipError_t launch_attn_decode(const AttnArgs &a, bool fused, hipStream_t s) {
    if (a.B <= 0) return hipSuccess;
    const int gqa = a.nh / a.nkv;
    if (a.hd > 64 || a.hd % 8 || gqa > 8 || a.nh % a.nkv || a.d % 4 || a.qd % 4)
        return hipErrorInvalidValue;
    const int N = a.qd + 2 * a.kd;
    const int nchunk = (a.max_seq + kChunkPos - 1) / kChunkPos;
    const int nc = a.B * a.nkv * nchunk;
    if (fused) {
        if (!a.sync || !a.err || a.nqkv_tiles != tiles(N) * tiles(a.B)) return hipErrorInvalidValue;
        const int nq = tiles(N) * tiles(a.B) * slices(a.d);
        const int no = tiles(a.d) * tiles(a.B) * slices(a.qd);
        const bool ok = with_fast_shape(a.hd, gqa, [&](auto hd, auto g) {
            hipLaunchKernelGGL((attn_fused_kernel<decltype(hd)::value, decltype(g)::value>),
                               dim3((unsigned)(nq + nc + no)), dim3(256), 0, s, a, nq, nc);
        });
        if (!ok) return hipErrorInvalidValue;
        return hipGetLastError();
    }
    auto t16 = [](int n) { return (unsigned)((n + kPT - 1) / kPT); };
    hipLaunchKernelGGL(proj16_kernel<true>, dim3(t16(N), t16(a.B)), dim3(1024), 0, s, a);
    const bool fast = with_fast_shape(a.hd, gqa, [&](auto hd, auto g) {
        hipLaunchKernelGGL((attn_chunk_fast_kernel<decltype(hd)::value, decltype(g)::value>),
                           dim3((unsigned)nc), dim3(256), 0, s, a);
    });
    if (!fast) {
        hipLaunchKernelGGL(attn_chunk_kernel, dim3((unsigned)nc), dim3(256), 0, s, a);
        hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)((a.B * a.qd + 255) / 256)),
                           dim3(256), 0, s, a);
    }
    hipLaunchKernelGGL(proj16_kernel<false>, dim3(t16(a.d), t16(a.B)), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace moe
