// attention.hip — the attention half of the KV-cache decode step
// (src/inference.c:252-308) for B sequences at once, each at its own
// position, on gfx950:  x += W_O . Attn(RoPE(W_Q xn), RoPE(W_K xn), W_V xn)
// with xn = rms_norm(x) and the new k, v rows appended to the caches.
//
// Three launches:
//   QKV tiles     q, k, v = rms_norm(x) . [W_Q | W_K | W_V]: one 1024-thread
//                 workgroup per 16 x 16 output tile with the whole reduction
//                 (proj16_kernel; batches of at most 4 rows: one workgroup
//                 per output column quad, projv_kernel).  rms_norm's row scale 1/rms (:48-60) is
//                 taken out of the reduction: tiles multiply x * w_rms, sum
//                 x^2 on the side, scale by 1/sqrt(ss/d + eps), apply RoPE at
//                 the sequence's position from the caller's tables (:187-203)
//                 to q and k, and write q and the cache rows at pos.
//   chunks        one workgroup per (sequence, kv head, 128 positions)
//                 streams that K and V once for the kv head's query heads:
//                 scores times 1/sqrt(hd), exp against the chunk maximum,
//                 the V sum; the last chunk of a (sequence, kv head) merges
//                 the chunk partials (m, l, o) into o.  Bound by the K/V
//                 reads.
//   W_O tiles     x += o . W_O with the same tiles (the element add of :306).
// The chunks hand their partials to the merging chunk through device-scope
// coherent stores and a counter (the last to arrive merges; nothing waits).
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

// RoPE on the pair (v0, v1) = columns 2i, 2i + 1 of a head (:196-199).
__device__ inline void rope_pair(float &v0, float &v1, float c, float s) {
    const float a = v0, b = v1;
    v0 = a * c - b * s;
    v1 = a * s + b * c;
}

// Wave-wide max and sum through DPP instead of LDS permutes: four row_shr
// steps (lanes without a source take the identity) leave each 16-lane row's
// total in its lane 15; lanes 15, 31, 47 and 63 are then combined as
// (r0 op r1) op (r2 op r3), the same value in every lane.
template <int N> __device__ inline float shr_fill(float v, float fill) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v),
                                                      0x110 + N, 0xF, 0xF, false));
}
__device__ inline float lane_of(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ inline float wave_max(float v) {
    v = fmaxf(v, shr_fill<1>(v, -INFINITY));
    v = fmaxf(v, shr_fill<2>(v, -INFINITY));
    v = fmaxf(v, shr_fill<4>(v, -INFINITY));
    v = fmaxf(v, shr_fill<8>(v, -INFINITY));
    return fmaxf(fmaxf(lane_of(v, 15), lane_of(v, 31)), fmaxf(lane_of(v, 47), lane_of(v, 63)));
}
__device__ inline float wave_sum(float v) {
    v = v + shr_fill<1>(v, 0.0f);
    v = v + shr_fill<2>(v, 0.0f);
    v = v + shr_fill<4>(v, 0.0f);
    v = v + shr_fill<8>(v, 0.0f);
    return (lane_of(v, 15) + lane_of(v, 31)) + (lane_of(v, 47) + lane_of(v, 63));
}

__device__ inline float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ inline float comp(const float4 &v, int j) {
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
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
// ---------------------------------------------------------------------------
// Projection tiles without a split reduction: one 1024-thread workgroup per
// 16 x 16 output tile (tile column blockIdx.x, row blockIdx.y).  The X rows
// and W columns of a 512-long reduction chunk are staged in LDS: thread t
// loads float4 t % 128 of X rows t / 128 and 8 + t / 128, and float4s t and
// t + 1024 of the W block.  Wave w takes chunk rows 32w .. 32w + 31, lane
// (rr, cq) = (lane / 4, lane % 4) row rr and columns 4cq .. 4cq + 3; the
// sixteen waves' sums are added through LDS in wave order.  QKV: row r's
// sum of x^2 is each thread's k-ordered share, summed over its wave and
// then over the row's two waves; the epilogue scales by 1/rms, applies RoPE
// at the sequence's position to q and k and writes q and the cache rows at
// pos.  WO: x += the products.  One global round trip.
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
        // Every load reads a valid address (out-of-range elements read the
        // tile's first element) and is masked after: a select between the
        // load and a constant keeps all of them in flight together.
        float4 xv[2], wv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = r0 + xr0 + 8 * i;
            const bool in = row < a.B && k < M;
            xv[i] = masked4(in, *reinterpret_cast<const float4 *>(X + (in ? (size_t)row * M + k : 0)));
        }
        const float *wp = QKV ? a.wqkv_p : a.wo_p;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 1024 * i, kk = k0 + idx / (kPT / 4), cc = c0 + 4 * (idx % (kPT / 4));
            const bool in = kk < M && cc < N;
            const int kr = in ? kk : 0, cr = in ? cc : 0;
            const float *src;
            if (wp)                      src = wp + ((size_t)(cr >> 4) * M + kr) * 16 + (cr & 15);
            else if (!QKV)               src = a.wo + (size_t)kr * a.d + cr;
            else if (cr < a.qd)          src = a.wq + (size_t)kr * a.qd + cr;
            else if (cr < a.qd + a.kd)   src = a.wk + (size_t)kr * a.kd + (cr - a.qd);
            else                         src = a.wv + (size_t)kr * a.kd + (cr - a.qd - a.kd);
            wv[i] = masked4(in, *reinterpret_cast<const float4 *>(src));
        }
        float4 wr = zero;
        if (QKV) wr = masked4(k < M, *reinterpret_cast<const float4 *>(a.rms_w + (k < M ? k : 0)));
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
        for (int i = 0; i < 2; ++i) ss[i] = wave_sum(ss[i]);
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

// Projections of small batches (B <= kPVRows rows): one 256-thread
// workgroup per output column quad c0 .. c0 + 3 (N / 4 workgroups, where the
// 16 x 16 tiles would give N / 16 with 15 of 16 rows idle).  Thread t takes
// k = t, t + 256, ... of the reduction for every row, all its loads issued
// before the first product; the rows' sums (and QKV's sums of x^2) are added
// over each wave by DPP and over the four waves through LDS in wave order.
// Thread b < B then runs proj16's epilogue for row b.
constexpr int kPVRows = 4;
template <bool QKV>
__global__ __launch_bounds__(256) void projv_kernel(AttnArgs a) {
    constexpr int R = kPVRows, KU = 4;   // rows, k steps per thread per batch of loads
    const int M = QKV ? a.d : a.qd, N = QKV ? a.qd + 2 * a.kd : a.d;
    const float *X = QKV ? a.x : a.o;
    const float *wp = QKV ? a.wqkv_p : a.wo_p;
    const int c0 = 4 * blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int B = a.B;
    __shared__ float4 red[4][R];
    __shared__ float ssr[4][R];
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 acc[R];
    float ss[R];
#pragma unroll
    for (int b = 0; b < R; ++b) { acc[b] = zero; ss[b] = 0.0f; }
    for (int k0 = 0; k0 < M; k0 += 256 * KU) {
        float4 wv[KU];
        float xv[KU][R], wr[KU];
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int k = k0 + tid + 256 * u;
            const bool in = k < M;
            const int kr = in ? k : 0;
            const float *src;
            if (wp)                      src = wp + ((size_t)(c0 >> 4) * M + kr) * 16 + (c0 & 15);
            else if (!QKV)               src = a.wo + (size_t)kr * a.d + c0;
            else if (c0 < a.qd)          src = a.wq + (size_t)kr * a.qd + c0;
            else if (c0 < a.qd + a.kd)   src = a.wk + (size_t)kr * a.kd + (c0 - a.qd);
            else                         src = a.wv + (size_t)kr * a.kd + (c0 - a.qd - a.kd);
            wv[u] = masked4(in, *reinterpret_cast<const float4 *>(src));
#pragma unroll
            for (int b = 0; b < R; ++b) {
                const bool inb = in && b < B;
                const float v = X[inb ? (size_t)b * M + k : 0];
                xv[u][b] = inb ? v : 0.0f;
            }
            wr[u] = QKV ? (in ? a.rms_w[kr] : 0.0f) : 1.0f;
        }
#pragma unroll
        for (int u = 0; u < KU; ++u)
#pragma unroll
            for (int b = 0; b < R; ++b) {
                const float v = xv[u][b];
                float xw = v;
                if (QKV) {
                    ss[b] = fmaf(v, v, ss[b]);
                    xw = v * wr[u];
                }
                acc[b].x = fmaf(xw, wv[u].x, acc[b].x);
                acc[b].y = fmaf(xw, wv[u].y, acc[b].y);
                acc[b].z = fmaf(xw, wv[u].z, acc[b].z);
                acc[b].w = fmaf(xw, wv[u].w, acc[b].w);
            }
    }
#pragma unroll
    for (int b = 0; b < R; ++b) {
        if (b >= B) break;
        const float4 t = make_float4(wave_sum(acc[b].x), wave_sum(acc[b].y), wave_sum(acc[b].z),
                                     wave_sum(acc[b].w));
        const float q = QKV ? wave_sum(ss[b]) : 0.0f;
        if (lane == 0) {
            red[wave][b] = t;
            ssr[wave][b] = q;
        }
    }
    __syncthreads();
    if (tid >= B) return;
    const int b = tid;
    const int p = a.pos[b];
    if (p < 0 || p >= a.max_seq) return;   // (out of range: left untouched)
    float4 y = zero;
    for (int w = 0; w < 4; ++w) y = add4(y, red[w][b]);
    if (!QKV) {
        float4 *xo = reinterpret_cast<float4 *>(a.x + (size_t)b * a.d + c0);
        *xo = add4(*xo, y);
        return;
    }
    const float sq = (ssr[0][b] + ssr[1][b]) + (ssr[2][b] + ssr[3][b]);
    const float inv = 1.0f / sqrtf(sq / (float)M + a.eps);
    y = make_float4(y.x * inv, y.y * inv, y.z * inv, y.w * inv);
    const int col = c0 < a.qd ? c0 : c0 < a.qd + a.kd ? c0 - a.qd : c0 - a.qd - a.kd;
    if (c0 < a.qd + a.kd) {
        const int half = a.hd / 2, i0 = (col % a.hd) / 2;
        const float *cr = a.cos_t + (size_t)p * half + i0, *sr = a.sin_t + (size_t)p * half + i0;
        rope_pair(y.x, y.y, cr[0], sr[0]);
        rope_pair(y.z, y.w, cr[1], sr[1]);
    }
    float *dst = c0 < a.qd ? a.q + (size_t)b * a.qd
                           : (c0 < a.qd + a.kd ? a.kc : a.vc) + ((size_t)b * a.max_seq + p) * a.kd;
    *reinterpret_cast<float4 *>(dst + col) = y;
    (void)N;
}

// Merged output of one head at dimension dim from its chunk partials at
// float index ph + c * (hd + 2) = (m_c, l_c, o_c[hd]), c < nc:
// o = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c with M = max_c m_c,
// taken sixteen chunks at a time (online: the running sums are rescaled when
// the maximum grows), so contexts up to 2048 positions merge in one round
// trip (eight at a time: 0.25-0.3 us more per block at context 1024).  Loads
// past nc read chunk 0 and are masked, so every batch's loads are in flight
// together.
template <class RD>
__device__ inline float merge_head(const RD &rd, size_t ph, int nc, int hd, int dim) {
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += 16) {
        float m[16], l[16], o[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const size_t pc = ph + (size_t)(c0 + u < nc ? c0 + u : 0) * (hd + 2);
            m[u] = rd(pc);
            l[u] = rd(pc + 1);
            o[u] = rd(pc + 2 + dim);
        }
        float Mn = M;
#pragma unroll
        for (int u = 0; u < 16; ++u)
            if (c0 + u < nc) Mn = fmaxf(Mn, m[u]);
        const float f0 = expf(M - Mn);
        L *= f0;
        O *= f0;
#pragma unroll
        for (int u = 0; u < 16; ++u)
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

// K and V rows are read once per step: non-temporal (streaming) loads
// (the 64-sequence, 1025-position block: 32.5 -> 29.8 us per attention
// sublayer against default loads).
__device__ inline float4 ld_stream4(const float *p) {
    typedef float fx4 __attribute__((ext_vector_type(4)));
    const fx4 v = __builtin_nontemporal_load(reinterpret_cast<const fx4 *>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
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
// positions merges them into o.
template <int HD, int G>
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
    if (n <= 0) return;   // past the sequence (the merge reads chunks 0 .. pos / 128)
    float *part = a.part + ((size_t)(b * a.nh + kvh * G) * nchunk + c) * (HD + 2);
    const size_t head_stride = (size_t)nchunk * (HD + 2);
    const size_t base = ((size_t)b * a.max_seq + j0) * a.kd + kvh * HD + 4 * cq;
    // q, then the K rows, then the V rows, all issued before anything waits
    // (the scheduling barrier keeps the compiler from sinking the V loads
    // below the scores, which would cost a second memory round trip).
    float4 q[G];
#pragma unroll
    for (int h = 0; h < G; ++h)
        q[h] = *reinterpret_cast<const float4 *>(a.q + (size_t)b * a.qd + (kvh * G + h) * HD +
                                                 4 * cq);
    float4 kv[NI], vv[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = i * R + rg;
        const bool in = row < n;
        const size_t off = base + (size_t)(in ? row : 0) * a.kd;
        kv[i] = masked4(in, ld_stream4(a.kc + off));
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = i * R + rg;
        const bool in = row < n;
        const size_t off = base + (size_t)(in ? row : 0) * a.kd;
        vv[i] = masked4(in, ld_stream4(a.vc + off));
    }
    __builtin_amdgcn_sched_barrier(0);
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
        m = wave_max(m);
        float l = 0.0f;
        for (int t = lane; t < kChunkPos; t += 64) {
            const float e = t < n ? expf(sm.sc[h][t] - m) : 0.0f;
            sm.sc[h][t] = e;
            l += e;
        }
        l = wave_sum(l);
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
        ob[t] = merge_head(rd, (size_t)(t / HD) * head_stride, nc, HD, t % HD);
    }
}

// ---------------------------------------------------------------------------
// Kernels.

template <int HD, int G>
__global__ __launch_bounds__(256) void attn_chunk_fast_kernel(AttnArgs a) {
    __shared__ ChunkSmem<HD, G> sm;
    chunk<HD, G>(a, blockIdx.x, sm);
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
        m = wave_max(m);
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
        l = wave_sum(l);
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

// Head shapes with a fast chunk kernel.
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

hipError_t launch_attn_decode(const AttnArgs &a, hipStream_t s) {
    if (a.B <= 0) return hipSuccess;
    const int gqa = a.nh / a.nkv;
    if (a.hd > 64 || a.hd % 8 || gqa > 8 || a.nh % a.nkv || a.d % 4 || a.qd % 4)
        return hipErrorInvalidValue;
    const int N = a.qd + 2 * a.kd;
    const int nchunk = (a.max_seq + kChunkPos - 1) / kChunkPos;
    const int nc = a.B * a.nkv * nchunk;
    if (!a.cnt_merge) return hipErrorInvalidValue;
    auto t16 = [](int n) { return (unsigned)((n + kPT - 1) / kPT); };
    const bool small = a.B <= kPVRows;
    if (small) hipLaunchKernelGGL(projv_kernel<true>, dim3((unsigned)(N / 4)), dim3(256), 0, s, a);
    else       hipLaunchKernelGGL(proj16_kernel<true>, dim3(t16(N), t16(a.B)), dim3(1024), 0, s, a);
    const bool fast = with_fast_shape(a.hd, gqa, [&](auto hd, auto g) {
        hipLaunchKernelGGL((attn_chunk_fast_kernel<decltype(hd)::value, decltype(g)::value>),
                           dim3((unsigned)nc), dim3(256), 0, s, a);
    });
    if (!fast) {
        hipLaunchKernelGGL(attn_chunk_kernel, dim3((unsigned)nc), dim3(256), 0, s, a);
        hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)((a.B * a.qd + 255) / 256)),
                           dim3(256), 0, s, a);
    }
    if (small) hipLaunchKernelGGL(projv_kernel<false>, dim3((unsigned)(a.d / 4)), dim3(256), 0, s, a);
    else       hipLaunchKernelGGL(proj16_kernel<false>, dim3(t16(a.d), t16(a.B)), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace moe
