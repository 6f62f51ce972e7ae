// route.hip — router logits, softmax, top-k gating and the stable expert
// dispatch for gfx950.
//
// Bit-exactness contract (reference paths relative to the reference root):
//  * logits: one fused-multiply-add chain per (token, expert), k ascending
//    from +0.0f, skipping x == 0 — the AVX2+FMA mat_mul (src/matrix.c:381-400
//    with axpy_avx2fma :278-303).  Register-blocked VALU FMAs keep every
//    accumulator its own ascending chain, so blocking changes no bit.
//  * softmax: softmax_rows (src/matrix.c:529-586): 8-lane blocks through the
//    exp_avx2 polynomial (:82-116) with lane sums folded in hsum256 order
//    (include/simd.h:110-121), glibc expf on the E % 8 tail, 1/sum times each.
//  * top-k: src/transformer.c:317-337 (strict '>', best = -1, ties -> lowest
//    expert, renormalised gate weights).
//  * The reference executables run with FTZ/DAZ (-ffast-math startup code);
//    this file is built with fp32 denormal flushing and the explicit flushes
//    below mirror that.
//  * dispatch: stable counting sort of the (token, slot) assignments by expert
//    through per-wave LDS histograms, an exclusive scan and ballot ranks.
#include "moe_internal.h"
#include "moe_math.h"
#include "route_rows.h"

namespace moe {
namespace {

// Softmax of one row in place (src/matrix.c:529-586, AVX2+FMA build, with
// the tail division compiled as a multiply by 1/sum).
__device__ inline void softmax_row(float *row, int E) {
    int nb = E >> 3;
    float lane_max[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) lane_max[l] = -1e38f;
    for (int b = 0; b < nb; ++b)
#pragma unroll
        for (int l = 0; l < 8; ++l) lane_max[l] = fmaxf(lane_max[l], row[8 * b + l]);
    float mx = lane_max[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) mx = fmaxf(mx, lane_max[l]);
    for (int j = nb * 8; j < E; ++j) if (row[j] > mx) mx = row[j];

    float vs[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) vs[l] = 0.0f;
    for (int b = 0; b < nb; ++b)
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            float ex = exp_poly(row[8 * b + l] - mx);
            row[8 * b + l] = ex;
            vs[l] = vs[l] + ex;
        }
    float sum = ((vs[0] + vs[4]) + (vs[1] + vs[5])) + ((vs[2] + vs[6]) + (vs[3] + vs[7]));
    for (int j = nb * 8; j < E; ++j) {
        float ex = glibc_expf(row[j] - mx);
        row[j] = ex;
        sum = sum + ex;
    }
    float inv = 1.0f / sum;
    for (int j = 0; j < E; ++j) row[j] = ftz_f(row[j] * inv);
}

// ---------------------------------------------------------------------------
// Dispatch: one workgroup of 16 waves.  Wave w owns the contiguous run
// [w*chunk, (w+1)*chunk) of the flattened assignments a = t*k + slot.
//   pass 1: per-wave expert histograms in LDS;
//   scan:   counts, offsets (exclusive), per-(wave, expert) bases in
//           expert-major, wave-minor order;
//   pass 2: each wave walks its run in order; a lane's rank among earlier
//           lanes with the same expert comes from bit-sliced ballots.
// The result is the stable counting sort: pos(a) = offsets[e] + #{a' < a
// with the same expert}.
// ---------------------------------------------------------------------------
// Counting sort body run by the NW waves (64*NW threads) of one workgroup.
// hist: [NW][kMaxExperts] ints of LDS, offs: [kMaxExperts + 1].
template <int NW>
__device__ void dispatch_body(const DispatchArgs &a, int (*hist)[kMaxExperts], int *offs,
                              int *toff) {
    constexpr int NT = 64 * NW;
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int E = a.E, n = a.n;
    for (int x = lane; x < E; x += 64) hist[w][x] = 0;   // (the experts in use)
    __syncthreads();

    const int chunk = ((n + NW * 64 - 1) / (NW * 64)) * 64;
    const int beg = w * chunk;
    const int end = min(n, beg + chunk);
    // Expert ids in groups of 8 per lane, every load of a group in flight
    // before its LDS atomics.
    constexpr int kG = 8;
    for (int i0 = beg; i0 < end; i0 += 64 * kG) {
        int v[kG];
#pragma unroll
        for (int u = 0; u < kG; ++u) {
            const int i = i0 + 64 * u + lane;
            v[u] = i < end ? a.ids[i] : -1;
        }
#pragma unroll
        for (int u = 0; u < kG; ++u)
            if (v[u] >= 0) atomicAdd(&hist[w][v[u]], 1);
    }
    __syncthreads();

    // Wave 0 scans counts and m-tiles over the experts, kEpl consecutive
    // experts per lane.
    if (w == 0) {
        constexpr int kEpl = kMaxExperts / 64;
        int c[kEpl], m[kEpl], cs = 0, ms = 0;
#pragma unroll
        for (int j = 0; j < kEpl; ++j) {
            const int e = kEpl * lane + j;
            c[j] = 0;
            for (int ww = 0; ww < NW; ++ww)
                if (e < E) c[j] += hist[ww][e];
            if (e < E) a.counts[e] = c[j];
            m[j] = (c[j] + a.bm - 1) / a.bm;
            cs += c[j];
            ms += m[j];
        }
        const int c_own = cs, m_own = ms;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(cs, o), v = __shfl_up(ms, o);
            if (lane >= o) { cs += u; ms += v; }
        }
        int cb = cs - c_own, mb = ms - m_own;
#pragma unroll
        for (int j = 0; j < kEpl; ++j) {
            const int e = kEpl * lane + j;
            if (e < E) { offs[e] = cb; toff[e] = mb; }
            cb += c[j];
            mb += m[j];
        }
        if (lane == 63) { offs[E] = cs; toff[E] = ms; }
    }
    __syncthreads();
    for (int e = tid; e <= E; e += NT) {
        a.offsets[e] = offs[e];
        a.tile_off[e] = toff[e];
    }
    if (a.tile_expert)
        for (int e = tid; e < E; e += NT)
            for (int t = toff[e]; t < toff[e + 1]; ++t) a.tile_expert[t] = e;
    for (int e = tid; e < E; e += NT) {
        int base = offs[e];
        for (int ww = 0; ww < NW; ++ww) {
            int c = hist[ww][e];
            hist[ww][e] = base;
            base += c;
        }
    }
    __syncthreads();

    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int ev[kG];   // the next group of ids, loaded ahead of the ballots
    for (int i0 = beg; i0 < end; i0 += 64) {
        const int u = ((i0 - beg) >> 6) % kG;
        if (u == 0)
#pragma unroll
            for (int q = 0; q < kG; ++q) {
                const int iq = i0 + 64 * q + lane;
                ev[q] = iq < end ? a.ids[iq] : 0;
            }
        const int i = i0 + lane;
        const bool valid = i < end;
        int e = 0;
#pragma unroll
        for (int q = 0; q < kG; ++q)
            if (q == u) e = ev[q];
        uint64_t peers = __ballot(valid);
        for (int b = 0; b < nbits; ++b) {
            uint64_t m = __ballot(valid && ((e >> b) & 1));
            peers &= ((e >> b) & 1) ? m : ~m;
        }
        int base = 0;
        if (valid) base = hist[w][e];
        const int rank = __popcll(peers & below);
        if (valid) a.perm[base + rank] = i;
        // The highest lane of each peer group advances that expert's base.
        const bool last = valid && ((peers >> lane) >> 1) == 0ull;
        __builtin_amdgcn_wave_barrier();
        if (last) hist[w][e] = base + rank + 1;
        __builtin_amdgcn_wave_barrier();
    }
}

constexpr int kDispWaves = 16, kDispMaxGroups = 32;

// The same counting sort over G workgroups of 16 waves (dispatch_groups):
// the assignments fall into G * 16 wave chunks of CH (a multiple of 64)
// consecutive entries, chunk c = gg * 16 + w.  Every workgroup counts all
// of them into per-range histograms (wave w taking chunks gg * 16 + w for
// every gg), and its own range's chunks into per-wave ones.  Workgroup g
// then places its own 16 chunks: a wave's running base per expert lives in
// lane x, an entry's base comes from its expert's lane (a shuffle), its rank
// among the group's earlier lanes from the expert bits' ballots, which also
// give each lane x the group's count of experts x, x + 64, ....  Workgroup 0
// writes counts, offsets, tile_off and tile_expert.
// (Both loops run to the largest bit count, 8 for 256 experts, with
// constant indices, so the masks stay in registers.)
constexpr int kExpertBits = 8;
static_assert((1 << kExpertBits) >= kMaxExperts, "expert bits");
struct GroupMasks {
    uint64_t valid, bit[kExpertBits];
    // Lanes of the group whose expert is x.
    __device__ uint64_t of(int x, int nbits) const {
        uint64_t m = valid;
#pragma unroll
        for (int b = 0; b < kExpertBits; ++b)
            if (b < nbits) m &= ((x >> b) & 1) ? bit[b] : ~bit[b];
        return m;
    }
};
__device__ inline GroupMasks group_masks(bool valid, int e, int nbits) {
    GroupMasks g;
    g.valid = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kExpertBits; ++b) g.bit[b] = __ballot(b < nbits && valid && ((e >> b) & 1));
    return g;
}

__global__ __launch_bounds__(1024) void dispatch_groups_kernel(DispatchArgs a, int CH) {
    __shared__ int hg[kDispMaxGroups][kMaxExperts];   // per-workgroup-range counts
    __shared__ int hw[kDispWaves][kMaxExperts];       // this range's per-wave counts, then bases
    __shared__ int tot[kMaxExperts], pre[kMaxExperts];
    __shared__ int offs[kMaxExperts + 1], toff[kMaxExperts + 1];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int G = gridDim.x, g = blockIdx.x, E = a.E, n = a.n;
    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;
    // (Only the rows and columns in use are cleared: G ranges, E experts.)
    for (int gg = w; gg < G; gg += kDispWaves)
        for (int x = lane; x < E; x += 64) hg[gg][x] = 0;
    for (int x = lane; x < E; x += 64) hw[w][x] = 0;
    __syncthreads();

    // Pass 1: wave w counts chunks gg * 16 + w, gg < G (LDS atomics per
    // entry), 8 groups' loads at a time; (gg, sub) advance without
    // divisions.
    const int per = CH / 64, Q = G * per;
    int gg_n = 0, sub_n = 0;   // the next group to load
    for (int q0 = 0; q0 < Q; q0 += 8) {
        int v[8], gq[8];
        bool ok[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = (gg_n * kDispWaves + w) * CH + sub_n * 64 + lane;
            ok[u] = q0 + u < Q && i < n;
            gq[u] = gg_n;
            v[u] = a.ids[min(i, n - 1)];
            if (++sub_n == per) {
                sub_n = 0;
                ++gg_n;
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (ok[u]) {
                atomicAdd(&hg[gq[u]][v[u]], 1);
                if (gq[u] == g) atomicAdd(&hw[w][v[u]], 1);
            }
    }
    __syncthreads();

    // Totals, the counts before this workgroup's range, offsets (a scan in
    // expert order), then each wave's bases.
    for (int x = tid; x < E; x += 1024) {
        int t = 0, p = 0;
        for (int gg = 0; gg < G; ++gg) {
            const int c = hg[gg][x];
            t += c;
            if (gg < g) p += c;
        }
        tot[x] = t;
        pre[x] = p;
    }
    __syncthreads();
    if (tid == 0) {
        int cs = 0, ms = 0;
        for (int x = 0; x < E; ++x) {
            offs[x] = cs;
            toff[x] = ms;
            cs += tot[x];
            ms += (tot[x] + a.bm - 1) / a.bm;
        }
        offs[E] = cs;
        toff[E] = ms;
    }
    __syncthreads();
    for (int x = tid; x < E; x += 1024) {
        int b = offs[x] + pre[x];
        for (int ww = 0; ww < kDispWaves; ++ww) {
            const int c = hw[ww][x];
            hw[ww][x] = b;
            b += c;
        }
    }
    if (g == 0) {
        for (int x = tid; x < E; x += 1024) a.counts[x] = tot[x];
        for (int x = tid; x <= E; x += 1024) {
            a.offsets[x] = offs[x];
            a.tile_off[x] = toff[x];
        }
        if (a.tile_expert)
            for (int x = tid; x < E; x += 1024)
                for (int t = toff[x]; t < toff[x + 1]; ++t) a.tile_expert[t] = x;
    }
    __syncthreads();

    // Pass 2: this workgroup's chunk g * 16 + w, in order.
    constexpr int kEpl = kMaxExperts / 64;   // running bases per lane: experts lane + 64 j
    int bs[kEpl];
#pragma unroll
    for (int j = 0; j < kEpl; ++j) bs[j] = lane + 64 * j < E ? hw[w][lane + 64 * j] : 0;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int beg = (g * kDispWaves + w) * CH;
    for (int s0 = 0; s0 < per; s0 += 8) {
        int v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = a.ids[min(beg + min(s0 + u, per - 1) * 64 + lane, n - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (s0 + u >= per) break;
            const int i = beg + (s0 + u) * 64 + lane;
            const bool valid = i < n;
            const int e = v[u];
            const GroupMasks m = group_masks(valid, e, nbits);
            const uint64_t peers = m.of(e, nbits);
            int base = 0;
#pragma unroll
            for (int j = 0; j < kEpl; ++j)
                if (64 * j < E) {
                    const int bj = __shfl(bs[j], e & 63);
                    if ((e >> 6) == j) base = bj;
                }
            if (valid) a.perm[base + __popcll(peers & below)] = i;
#pragma unroll
            for (int j = 0; j < kEpl; ++j)
                if (64 * j < E) bs[j] += __popcll(m.of(lane + 64 * j, nbits));
        }
    }
}

// Workgroups of the grouped dispatch for n assignments (about one 64-entry
// group per wave), and the chunk length CH.
inline void dispatch_groups(int n, int &G, int &CH) {
    G = std::max(1, std::min(kDispMaxGroups, (n + kDispWaves * 64 - 1) / (kDispWaves * 64)));
    const int wc = G * kDispWaves;
    CH = ((n + wc - 1) / wc + 63) / 64 * 64;
}

hipError_t launch_dispatch_groups(const DispatchArgs &da, hipStream_t s) {
    if (da.n <= 0) return hipSuccess;
    int G, CH;
    dispatch_groups(da.n, G, CH);
    hipLaunchKernelGGL(dispatch_groups_kernel, dim3((unsigned)G), dim3(1024), 0, s, da, CH);
    return hipGetLastError();
}

// The token x expert tile router (router_kernel) takes up to 128 experts;
// wider layers route through the row-block router.
constexpr int kTileRouterMaxExperts = 128;

// Softmax, top-k and gate weights of token t from its logits row (in LDS),
// which is left holding the probabilities.  The reference's "already chosen"
// scan over ids[0..ki) (src/transformer.c:321-325) is a set membership test;
// a bit set keeps it (and every index below) in registers.  The gate weight
// uses probs[ids[ki]], as the reference does even when no candidate beat -1.
__device__ inline void finish_token(const RouteArgs &a, float *row, int t) {
    const int E = a.E, k = a.k;
    softmax_row(row, E);
    uint64_t chosen[kTileRouterMaxExperts / 64] = {};
    float pk[kMaxTopK];
    int idk[kMaxTopK];
#pragma unroll
    for (int ki = 0; ki < kMaxTopK; ++ki) {
        if (ki < k) {
            float best = -1.0f;
            int best_e = 0;
            for (int e = 0; e < E; ++e) {
                const bool already = (chosen[e >> 6] >> (e & 63)) & 1ull;
                if (!already && row[e] > best) { best = row[e]; best_e = e; }
            }
            chosen[best_e >> 6] |= 1ull << (best_e & 63);
            idk[ki] = best_e;
            pk[ki] = row[best_e];
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int ki = 0; ki < kMaxTopK; ++ki)
        if (ki < k) s = s + pk[ki];
    float inv = (s > 1e-9f) ? 1.0f / s : 0.0f;
#pragma unroll
    for (int ki = 0; ki < kMaxTopK; ++ki) {
        if (ki < k) {
            if (a.ids) a.ids[(size_t)t * k + ki] = idk[ki];
            if (a.gw) a.gw[(size_t)t * k + ki] = ftz_f(pk[ki] * inv);
        }
    }
}

// kend steps of the per-thread FMA chains from one LDS chunk.  The LDS reads
// of 8 steps are issued ahead of their FMAs; each accumulator still adds its
// terms in ascending k.  SKIP applies the reference's zero-skip.
template <int RT, int RE, int TM, int EP, int KC, bool SKIP>
__device__ inline void chain_steps(const float *xs, const float *ws, int kend, int tx, int ty,
                                   float (&acc)[RT][RE]) {
    int kk = 0;
    for (; kk + 8 <= kend; kk += 8) {
        float xv[8][RT], wv[8][RE];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
#pragma unroll
            for (int i = 0; i < RT; ++i) xv[u][i] = xs[(kk + u) * TM + ty * RT + i];
#pragma unroll
            for (int j = 0; j < RE; ++j) wv[u][j] = ws[(kk + u) * EP + tx * RE + j];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int j = 0; j < RE; ++j) {
                    if (SKIP) acc[i][j] = (xv[u][i] != 0.0f) ? fmaf(xv[u][i], wv[u][j], acc[i][j])
                                                            : acc[i][j];
                    else      acc[i][j] = fmaf(xv[u][i], wv[u][j], acc[i][j]);
                }
    }
    for (; kk < kend; ++kk) {
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const float xv = xs[kk * TM + ty * RT + i];
#pragma unroll
            for (int j = 0; j < RE; ++j) {
                const float wv = ws[kk * EP + tx * RE + j];
                if (SKIP) acc[i][j] = (xv != 0.0f) ? fmaf(xv, wv, acc[i][j]) : acc[i][j];
                else      acc[i][j] = fmaf(xv, wv, acc[i][j]);
            }
        }
    }
}

// Router workgroup: 16*RT tokens x 16*RE expert slots, 256 threads.  Thread
// (tx, ty) owns tokens ty*RT .. ty*RT+RT-1 and experts tx*RE .. tx*RE+RE-1,
// each an independent ascending FMA chain.  K is staged through LDS in
// KC-wide chunks with the next chunk prefetched into registers.  When a
// chunk holds no exact zero among the live x values the zero-skip select is
// a no-op and the chunk runs plain FMAs (a uniform branch).
template <int RT, int RE, int KC, bool FUSE>
__global__ __launch_bounds__(256) void router_kernel(RouteArgs a, DispatchArgs da) {
    constexpr int TM = 16 * RT, EP = 16 * RE;
    constexpr int XQ = TM * KC / 4;                 // float4s of x per chunk
    constexpr int XL = (XQ + 255) / 256;
    constexpr int WQ = KC * EP;                     // floats of w per chunk
    constexpr int WL = (WQ + 255) / 256;
    __shared__ __align__(16) float xs[2][KC][TM];
    __shared__ __align__(16) float ws[2][KC][EP];
    __shared__ float lg[TM][EP + 1];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int t0 = blockIdx.x * TM;
    const int T = a.T, d = a.d, E = a.E;

    float acc[RT][RE];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < RE; ++j) acc[i][j] = 0.0f;

    float4 rx[XL];
    float rw[WL];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            int q = tid + 256 * i;
            int r = q / (KC / 4), c4 = q % (KC / 4);
            int t = t0 + r, kk = k0 + 4 * c4;
            rx[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (q < XQ && t < T && kk < d)
                rx[i] = *reinterpret_cast<const float4 *>(a.x + (size_t)t * d + kk);
        }
#pragma unroll
        for (int i = 0; i < WL; ++i) {
            int q = tid + 256 * i;
            int r = q / EP, c = q % EP;
            int kk = k0 + r;
            rw[i] = (q < WQ && kk < d && c < E) ? a.wr[(size_t)kk * E + c] : 0.0f;
        }
    };
    // Stores the prefetched chunk; returns 1 if a live x value is exactly 0
    // (after DAZ), which selects the zero-skip path for the chunk.
    auto sstore = [&](int buf, int k0) -> int {
        int z = 0;
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            int q = tid + 256 * i;
            if (q < XQ) {
                int r = q / (KC / 4), c4 = q % (KC / 4);
                bool live = (t0 + r < T) && (k0 + 4 * c4 < d);
                float v[4] = {rx[i].x, rx[i].y, rx[i].z, rx[i].w};
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    float u = ftz_f(v[m]);
                    if (u == 0.0f) { u = 0.0f; z |= live ? 1 : 0; }
                    xs[buf][4 * c4 + m][r] = u;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < WL; ++i) {
            int q = tid + 256 * i;
            if (q < WQ) ws[buf][q / EP][q % EP] = ftz_f(rw[i]);
        }
        return z;
    };

    const int nchunk = (d + KC - 1) / KC;
    gload(0);
    int zero = __syncthreads_or(sstore(0, 0));
    for (int c = 0; c < nchunk; ++c) {
        const int buf = c & 1;
        const int k0 = c * KC;
        if (c + 1 < nchunk) gload(k0 + KC);
        const int kend = min(KC, d - k0);
        if (!zero) chain_steps<RT, RE, TM, EP, KC, false>(&xs[buf][0][0], &ws[buf][0][0], kend,
                                                          tx, ty, acc);
        else       chain_steps<RT, RE, TM, EP, KC, true>(&xs[buf][0][0], &ws[buf][0][0], kend,
                                                         tx, ty, acc);
        int z = 0;
        if (c + 1 < nchunk) z = sstore(buf ^ 1, k0 + KC);
        zero = __syncthreads_or(z);
    }
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < RE; ++j) {
            int e = tx * RE + j;
            if (e < E) {
                float v = acc[i][j];
                if (a.bias) v = v + a.bias[e];
                lg[ty * RT + i][e] = v;
            }
        }
    __syncthreads();

    // One thread per token: softmax, top-k, gate weights.
    if (tid < TM && t0 + tid < T) finish_token(a, &lg[tid][0], t0 + tid);
    __syncthreads();
    if (a.probs) {
        for (int idx = tid; idx < TM * E; idx += 256) {
            int r = idx / E, e = idx % E;
            if (t0 + r < T) a.probs[(size_t)(t0 + r) * E + e] = lg[r][e];
        }
    }
    if (FUSE) {
        // The last workgroup to finish runs the dispatch over every token's
        // ids (release/acquire through the device-scope fences), then resets
        // the counter for the next launch.
        __shared__ int hist[4][kMaxExperts];
        __shared__ int offs[kMaxExperts + 1];
        __shared__ int toff[kMaxExperts + 1];
        __shared__ int is_last;
        __threadfence();
        __syncthreads();
        if (tid == 0) is_last = atomicAdd(da.counter, 1) == (int)gridDim.x - 1;
        __syncthreads();
        if (is_last) {
            __threadfence();
            dispatch_body<4>(da, hist, offs, toff);
            if (tid == 0) *da.counter = 0;
        }
    }
}

template <int NWV, int RE, int KC, bool SKIP, bool FUSE>
__global__ __launch_bounds__(64 * NWV) void router_rows_kernel(RouteArgs a, DispatchArgs da) {
    __shared__ __align__(16) float smem[RowsSmem<KC, rows_lw(NWV, RE)>::kFloats];
    __shared__ int is_last;
    const int tid = threadIdx.x;
    route_rows_block<NWV, RE, KC, SKIP>(a, blockIdx.x, smem);
    if (FUSE) {
        // The last workgroup to finish runs the dispatch over every token's
        // ids (release/acquire through the device-scope fences), then resets
        // the counter for the next launch.
        __shared__ int hist[NWV][kMaxExperts];
        __shared__ int offs[kMaxExperts + 1];
        __shared__ int toff[kMaxExperts + 1];
        __threadfence();
        __syncthreads();
        if (tid == 0) is_last = atomicAdd(da.counter, 1) == (int)gridDim.x - 1;
        __syncthreads();
        if (is_last) {
            __threadfence();
            dispatch_body<NWV>(da, hist, offs, toff);
            if (tid == 0) *da.counter = 0;
        }
    }
}

// dst[c][r] = src[r][c] for a rows x cols matrix.
__global__ __launch_bounds__(256) void transpose_kernel(const float *src, float *dst, int rows,
                                                        int cols) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int i = ty; i < 32; i += 8)
        if (r0 + i < rows && c0 + tx < cols) tile[i][tx] = src[(size_t)(r0 + i) * cols + c0 + tx];
    __syncthreads();
    for (int i = ty; i < 32; i += 8)
        if (c0 + i < cols && r0 + tx < rows) dst[(size_t)(c0 + i) * rows + r0 + tx] = tile[tx][i];
}

// rms_norm (src/matrix.c:666-711) rows: y = (x * inv_rms) * w.  Four lanes
// per row, lane q owning columns 16b + 4q .. 16b + 4q + 3 of every 16-column
// block, i.e. the reference's accumulator lanes l = 4q .. 4q + 3 (l < 8 of
// its first 8-wide register, l - 8 of its second).  Then: first += second
// lane-wise, one 8-column block into the first, hsum256's fold
// ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)), the scalar tail as FMAs, and
// inv_rms = 1 / sqrt(fma(ss, 1/cols, eps)) correctly rounded (the reference
// build estimates it with RSQRTSS and one Newton-Raphson step).
// NB > 0: cols == 16 * NB; sixteen lanes per row, lane l holding the
// reference accumulator lane l (columns 16b + l) in registers, all its loads
// in flight at once; four rows per 64-thread workgroup.  The lanes are then
// folded in the same association: v_l = acc_l + acc_(l+8), s_i = v_i +
// v_(i+4), ((s_0 + s_1) + (s_2 + s_3)).  NB == 0: any cols, four lanes per
// row as described above, loads unrolled eight column blocks at a time.
template <int NB>
__global__ __launch_bounds__(NB > 0 ? 64 : 256) void rms_norm_kernel(
    const float *x, const float *w, float eps, int rows, int cols, float rcp_cols, float *y) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (NB > 0) {
        const int l = threadIdx.x & 15;
        const int row = blockIdx.x * 4 + (threadIdx.x >> 4);
        const bool live = row < rows;
        const float *xr = x + (size_t)(live ? row : 0) * cols;
        float v[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) v[b] = xr[16 * b + l];
        float acc = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) acc = fmaf(v[b], v[b], acc);
        acc = acc + row_down<8>(acc);
        acc = acc + row_down<4>(acc);
        acc = acc + row_down<1>(acc);
        acc = acc + row_down<2>(acc);
        const float inv = row_lane0(1.0f / sqrtf(fmaf(acc, rcp_cols, eps)));
        if (!live) return;
        float *yr = y + (size_t)row * cols;
#pragma unroll
        for (int b = 0; b < NB; ++b) yr[16 * b + l] = (v[b] * inv) * w[16 * b + l];
        return;
    }
    const int q = threadIdx.x & 3;
    const int row = blockIdx.x * 64 + (threadIdx.x >> 2);
    const bool live = row < rows;
    const float *xr = x + (size_t)(live ? row : 0) * cols;
    const int nb = cols / 16;
#pragma unroll 8
    for (int b = 0; b < nb; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = xr[16 * b + 4 * q + i];
            a[i] = fmaf(v, v, a[i]);
        }
    // Lanes 0, 1 hold accumulator lanes 0..7; add lanes 8..15 from 2, 3.
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = a[i] + __shfl_down(a[i], 2, 4);
    int j = 16 * nb;
    if (j + 8 <= cols) {
        if (q < 2)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = xr[j + 4 * q + i];
                a[i] = fmaf(v, v, a[i]);
            }
        j += 8;
    }
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = a[i] + __shfl_down(a[i], 1, 4);   // v_i + v_{i+4}
    float ss = (s[0] + s[1]) + (s[2] + s[3]);
    for (int t = j; t < cols; ++t) ss = fmaf(xr[t], xr[t], ss);
    const float inv = __shfl(1.0f / sqrtf(fmaf(ss, rcp_cols, eps)), 0, 4);
    if (!live) return;
    float *yr = y + (size_t)row * cols;
#pragma unroll 4
    for (int c = 4 * q; c < cols; c += 16)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (c + i < cols) yr[c + i] = (xr[c + i] * inv) * w[c + i];
}

__global__ __launch_bounds__(256) void eval_exp_kernel(int which, const float *x, float *y,
                                                      size_t n) {
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        y[i] = which == 0 ? exp_poly(x[i]) : glibc_expf(x[i]);
}

}  // namespace

hipError_t launch_transpose(const float *src, float *dst, int rows, int cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    dim3 grid((cols + 31) / 32, (rows + 31) / 32);
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(256), 0, s, src, dst, rows, cols);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float *x, const float *w, float eps, int rows, int cols,
                           float *y, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const float rc = 1.0f / (float)cols;
    const dim3 g4((unsigned)((rows + 3) / 4)), g64((unsigned)((rows + 63) / 64));
    switch (cols) {
    case 128:  hipLaunchKernelGGL(rms_norm_kernel<8>, g4, dim3(64), 0, s, x, w, eps, rows, cols, rc, y); break;
    case 256:  hipLaunchKernelGGL(rms_norm_kernel<16>, g4, dim3(64), 0, s, x, w, eps, rows, cols, rc, y); break;
    case 512:  hipLaunchKernelGGL(rms_norm_kernel<32>, g4, dim3(64), 0, s, x, w, eps, rows, cols, rc, y); break;
    case 1024: hipLaunchKernelGGL(rms_norm_kernel<64>, g4, dim3(64), 0, s, x, w, eps, rows, cols, rc, y); break;
    default:   hipLaunchKernelGGL(rms_norm_kernel<0>, g64, dim3(256), 0, s, x, w, eps, rows, cols, rc, y);
    }
    return hipGetLastError();
}

hipError_t launch_eval_exp(int which, const float *x, float *y, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    unsigned blocks = (unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    hipLaunchKernelGGL(eval_exp_kernel, dim3(blocks), dim3(256), 0, s, which, x, y, n);
    return hipGetLastError();
}

namespace {

template <bool FUSE>
hipError_t launch_router(const RouteArgs &a, const DispatchArgs &da, hipStream_t s) {
    const bool big = a.T >= 2048;
    const int TM = big ? 64 : 16;
    dim3 grid((a.T + TM - 1) / TM), block(256);
    if (big) {
        if (a.E <= 16)       hipLaunchKernelGGL((router_kernel<4, 1, 64, FUSE>), grid, block, 0, s, a, da);
        else if (a.E <= 32)  hipLaunchKernelGGL((router_kernel<4, 2, 64, FUSE>), grid, block, 0, s, a, da);
        else if (a.E <= 64)  hipLaunchKernelGGL((router_kernel<4, 4, 32, FUSE>), grid, block, 0, s, a, da);
        else if (a.E <= 128) hipLaunchKernelGGL((router_kernel<4, 8, 16, FUSE>), grid, block, 0, s, a, da);
        else return hipErrorInvalidValue;
    } else {
        if (a.E <= 16)       hipLaunchKernelGGL((router_kernel<1, 1, 128, FUSE>), grid, block, 0, s, a, da);
        else if (a.E <= 32)  hipLaunchKernelGGL((router_kernel<1, 2, 128, FUSE>), grid, block, 0, s, a, da);
        else if (a.E <= 64)  hipLaunchKernelGGL((router_kernel<1, 4, 64, FUSE>), grid, block, 0, s, a, da);
        else if (a.E <= 128) hipLaunchKernelGGL((router_kernel<1, 8, 32, FUSE>), grid, block, 0, s, a, da);
        else return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int NWV, int RE, int KC, bool FUSE>
void launch_rows(const RouteArgs &a, const DispatchArgs &da, hipStream_t s) {
    dim3 grid((a.T + 15) / 16), block(64 * NWV);
    if (a.wr_nonfinite)
        hipLaunchKernelGGL((router_rows_kernel<NWV, RE, KC, true, FUSE>), grid, block, 0, s, a, da);
    else
        hipLaunchKernelGGL((router_rows_kernel<NWV, RE, KC, false, FUSE>), grid, block, 0, s, a, da);
}

// Waves and experts per lane: 4 * NWV * RE >= E.  Chunks of 128 k when d
// allows (d % 64 == 0 always holds).
template <int KC, bool FUSE>
hipError_t launch_rows_kc(const RouteArgs &a, const DispatchArgs &da, hipStream_t s) {
    if (a.E <= 8)        launch_rows<2, 1, KC, FUSE>(a, da, s);
    else if (a.E <= 16)  launch_rows<4, 1, KC, FUSE>(a, da, s);
    else if (a.E <= 32)  launch_rows<4, 2, KC, FUSE>(a, da, s);
    else {
        if constexpr (KC == 512) {
            return hipErrorInvalidValue;
        } else {
            if (a.E <= 64)       launch_rows<4, 4, KC, FUSE>(a, da, s);
            else if (a.E <= 128) launch_rows<4, 8, KC, FUSE>(a, da, s);
            else if (a.E <= 256) launch_rows<8, 8, KC, FUSE>(a, da, s);
            else return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

// k chunk: 512 when d allows and the router rows fit in registers (up to 32
// experts), so a d = 512 layer stages x once; else 128 or 64 (d % 64 == 0
// always holds).
template <bool FUSE>
hipError_t launch_rows_router(const RouteArgs &a, const DispatchArgs &da, hipStream_t s) {
    if (a.d % 512 == 0 && a.E <= 32) return launch_rows_kc<512, FUSE>(a, da, s);
    if (a.d % 128 == 0) return launch_rows_kc<128, FUSE>(a, da, s);
    return launch_rows_kc<64, FUSE>(a, da, s);
}

}  // namespace

// Routing followed by dispatch.  For small launches (at most
// kFusedDispatchMax assignments and kFusedDispatchMaxBlocks router
// workgroups) the router's last workgroup sorts them in the same launch; its
// device-scope fences write back and invalidate L2, which is cheap for a
// handful of workgroups only.  Otherwise dispatch_groups_kernel sorts them
// (about one 64-entry group per wave, over up to 32 workgroups).
hipError_t launch_route_dispatch(const RouteArgs &a, const DispatchArgs &da, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    if (a.E > kMaxExperts || a.k > kMaxTopK) return launch_route_wide(a, da, s);
    if (a.rms_w && !(a.wrT && a.d % 16 == 0)) {
        // Only the row-block router normalises its rows itself.
        hipError_t e = launch_rms_norm(a.x_raw, a.rms_w, a.rms_eps, a.T, a.d, a.xn_out, s);
        if (e != hipSuccess) return e;
        RouteArgs b = a;
        b.rms_w = nullptr;
        return launch_route_dispatch(b, da, s);
    }
    if (a.no_dispatch)
        return a.wrT ? launch_rows_router<false>(a, da, s) : launch_router<false>(a, da, s);
    if (a.wrT) {
        const int blocks = (a.T + 15) / 16;
        const bool fuse = da.counter && da.n <= kFusedDispatchMax && blocks <= kRowsFusedMaxBlocks;
        hipError_t e = fuse ? launch_rows_router<true>(a, da, s) : launch_rows_router<false>(a, da, s);
        if (e != hipSuccess || fuse) return e;
        return launch_dispatch_groups(da, s);
    }
    const int grid = (a.T + (a.T >= 2048 ? 64 : 16) - 1) / (a.T >= 2048 ? 64 : 16);
    if (da.n <= kFusedDispatchMax && grid <= kFusedDispatchMaxBlocks && da.counter)
        return launch_router<true>(a, da, s);
    hipError_t e = launch_router<false>(a, da, s);
    if (e != hipSuccess) return e;
    return launch_dispatch_groups(da, s);
}


}  // namespace moe
