// decode_gemv.h — building blocks of the bandwidth-bound decode expert
// products (decode.hip).
//
// Weights stream from HBM straight into v_mfma_f32_16x16x4f32 operands: a
// lane holds a 16-byte piece of one weight row (K contiguous), the MFMA's
// k-row h (lane/16) takes the piece's 4 elements in turn, and the
// activations come from LDS as 128-bit reads with the same k mapping.
// Weights are in the unit layout (16 x 16 tiles in MFMA operand order, see
// gemm.hip): a K step of 16 is one contiguous 1 KB unit per wave.
#pragma once
#include <type_traits>

#include "handoff.h"
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
// workgroup's NW waves with ballots, and (tok != nullptr) the token a / topk
// of each; returns the list length.  Every thread calls this, with id0 =
// ids[threadIdx.x] (or -1 past n) loaded by the caller before its first
// weight loads so that waiting for it does not wait for them; wcnt is NW
// ints of LDS.
template <int NW>
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
#pragma unroll
    for (int w = 0; w < NW; ++w) total += wcnt[w];
    __syncthreads();
}

template <int NW = 4>
__device__ int expert_slots(const int *ids, int n, int e, int id0, int topk, int *list, int *tok,
                            int *wcnt) {
    int total = 0;
    slot_chunk<NW>(threadIdx.x, n, e, id0, topk, list, tok, wcnt, total);
    for (int base = 64 * NW; base < n; base += 64 * NW) {
        const int i = base + threadIdx.x;
        slot_chunk<NW>(i, n, e, ids[min(i, n - 1)], topk, list, tok, wcnt, total);
    }
    return total;
}

// Staging of rows rowlist[pos0 .. pos0 + rows) of src, columns [k0, k0 + kc),
// into LDS rows of stride kLd by global-to-LDS DMA (no registers): wave w of
// NW copies rows w, w + NW, ... as two 1 KB pieces each (64 lanes x 16
// bytes), columns clamped to the source row.  Columns past kc and rows past
// rows are never read.
template <int NW = 4>
__device__ inline void stage_lds(float *xs, const float *src, int ld, const int *rowlist,
                                 int pos0, int rows, int k0, int kc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int r = wave; r < rows; r += NW) {
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

// After the rows staged by DMA are known to have landed (an explicit wait):
// one read of them, so that the compiler's own wait tracking also counts the
// DMA as complete.  Otherwise it assumes the DMA may still be writing LDS
// and waits for every outstanding load before each later LDS read, which
// drains the weight stream in every loop iteration.
__device__ inline void dma_landed(const float *xs) {
    const float v = xs[threadIdx.x & 63];
    asm volatile("" ::"v"(v));
}

// Streams NB weight rows (NB = 2: gate and up of the lane's feature, NB = 1:
// one down row) over nq 16-wide K steps against RB 16-row activation blocks
// in LDS.  The stream is cut into groups of kU = 8/NB steps held in two
// register sets; the loads of group g + 2 are issued as soon as group g's
// MFMAs are done, so one to two groups (8 to 16 16-byte loads per lane) stay
// in flight.
template <int NB> struct Unroll { static constexpr int kU = 8 / NB; };

template <int NB>
using WGroup = floatx4[Unroll<NB>::kU][NB];

// One expert's packed weight block as a buffer resource (four SGPRs,
// range-checked against the block's size) plus the lane's byte offset lo
// (one VGPR): every weight load is then lo + a wave-uniform byte offset
// (SGPR and immediate), which keeps address arithmetic off the VGPRs.
// Blocks stay below 2 GiB (the host checks), so offsets fit an int.
struct WSrc {
    __amdgpu_buffer_rsrc_t r;
    unsigned lo;
};

__device__ inline WSrc wsrc(const float *block, size_t nfloats, unsigned lo) {
    // dword 3 = 0x00020000: 32-bit data format, the gfx9 raw-buffer form.
    return WSrc{__builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(block), (short)0,
                                                  (int)(nfloats * sizeof(float)), 0x00020000),
                lo};
}

// The 16-byte piece at byte offset off (wave-uniform) of a weight row, as a
// non-temporal (streaming) load: every weight byte is read once per step, and
// a plain read of 192 MiB over 256 workgroups runs at 5.9-6.0 TB/s this way
// against 5.5 TB/s with the default policy (the decode layer: 46.4-46.9 ->
// 44.1-44.8 us).
constexpr int kCachePolicyNt = 2;
__device__ inline floatx4 ldw(const WSrc &s, int off) {
    return __builtin_amdgcn_raw_buffer_load_b128(s.r, s.lo, off, kCachePolicyNt);
}

// Byte size of a unit (a 16-wide K step of 16 rows).
constexpr int kUnitBytes = kUnit * (int)sizeof(float);

// Loads steps q .. q + kU - 1 of the stream rows at byte offsets ob[b], each
// clamped to step last (CLAMP; so a short chunk never reads past its
// weights).
template <int NB, bool CLAMP = true>
__device__ inline void wload(const WSrc &s, const int (&ob)[2], int q, int last, WGroup<NB> &w) {
#pragma unroll
    for (int u = 0; u < Unroll<NB>::kU; ++u)
#pragma unroll
        for (int b = 0; b < NB; ++b)
            w[u][b] = ldw(s, ob[b] + kUnitBytes * (CLAMP ? min(q + u, last) : q + u));
}

// First step of stream group g when the stream of ng whole groups starts at
// group g0 (0 < g0 < ng, so that the workgroups sharing the memory system
// are spread over it) and wraps around; g0 = 0: group g itself.
template <int NB>
__device__ inline int group_step(int g, int g0, int ng) {
    const int r = g + g0;
    return Unroll<NB>::kU * (g0 && r >= ng ? r - ng : r);
}

// Issues the loads of groups 0 and 1 of a chunk of nq steps, unconditionally
// (wait counts stay exact); groups the chunk lacks are never used.  g0: the
// rotation gemv_loop is given (nonzero only for chunks of whole groups).
template <int NB>
__device__ inline void gemv_prime(const WSrc &s, int o0, int o1, int nq, WGroup<NB> &wa,
                                  WGroup<NB> &wb, int g0 = 0) {
    const int ng = nq / Unroll<NB>::kU;
    const int ob[2] = {o0, o1};
    wload<NB>(s, ob, group_step<NB>(0, g0, ng), nq - 1, wa);
    wload<NB>(s, ob, group_step<NB>(1, g0, ng), nq - 1, wb);
}

// as0 / as1: the lane's activation row of 16-row block 0 / 1 (as1 is read
// only when RB == 2).
template <int NB, int RB>
__device__ inline void gemv_group(const float *as0, const float *as1, int q, const WGroup<NB> &w,
                                  floatx4 (&acc)[2][NB]) {
#pragma unroll
    for (int u = 0; u < Unroll<NB>::kU; ++u) {
        floatx4 a0 = *reinterpret_cast<const floatx4 *>(as0 + 16 * (q + u));
        floatx4 a1;
        if (RB == 2) a1 = *reinterpret_cast<const floatx4 *>(as1 + 16 * (q + u));
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                acc[0][b] = mfma16(a0[s], w[u][b][s], acc[0][b]);
                if (RB == 2) acc[1][b] = mfma16(a1[s], w[u][b][s], acc[1][b]);
            }
    }
}

// Down-projection units of the fused kernel: 8 units per group (8 / NW
// 16-column blocks of NW feature units each), clamped to the wave's last
// unit.
template <int NW>
__device__ inline void dload(const WSrc &s, int od, int fq, int g, int last, floatx4 (&w)[8]) {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
        const int q = min(8 * g + v, last);
        w[v] = ldw(s, od + kUnitBytes * ((q / NW) * fq + q % NW));
    }
}

// Where the fused kernel's down stream starts: its first two groups go out
// from the tail of the last gate/up chunk (into the registers that chunk
// frees), so the weight stream does not drain between the two products.
template <int NW>
struct DownHead {
    WSrc s;
    int od, fq, last;
    int g0, ng;   // the down stream's ng groups start at group g0 (see group_step)
    __device__ int rot(int g) const { return g0 && g + g0 >= ng ? g + g0 - ng : g + g0; }
};

// wa / wb must hold groups 0 / 1 (gemv_prime, same g0).  g0 != 0 rotates
// the stream (requires nq = kU * ng).
// HEAD: also issues the first two down groups into wa and wb (NB = 2 only).
template <int NB, int RB, bool HEAD = false, int NW = 4>
__device__ inline void gemv_loop(const WSrc &s, int o0, int o1, const float *as0, const float *as1,
                                 int nq,
                                 floatx4 (&acc)[2][NB], WGroup<NB> &wa, WGroup<NB> &wb,
                                 const DownHead<NW> &dh = DownHead<NW>{}, int g0 = 0) {
    constexpr int kU = Unroll<NB>::kU;
    static_assert(!HEAD || NB == 2, "the down stream reuses the gate/up registers");
    auto head = [&](int g, WGroup<NB> &w) {
        if constexpr (HEAD)
            dload<NW>(dh.s, dh.od, dh.fq, dh.rot(g), dh.last, reinterpret_cast<floatx4 (&)[8]>(w));
    };
    const int ob[2] = {o0, o1};
    const int ng = nq / kU;
    auto qg = [&](int gg) { return group_step<NB>(gg, g0, ng); };
    int g = 0;
    // Steady state with unconditional loads (exact wait counts); groups
    // g + 2 and g + 3 lie inside the chunk, so they go unclamped.
    // (Scheduling barriers keep each group's loads right after the MFMAs
    // that free its registers.)
    for (; g + 4 <= ng; g += 2) {
        gemv_group<NB, RB>(as0, as1, qg(g), wa, acc);
        __builtin_amdgcn_sched_barrier(0);
        wload<NB, false>(s, ob, qg(g + 2), nq - 1, wa);
        __builtin_amdgcn_sched_barrier(0);
        gemv_group<NB, RB>(as0, as1, qg(g + 1), wb, acc);
        __builtin_amdgcn_sched_barrier(0);
        wload<NB, false>(s, ob, qg(g + 3), nq - 1, wb);
        __builtin_amdgcn_sched_barrier(0);
    }
    const int left = ng - g;   // 0 .. 3 groups, the first two already loaded
    if (left == 3) {
        gemv_group<NB, RB>(as0, as1, qg(g), wa, acc);
        wload<NB>(s, ob, qg(g + 2), nq - 1, wa);
        gemv_group<NB, RB>(as0, as1, qg(g + 1), wb, acc);
        gemv_group<NB, RB>(as0, as1, qg(g + 2), wa, acc);
    } else if (left == 2 && nq == kU * ng) {
        // (the common case: each down group goes out as its registers free)
        gemv_group<NB, RB>(as0, as1, qg(g), wa, acc);
        __builtin_amdgcn_sched_barrier(0);
        head(0, wa);
        __builtin_amdgcn_sched_barrier(0);
        gemv_group<NB, RB>(as0, as1, qg(g + 1), wb, acc);
        __builtin_amdgcn_sched_barrier(0);
        head(1, wb);
        return;
    } else if (left == 2) {
        gemv_group<NB, RB>(as0, as1, qg(g), wa, acc);
        gemv_group<NB, RB>(as0, as1, qg(g + 1), wb, acc);
    } else if (left == 1) {
        gemv_group<NB, RB>(as0, as1, qg(g), wa, acc);
    }
    for (int q = kU * ng; q < nq; ++q) {
        floatx4 w[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) w[b] = ldw(s, ob[b] + kUnitBytes * q);
        floatx4 a0 = *reinterpret_cast<const floatx4 *>(as0 + 16 * q);
        floatx4 a1;
        if (RB == 2) a1 = *reinterpret_cast<const floatx4 *>(as1 + 16 * q);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                acc[0][b] = mfma16(a0[s], w[b][s], acc[0][b]);
                if (RB == 2) acc[1][b] = mfma16(a1[s], w[b][s], acc[1][b]);
            }
    }
    head(0, wa);
    head(1, wb);
}

// Padded LDS row of the fused kernel's H block (16 * NW features).
template <int NW> constexpr int hld() { return 16 * NW + 4; }

// MFMAs of one down group: column blocks CB*g .. CB*g + CB - 1 of the wave
// (CB = 8 / NW; those below nbw), K = the block's 16 * NW features (A
// operands from the H block in LDS at as), each block written at yoff + its
// column once complete (yoff < 0: a row past the pass); CS: with coherent
// (write-through) stores.
template <int RB, int NW, bool CS = false>
__device__ inline void dgroup(const floatx4 (&w)[8], const float *as, int g, int nbw, int cb0,
                              const int (&yoff)[2][4], float *yp, int j) {
    constexpr int CB = 8 / NW;
    floatx4 ha[2][NW];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int u = 0; u < NW; ++u)
            ha[b][u] = *reinterpret_cast<const floatx4 *>(as + b * 16 * hld<NW>() + 16 * u);
#pragma unroll
    for (int bi = 0; bi < CB; ++bi) {
        floatx4 acc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int u = 0; u < NW; ++u)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                acc[0] = mfma16(ha[0][u][s], w[NW * bi + u][s], acc[0]);
                if (RB == 2) acc[1] = mfma16(ha[1][u][s], w[NW * bi + u][s], acc[1]);
            }
        const int cb = CB * g + bi;
        if (cb < nbw) {
            const int col = 16 * (cb0 + cb) + j;
#pragma unroll
            for (int b = 0; b < RB; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (yoff[b][r] >= 0) {
                        if (CS) cstore(yp + yoff[b][r] + col, acc[b][r]);
                        else    yp[yoff[b][r] + col] = acc[b][r];
                    }
        }
    }
}

// Item (expert e, feature block fb) of workgroup b.  With E a multiple of 8
// an expert's items are the workgroups b = x + 8 j of one x, i.e. (as the
// hardware hands workgroups to the 8 XCDs in turn) all on one XCD, which
// shares the expert's staged activation rows in that XCD's L2 (measured 1.1-
// 1.6 us faster per 64-token, E = 16 layer than experts spread over XCDs).
__device__ inline void item_of(int b, int E, int nfb, int &e, int &fb) {
    if (E % 8 == 0) {
        const int x = b % 8, j = b / 8;
        e = x + 8 * (j / nfb);
        fb = j % nfb;
    } else {
        e = b / nfb;
        fb = b % nfb;
    }
}

// Where one gate/up item of NW waves reads its weights: expert e, features
// 16*NW*fb .. + 16*NW - 1 (16 per wave).  (e, fb and the wave index are
// uniform: weight addresses keep their common part in SGPRs, the lane's
// 16-byte column in lo.)
template <int NW>
struct ItemGeo {
    int lane, wave, j, h, f;
    WSrc gs, ds;
    int og, ou;           // gate / up rows of the wave's feature block
    int fq, nbw, last, ngd, od;
    int spread;
    DownHead<NW> dh;
    // Rotation of a gate/up chunk of nq steps: each wave starts its streams
    // at its own group (chunks of whole groups only), spreading the
    // concurrent reads over the memory system.
    __device__ int rot_of(int nq) const {
        const int ng = nq / Unroll<2>::kU;
        return nq % Unroll<2>::kU == 0 && ng >= 2 ? (5 * spread) % ng : 0;
    }
};

template <bool FUSED, int NW>
__device__ __forceinline__ ItemGeo<NW> item_geo(const DecodeArgs &a, int e, int fb) {
    static_assert(NW == 4 || NW == 8, "an item is 4 or 8 waves of 16 features");
    ItemGeo<NW> g;
    e = __builtin_amdgcn_readfirstlane(e);
    fb = __builtin_amdgcn_readfirstlane(fb);
    g.lane = threadIdx.x & 63;
    g.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const unsigned lo = 16u * g.lane;
    g.j = g.lane & 15;
    g.h = g.lane >> 4;
    const int m = NW * fb + g.wave;                 // this wave's 16-feature block
    g.f = 16 * m + g.j;
    // Gate rows of feature block m form unit row nbg (packed rows interleave
    // 32 gate and 32 up rows); up rows are 2 unit rows further.
    const int nbg = 4 * (m >> 1) + (m & 1);
    g.gs = wsrc(a.w + (size_t)e * 2 * a.F * a.d, (size_t)2 * a.F * a.d, lo);
    g.og = kUnitBytes * nbg * (a.d / 16);
    g.ou = g.og + kUnitBytes * 2 * (a.d / 16);
    // Down weights (FUSED): wave w's 16-column blocks w*nbw .. of the
    // expert's W_down, this item's NW feature units.
    g.fq = a.F / 16;
    g.nbw = a.d / (16 * NW);                        // 16-column blocks per wave
    g.last = NW * g.nbw - 1;
    g.ngd = (NW * g.nbw + 7) / 8;
    g.ds = wsrc(FUSED ? a.w2 + (size_t)e * a.d * a.F : a.w, (size_t)a.d * a.F, lo);
    g.od = kUnitBytes * ((g.wave * g.nbw) * g.fq + NW * fb);
    g.spread = NW * (e * (a.F / (16 * NW)) + fb) + g.wave;
    g.dh = DownHead<NW>{g.ds, g.od, g.fq, g.last, g.ngd >= 2 ? (3 * g.spread) % g.ngd : 0, g.ngd};
    return g;
}

// The fused item's down projection for one pass of rows list[r0 ..
// r0 + rows): the gate/up accumulators become the H block [rows][16 * NW] in
// LDS at hs, which multiplies the matching rows of W_down; the split-K
// partial goes to Yp[fb][a][0 .. d) by assignment a (CS: write-through
// stores).  wa / wb arrive holding the down stream's first two groups.
template <int NW, bool CS>
__device__ __forceinline__ void fused_down_pass(const DecodeArgs &a, const ItemGeo<NW> &g, int fb,
                                       const floatx4 (&acc)[2][2], int rows, const int *list,
                                       int r0, float *hs, WGroup<2> &wa, WGroup<2> &wb) {
    const int j = g.j, h = g.h;
    // The gate/up weight registers carry the down stream.
    floatx4 (&da)[8] = reinterpret_cast<floatx4 (&)[8]>(wa);
    floatx4 (&db)[8] = reinterpret_cast<floatx4 (&)[8]>(wb);
    // (every wave is past the activation rows, which hs may overlay)
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0) only
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            hs[(b * 16 + 4 * h + r) * hld<NW>() + g.wave * 16 + j] =
                swiglu_fast(acc[b][0][r], acc[b][1][r]);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    const float *as = hs + j * hld<NW>() + 4 * h;
    // Partial offsets fit in 32 bits: the host caps the partial buffer.
    int yoff[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = b * 16 + 4 * h + r;
            yoff[b][r] = row < rows ? (fb * a.nslots + list[r0 + row]) * a.d : -1;
        }
    const int cb0 = g.wave * g.nbw, nbw = g.nbw, ngd = g.ngd;
    const DownHead<NW> &dh = g.dh;
    auto run = [&](auto rb) {
        constexpr int RB = decltype(rb)::value;
        int q = 0;
        for (; q + 4 <= ngd; q += 2) {
            dgroup<RB, NW, CS>(da, as, dh.rot(q), nbw, cb0, yoff, a.out, j);
            __builtin_amdgcn_sched_barrier(0);
            dload<NW>(g.ds, g.od, g.fq, dh.rot(q + 2), g.last, da);
            __builtin_amdgcn_sched_barrier(0);
            dgroup<RB, NW, CS>(db, as, dh.rot(q + 1), nbw, cb0, yoff, a.out, j);
            __builtin_amdgcn_sched_barrier(0);
            dload<NW>(g.ds, g.od, g.fq, dh.rot(q + 3), g.last, db);
            __builtin_amdgcn_sched_barrier(0);
        }
        const int left = ngd - q;
        if (left == 3) {
            dgroup<RB, NW, CS>(da, as, dh.rot(q), nbw, cb0, yoff, a.out, j);
            dload<NW>(g.ds, g.od, g.fq, dh.rot(q + 2), g.last, da);
            dgroup<RB, NW, CS>(db, as, dh.rot(q + 1), nbw, cb0, yoff, a.out, j);
            dgroup<RB, NW, CS>(da, as, dh.rot(q + 2), nbw, cb0, yoff, a.out, j);
        } else if (left == 2) {
            dgroup<RB, NW, CS>(da, as, dh.rot(q), nbw, cb0, yoff, a.out, j);
            dgroup<RB, NW, CS>(db, as, dh.rot(q + 1), nbw, cb0, yoff, a.out, j);
        } else if (left == 1) {
            dgroup<RB, NW, CS>(da, as, dh.rot(q), nbw, cb0, yoff, a.out, j);
        }
    };
    if (rows > 16) run(std::integral_constant<int, 2>{});
    else           run(std::integral_constant<int, 1>{});
}

// One gate/up item of NW waves: expert e, features 16*NW*fb .. + 16*NW - 1
// (16 per wave).  FUSED = false: writes H [n x F] by assignment.  FUSED =
// true: keeps the item's H columns in LDS and multiplies them by the matching
// rows of W_down, writing the split-K partial Yp[fb][a][0 .. d) (the combine
// adds the F/(16*NW) partials in order).  xs: the dynamic LDS (rows, slot
// list, token list); wcnt: NW ints of LDS.  CS: partials go out with
// coherent (write-through) stores.
template <bool FUSED, int NW = 4, bool CS = false>
__device__ void gateup_item(const DecodeArgs &a, int e, int fb, float *xs, int *wcnt) {
    int *list = reinterpret_cast<int *>(xs + kRows * kLd);
    int *tok = list + a.nslots;
    const ItemGeo<NW> g = item_geo<FUSED, NW>(a, e, fb);
    const int j = g.j, h = g.h;

    // The slot list first (its loads are not queued behind weight loads),
    // then per chunk the activation rows (DMA), the first two weight groups
    // and a wait for the rows only.
    WGroup<2> wa, wb;
    const int id0 = (int)threadIdx.x < a.nslots ? a.ids[threadIdx.x] : -1;
    const int cnt = expert_slots<NW>(a.ids, a.nslots, e, id0, a.topk, list, tok, wcnt);
    if (cnt == 0) return;
    for (int r0 = 0; r0 < cnt; r0 += kRows) {
        const int rows = min(kRows, cnt - r0);
        floatx4 acc[2][2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int q = 0; q < 2; ++q) acc[b][q] = floatx4{0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < a.d; k0 += kChunk) {
            const int kc = min(kChunk, a.d - k0);
            __syncthreads();   // every wave is done with the previous rows
            stage_lds<NW>(xs, a.x, a.d, tok, r0, rows, k0, kc);
            // The counted wait below takes the rows' DMA as issued before the
            // weight loads, and other waves read those rows after the barrier:
            // keep the compiler from moving weight loads above the DMA.
            __builtin_amdgcn_sched_barrier(0);
            const int g0 = g.rot_of(kc / 16);
            gemv_prime<2>(g.gs, g.og + 64 * k0, g.ou + 64 * k0, kc / 16, wa, wb, g0);
            WAIT_VMCNT(4 * Unroll<2>::kU);   // the rows, not the weights behind them
            __builtin_amdgcn_s_barrier();   // (a fence here would wait for the weights too)
            dma_landed(xs);
            const float *as0 = xs + j * kLd + 4 * h, *as1 = as0 + 16 * kLd;
            const int go = g.og + 64 * k0, uo = g.ou + 64 * k0;   // (16 floats per K column)
            if (FUSED && k0 + kc == a.d) {   // last chunk: hand over to the down stream
                if (rows > 16)
                    gemv_loop<2, 2, true, NW>(g.gs, go, uo, as0, as1, kc / 16, acc, wa, wb, g.dh, g0);
                else
                    gemv_loop<2, 1, true, NW>(g.gs, go, uo, as0, as1, kc / 16, acc, wa, wb, g.dh, g0);
            } else {
                if (rows > 16)
                    gemv_loop<2, 2, false, NW>(g.gs, go, uo, as0, as1, kc / 16, acc, wa, wb, g.dh, g0);
                else
                    gemv_loop<2, 1, false, NW>(g.gs, go, uo, as0, as1, kc / 16, acc, wa, wb, g.dh, g0);
            }
        }
        // 16x16 accumulator: lane holds rows 4*(lane/16) + r, column lane%16.
        if (!FUSED) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = b * 16 + 4 * h + r;
                    if (row < rows)
                        a.out[(size_t)list[r0 + row] * a.F + g.f] =
                            swiglu_fast(acc[b][0][r], acc[b][1][r]);
                }
            continue;
        }
        // (the next pass, if any, primes the gate/up groups again)
        fused_down_pass<NW, CS>(a, g, fb, acc, rows, list, r0, xs, wa, wb);
    }
}


}  // namespace
}  // namespace moe
