// gemm.hip — grouped expert GEMMs on the fp32 matrix cores of gfx950, plus
// the combine, weight packing and synthetic fill kernels.
//
// Layout (device, packed once at upload), per expert a matrix of N packed
// rows by K, stored as 16 x 16 tiles ("units", 1 KB) in MFMA operand order:
//   unit (nb, qb) at ((nb * K/16) + qb) * 256 floats holds rows
//   16nb..16nb+15, k = 16qb..16qb+15; element (row 16nb + j, k = 16qb + 4h + s)
//   sits at h*64 + j*4 + s, so lane 16h + j of a wave loads its 16-byte
//   piece at lane*4 and one wave instruction reads one contiguous unit; the
//   units of one row block follow each other along K.
//   gate/up  wgu [E][2F rows][d]: packed rows 64*fb + c hold gate feature
//            32*fb + c (c < 32) and up feature 32*fb + c - 32 (c >= 32).
//   down     wdT [E][d rows][F]: row n holds W_down[:, n].
// The rows of one expert's m-tile are consecutive dispatch positions
// offsets[e] + m; gate/up gathers them straight from x through perm.
//
// Work decomposition: the grid enumerates (m-tile, n-tile) pairs over the
// flat per-expert m-tile list built by the dispatch kernel (tile_off), so a
// hot expert simply owns more tiles; blocks past the live tile count exit.
//
// Each workgroup computes a 128 x (64*WN) tile with 2 x WN waves of 64 x 64.
// A wave issues v_mfma_f32_32x32x2f32 on 2 x 2 sub-tiles.  K is staged
// through LDS in 32-wide slices (three buffers for 256-column tiles, two for
// narrower ones); a lane of half h (lane/32) feeds the MFMA's k-row h with
// the slice's elements 16h..16h+15 in turn, so both operands come from LDS
// as 128-bit reads.
// Both operands go global -> LDS by DMA (global_load_lds_dwordx4, one wave
// instruction = 64 lanes x 16 bytes into 1 KB of LDS), one or two slices
// ahead of the MFMAs: no registers or LDS store instructions carry the tiles.
//   B  the packed 1 KB units are copied whole (unit layout in LDS);
//   A  a unit is 8 whole gathered rows (128 B each, full cache lines), each
//      row's eight 16-byte chunks permuted by XOR with row % 8 so the
//      fragment reads are free of bank conflicts.
// Measured on the gate/up GEMM of the large layer (ms): register staging
// with the fill in one burst 35.3, spread over the slice 34.5, B by DMA 33.8,
// both by DMA 33.1.  The DMA is waited for explicitly (vmcnt) before the
// barrier that ends the slice: s_barrier orders LDS accesses, not loads in
// flight.
// Fragments: a wave reads the slice's four quarter-steps into four register
// sets, set q + 1 while set q's MFMAs run; the last quarter's MFMAs run
// after the barrier, under the next slice's first reads.  A register that an
// MFMA still in the pipe reads is never written meanwhile (such a write
// waits for that MFMA to complete, draining the pipe): 33.0 -> 32.6 ms.
#include "moe_internal.h"
#include "moe_math.h"
#include "synth.h"
#include <algorithm>
#include <type_traits>

namespace moe {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = kGemmBM;   // 128
constexpr int KT = 32;
// LDS buffers per operand: three for 256-column tiles (144 KB, one
// workgroup per CU either way), two for narrower tiles (whose workgroups
// share a CU).
constexpr int gemm_stages(int wn) { return wn == 4 ? 3 : 2; }

// One wave instruction of LDS DMA: lane i's 16 bytes at g go to LDS byte
// address lds + 16 i (lds wave-uniform, passed in M0).  Written as asm: the
// compiler books its own LDS DMA builtin as an LDS access as well as a
// vector load, and then waits for every LDS read with lgkmcnt(0) while a DMA
// is in flight, which would stall each fragment read ahead.  The DMA counts
// on vmcnt only, and every slice waits for it (GEMM_WAIT_VMCNT) before the
// barrier after which its LDS is read.
__device__ __forceinline__ void gemm_dma16(const float *g, unsigned lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(g), "{m0}"(lds) : "memory");
}
// An empty use of four fragments: keeps their registers allocated (and so
// not reused) up to this point.
__device__ __forceinline__ void keep_regs(floatx4 a, floatx4 b, floatx4 c, floatx4 d) {
    asm volatile("" :: "v"(a), "v"(b), "v"(c), "v"(d));
}
// s_waitcnt limiting only the vector-memory count (expcnt, lgkmcnt at max).
#define GEMM_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | 0x0F70)

// One tile (m-tile mtg, n-tile nt) over the nk K slices from element kb;
// the down projection writes its partial to slot `slot` (c + slot *
// split_stride) and, with npieces > 0, records npieces for the tile's rows.
// Every thread of the workgroup calls this together.
template <int MODE, int WN>
__device__ __forceinline__ void gemm_tile(const GemmArgs &a, float *smem, int mtg, int nt, int kb,
                                          int nk, int slot, int npieces, float *part = nullptr) {
    constexpr int BN = 64 * WN;
    constexpr int ST = gemm_stages(WN);
    // ST buffers each: A as 128 rows of 32 swizzled floats, B as
    // (BN/16) x 2 packed 1 KB units (BN rows of 32 floats' worth).
    float *As = smem;
    float *Bs = smem + ST * BM * KT;
    const int e = a.tile_expert[mtg];
    const int row0 = a.offsets[e] + (mtg - a.tile_off[e]) * BM;
    const int rows = min(BM, a.offsets[e + 1] - row0);
    const int K = a.K;
    const float *B = a.b + (size_t)e * a.N * K;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    // Waves are dealt to the 4 SIMDs in turn, so with 8 waves SIMD s runs
    // waves s and s + 4; wm = wave / WN makes them an upper-half and a
    // lower-half wave.  When an expert's last tile is short, the MFMAs the
    // lower-half wave skips leave its SIMD to the upper-half wave.
    const int wm = wave / WN, wn = wave % WN;
    // Valid 32-row MFMA blocks of this wave (0, 1 or 2); uniform per wave.
    const int nmb = max(0, min(2, (rows - wm * 64 + 31) / 32));
    const int li = lane & 31, lh = lane >> 5;

    // Rows past the expert's last row reuse its last row: their accumulator
    // rows are never stored, and every DMA lane stays in bounds.
    // A tile = 16 units of 8 whole rows (32 floats = 128 B each), copied by
    // LDS DMA: lane i of a unit's DMA brings row i / 8's 16-byte chunk
    // (i % 8) ^ (row % 8), so row r's chunk c sits at r * 32 + 4 (c ^ (r % 8))
    // floats and the fragment reads below are free of bank conflicts.
    constexpr int AUW = (BM / 8) / (2 * WN);
    const int wu = __builtin_amdgcn_readfirstlane(wave);   // (uniform: LDS DMA bases)
    const unsigned lds0 = __builtin_amdgcn_readfirstlane(
        (unsigned)(size_t)(const __attribute__((address_space(3))) float *)smem);
    const float *a_src[AUW];
#pragma unroll
    for (int i = 0; i < AUW; ++i) {
        const int r = 8 * (wu * AUW + i) + (lane >> 3);
        const int c = (lane & 7) ^ (r & 7);
        const int rr = min(r, rows - 1);
        size_t src_row;
        if (MODE == 0 || MODE == 2) src_row = (size_t)(a.perm[row0 + rr] / a.topk);
        else           src_row = (size_t)(row0 + rr);
        a_src[i] = a.a + src_row * K + 4 * c;
    }
    auto adma = [&](int k0, int buf) {
#pragma unroll
        for (int i = 0; i < AUW; ++i)
            gemm_dma16(a_src[i] + k0, lds0 + 4u * (buf * BM * KT + (wu * AUW + i) * 256));
    };
    // B tile = (BN/16) x 2 units, copied whole by LDS DMA: wave w the units
    // w * BUW .. in the packed unit layout (unit u at u * 256 floats).
    constexpr int BUW = (BN / 16 * 2) / (2 * WN);
    const float *b_src[BUW];
#pragma unroll
    for (int i = 0; i < BUW; ++i) {
        const int u = wu * BUW + i, nbl = u >> 1, qbl = u & 1;
        b_src[i] = B + ((size_t)(nt * (BN / 16) + nbl) * (K / 16) + qbl) * 256 + 4 * lane;
    }
    auto bdma = [&](int k0, int buf) {
#pragma unroll
        for (int i = 0; i < BUW; ++i)
            gemm_dma16(b_src[i] + (size_t)16 * k0,
                       lds0 + 4u * (ST * BM * KT + buf * BN * KT + (wu * BUW + i) * 256));
    };
    // Slice j of the tile into buffer j % ST.  With three buffers slice
    // kt + 2 is issued during slice kt, so before the barrier that ends
    // slice kt only the wave's newest NDMA transfers may still be in
    // flight.
    constexpr int NDMA = AUW + BUW;
    auto dma = [&](int j, int buf) {
        adma(kb + j * KT, buf);
        bdma(kb + j * KT, buf);
    };
    auto wait_next = [&](int kt) {
        if (ST == 3 && kt + 2 < nk) GEMM_WAIT_VMCNT(NDMA);
        else GEMM_WAIT_VMCNT(0);
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[m][n][r] = 0.0f;

    dma(0, 0);
    if (ST == 3 && nk > 1) {
        dma(1, 1);
        GEMM_WAIT_VMCNT(NDMA);
    } else {
        GEMM_WAIT_VMCNT(0);
    }
    __syncthreads();
    // Row (li) of this lane's A blocks has r % 8 = li % 8: the 16-byte chunk
    // 4 lh + q of K step q sits at 4 ((4 lh + q) ^ (li % 8)) floats.
    int aoff[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) aoff[q] = 4 * ((4 * lh + q) ^ (li & 7));
    if (nmb == 2) {
        // Set q holds quarter-step q's fragments (a0, a1 of the two 32-row
        // blocks, b0, b1 of the two 32-column blocks).  Order per slice:
        // read set 1, MFMAs of set 0, read set 2, MFMAs of set 1, read set 3,
        // issue the DMA of slice kt + ST - 1, MFMAs of set 2, wait for the
        // next slice, barrier, read the next slice's set 0, MFMAs of set 3.
        // keep() holds set q's registers until the following quarter's
        // MFMAs have issued: they wait on set q's results, so by then no
        // MFMA reads set q and it can be refilled.  The DMA goes out after
        // the slice's last fragment reads: LDS reads issued behind an LDS
        // DMA of the same wave measured slower (the loop took 3 % longer
        // with the DMA at the top of the slice).
        floatx4 fa0[4], fa1[4], fb0[4], fb1[4];
        const float *ap = As + (wm * 64 + li) * KT;
        const float *bp = Bs + ((wn * 4 + (li >> 4)) * 2 + lh) * 256 + (li & 15) * 4;
        auto rd = [&](auto bufc, auto qc) {
            constexpr int buf = decltype(bufc)::value, q = decltype(qc)::value;
            fa0[q] = *reinterpret_cast<const floatx4 *>(ap + buf * BM * KT + aoff[q]);
            fa1[q] = *reinterpret_cast<const floatx4 *>(ap + buf * BM * KT + 32 * KT + aoff[q]);
            fb0[q] = *reinterpret_cast<const floatx4 *>(bp + buf * BN * KT + 64 * q);
            fb1[q] = *reinterpret_cast<const floatx4 *>(bp + buf * BN * KT + 4 * 256 + 64 * q);
        };
        auto mm = [&](auto qc) {
            constexpr int q = decltype(qc)::value;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[q][s], fb0[q][s], acc[0][0], 0, 0, 0);
                acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[q][s], fb1[q][s], acc[0][1], 0, 0, 0);
                acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[q][s], fb0[q][s], acc[1][0], 0, 0, 0);
                acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[q][s], fb1[q][s], acc[1][1], 0, 0, 0);
            }
        };
        auto keep = [&](auto qc) {
            constexpr int q = decltype(qc)::value;
            keep_regs(fa0[q], fa1[q], fb0[q], fb1[q]);
        };
        using Q0 = std::integral_constant<int, 0>;
        using Q1 = std::integral_constant<int, 1>;
        using Q2 = std::integral_constant<int, 2>;
        using Q3 = std::integral_constant<int, 3>;
        // One slice from LDS buffer buf (a constant, so every fragment
        // address is a register plus an immediate offset).  The scheduling
        // barriers keep the reads ahead of the MFMAs they overlap.
        auto slice = [&](int kt, auto bufc) {
            constexpr int buf = decltype(bufc)::value;
            rd(bufc, Q1{});
            __builtin_amdgcn_sched_barrier(0);
            mm(Q0{});
            keep(Q3{});
            __builtin_amdgcn_sched_barrier(0);
            rd(bufc, Q2{});
            __builtin_amdgcn_sched_barrier(0);
            mm(Q1{});
            keep(Q0{});
            __builtin_amdgcn_sched_barrier(0);
            rd(bufc, Q3{});
            __builtin_amdgcn_sched_barrier(0);
            if (kt + ST - 1 < nk) dma(kt + ST - 1, (buf + ST - 1) % ST);
            __builtin_amdgcn_sched_barrier(0);
            mm(Q2{});
            keep(Q1{});
            __builtin_amdgcn_sched_barrier(0);
            wait_next(kt);   // slice kt + 1 has landed
            __syncthreads();
            if (kt + 1 < nk) rd(std::integral_constant<int, (buf + 1) % ST>{}, Q0{});
            __builtin_amdgcn_sched_barrier(0);
            mm(Q3{});
            keep(Q2{});
            __builtin_amdgcn_sched_barrier(0);
        };
#pragma unroll
        for (int q = 1; q < 4; ++q) fa0[q] = fa1[q] = fb0[q] = fb1[q] = floatx4{0.f, 0.f, 0.f, 0.f};
        rd(Q0{}, Q0{});
        for (int kt = 0; kt < nk; kt += ST) {
            slice(kt, Q0{});
            if (kt + 1 < nk) slice(kt + 1, Q1{});
            if (ST == 3 && kt + 2 < nk) slice(kt + 2, std::integral_constant<int, 2 % ST>{});
        }
    } else {
        // One 32-row block (the expert's last, short tile) or none.
        for (int kt = 0; kt < nk; ++kt) {
            const int buf = kt % ST;
            // Slice kt + ST - 1 into the buffer slice kt - 1 used (free since
            // the barrier that ended slice kt - 1), in flight meanwhile.
            if (kt + ST - 1 < nk) dma(kt + ST - 1, (kt + ST - 1) % ST);
            const float *as = As + buf * BM * KT + (wm * 64 + li) * KT;
            const float *bs = Bs + buf * BN * KT + ((wn * 4 + (li >> 4)) * 2 + lh) * 256 + (li & 15) * 4;
            if (nmb == 1) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    floatx4 a0 = *reinterpret_cast<const floatx4 *>(as + aoff[q]);
                    floatx4 b0 = *reinterpret_cast<const floatx4 *>(bs + 64 * q);
                    floatx4 b1 = *reinterpret_cast<const floatx4 *>(bs + 4 * 256 + 64 * q);
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[s], b0[s], acc[0][0], 0, 0, 0);
                        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[s], b1[s], acc[0][1], 0, 0, 0);
                    }
                }
            }
            wait_next(kt);   // slice kt + 1 has landed
            __syncthreads();
        }
    }

    // Accumulator layout of a 32x32 block: lane l, register r holds
    // row 8*(r/4) + 4*(l/32) + (r%4), column l%32.
    if (MODE != 1 && part) {
        // A piece of a split tile: raw sums, [row][tile column].
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                int row = wm * 64 + m * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (row < rows)
#pragma unroll
                    for (int n = 0; n < 2; ++n)
                        part[row * BN + wn * 64 + n * 32 + li] = acc[m][n][r];
            }
    } else if (MODE == 0) {
        const int f = ((nt * BN + wn * 64) >> 1) + li;   // feature index
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                int row = wm * 64 + m * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (row < rows)
                    a.c[(size_t)(row0 + row) * a.ldc + f] = swiglu_fast(acc[m][0][r], acc[m][1][r]);
            }
    } else if (MODE == 2) {
        // Raw gate and up columns (packed order, dispatch-ordered rows) and H.
        const int f = ((nt * BN + wn * 64) >> 1) + li;
        const int col = nt * BN + wn * 64 + li;
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                int row = wm * 64 + m * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (row < rows) {
                    const size_t p = (size_t)(row0 + row);
                    const float g = acc[m][0][r], u = acc[m][1][r];
                    a.c[p * a.ldc + col] = g;
                    a.c[p * a.ldc + col + 32] = u;
                    a.c2[p * a.ldc2 + f] = swiglu_fast(g, u);
                }
            }
    } else if (MODE == 3) {
        // acc = dH for features f = nt*BN + wn*64 + 32n + li; the gate and up
        // values of f sit at packed columns 64(f/32) + f%32 and 32 past it,
        // and are replaced by dG = dH u silu'(g), dU = dH silu(g).
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                int row = wm * 64 + m * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (row < rows) {
                    float *gu = a.c + (size_t)(row0 + row) * a.ldc;
#pragma unroll
                    for (int n = 0; n < 2; ++n) {
                        const int col = 2 * (nt * BN + wn * 64) + 64 * n + li;
                        const float g = gu[col], u = gu[col + 32], dh = acc[m][n][r];
                        const float sg = 1.0f / (1.0f + expf(-g));
                        gu[col] = dh * u * fmaf(g * sg, 1.0f - sg, sg);
                        gu[col + 32] = dh * g * sg;
                    }
                }
            }
    } else {
        float *c = a.c + (size_t)slot * a.split_stride;
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                int row = wm * 64 + m * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (row < rows) {
                    size_t dst = (size_t)a.perm[row0 + row] * a.ldc;
#pragma unroll
                    for (int n = 0; n < 2; ++n)
                        c[dst + nt * BN + wn * 64 + n * 32 + li] = acc[m][n][r];
                }
            }
        if (npieces > 0)
            for (int r = tid; r < rows; r += 128 * WN)
                a.pieces[(size_t)a.perm[row0 + r] * (a.N / BN) + nt] = npieces;
    }
}

// The split tail of a gate/up launch: whole tiles [0, dp); r tiles left over
// (dp .. dp + r - 1), each in s pieces; r = s = 0 when the tail is not split.
struct TailLayout { int dp, r, s; };
__device__ __forceinline__ TailLayout tail_layout(const GemmArgs &a, int ntiles, int nks) {
    const int live = a.tile_off[a.E] * ntiles;
    const int g = a.tail_groups;
    const int r = live % g;
    const int sp = r ? min(min(nks, 4), g / r) : 0;
    if (sp < 2) return TailLayout{live, 0, 0};
    return TailLayout{live - r, r, sp};
}

// Grid: the (m-tile, n-tile) pairs, times the reduction splits.  Down
// projection in stream-K form (a.streamk): workgroup g takes units
// [g per, (g + 1) per) of the flat list of (live tile, K slice) units, per =
// ceil(units / grid); each tile it touches is a piece whose index within
// the tile (0 for the workgroup holding the tile's first slice) is the
// partial slot it writes, and piece 0 records the tile's piece count for
// the combine.  Slots, pieces and counts follow from the live tile count
// alone, so results are deterministic.
template <int MODE, int WN>
__global__ __launch_bounds__(128 * WN) void grouped_gemm_kernel(GemmArgs a) {
    constexpr int BN = 64 * WN;
    extern __shared__ __align__(16) float smem[];
    const int ntiles = a.N / BN;
    const int nks = a.K / KT;
    if (MODE == 1 && a.streamk) {
        const long units = (long)a.tile_off[a.E] * ntiles * nks;
        const long per = (units + gridDim.x - 1) / gridDim.x;
        long u = (long)blockIdx.x * per;
        const long uend = u + per < units ? u + per : units;
        while (u < uend) {
            const int tile = (int)(u / nks);
            const int k0 = (int)(u - (long)tile * nks);
            const int k1 = (int)(k0 + (uend - u) < nks ? k0 + (uend - u) : nks);
            const long tstart = (long)tile * nks;
            const int first = (int)(tstart / per);   // workgroup of the tile's first slice
            const int slot = (int)blockIdx.x - first;
            const int npieces = (int)((tstart + nks - 1) / per) - first + 1;
            gemm_tile<MODE, WN>(a, smem, tile / ntiles, tile % ntiles, k0 * KT, k1 - k0, slot,
                                slot == 0 ? npieces : 0);
            u += k1 - k0;
        }
        return;
    }
    if (MODE != 1 && a.tail_groups > 0) {
        // Whole tiles in the grid's first dp workgroups, then the pieces of
        // the split tail: piece s of tail tile r covers K slices
        // [s nks / S, (s + 1) nks / S).  (Grid: the m-tile bound's tiles plus
        // tail_groups.)
        const TailLayout tl = tail_layout(a, ntiles, nks);
        const int b = blockIdx.x;
        if (b < tl.dp) {
            gemm_tile<MODE, WN>(a, smem, b / ntiles, b % ntiles, 0, nks, 0, 0);
            return;
        }
        const int j = b - tl.dp;
        if (j >= tl.r * tl.s) return;
        const int r = j / tl.s, sp = j - r * tl.s;
        const int tile = tl.dp + r;
        const int k0 = sp * nks / tl.s, k1 = (sp + 1) * nks / tl.s;
        gemm_tile<MODE, WN>(a, smem, tile / ntiles, tile % ntiles, k0 * KT, k1 - k0, 0, 0,
                            a.tail_part + (size_t)j * BM * BN);
        return;
    }
    const int per_split = a.max_mtiles * ntiles;
    const int ks = blockIdx.x / per_split;       // reduction split (down projection)
    const int nt = (blockIdx.x % per_split) % ntiles;
    int mtg = (blockIdx.x % per_split) / ntiles;
    if (mtg >= a.tile_off[a.E]) return;
    if (a.order) mtg = a.order[mtg];
    const int nk = nks / a.ksplit;   // K steps of this split
    gemm_tile<MODE, WN>(a, smem, mtg, nt, ks * nk * KT, nk, ks, 0);
}

template <int MODE, int WN>
hipError_t launch_grouped(const GemmArgs &a, hipStream_t s) {
    constexpr int BN = 64 * WN;
    const size_t lds = (size_t)gemm_stages(WN) * (BM + BN) * KT * sizeof(float);
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t err = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&grouped_gemm_kernel<MODE, WN>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (err != hipSuccess) return err;
        attr_set = true;
    }
    const int ntiles = a.N / BN;
    dim3 grid((unsigned)(a.max_mtiles * ntiles * a.ksplit + (MODE != 1 ? a.tail_groups : 0)));
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE, WN>), grid, dim3(128 * WN), lds, s, a);
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_mode(const GemmArgs &a, hipStream_t s) {
    const GemmPlan pl = gemm_plan(a.N, a.K, a.max_mtiles, MODE == 1);
    if (a.ksplit != (MODE == 1 ? pl.ksplit : 1)) return hipErrorInvalidValue;
    switch (pl.bn) {
        case 256: return launch_grouped<MODE, 4>(a, s);
        case 128: return launch_grouped<MODE, 2>(a, s);
        case 64:  return launch_grouped<MODE, 1>(a, s);
        default:  return hipErrorInvalidValue;
    }
}

// out[t] = sum over slots of gw * y, one FMA per slot in slot order
// (src/transformer.c:355-358 after contraction), optionally added into out.
// With ksplit > 1 each slot's y is the sum of its split partials, added in
// split order (with pieces: as many as its column block's tile had).  With
// PARTS (ksplit > 1 or pieces) the first 8 partials of a slot are loaded
// together (clamped, masked), and with KS > 0 (k = KS) every slot's loads
// go out before the first sum, so no load waits for another.
template <int KS, bool PARTS>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    constexpr int KB = KS > 0 ? KS : 1;   // slots whose loads go out together
    constexpr int NQ = PARTS ? 8 : 1;     // partials loaded together
    const int d4 = a.d >> 2;
    const size_t total = (size_t)a.T * d4;
    const int k = KS > 0 ? KS : a.k;
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        const int t = (int)(i / d4), c = (int)(i % d4);
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < k; k0 += KB) {
            floatx4 q[KB][NQ];
            float w[KB];
            int np[KB];
            const float *yp[KB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const size_t slot = (size_t)t * a.k + k0 + kb;
                w[kb] = a.gw[slot];
                yp[kb] = a.ys + slot * a.d + 4 * c;
                np[kb] = !PARTS ? 1
                         : a.pieces ? a.pieces[slot * (a.d / a.pieces_cols) + 4 * c / a.pieces_cols]
                                    : a.ksplit;
                np[kb] = max(np[kb], 1);
#pragma unroll
                for (int u = 0; u < NQ; ++u)
                    q[kb][u] = *reinterpret_cast<const floatx4 *>(
                        yp[kb] + (size_t)min(u, np[kb] - 1) * a.split_stride);
            }
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                floatx4 y = q[kb][0];
#pragma unroll
                for (int u = 1; u < NQ; ++u)
                    if (u < np[kb])
#pragma unroll
                        for (int j = 0; j < 4; ++j) y[j] = y[j] + q[kb][u][j];
                for (int sp = NQ; sp < np[kb]; ++sp) {
                    const floatx4 p = *reinterpret_cast<const floatx4 *>(
                        yp[kb] + (size_t)sp * a.split_stride);
#pragma unroll
                    for (int j = 0; j < 4; ++j) y[j] = y[j] + p[j];
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[j] = fmaf(w[kb], y[j], acc[j]);
            }
        }
        floatx4 *o = reinterpret_cast<floatx4 *>(a.out + (size_t)t * a.d + 4 * c);
        if (a.accumulate) {
            floatx4 v = *o;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = v[j] + acc[j];
            *o = v;
        } else {
            *o = acc;
        }
    }
}

// The same for many split-K partials (the fused decode kernel writes one per
// 64 features): G lanes share an output float4, each summing up to 8
// consecutive partials of a slot in split order (PL: 2 for steps of a few
// tokens, so that more workgroups share the loads); lane 0 adds the G group
// sums in a fixed tree order and applies the slot's gate weight.  KS > 0:
// k = KS at compile time, and every load of the lane (partials, gate
// weights, the accumulated output) is issued before the first sum.
template <int G, int KS, int PL = 8>
__global__ __launch_bounds__(256) void combine_groups_kernel(CombineArgs a) {
    constexpr int KB = KS > 0 ? KS : 1;   // slots whose loads go out together
    const int d4 = a.d >> 2;
    const size_t gid = ((size_t)blockIdx.x * 256 + threadIdx.x) / G;
    const int g = threadIdx.x % G;
    const bool valid = gid < (size_t)a.T * d4;
    const int t = valid ? (int)(gid / d4) : 0, c4 = valid ? (int)(gid % d4) : 0;
    const int s0 = PL * g, s1 = min(s0 + PL, a.ksplit);
    const int k = KS > 0 ? KS : a.k;
    floatx4 *o = reinterpret_cast<floatx4 *>(a.out + (size_t)t * a.d + 4 * c4);
    floatx4 prev = {0.f, 0.f, 0.f, 0.f};
    if (KS > 0 && a.accumulate && g == 0) prev = *o;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < k; k0 += KB) {
        floatx4 p[KB][PL];
        float w[KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const float *yp = a.ys + ((size_t)t * a.k + k0 + kb) * a.d + 4 * c4;
#pragma unroll
            for (int u = 0; u < PL; ++u)
                p[kb][u] = *reinterpret_cast<const floatx4 *>(
                    yp + (size_t)min(s0 + u, a.ksplit - 1) * a.split_stride);
            w[kb] = a.gw[(size_t)t * a.k + k0 + kb];
        }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            floatx4 y = {0.f, 0.f, 0.f, 0.f};
            if (s0 < s1) y = p[kb][0];
#pragma unroll
            for (int u = 1; u < PL; ++u)
                if (s0 + u < s1)
#pragma unroll
                    for (int j = 0; j < 4; ++j) y[j] = y[j] + p[kb][u][j];
#pragma unroll
            for (int m = G / 2; m >= 1; m >>= 1)
#pragma unroll
                for (int j = 0; j < 4; ++j) y[j] = y[j] + __shfl_xor(y[j], m, G);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = fmaf(w[kb], y[j], acc[j]);
        }
    }
    if (valid && g == 0) {
        if (a.accumulate) {
            floatx4 v = KS > 0 ? prev : *o;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = v[j] + acc[j];
            *o = v;
        } else {
            *o = acc;
        }
    }
}

// Packs source matrix src [K x N] (reference layout) into the unit layout
// (unpack != 0: the inverse).  Source column c goes to packed row
// c (mode 0, down), 64*(c/32) + c%32 (mode 1, gate) or that + 32 (mode 2,
// up).  One workgroup moves a 32 x 32 block = 4 units through LDS; grid z
// runs over experts whose matrices are src_e and dst_e floats apart.
__global__ __launch_bounds__(256) void pack_kernel(float *src, float *dst, int K, int N,
                                                    int mode, int unpack, size_t src_e = 0,
                                                    size_t dst_e = 0) {
    __shared__ float tile[32][33];
    src += blockIdx.z * src_e;
    dst += blockIdx.z * dst_e;
    const int c0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    const int row0 = mode == 0 ? c0 : 64 * (c0 >> 5) + (mode == 2 ? 32 : 0);
    const int t = threadIdx.x;
    const int h = t >> 6, j = (t >> 2) & 15, sx = t & 3;
    if (!unpack) {
        for (int r = ty; r < 32; r += 8) tile[r][tx] = src[(size_t)(k0 + r) * N + c0 + tx];
        __syncthreads();
        for (int u = 0; u < 4; ++u) {
            const int nbl = u >> 1, qbl = u & 1;
            const size_t unit = (size_t)((row0 >> 4) + nbl) * (K / 16) + (k0 >> 4) + qbl;
            dst[unit * 256 + t] = tile[qbl * 16 + 4 * h + sx][nbl * 16 + j];
        }
    } else {
        for (int u = 0; u < 4; ++u) {
            const int nbl = u >> 1, qbl = u & 1;
            const size_t unit = (size_t)((row0 >> 4) + nbl) * (K / 16) + (k0 >> 4) + qbl;
            tile[qbl * 16 + 4 * h + sx][nbl * 16 + j] = dst[unit * 256 + t];
        }
        __syncthreads();
        for (int r = ty; r < 32; r += 8) src[(size_t)(k0 + r) * N + c0 + tx] = tile[r][tx];
    }
}

// dst[e] = the transpose of src[e] in the unit layout: src [E][R rows][C],
// dst [E][C rows][R].  Four 16 x 16 units per workgroup, 64 threads each;
// thread q writes destination floats o = 4q..4q+3 of its unit (row 16rb + j,
// k = 16kb + 4h + s for o = 64h + 4j + s), read from source row
// 16kb + 4h + s, k = 16rb + j.
__global__ __launch_bounds__(256) void transpose_units_kernel(const float *src, float *dst, int R,
                                                              int C) {
    const int units = (R / 16) * (C / 16);
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (u >= units) return;
    const int rb = u % (C / 16), kb = u / (C / 16);
    const size_t base = (size_t)blockIdx.y * R * C;
    const int q = threadIdx.x & 63, h = q >> 4, j = q & 15;
    const float *sp = src + base + ((size_t)kb * (C / 16) + rb) * 256 + (j >> 2) * 64 + (j & 3);
    floatx4 v;
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) v[sl] = sp[(4 * h + sl) * 4];
    *reinterpret_cast<floatx4 *>(dst + base + ((size_t)rb * (R / 16) + kb) * 256 + 4 * q) = v;
}

__global__ __launch_bounds__(256) void fill_normal_kernel(float *dst, size_t n, uint64_t seed,
                                                           uint64_t stream_id, float mean,
                                                           float std) {
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        dst[i] = synth_normal(seed, stream_id, i, mean, std);
}

__global__ __launch_bounds__(256) void zero_ints_kernel(int *p, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0;
}

// Workgroup 8 r + q: rows 16 q .. 16 q + 15 of tail tile r of a launch with
// a split tail, one thread per (row, 4 columns in each 32-column half of a
// 64-column group).  The sums are the tile's S pieces added in piece order
// (loads of four pieces in flight at a time); the tile engine's epilogue of
// MODE then runs on them.
template <int MODE>
__global__ __launch_bounds__(512) void tail_fixup_kernel(GemmArgs a) {
    constexpr int BN = 256;
    const int ntiles = a.N / BN;
    const TailLayout tl = tail_layout(a, ntiles, a.K / KT);
    const int r = blockIdx.x >> 3;
    if (r >= tl.r) return;
    const int tile = tl.dp + r, mtg = tile / ntiles, nt = tile - mtg * ntiles;
    const int e = a.tile_expert[mtg];
    const int row0 = a.offsets[e] + (mtg - a.tile_off[e]) * BM;
    const int rows = min(BM, a.offsets[e + 1] - row0);
    const int row = 16 * (blockIdx.x & 7) + (threadIdx.x >> 5);
    if (row >= rows) return;
    const int g = (threadIdx.x >> 3) & 3, c = (threadIdx.x & 7) * 4;
    const float *src = a.tail_part + (size_t)r * tl.s * BM * BN + row * BN + 64 * g + c;
    constexpr size_t PS = (size_t)BM * BN;   // floats per piece
    // v0: columns 64 g + c .., v1: 32 further (gate and up, or dH of two
    // feature runs for MODE 3).
    floatx4 v0 = {0.f, 0.f, 0.f, 0.f}, v1 = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < tl.s; s0 += 4) {
        floatx4 p0[4], p1[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {   // (clamped: every load goes out together)
            const size_t sq = (size_t)min(s0 + q, tl.s - 1) * PS;
            p0[q] = *reinterpret_cast<const floatx4 *>(src + sq);
            p1[q] = *reinterpret_cast<const floatx4 *>(src + sq + 32);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (s0 + q < tl.s) {
                if (s0 + q == 0) { v0 = p0[0]; v1 = p1[0]; }
                else { v0 += p0[q]; v1 += p1[q]; }
            }
    }
    const size_t p = (size_t)(row0 + row);
    if (MODE == 0 || MODE == 2) {
        // Gate (v0) and up (v1) of features 128 nt + 32 g + c ..
        floatx4 h;
#pragma unroll
        for (int q = 0; q < 4; ++q) h[q] = swiglu_fast(v0[q], v1[q]);
        if (MODE == 0) {
            *reinterpret_cast<floatx4 *>(a.c + p * a.ldc + nt * (BN / 2) + 32 * g + c) = h;
        } else {
            float *gu = a.c + p * a.ldc + nt * BN + 64 * g + c;
            *reinterpret_cast<floatx4 *>(gu) = v0;
            *reinterpret_cast<floatx4 *>(gu + 32) = v1;
            *reinterpret_cast<floatx4 *>(a.c2 + p * a.ldc2 + nt * (BN / 2) + 32 * g + c) = h;
        }
    } else {
        // dH of features 256 nt + 64 g + 32 n + c .. (n = 0: v0, 1: v1); the
        // gate and up values of feature f sit at packed columns
        // 64 (f / 32) + f % 32 and 32 past it, replaced by dG and dU.
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            float *gu = a.c + p * a.ldc + 2 * (nt * BN + 64 * g) + 64 * n + c;
            const floatx4 dhv = n ? v1 : v0;
            floatx4 gv = *reinterpret_cast<const floatx4 *>(gu);
            floatx4 uv = *reinterpret_cast<const floatx4 *>(gu + 32);
            floatx4 dg, du;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float gq = gv[q], uq = uv[q], dh = dhv[q];
                const float sg = 1.0f / (1.0f + expf(-gq));
                dg[q] = dh * uq * fmaf(gq * sg, 1.0f - sg, sg);
                du[q] = dh * gq * sg;
            }
            *reinterpret_cast<floatx4 *>(gu) = dg;
            *reinterpret_cast<floatx4 *>(gu + 32) = du;
        }
    }
}

// The short-first m-tile order: thread t takes experts [t EPT, (t + 1)
// EPT); the count of short last m-tiles before each expert comes from a
// workgroup scan (wave shuffles, then the wave totals).
constexpr int kOrderThreads = 1024;
__global__ __launch_bounds__(kOrderThreads) void short_first_order_kernel(const int *offsets,
                                                                          const int *tile_off,
                                                                          int E, int *order) {
    __shared__ int wtot[kOrderThreads / 64];
    __shared__ int nshort;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ept = (E + kOrderThreads - 1) / kOrderThreads;
    const int e0 = min(E, tid * ept), e1 = min(E, e0 + ept);
    auto is_short = [&](int e) {
        const int m = tile_off[e + 1] - tile_off[e];
        return m > 0 && offsets[e + 1] - offsets[e] - BM * (m - 1) <= 96;
    };
    int c = 0;
    for (int e = e0; e < e1; ++e) c += is_short(e);
    int v = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    if (lane == 63) wtot[w] = v;
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int i = 0; i < kOrderThreads / 64; ++i) {
            const int t = wtot[i];
            wtot[i] = run;
            run += t;
        }
        nshort = run;
    }
    __syncthreads();
    int sb = wtot[w] + v - c;   // short m-tiles of the experts before e0
    const int ns = nshort;
    for (int e = e0; e < e1; ++e) {
        const int t0 = tile_off[e], m = tile_off[e + 1] - t0;
        const bool sh = is_short(e);
        for (int j = 0; j < m; ++j) {
            const int mt = t0 + j;
            if (sh && j == m - 1) order[sb] = mt;
            else order[ns + mt - sb] = mt;
        }
        sb += sh;
    }
}

}  // namespace

// Compute units of the current device (cached; 256 on MI355X).
int device_cus() {
    static int cus = 0;
    if (cus <= 0) {
        int dev = 0, n = 0;
        cus = hipGetDevice(&dev) == hipSuccess &&
                      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) ==
                          hipSuccess && n > 0
                  ? n : 256;
    }
    return cus;
}

GemmPlan gemm_plan(int N, int K, int max_mtiles, bool allow_split) {
    GemmPlan p{0, 1};
    if (N % 256 == 0) p.bn = 256;
    else if (N % 128 == 0) p.bn = 128;
    else if (N % 64 == 0) p.bn = 64;
    else return p;
    if (allow_split) {
        // Down projection: the widest tile, and the reduction split (its
        // partials are added by the combine) until the workgroups cover the
        // CUs once: blocks of 256 columns hold a CU each, narrower ones share
        // it 2 or 3 ways.  A split keeps >= 512 reduction elements (16 LDS
        // slices) unless the grid is tiny.  Measured at T=4096, d=512,
        // F=2048, E=8: no split 0.568 ms per layer, 2 splits 0.489, 4 0.501.
        const long slots = (long)device_cus() * (p.bn == 256 ? 1 : p.bn == 128 ? 2 : 3);
        const long blocks = (long)max_mtiles * (N / p.bn);
        const int min_k = blocks * 4 < slots ? 128 : 512;
        while (p.ksplit < 4 && blocks * p.ksplit < slots && K % (2 * p.ksplit * KT) == 0 &&
               K / (2 * p.ksplit) >= min_k)
            p.ksplit *= 2;
        return p;
    }
    // Without a split: waves in flight for tile width bn (bn / 32 waves per
    // workgroup); aim for ~4 per SIMD.  Wider tiles reuse each loaded tile
    // across more waves, so they shrink only to 128 columns, and only tiny
    // grids go to 64.
    constexpr size_t kTarget = 1024;
    auto waves = [&](int bn) { return (size_t)max_mtiles * (N / bn) * (bn / 32); };
    while (p.bn > 128 && waves(p.bn) < kTarget) p.bn /= 2;
    if (p.bn > 64 && waves(p.bn) < kTarget / 4 && N % 64 == 0) p.bn = 64;
    return p;
}

DownPlan down_plan(int N, int K, int max_mtiles, size_t n) {
    const GemmPlan g = gemm_plan(N, K, max_mtiles, true);
    DownPlan p{g.bn, g.ksplit, 0, 0};
    if (g.bn != 256 || K % KT) return p;
    // Stream-K when the tiles make fewer than ~4 rounds of one workgroup per
    // CU: every CU gets the same number of K slices, where whole tiles (or
    // tiles split a fixed 2 or 4 ways) leave a partial last round.
    const long cus = device_cus();
    const long tiles_max = (long)max_mtiles * (N / 256);
    if (tiles_max >= 4 * cus) return p;
    const long nks = K / KT;
    // The fewest live tiles n rows can make (all rows in full m-tiles) set
    // the shortest run per workgroup, hence the most pieces a tile can have.
    const long tiles_min = (long)((n + BM - 1) / BM) * (N / 256);
    const long units_min = tiles_min * nks;
    // At least 4 slices per workgroup on small problems.
    const long groups = std::max(1L, std::min(cus, units_min / 4));
    const long per_min = (units_min + groups - 1) / groups;
    p.streamk = 1;
    p.groups = (int)groups;
    p.slots = (int)((nks - 1 + per_min - 1) / per_min + 1);
    return p;
}

int gateup_tail_groups(int N, int K, int max_mtiles) {
    const GemmPlan g = gemm_plan(N, K, max_mtiles, false);
    const long cus = device_cus();
    if (g.bn != 256 || K % KT || K / KT < 2 || (long)max_mtiles * (N / 256) >= 4 * cus) return 0;
    return (int)cus;
}

hipError_t launch_gemm_gateup(const GemmArgs &a, hipStream_t s) {
    if (a.tail_groups > 0 && (!a.tail_part || a.N % 256 || a.K % KT ||
                              gemm_plan(a.N, a.K, a.max_mtiles, false).bn != 256))
        return hipErrorInvalidValue;
    return launch_mode<0>(a, s);
}

hipError_t launch_tail_fixup(const GemmArgs &a, int mode, hipStream_t s) {
    if (a.tail_groups <= 0) return hipSuccess;
    if (!a.tail_part || a.N % 256 || a.ldc % 4 || (mode == 2 && a.ldc2 % 4)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)a.tail_groups * 8);
    switch (mode) {
        case 0: hipLaunchKernelGGL(tail_fixup_kernel<0>, grid, dim3(512), 0, s, a); break;
        case 2: hipLaunchKernelGGL(tail_fixup_kernel<2>, grid, dim3(512), 0, s, a); break;
        case 3: hipLaunchKernelGGL(tail_fixup_kernel<3>, grid, dim3(512), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gateup_fixup(const GemmArgs &a, hipStream_t s) { return launch_tail_fixup(a, 0, s); }
hipError_t launch_gemm_down(const GemmArgs &a, hipStream_t s) {
    if (!a.streamk) return launch_mode<1>(a, s);
    if (!a.pieces || a.sk_groups <= 0 || a.N % 256 || a.K % KT) return hipErrorInvalidValue;
    constexpr size_t lds = (size_t)gemm_stages(4) * (BM + 256) * KT * sizeof(float);
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void *>(&grouped_gemm_kernel<1, 4>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (err != hipSuccess) return err;
        attr_set = true;
    }
    hipLaunchKernelGGL((grouped_gemm_kernel<1, 4>), dim3((unsigned)a.sk_groups), dim3(512), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_short_first_order(const int *offsets, const int *tile_off, int E, int *order,
                                    hipStream_t s) {
    if (E <= 0 || E > 4 * kOrderThreads || !order) return hipErrorInvalidValue;
    hipLaunchKernelGGL(short_first_order_kernel, dim3(1), dim3(kOrderThreads), 0, s, offsets,
                       tile_off, E, order);
    return hipGetLastError();
}

hipError_t launch_gemm_bwd(const GemmArgs &a, int mode, hipStream_t s) {
    if (a.ksplit != 1) return hipErrorInvalidValue;
    const GemmPlan pl = gemm_plan(a.N, a.K, a.max_mtiles, false);
    if (a.K % KT || (mode != 2 && mode != 3)) return hipErrorInvalidValue;
    if (a.tail_groups > 0 && (!a.tail_part || a.N % 256 || pl.bn != 256)) return hipErrorInvalidValue;
#define MOE_BWD_CASE(M)                                              \
    switch (pl.bn) {                                                 \
        case 256: return launch_grouped<M, 4>(a, s);                 \
        case 128: return launch_grouped<M, 2>(a, s);                 \
        case 64:  return launch_grouped<M, 1>(a, s);                 \
        default:  return hipErrorInvalidValue;                       \
    }
    if (mode == 2) { MOE_BWD_CASE(2) }
    MOE_BWD_CASE(3)
#undef MOE_BWD_CASE
}

hipError_t launch_combine(const CombineArgs &a, hipStream_t s) {
    if (a.pieces && (a.pieces_cols <= 0 || a.pieces_cols % 4 || a.d % a.pieces_cols))
        return hipErrorInvalidValue;
    if (!a.pieces && a.T <= 8 && a.ksplit > 8 && a.ksplit <= 128) {
        // A few tokens: two partials per lane, up to 64 lanes per output.
        const int groups = (a.ksplit + 1) / 2;
        const size_t n = (size_t)a.T * (a.d >> 2);
        if (n == 0) return hipSuccess;
        auto go = [&](auto kern, int G) {
            hipLaunchKernelGGL(kern, dim3((unsigned)((n * G + 255) / 256)), dim3(256), 0, s, a);
        };
        auto by_k = [&](auto gc) {
            constexpr int G = decltype(gc)::value;
            if (a.k == 1)      go(combine_groups_kernel<G, 1, 2>, G);
            else if (a.k == 2) go(combine_groups_kernel<G, 2, 2>, G);
            else               go(combine_groups_kernel<G, 0, 2>, G);
        };
        if (groups <= 8)       by_k(std::integral_constant<int, 8>{});
        else if (groups <= 16) by_k(std::integral_constant<int, 16>{});
        else if (groups <= 32) by_k(std::integral_constant<int, 32>{});
        else                   by_k(std::integral_constant<int, 64>{});
        return hipGetLastError();
    }
    if (!a.pieces && a.ksplit > 8 && a.ksplit <= 128) {
        const int groups = (a.ksplit + 7) / 8;
        const size_t n = (size_t)a.T * (a.d >> 2);
        if (n == 0) return hipSuccess;
        auto go = [&](auto kern, int G) {
            hipLaunchKernelGGL(kern, dim3((unsigned)((n * G + 255) / 256)), dim3(256), 0, s, a);
        };
        auto by_k = [&](auto gc) {
            constexpr int G = decltype(gc)::value;
            if (a.k == 1)      go(combine_groups_kernel<G, 1>, G);
            else if (a.k == 2) go(combine_groups_kernel<G, 2>, G);
            else               go(combine_groups_kernel<G, 0>, G);
        };
        if (groups <= 2)       by_k(std::integral_constant<int, 2>{});
        else if (groups <= 4)  by_k(std::integral_constant<int, 4>{});
        else if (groups <= 8)  by_k(std::integral_constant<int, 8>{});
        else if (groups <= 16) by_k(std::integral_constant<int, 16>{});
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    size_t total = (size_t)a.T * (a.d >> 2);
    if (total == 0) return hipSuccess;
    unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 8192);
    auto go = [&](auto parts) {
        constexpr bool P = decltype(parts)::value;
        if (a.k == 1)      hipLaunchKernelGGL((combine_kernel<1, P>), dim3(blocks), dim3(256), 0, s, a);
        else if (a.k == 2) hipLaunchKernelGGL((combine_kernel<2, P>), dim3(blocks), dim3(256), 0, s, a);
        else if (a.k == 4) hipLaunchKernelGGL((combine_kernel<4, P>), dim3(blocks), dim3(256), 0, s, a);
        else               hipLaunchKernelGGL((combine_kernel<0, P>), dim3(blocks), dim3(256), 0, s, a);
    };
    if (a.pieces || a.ksplit > 1) go(std::true_type{});
    else                          go(std::false_type{});
    return hipGetLastError();
}

// dst[r][c] = src[r][c] for c < min(sc, dc), 0 for sc <= c < dc: rows widened
// with zeros, or cut to their first dc columns.
__global__ __launch_bounds__(256) void copy_rows_kernel(const float *src, int rows, int sc,
                                                        float *dst, int dc) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)rows * dc) return;
    const size_t r = i / dc;
    const int c = (int)(i - r * dc);
    dst[i] = c < sc ? src[r * sc + c] : 0.0f;
}

hipError_t launch_copy_rows(const float *src, int rows, int src_cols, float *dst, int dst_cols,
                            hipStream_t s) {
    const size_t n = (size_t)rows * dst_cols;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(copy_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src,
                       rows, src_cols, dst, dst_cols);
    return hipGetLastError();
}

hipError_t launch_pack_gateup(const float *wg, const float *wu, float *dst, int d, int F,
                              hipStream_t s) {
    dim3 grid(F / 32, d / 32);
    hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, s, const_cast<float *>(wg), dst, d, F, 1, 0);
    hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, s, const_cast<float *>(wu), dst, d, F, 2, 0);
    return hipGetLastError();
}

hipError_t launch_unpack_gateup(const float *src, float *wg, float *wu, int d, int F,
                                hipStream_t s) {
    dim3 grid(F / 32, d / 32);
    hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, s, wg, const_cast<float *>(src), d, F, 1, 1);
    hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, s, wu, const_cast<float *>(src), d, F, 2, 1);
    return hipGetLastError();
}

hipError_t launch_unpack_experts(const float *wgu, const float *wdT, float *wg, float *wu,
                                 float *wd, int E, int d, int F, hipStream_t s) {
    const size_t dF = (size_t)d * F;
    dim3 ggu(F / 32, d / 32, E), gdn(d / 32, F / 32, E);
    hipLaunchKernelGGL(pack_kernel, ggu, dim3(256), 0, s, wg, const_cast<float *>(wgu), d, F, 1, 1,
                       dF, 2 * dF);
    hipLaunchKernelGGL(pack_kernel, ggu, dim3(256), 0, s, wu, const_cast<float *>(wgu), d, F, 2, 1,
                       dF, 2 * dF);
    hipLaunchKernelGGL(pack_kernel, gdn, dim3(256), 0, s, wd, const_cast<float *>(wdT), F, d, 0, 1,
                       dF, dF);
    return hipGetLastError();
}

hipError_t launch_transpose_units(const float *src, float *dst, int R, int C, int E,
                                  hipStream_t s) {
    if (R % 16 || C % 16 || E <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(transpose_units_kernel,
                       dim3((unsigned)(((R / 16) * (C / 16) + 3) / 4), (unsigned)E),
                       dim3(256), 0, s, src, dst, R, C);
    return hipGetLastError();
}

hipError_t launch_pack_down(const float *wd, float *dst, int F, int d, hipStream_t s) {
    dim3 grid(d / 32, F / 32);
    hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, s, const_cast<float *>(wd), dst, F, d, 0, 0);
    return hipGetLastError();
}

hipError_t launch_unpack_down(const float *src, float *wd, int F, int d, hipStream_t s) {
    dim3 grid(d / 32, F / 32);
    hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, s, wd, const_cast<float *>(src), F, d, 0, 1);
    return hipGetLastError();
}

hipError_t launch_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t stream_id,
                              float mean, float std, hipStream_t s) {
    if (n == 0) return hipSuccess;
    unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(fill_normal_kernel, dim3(blocks), dim3(256), 0, s, dst, n, seed,
                       stream_id, mean, std);
    return hipGetLastError();
}

// A read of known size through one load path (counter calibration): MODE 0
// the grouped GEMMs' LDS DMA (global_load_lds_dwordx4), 1 buffer loads into
// registers with the default cache policy, 2 the same loads non-temporal
// (the decode weight stream).  Workgroup b (4 waves) reads bytes [b span,
// (b + 1) span) in 4 KB steps, eight 1 KB wave instructions in flight; the
// sum of what it read (MODE 0: of its LDS) goes to out[b].
constexpr int kProbeGroups = 1024;
template <int MODE>
__global__ __launch_bounds__(256) void read_probe_kernel(const float *src, size_t span,
                                                         float *out) {
    __shared__ __align__(16) float lds[4][8][256];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const char *base = reinterpret_cast<const char *>(src) + (size_t)blockIdx.x * span;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (size_t off = 0; off < span; off += 4096 * 8) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const char *g = base + off + 4096 * i + 1024 * wave;
            if (MODE == 0) {
                gemm_dma16(reinterpret_cast<const float *>(g) + 4 * lane,
                           (unsigned)(size_t)(const __attribute__((address_space(3))) float *)
                               &lds[wave][i][0]);
            } else {
                const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<char *>(g), (short)0, 1024, 0x00020000);
                acc += __builtin_amdgcn_raw_buffer_load_b128(r, 16 * lane, 0, MODE == 2 ? 2 : 0);
            }
        }
        if (MODE == 0) GEMM_WAIT_VMCNT(0);
    }
    if (MODE == 0) {
        __syncthreads();
        acc[0] = lds[wave][lane & 7][threadIdx.x & 255];
    }
    if (threadIdx.x == 0) out[blockIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

hipError_t launch_read_probe(const float *src, size_t bytes, int mode, float *out,
                             hipStream_t s) {
    const size_t step = (size_t)kProbeGroups * 4096 * 8;
    if (bytes == 0 || bytes % step != 0 || mode < 0 || mode > 2) return hipErrorInvalidValue;
    const size_t span = bytes / kProbeGroups;
    if (mode == 0)
        hipLaunchKernelGGL(read_probe_kernel<0>, dim3(kProbeGroups), dim3(256), 0, s, src, span, out);
    else if (mode == 1)
        hipLaunchKernelGGL(read_probe_kernel<1>, dim3(kProbeGroups), dim3(256), 0, s, src, span, out);
    else
        hipLaunchKernelGGL(read_probe_kernel<2>, dim3(kProbeGroups), dim3(256), 0, s, src, span, out);
    return hipGetLastError();
}

// dst = src, n16 16-byte units; either side may be pinned host memory,
// which the kernel then reads or writes across the bus itself.
__global__ __launch_bounds__(256) void copy16_kernel(const uint4 *src, uint4 *dst, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
        dst[i] = src[i];
}

hipError_t launch_copy16(void *dst, const void *src, size_t bytes, hipStream_t s) {
    if (bytes == 0) return hipSuccess;
    if (bytes % 16 || reinterpret_cast<uintptr_t>(dst) % 16 || reinterpret_cast<uintptr_t>(src) % 16)
        return hipErrorInvalidValue;
    const size_t n16 = bytes / 16;
    const unsigned blocks = (unsigned)std::min<size_t>((n16 + 255) / 256, 1024);
    hipLaunchKernelGGL(copy16_kernel, dim3(blocks), dim3(256), 0, s, static_cast<const uint4 *>(src),
                       static_cast<uint4 *>(dst), n16);
    return hipGetLastError();
}

hipError_t launch_zero_ints(int *p, int n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(zero_ints_kernel, dim3((unsigned)std::min(1024, (n + 255) / 256)), dim3(256),
                       0, s, p, n);
    return hipGetLastError();
}

}  // namespace moe
