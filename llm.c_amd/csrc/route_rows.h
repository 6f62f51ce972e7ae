// route_rows.h — the row-block router as a device function of the routing
// kernel (route.hip), built with fp32 denormal flushing, matching the
// FTZ/DAZ mode of the reference's -ffast-math executables.
#pragma once
#include "moe_internal.h"
#include "moe_math.h"

namespace moe {
namespace {

// ---------------------------------------------------------------------------
// Row-block router.  A workgroup owns 16 tokens and every expert, so routing
// needs no cross-workgroup exchange.  Lane 16*r + c of wave w runs the
// chains of token t0 + c with experts 4*(w*RE + j) + r, j < RE, over k
// ascending.  x reaches the lanes through LDS (float4 reads; the four 16-lane
// rows read the same token row); each expert's router row sits in VGPRs
// sixteen k-values at a time (lane c of row r holds k0 + c of row r's
// expert) and reaches all lanes of the row through DPP row_newbcast inside
// the FMA, so the broadcast costs no instruction.
//
// Zero-skip: the reference skips x == 0 (src/matrix.c:394).  For finite
// router weights fma(0, w, acc) returns acc up to the sign of a zero
// accumulator, and a logit of +0 or -0 gives the same probabilities bit for
// bit (every path of the softmax maps both to the same value), so SKIP = false
// is exact for them.  Router weights holding an inf or NaN (0 * inf = NaN)
// take the SKIP = true variant, which applies the skip per step.
// ---------------------------------------------------------------------------

// acc = fma(w from lane 16*row + J, x[J], acc) for J = 0..15 in order.  The
// leading s_nop gives the wait states a DPP source read needs after a VALU
// write of that register or of EXEC.
__device__ inline void chain16_dpp(float &acc, float w, const float (&x)[16]) {
    asm("s_nop 4\n\t"
        "v_fmac_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %3 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %4 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %5 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %10 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %11 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %12 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %13 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %14 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %15 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %16 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %17 row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
        : "+v"(acc)
        : "v"(w), "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]), "v"(x[8]), "v"(x[9]), "v"(x[10]), "v"(x[11]), "v"(x[12]), "v"(x[13]), "v"(x[14]), "v"(x[15]));
}

// The same chain with the router row held as float4s: lane c of a 16-lane
// row holds k = 4c .. 4c + 3 of a 64-wide k block, so the sixteen steps of
// quarter Q (k = 16Q + J) take component J % 4 of lane 4Q + J / 4.  x[J] is
// x at k = 16Q + J of that block.
#define MOE_CHAIN_DPP4(L0, L1, L2, L3)                                                        \
    asm("s_nop 4\n\t"                                                                         \
        "v_fmac_f32_dpp %0, %1, %5 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"       \
        "v_fmac_f32_dpp %0, %2, %6 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"       \
        "v_fmac_f32_dpp %0, %3, %7 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"       \
        "v_fmac_f32_dpp %0, %4, %8 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"       \
        "v_fmac_f32_dpp %0, %1, %9 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"       \
        "v_fmac_f32_dpp %0, %2, %10 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %3, %11 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %4, %12 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %1, %13 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %2, %14 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %3, %15 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %4, %16 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %1, %17 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %2, %18 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %3, %19 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %4, %20 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        : "+v"(acc)                                                                           \
        : "v"(w.x), "v"(w.y), "v"(w.z), "v"(w.w), "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), \
          "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]), "v"(x[8]), "v"(x[9]), "v"(x[10]),       \
          "v"(x[11]), "v"(x[12]), "v"(x[13]), "v"(x[14]), "v"(x[15]))

// Two chains of the same x (two experts of one token) interleaved step by
// step, so that each FMA's predecessor in its chain is two instructions back.
#define MOE_CHAIN2_DPP4(L0, L1, L2, L3)                                                       \
    asm("s_nop 4\n\t"                                                                         \
        "v_fmac_f32_dpp %0, %2, %10 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %6, %10 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %3, %11 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %7, %11 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %4, %12 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %8, %12 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %5, %13 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %9, %13 row_newbcast:" #L0 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %2, %14 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %6, %14 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %3, %15 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %7, %15 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %4, %16 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %8, %16 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %5, %17 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %9, %17 row_newbcast:" #L1 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %2, %18 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %6, %18 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %3, %19 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %7, %19 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %4, %20 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %8, %20 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %5, %21 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %9, %21 row_newbcast:" #L2 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %2, %22 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %6, %22 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %3, %23 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %7, %23 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %4, %24 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %8, %24 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %0, %5, %25 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        "v_fmac_f32_dpp %1, %9, %25 row_newbcast:" #L3 " row_mask:0xf bank_mask:0xf\n\t"      \
        : "+v"(a0), "+v"(a1)                                                                  \
        : "v"(w0.x), "v"(w0.y), "v"(w0.z), "v"(w0.w), "v"(w1.x), "v"(w1.y), "v"(w1.z),       \
          "v"(w1.w), "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]),        \
          "v"(x[6]), "v"(x[7]), "v"(x[8]), "v"(x[9]), "v"(x[10]), "v"(x[11]), "v"(x[12]),     \
          "v"(x[13]), "v"(x[14]), "v"(x[15]))

// chain16_dpp4 on two accumulators (router rows w0 and w1) at once.
template <int Q>
__device__ inline void chain16x2_dpp4(float &a0, float &a1, const float4 &w0, const float4 &w1,
                                      const float (&x)[16]) {
    static_assert(Q >= 0 && Q < 4, "a quarter of a 64-wide k block");
    if constexpr (Q == 0) MOE_CHAIN2_DPP4(0, 1, 2, 3);
    else if constexpr (Q == 1) MOE_CHAIN2_DPP4(4, 5, 6, 7);
    else if constexpr (Q == 2) MOE_CHAIN2_DPP4(8, 9, 10, 11);
    else MOE_CHAIN2_DPP4(12, 13, 14, 15);
}
#undef MOE_CHAIN2_DPP4

template <int Q>
__device__ inline void chain16_dpp4(float &acc, const float4 &w, const float (&x)[16]) {
    static_assert(Q >= 0 && Q < 4, "a quarter of a 64-wide k block");
    if constexpr (Q == 0) MOE_CHAIN_DPP4(0, 1, 2, 3);
    else if constexpr (Q == 1) MOE_CHAIN_DPP4(4, 5, 6, 7);
    else if constexpr (Q == 2) MOE_CHAIN_DPP4(8, 9, 10, 11);
    else MOE_CHAIN_DPP4(12, 13, 14, 15);
}
#undef MOE_CHAIN_DPP4

template <int J>
__device__ inline float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + J, 0xF, 0xF, true));
}

// The same chain with the reference's per-step zero-skip.
template <int J>
struct SkipChain {
    __device__ static inline void run(float &acc, float w, const float (&x)[16]) {
        SkipChain<J - 1>::run(acc, w, x);
        const float wj = row_bcast<J - 1>(w);
        acc = (x[J - 1] != 0.0f) ? fmaf(x[J - 1], wj, acc) : acc;
    }
};
template <>
struct SkipChain<0> {
    __device__ static inline void run(float &, float, const float (&)[16]) {}
};

// Lane l of each aligned group of 8 lanes reads lane l ^ M (DPP moves).
template <int CTRL>
__device__ inline int dpp_mov(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int M> __device__ inline int xor8(int v);
template <> __device__ inline int xor8<1>(int v) { return dpp_mov<0xB1>(v); }   // quad_perm [1,0,3,2]
template <> __device__ inline int xor8<2>(int v) { return dpp_mov<0x4E>(v); }   // quad_perm [2,3,0,1]
template <> __device__ inline int xor8<4>(int v) {
    const int up = dpp_mov<0x104>(v);   // row_shl:4, lane i reads lane i + 4
    const int dn = dpp_mov<0x114>(v);   // row_shr:4, lane i reads lane i - 4
    return (threadIdx.x & 4) ? dn : up;
}
template <int M> __device__ inline float xor8f(float v) {
    return __int_as_float(xor8<M>(__float_as_int(v)));
}

// Eight consecutive lanes finish one token: lane l plays lane l of the
// reference's 8-wide vectors, so softmax_rows (src/matrix.c:529-586) keeps
// its per-lane maxima and sums and hsum256's fold order
// (include/simd.h:110-121) becomes three butterfly steps; every lane then
// runs the scalar tail in the reference's order.  Top-k
// (src/transformer.c:317-331) is k rounds of an argmax over the experts not
// yet chosen, ties to the lowest index, reduced across the eight lanes; lane
// 0 records each round's expert and probability in id_out / p_out and the
// returned value is the renormalisation factor (src/transformer.c:334-336).
// Every lane of the wave calls this together.
template <int NBM>
__device__ inline float finish_token8(const RouteArgs &a, float *row, int l, int *id_out,
                                      float *p_out) {
    // Lane l keeps its vector elements 8*b + l (b < nb <= NBM) in registers;
    // the E % 8 tail stays in LDS, read by every lane in order.
    const int E = a.E, k = a.k;
    const int nb = E >> 3, tail = E - 8 * nb;
    float v[NBM];
#pragma unroll
    for (int b = 0; b < NBM; ++b) v[b] = b < nb ? row[8 * b + l] : 0.0f;
    float m = -1e38f;
#pragma unroll
    for (int b = 0; b < NBM; ++b)
        if (b < nb) m = fmaxf(m, v[b]);
    m = fmaxf(m, xor8f<4>(m));
    m = fmaxf(m, xor8f<2>(m));
    m = fmaxf(m, xor8f<1>(m));
    for (int j = 8 * nb; j < E; ++j) {
        const float t = row[j];
        if (t > m) m = t;
    }
    float vs = 0.0f;
#pragma unroll
    for (int b = 0; b < NBM; ++b)
        if (b < nb) {
            v[b] = exp_poly(v[b] - m);
            vs = vs + v[b];
        }
    vs = vs + xor8f<4>(vs);   // v_l + v_(l+4)
    vs = vs + xor8f<1>(vs);   // (v0+v4) + (v1+v5) and (v2+v6) + (v3+v7)
    vs = vs + xor8f<2>(vs);   // the two halves
    for (int j = 8 * nb; j < E; ++j) {
        const float ex = glibc_expf(row[j] - m);
        vs = vs + ex;
        if (l == 0) row[j] = ex;
    }
    const float inv = 1.0f / vs;
#pragma unroll
    for (int b = 0; b < NBM; ++b)
        if (b < nb) {
            v[b] = ftz_f(v[b] * inv);
            row[8 * b + l] = v[b];
        }
    float tv = 0.0f;
    if (l < tail) {
        tv = ftz_f(row[8 * nb + l] * inv);
        row[8 * nb + l] = tv;
    }

    // The chosen set: one bit per expert in NW words, every word index a
    // constant after unrolling (a runtime index would put them in scratch).
    constexpr int NW = (8 * NBM + 63) / 64;
    uint64_t chosen[NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) chosen[q] = 0;
    auto is_chosen = [&](int e) {
        uint64_t bit = 0;
#pragma unroll
        for (int q = 0; q < NW; ++q)
            if ((e >> 6) == q) bit = (chosen[q] >> (e & 63)) & 1ull;
        return bit != 0;
    };
    float s = 0.0f;
    for (int ki = 0; ki < k; ++ki) {
        float best = -1.0f;
        int be = 0x7fffffff;
        auto consider = [&](int e, float p) {
            if (!is_chosen(e) && p > best) { best = p; be = e; }
        };
#pragma unroll
        for (int b = 0; b < NBM; ++b)
            if (b < nb) consider(8 * b + l, v[b]);
        if (l < tail) consider(8 * nb + l, tv);
        auto merge = [&](float ob, int oe) {
            if (ob > best || (ob == best && oe < be)) { best = ob; be = oe; }
        };
        merge(xor8f<4>(best), xor8<4>(be));
        merge(xor8f<2>(best), xor8<2>(be));
        merge(xor8f<1>(best), xor8<1>(be));
        float p = best;   // the chosen probability itself
        if (be == 0x7fffffff) {   // nothing beat -1: the reference keeps best_e = 0
            be = 0;
            p = row[0];
        }
#pragma unroll
        for (int q = 0; q < NW; ++q)
            if ((be >> 6) == q) chosen[q] |= 1ull << (be & 63);
        s = s + p;
        if (l == 0) { id_out[ki] = be; p_out[ki] = p; }
    }
    return (s > 1e-9f) ? 1.0f / s : 0.0f;
}

// Logits row width of a router block covering 4 NWV RE experts: 129 floats
// up to 128 experts, 257 up to 256.
constexpr int rows_lw(int nwv, int re) { return 4 * nwv * re > 128 ? 257 : 129; }

// LDS layout of route_rows_block (floats): x chunks, logits rows, chosen
// probabilities and experts, renormalisation factors.
template <int KC, int LW = 129>
struct RowsSmem {
    static constexpr int kLd = KC + 4;
    static constexpr int kLg = 2 * 16 * kLd;
    static constexpr int kLw = LW;   // logits row (floats): the experts + 1
    static constexpr int kPSel = kLg + 16 * LW;
    static constexpr int kIdSel = kPSel + 16 * kMaxTopK;
    static constexpr int kInv = kIdSel + 16 * kMaxTopK;
    static constexpr int kFloats = kInv + 16;
};

// Routes token block tb (tokens 16*tb ..) with NWV waves; every thread of
// the workgroup calls this.  smem: RowsSmem<KC, rows_lw(NWV, RE)>::kFloats floats of LDS,
// 16-byte aligned.
template <int NWV, int RE, int KC, bool SKIP>
__device__ void route_rows_block(const RouteArgs &a, int tb, float *smem) {
    static_assert(NWV >= 2, "two waves finish the block's 16 tokens");
    constexpr int NT = 64 * NWV;
    constexpr int LD = KC + 4;                     // padded LDS row of x (floats)
    constexpr int XQ = 16 * KC / 4;                // float4s of x per chunk
    constexpr int XL = (XQ + NT - 1) / NT;
    constexpr int WV = KC / 16;                    // router VGPRs per expert per chunk
    using S = RowsSmem<KC, rows_lw(NWV, RE)>;
    float (*xs)[16][LD] = reinterpret_cast<float (*)[16][LD]>(smem);
    float (*lg)[S::kLw] = reinterpret_cast<float (*)[S::kLw]>(smem + S::kLg);
    float (*p_sel)[kMaxTopK] = reinterpret_cast<float (*)[kMaxTopK]>(smem + S::kPSel);
    int (*id_sel)[kMaxTopK] = reinterpret_cast<int (*)[kMaxTopK]>(smem + S::kIdSel);
    float *inv_sel = smem + S::kInv;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane >> 4, c = lane & 15;
    const int T = a.T, d = a.d, E = a.E, k = a.k;
    const int t0 = tb * 16;

    // Experts past E repeat expert E - 1 and store nothing; rows past T read
    // row T - 1 (all lanes stay active for the DPP reads) and store nothing.
    const float *wrow[RE];
#pragma unroll
    for (int j = 0; j < RE; ++j)
        wrow[j] = a.wrT + (size_t)min(4 * (w * RE + j) + r, E - 1) * d + c;

    float4 rx[XL];
    float rw[RE][WV], wc[RE][WV];
    auto gload = [&](int k0, bool with_x = true) {
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            if (!with_x) break;
            const int q = min(tid + NT * i, XQ - 1);
            const int rr = q / (KC / 4), c4 = q % (KC / 4);
            const int t = min(t0 + rr, T - 1);
            rx[i] = *reinterpret_cast<const float4 *>(a.x + (size_t)t * d + k0 + 4 * c4);
        }
#pragma unroll
        for (int j = 0; j < RE; ++j)
#pragma unroll
            for (int s4 = 0; s4 < WV; ++s4) rw[j][s4] = wrow[j][k0 + 16 * s4];
    };
    auto sstore = [&](int buf, bool with_x = true) {
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            if (!with_x) break;
            const int q = tid + NT * i;
            if (XQ % NT == 0 || q < XQ) {
                const int rr = q / (KC / 4), c4 = q % (KC / 4);
                float4 v = rx[i];
                if (SKIP) v = make_float4(ftz_f(v.x), ftz_f(v.y), ftz_f(v.z), ftz_f(v.w));
                *reinterpret_cast<float4 *>(&xs[buf][rr][4 * c4]) = v;
            }
        }
#pragma unroll
        for (int j = 0; j < RE; ++j)
#pragma unroll
            for (int s4 = 0; s4 < WV; ++s4) wc[j][s4] = rw[j][s4];
    };

    const int nchunk = d / KC;
    // With a.rms_w the block's rows are first normalised from x_raw (sixteen
    // lanes per row, the reference's accumulator order) into a.x; in one
    // chunk (d == KC) straight into the LDS rows as well, else read back.
    const bool pre = a.rms_w && nchunk == 1;
    if (pre) gload(0, false);   // (router rows in flight during the normalisation)
    if (a.rms_w) {
        for (int rr = tid >> 4; rr < 16; rr += NT / 16) {
            const int t = min(t0 + rr, T - 1);
            const float *xr = a.x_raw + (size_t)t * d;
            rms_row16([&](int i) { return xr[i]; }, a.rms_w, d / 16, a.rms_eps, a.rms_rcp,
                      a.xn_out + (size_t)t * d, t0 + rr < T, pre ? &xs[0][rr][0] : nullptr, SKIP);
        }
        if (!pre) {
            __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the rows are stored
            __syncthreads();
        }
    }
    float acc[RE];
#pragma unroll
    for (int j = 0; j < RE; ++j) acc[j] = 0.0f;
    if (!pre) gload(0);
    sstore(0, !pre);
    __syncthreads();
    for (int ch = 0; ch < nchunk; ++ch) {
        const int buf = ch & 1;
        if (ch + 1 < nchunk) gload((ch + 1) * KC);
        // x of the next 16 steps is read while the FMAs of these run.
        auto xread = [&](float (&xv)[16], int s4) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = *reinterpret_cast<const float4 *>(&xs[buf][c][16 * s4 + 4 * q]);
                xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
            }
        };
        auto chains = [&](const float (&xv)[16], int s4) {
#pragma unroll
            for (int j = 0; j < RE; ++j) {
                if (SKIP) SkipChain<16>::run(acc[j], wc[j][s4], xv);
                else      chain16_dpp(acc[j], wc[j][s4], xv);
            }
        };
        float xa[16], xb[16];
        xread(xa, 0);
#pragma unroll
        for (int s4 = 0; s4 < WV; s4 += 2) {
            xread(xb, s4 + 1);
            chains(xa, s4);
            if (s4 + 2 < WV) xread(xa, s4 + 2);
            chains(xb, s4 + 1);
        }
        if (ch + 1 < nchunk) sstore(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < RE; ++j) {
        const int e = 4 * (w * RE + j) + r;
        if (e < E) lg[c][e] = a.bias ? acc[j] + a.bias[e] : acc[j];
    }
    __syncthreads();
    if (tid < 128) {
        const int ct = tid >> 3, l = tid & 7;
        const float inv = finish_token8<(4 * NWV * RE + 7) / 8>(a, &lg[ct][0], l, &id_sel[ct][0],
                                                                &p_sel[ct][0]);
        if (l == 0) inv_sel[ct] = inv;
    }
    __syncthreads();
    const int tn = min(16, T - t0);
    if (a.ids || a.gw)
        for (int i = tid; i < tn * k; i += NT) {
            const int ct = i / k, ki = i - ct * k;
            const size_t o = (size_t)(t0 + ct) * k + ki;
            if (a.ids) a.ids[o] = id_sel[ct][ki];
            if (a.gw) a.gw[o] = ftz_f(p_sel[ct][ki] * inv_sel[ct]);
        }
    if (a.probs)
        for (int i = tid; i < tn * E; i += NT) {
            const int ct = i / E, e = i - ct * E;
            a.probs[(size_t)(t0 + ct) * E + e] = lg[ct][e];
        }
}

}  // namespace
}  // namespace moe
