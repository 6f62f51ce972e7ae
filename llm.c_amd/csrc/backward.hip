// backward.hip — backward pass of the MoE layer and its load-balancing loss.
//
// The reference has neither: its block backward (src/transformer.c:975-1013)
// skips the FFN/MoE half, and the auxiliary loss exists only as the comment
// aux = n_experts * sum_e f_e * P_e (src/transformer.c:280-282).  Here, for
// the layer of src/transformer.c:287-366 with the routing held as the
// forward decided it, the gradients of L = sum(dout * out) + aux_coef * aux
// (f_e = assignments to e / (T k), a count; P_e = mean_t probs[t][e]):
//
//   recompute  G, U = x W_g, x W_u (rows in dispatch order), H = silu(G) U,
//              Y = H W_d
//   slots      dgw = <Y, dout[t]>, dY = gw dout[t]
//   experts    dH = dY W_d^T, dG = dH U silu'(G), dU = dH silu(G),
//              dXr = dG W_g^T + dU W_u^T; dW_d = H^T dY, dW_g = X^T dG,
//              dW_u = X^T dU over each expert's rows
//   router     gw = p_sel / S: dp_sel = (dgw - <dgw, gw>) / S; dp += aux_coef
//              E f / T; dlogits = p (dp - <dp, p>); dW_r = X^T dlogits
//   dx         = sum over the token's slots of dXr + dlogits W_r^T
//
// Two fp32 tiled GEMMs do the products: rows_gemm over the dispatch tile
// schedule (one expert per 128-row tile), reduce_gemm with the reduction
// over an expert's rows.  Every sum runs in a fixed order (deterministic).
#include "moe_internal.h"
#include "moe_math.h"

namespace moe {
namespace {

constexpr int kRM = 128, kRN = 64, kRK = 16;   // rows_gemm tile
constexpr int kQM = 64, kQN = 64, kQR = 16;    // reduce_gemm tile

// C[pos][n] (+)= sum_kk A(pos, kk) B_e(kk, n) for the rows pos of each
// 128-row tile (expert e).  A(pos, kk) = a[arow * lda + kk] with arow =
// perm[pos] / topk (GATHER) or pos; B_e(kk, n) = b[e * b_e + kk * ldb + n]
// or, BT, b[e * b_e + n * ldb + kk].  Thread (tr, tc) = (tid / 16, tid % 16)
// owns rows 8tr .. 8tr + 7 and columns 4tc .. 4tc + 3; K slices of 16 in LDS.
struct RowsGemm {
    const float *a;
    int lda;
    const int *perm;
    int topk;
    const float *b;
    size_t b_e;
    int ldb;
    float *c;
    int ldc;
    const int *offsets, *tile_off, *tile_expert;
    int E, K, N, max_mtiles, accumulate;
};

template <bool GATHER, bool BT>
__global__ __launch_bounds__(256) void rows_gemm_kernel(RowsGemm g) {
    __shared__ __align__(16) float As[kRK][kRM + 4];
    __shared__ __align__(16) float Bs[kRK][kRN + 4];
    const int ntn = (g.N + kRN - 1) / kRN;
    const int nt = blockIdx.x % ntn, mtg = blockIdx.x / ntn;
    if (mtg >= g.tile_off[g.E]) return;
    const int e = g.tile_expert[mtg];
    const int row0 = g.offsets[e] + (mtg - g.tile_off[e]) * kRM;
    const int rows = min(kRM, g.offsets[e + 1] - row0);
    const int n0 = nt * kRN;
    const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;

    const float *arow[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = min((tid >> 2) + 64 * i, rows - 1);
        const size_t src = GATHER ? (size_t)(g.perm[row0 + r] / g.topk) : (size_t)(row0 + r);
        arow[i] = g.a + src * g.lda + 4 * (tid & 3);
    }
    const float *bb = g.b + (size_t)e * g.b_e;
    float acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;

    for (int k0 = 0; k0 < g.K; k0 += kRK) {
        float4 av[2], bv;
#pragma unroll
        for (int i = 0; i < 2; ++i) av[i] = *reinterpret_cast<const float4 *>(arow[i] + k0);
        int bk, bn;
        if (!BT) {   // 16 k rows x 16 column quads
            bk = tid >> 4;
            bn = 4 * (tid & 15);
            const bool in = n0 + bn < g.N;
            bv = masked4(in, *reinterpret_cast<const float4 *>(bb + (size_t)(k0 + bk) * g.ldb +
                                                              (in ? n0 + bn : 0)));
        } else {     // 64 columns x 4 k quads
            bn = tid >> 2;
            bk = 4 * (tid & 3);
            const bool in = n0 + bn < g.N;
            bv = masked4(in, *reinterpret_cast<const float4 *>(bb + (size_t)(in ? n0 + bn : 0) * g.ldb +
                                                              k0 + bk));
        }
        __syncthreads();   // the previous slice is consumed
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = (tid >> 2) + 64 * i, kq = 4 * (tid & 3);
            As[kq][r] = av[i].x;
            As[kq + 1][r] = av[i].y;
            As[kq + 2][r] = av[i].z;
            As[kq + 3][r] = av[i].w;
        }
        if (!BT) {
            *reinterpret_cast<float4 *>(&Bs[bk][bn]) = bv;
        } else {
            Bs[bk][bn] = bv.x;
            Bs[bk + 1][bn] = bv.y;
            Bs[bk + 2][bn] = bv.z;
            Bs[bk + 3][bn] = bv.w;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kRK; ++kk) {
            const float4 a0 = *reinterpret_cast<const float4 *>(&As[kk][8 * tr]);
            const float4 a1 = *reinterpret_cast<const float4 *>(&As[kk][8 * tr + 4]);
            const float4 b4 = *reinterpret_cast<const float4 *>(&Bs[kk][4 * tc]);
            const float a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            const float b[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
    }
    const int n = n0 + 4 * tc;
    if (n >= g.N) return;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = 8 * tr + i;
        if (r >= rows) break;
        float4 *cp = reinterpret_cast<float4 *>(g.c + (size_t)(row0 + r) * g.ldc + n);
        float4 v = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
        if (g.accumulate) {
            const float4 o = *cp;
            v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
        }
        *cp = v;
    }
}

// The same product on the matrix cores (v_mfma_f32_32x32x2f32): a 128 x 64
// tile per workgroup of two waves, wave w rows 64w .. 64w + 63 and all 64
// columns (2 x 2 blocks of 32 x 32).  K slices of 32 sit in LDS with K
// contiguous per row (As) and per column (Bs); lane (li, lh) = (l % 32,
// l / 32) feeds k = 16 lh + 4q + s of MFMA (q, s), as in the forward's
// grouped GEMM.  The next slice is loaded into registers while the MFMAs
// of this one run.
typedef float fx4 __attribute__((ext_vector_type(4)));
typedef float fx16 __attribute__((ext_vector_type(16)));
constexpr int kMK = 32, kMLd = kMK + 4;

template <bool GATHER, bool BT>
__global__ __launch_bounds__(128) void rows_mfma_kernel(RowsGemm g) {
    __shared__ __align__(16) float As[kRM][kMLd];
    __shared__ __align__(16) float Bs[kRN][kMLd];
    const int ntn = (g.N + kRN - 1) / kRN;
    const int nt = blockIdx.x % ntn, mtg = blockIdx.x / ntn;
    if (mtg >= g.tile_off[g.E]) return;
    const int e = g.tile_expert[mtg];
    const int row0 = g.offsets[e] + (mtg - g.tile_off[e]) * kRM;
    const int rows = min(kRM, g.offsets[e + 1] - row0);
    const int n0 = nt * kRN;
    const int tid = threadIdx.x, lane = tid & 63, wm = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    const fx4 zero = {0.f, 0.f, 0.f, 0.f};

    // A: 128 rows x 8 k-quads = 1024 float4s, 8 per thread.
    const float *asrc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int q = tid + 128 * i, r = min(q >> 3, rows - 1);
        const size_t src = GATHER ? (size_t)(g.perm[row0 + r] / g.topk) : (size_t)(row0 + r);
        asrc[i] = g.a + src * g.lda + 4 * (q & 7);
    }
    const float *bb = g.b + (size_t)e * g.b_e;
    fx4 ra[8], rb[4];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) ra[i] = *reinterpret_cast<const fx4 *>(asrc[i] + k0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = tid + 128 * i;
            if (BT) {   // 64 columns x 8 k-quads
                const int n = n0 + (q >> 3);
                rb[i] = n < g.N ? *reinterpret_cast<const fx4 *>(bb + (size_t)n * g.ldb + k0 +
                                                                   4 * (q & 7))
                                : zero;
            } else {    // 32 k rows x 16 column quads
                const int n = n0 + 4 * (q & 15);
                rb[i] = n < g.N ? *reinterpret_cast<const fx4 *>(bb + (size_t)(k0 + (q >> 4)) *
                                                                           g.ldb + n)
                                : zero;
            }
        }
    };
    auto sstore = [&]() {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = tid + 128 * i;
            *reinterpret_cast<fx4 *>(&As[q >> 3][4 * (q & 7)]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = tid + 128 * i;
            if (BT) {
                *reinterpret_cast<fx4 *>(&Bs[q >> 3][4 * (q & 7)]) = rb[i];
            } else {
                const int k = q >> 4, n = 4 * (q & 15);
                Bs[n][k] = rb[i][0];
                Bs[n + 1][k] = rb[i][1];
                Bs[n + 2][k] = rb[i][2];
                Bs[n + 3][k] = rb[i][3];
            }
        }
    };
    fx16 acc[2][2];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[m][n][r] = 0.f;
    const int nk = g.K / kMK;
    gload(0);
    for (int kt = 0; kt < nk; ++kt) {
        if (kt > 0) __syncthreads();   // this slice's LDS is free
        sstore();
        __syncthreads();
        if (kt + 1 < nk) gload((kt + 1) * kMK);
        const float *as = &As[wm * 64 + li][16 * lh];
        const float *bs = &Bs[li][16 * lh];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const fx4 a0 = *reinterpret_cast<const fx4 *>(as + 4 * q);
            const fx4 a1 = *reinterpret_cast<const fx4 *>(as + 32 * kMLd + 4 * q);
            const fx4 b0 = *reinterpret_cast<const fx4 *>(bs + 4 * q);
            const fx4 b1 = *reinterpret_cast<const fx4 *>(bs + 32 * kMLd + 4 * q);
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[s2], b0[s2], acc[0][0], 0, 0, 0);
                acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[s2], b1[s2], acc[0][1], 0, 0, 0);
                acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[s2], b0[s2], acc[1][0], 0, 0, 0);
                acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[s2], b1[s2], acc[1][1], 0, 0, 0);
            }
        }
    }
    // Block (m, n), register r: row 8 (r / 4) + 4 lh + r % 4, column li.
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = wm * 64 + m * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (row >= rows) continue;
            float *cr = g.c + (size_t)(row0 + row) * g.ldc;
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                const int col = n0 + n * 32 + li;
                if (col < g.N) cr[col] = g.accumulate ? cr[col] + acc[m][n][r] : acc[m][n][r];
            }
        }
}

// C_e[m][n] (+)= sum over the rows pos of group e (offsets[e] ..
// offsets[e + 1], or 0 .. nrows without offsets) of A(pos, m) B(pos, n),
// A(pos, m) = a[arow * lda + m] (arow = perm[pos] / topk with GATHER),
// B(pos, n) = b[pos * ldb + n].  Thread (tm, tn) = (tid / 16, tid % 16)
// owns rows 4tm .. and columns 4tn .. of the 64 x 64 tile (blockIdx.y,
// blockIdx.x) of group blockIdx.z; rows in slices of 16 through LDS.
struct ReduceGemm {
    const float *a;
    int lda;
    const int *perm;
    int topk;
    const float *b;
    int ldb;
    float *c;
    size_t c_e;
    int ldc;
    const int *offsets;
    int nrows, chunk, M, N, accumulate, vec_a, vec_b;
    // reduce_mfma_kernel only: N runs over [G | U]'s 2F packed columns and
    // column n's product goes to c (gate, n % 64 < 32) or c_up (up) at
    // feature 32 (n / 64) + n % 32.
    float *c_up = nullptr;
};

template <bool GATHER>
__global__ __launch_bounds__(256) void reduce_gemm_kernel(ReduceGemm g) {
    __shared__ __align__(16) float As[kQR][kQM + 4];
    __shared__ __align__(16) float Bs[kQR][kQN + 4];
    // Groups: the experts' row ranges, or (no offsets) chunks of nrows rows
    // of `chunk` each, whose partials go to C + z * c_e.
    const int e = blockIdx.z, m0 = blockIdx.y * kQM, n0 = blockIdx.x * kQN;
    const int r0 = g.offsets ? g.offsets[e] : e * g.chunk;
    const int r1 = g.offsets ? g.offsets[e + 1] : min(g.nrows, (e + 1) * g.chunk);
    const int tid = threadIdx.x, tm = tid >> 4, tn = tid & 15;
    const int lr = tid >> 4, lq = 4 * (tid & 15);   // load row and column quad
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    for (int r = r0; r < r1; r += kQR) {
        const int row = r + lr;
        const bool in = row < r1;
        float av[4], bv[4];
        const size_t arow = in ? (GATHER ? (size_t)(g.perm[row] / g.topk) : (size_t)row) : 0;
        if (g.vec_a && in && m0 + lq < g.M) {   // (M, lda multiples of 4)
            const float4 v = *reinterpret_cast<const float4 *>(g.a + arow * g.lda + m0 + lq);
            av[0] = v.x; av[1] = v.y; av[2] = v.z; av[3] = v.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                av[j] = in && m0 + lq + j < g.M ? g.a[arow * g.lda + m0 + lq + j] : 0.f;
        }
        if (g.vec_b && in && n0 + lq < g.N) {   // (N, ldb multiples of 4)
            const float4 v = *reinterpret_cast<const float4 *>(g.b + (size_t)row * g.ldb + n0 + lq);
            bv[0] = v.x; bv[1] = v.y; bv[2] = v.z; bv[3] = v.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bv[j] = in && n0 + lq + j < g.N ? g.b[(size_t)row * g.ldb + n0 + lq + j] : 0.f;
        }
        __syncthreads();
        *reinterpret_cast<float4 *>(&As[lr][lq]) = make_float4(av[0], av[1], av[2], av[3]);
        *reinterpret_cast<float4 *>(&Bs[lr][lq]) = make_float4(bv[0], bv[1], bv[2], bv[3]);
        __syncthreads();
#pragma unroll
        for (int rr = 0; rr < kQR; ++rr) {
            const float4 a4 = *reinterpret_cast<const float4 *>(&As[rr][4 * tm]);
            const float4 b4 = *reinterpret_cast<const float4 *>(&Bs[rr][4 * tn]);
            const float a[4] = {a4.x, a4.y, a4.z, a4.w}, b[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
    }
    float *ce = g.c + (size_t)e * g.c_e;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * tm + i;
        if (m >= g.M) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + 4 * tn + j;
            if (n >= g.N) break;
            float *cp = ce + (size_t)m * g.ldc + n;
            *cp = g.accumulate ? *cp + acc[i][j] : acc[i][j];
        }
    }
}

// The same product on the matrix cores for M, N multiples of 64 WM and
// 64 WN over the experts' row ranges: a 64 WM x 64 WN tile per workgroup,
// NWM x NWN waves of 32 x 32 blocks of v_mfma_f32_32x32x2f32 (lane half h
// feeds rows 2i + h of the slice).  Rows go through LDS in
// double-buffered slices of 32, the next two slices' loads in registers
// while the current one is multiplied; rows past the range enter LDS as zeros.  Row
// strides of 32 mod 64 floats: the two half-waves' rows fall in disjoint
// banks.  The larger tiles read each operand row once per 128 columns
// instead of once per 64.
constexpr int kMR = 32;

template <bool GATHER, int WM, int WN, int NWM, int NWN>
__global__ __launch_bounds__(64 * NWM * NWN) void reduce_mfma_kernel(ReduceGemm g) {
    // NWM x NWN waves, each BM x BN blocks of 32 x 32.
    constexpr int NT = 64 * NWM * NWN, BM = 2 * WM / NWM, BN = 2 * WN / NWN;
    static_assert(BM >= 1 && BN >= 1 && BM * NWM == 2 * WM && BN * NWN == 2 * WN, "wave layout");
    constexpr int TM = 64 * WM, TN = 64 * WN, LDA = TM + 32, LDB = TN + 32;
    constexpr int QA = TM / 4, QB = TN / 4;       // float4s per slice row
    constexpr int RA = NT / QA, RB = NT / QB;     // rows per load pass
    constexpr int PA = kMR / RA, PB = kMR / RB;   // load passes
    // The wider tiles fill the CUs in about one round: unused rows past the
    // slices take the LDS above half a CU's 160 KB, so that no two of these
    // workgroups share a CU while another CU idles.
    constexpr int kBase = 2 * kMR * (LDA + LDB) * 4, kHalf = 80 * 1024;
    constexpr int XR = WM * WN > 1 && kBase <= kHalf ? (kHalf - kBase) / (2 * LDA * 4) + 1 : 0;
    __shared__ __align__(16) float As[2][kMR + XR][LDA];
    __shared__ __align__(16) float Bs[2][kMR][LDB];
    const int e = blockIdx.z, m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
    const int r0 = g.offsets[e], r1 = g.offsets[e + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / NWN, wn = wave % NWN, li = lane & 31, lh = lane >> 5;
    const int la = tid / QA, qa = 4 * (tid % QA), lb = tid / QB, qb = 4 * (tid % QB);
    // Two register sets take the loads of the next two slices, so each load
    // has a slice and a half of MFMAs to arrive; the perm entries (GATHER)
    // of a slice are loaded a slice earlier still, into a set of their own
    // (pix, by slice parity; divided when used).  Every load is issued
    // unconditionally, rows clamped to r1 - 1 (rows past the range are
    // zeroed when stored to LDS), so the wait counts stay exact and no load
    // waits for a younger one.
    fx4 ra[2][PA], rb[2][PB];
    int pix[2][PA];
    auto pload = [&](auto set, int r) {
        constexpr int S = decltype(set)::value;
#pragma unroll
        for (int i = 0; i < PA; ++i) {
            const int row = min(r + la + RA * i, r1 - 1);
            pix[S][i] = GATHER ? g.perm[row] : row;
        }
    };
    auto gload = [&](auto set, int r) {
        constexpr int S = decltype(set)::value;
#pragma unroll
        for (int i = 0; i < PA; ++i)
            ra[S][i] = *reinterpret_cast<const fx4 *>(
                g.a + (size_t)(GATHER ? pix[S][i] / g.topk : pix[S][i]) * g.lda + m0 + qa);
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            const int row = min(r + lb + RB * i, r1 - 1);
            rb[S][i] = *reinterpret_cast<const fx4 *>(g.b + (size_t)row * g.ldb + n0 + qb);
        }
    };
    // Store p (< PA + PB) of register set S as LDS rows of buffer buf, slice r.
    auto sstore1 = [&](auto set, int p, int buf, int r) {
        constexpr int S = decltype(set)::value;
        const fx4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < PA; ++i)
            if (p == i)
                *reinterpret_cast<fx4 *>(&As[buf][la + RA * i][qa]) =
                    r + la + RA * i < r1 ? ra[S][i] : z;
#pragma unroll
        for (int i = 0; i < PB; ++i)
            if (p == PA + i)
                *reinterpret_cast<fx4 *>(&Bs[buf][lb + RB * i][qb]) =
                    r + lb + RB * i < r1 ? rb[S][i] : z;
    };
    auto sstore = [&](auto set, int buf, int r) {
#pragma unroll
        for (int p = 0; p < PA + PB; ++p) sstore1(set, p, buf, r);
    };
    fx16 acc[BM][BN];
#pragma unroll
    for (int i = 0; i < BM; ++i)
#pragma unroll
        for (int j = 0; j < BN; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;
    const int am = wm * 32 * BM + li, bn = wn * 32 * BN + li;
    // The slice in LDS buffer buf; operands of step kk + 2 are read while
    // step kk multiplies.  mid(p) runs after step 2 + p's MFMAs have issued
    // (the next slice's LDS stores, one per step under the MFMAs, so that no
    // step waits for more than one of them).
    static_assert(PA + PB + 2 <= kMR / 2, "stores per slice");
    auto mm = [&](int buf, auto &&mid) {
        float av[2][BM], bv[2][BN];
        auto rd = [&](int st, int kk) {
#pragma unroll
            for (int i = 0; i < BM; ++i) av[st][i] = As[buf][kk + lh][am + 32 * i];
#pragma unroll
            for (int j = 0; j < BN; ++j) bv[st][j] = Bs[buf][kk + lh][bn + 32 * j];
        };
        rd(0, 0);
#pragma unroll
        for (int kk = 0; kk < kMR; kk += 2) {
            const int st = (kk >> 1) & 1;
            if (kk + 2 < kMR) rd(st ^ 1, kk + 2);
            __builtin_amdgcn_sched_barrier(0);   // (the reads go out before the MFMAs)
#pragma unroll
            for (int i = 0; i < BM; ++i)
#pragma unroll
                for (int j = 0; j < BN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[st][i], bv[st][j],
                                                                     acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            const int p = kk / 2 - 2;
            if (p >= 0 && p < PA + PB) {
                mid(p);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    // Slice r (parity S), held by register set S and already in LDS buffer
    // S: the perm entries of slice r + 3 kMR go to pix set S ^ 1, register
    // set S takes slice r + 2 kMR (perm entries in pix set S), buffer S is
    // multiplied, and slice r + kMR (register set S ^ 1) goes to buffer
    // S ^ 1, which every wave finished reading before the barrier that ended
    // the previous slice.
    auto step = [&](auto set, int r) {
        constexpr int S = decltype(set)::value;
        using O = std::integral_constant<int, S ^ 1>;
        pload(O{}, r + 3 * kMR);
        gload(set, r + 2 * kMR);
        mm(S, [&](int p) { sstore1(O{}, p, S ^ 1, r + kMR); });
        __syncthreads();
    };
    if (r0 < r1) {
        pload(S0{}, r0);
        pload(S1{}, r0 + kMR);
        gload(S0{}, r0);
        pload(S0{}, r0 + 2 * kMR);
        gload(S1{}, r0 + kMR);
        sstore(S0{}, 0, r0);
        __syncthreads();
        int r = r0;
        for (; r + kMR < r1; r += 2 * kMR) {
            step(S0{}, r);
            step(S1{}, r + kMR);
        }
        if (r < r1) step(S0{}, r);   // an odd last slice
    }
    // Lane l, register q of a block: row 8 (q / 4) + 4 (l / 32) + q % 4,
    // column l % 32.
#pragma unroll
    for (int j = 0; j < BN; ++j) {
        const int n = n0 + bn + 32 * j;
        float *ce = (g.c_up && (n & 32) ? g.c_up : g.c) + (size_t)e * g.c_e;
        const int col = g.c_up ? 32 * (n >> 6) + (n & 31) : n;
#pragma unroll
        for (int i = 0; i < BM; ++i)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int m = m0 + wm * 32 * BM + 32 * i + 8 * (q >> 2) + 4 * lh + (q & 3);
                float *cp = ce + (size_t)m * g.ldc + col;
                *cp = g.accumulate ? *cp + acc[i][j][q] : acc[i][j][q];
            }
    }
}

// dW_r = X^T dlogits over all T rows, and (CS set) the column sums of
// probs for the aux loss.  Workgroup (column block cb of 64 x columns, row
// chunk z of R rows); thread (c, p) = (t % 64, t / 64) runs the FMA chains of
// kRgEB experts at a time over rows zR + p, zR + p + 4, ..., and the 4 row
// phases are added in phase order through LDS into P[z][d][E].  Every load
// is unconditional (indices clamped, masked terms multiplied by zero).  The
// workgroups of column block 0 also sum probs over their rows into CS[z][E].
// router_grad_final_kernel adds the chunks in order.
constexpr int kRgEB = 8;

__global__ __launch_bounds__(256) void router_grad_kernel(const float *x, const float *dl,
                                                          const float *probs, int T, int d,
                                                          int E, int R, float *P, float *CS) {
    __shared__ float red[4][64][kRgEB + 1];
    const int cb = blockIdx.x, z = blockIdx.y;
    const int t = threadIdx.x, c = t & 63, p = t >> 6;
    const int col = min(cb * 64 + c, d - 1);
    const int r0 = z * R, r1 = min(T, r0 + R);
    for (int e0 = 0; e0 < E; e0 += kRgEB) {
        float acc[kRgEB];
#pragma unroll
        for (int j = 0; j < kRgEB; ++j) acc[j] = 0.f;
        // Rows in batches of 8 (every load of a batch in flight together).
        for (int rb = r0 + p; rb < r1; rb += 32) {
            float xv[8], w[8][kRgEB];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int r = min(rb + 4 * u, r1 - 1);
                xv[u] = x[(size_t)r * d + col];
#pragma unroll
                for (int j = 0; j < kRgEB; ++j) w[u][j] = dl[(size_t)r * E + min(e0 + j, E - 1)];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int j = 0; j < kRgEB; ++j)
                    acc[j] = fmaf(rb + 4 * u < r1 ? xv[u] : 0.f, e0 + j < E ? w[u][j] : 0.f,
                                  acc[j]);
        }
#pragma unroll
        for (int j = 0; j < kRgEB; ++j) red[p][c][j] = acc[j];
        __syncthreads();
        for (int i = t; i < 64 * kRgEB; i += 256) {
            const int cc = i / kRgEB, j = i % kRgEB, oc = cb * 64 + cc;
            if (oc < d && e0 + j < E)
                P[((size_t)z * d + oc) * E + e0 + j] =
                    ((red[0][cc][j] + red[1][cc][j]) + red[2][cc][j]) + red[3][cc][j];
        }
        __syncthreads();
    }
    if (CS && cb == 0)
        for (int e = t; e < E; e += 256) {
            float sum = 0.f;
            for (int rb = r0; rb < r1; rb += 16) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) v[u] = probs[(size_t)min(rb + u, r1 - 1) * E + e];
#pragma unroll
                for (int u = 0; u < 16; ++u)
                    if (rb + u < r1) sum += v[u];
            }
            CS[(size_t)z * E + e] = sum;
        }
}

// base + sum over z < nz (in order) of P[z n + i], 16 chunks' loads in
// flight at a time.
__device__ inline float sum_chunks(const float *P, int nz, int n, int i, float base) {
    float v = 0.f;
    for (int z0 = 0; z0 < nz; z0 += 16) {
        float q[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) q[u] = P[(size_t)min(z0 + u, nz - 1) * n + i];
#pragma unroll
        for (int u = 0; u < 16; ++u)
            if (z0 + u < nz) v += q[u];
    }
    return base + v;
}

// dwr (+)= sum over z (in order) of P[z] (n = d E floats); with aux, one
// more workgroup adds the column sums CS over z (in order) and takes
// aux = E sum_e f_e P_e, f_e = counts[e] / (T k), P_e = colsum[e] / T.
__global__ __launch_bounds__(256) void router_grad_final_kernel(const float *P, int nz, int n,
                                                                int accumulate, float *dwr,
                                                                const float *CS,
                                                                const int *counts, int T, int E,
                                                                int k, float *aux) {
    __shared__ float cs[kMaxExperts];
    const int nb = (n + 255) / 256;
    if ((int)blockIdx.x < nb) {
        const int i = blockIdx.x * 256 + threadIdx.x;
        if (i < n) dwr[i] = sum_chunks(P, nz, n, i, accumulate ? dwr[i] : 0.f);
        return;
    }
    for (int e = threadIdx.x; e < E; e += 256) cs[e] = sum_chunks(CS, nz, E, e, 0.f);
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.f;
        for (int e = 0; e < E; ++e)
            total = fmaf((float)counts[e] / ((float)T * (float)k), cs[e] / (float)T, total);
        *aux = (float)E * total;
    }
}

// H = silu(G) * U, the forward's SwiGLU.
__global__ __launch_bounds__(256) void act_kernel(const float *G, const float *U, float *H,
                                                  size_t n) {
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        H[i] = swiglu_fast(G[i], U[i]);
}

// In place: G <- dG = dH U silu'(G), U <- dU = dH silu(G).
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(float *G, float *U, const float *dH,
                                                         size_t n) {
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float g = G[i], u = U[i], dh = dH[i];
        const float s = 1.0f / (1.0f + expf(-g));
        G[i] = dh * u * fmaf(g * s, 1.0f - s, s);
        U[i] = dh * g * s;
    }
}

// Where an expert GEMM left its [T k x d] rows: by dispatch position, or by
// slot as ns partials ys apart (summed in order).
// With pieces (a stream-K GEMM): slot a's columns [pcols j, pcols (j + 1))
// hold pieces[a * (d / pcols) + j] partials instead of ns.
struct SlotRows {
    const float *p;
    int by_slot, ns;
    size_t ys;
    const int *pieces = nullptr;
    int pcols = 0;
    __device__ int count(int a, int d, int c) const {
        return pieces ? pieces[(size_t)a * (d / pcols) + c / pcols] : ns;
    }
    // The partials of (row, column c) added in order; the first 8 are
    // loaded together (clamped, masked), so none waits for another.
    __device__ float at(int pos, int a, int d, int c) const {
        const float *r = p + (size_t)(by_slot ? a : pos) * d + c;
        const int n = max(count(a, d, c), 1);
        float q[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) q[u] = r[(size_t)min(u, n - 1) * ys];
        float v = q[0];
#pragma unroll
        for (int u = 1; u < 8; ++u)
            if (u < n) v += q[u];
        for (int s = 8; s < n; ++s) v += r[(size_t)s * ys];
        return v;
    }
    // The same for the four columns c .. c + 3 (16-byte aligned).
    __device__ fx4 at4(int row, int a, int d, int c) const {
        const float *r = p + (size_t)row * d + c;
        const int n = max(count(a, d, c), 1);
        fx4 q[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) q[u] = *reinterpret_cast<const fx4 *>(r + (size_t)min(u, n - 1) * ys);
        fx4 v = q[0];
#pragma unroll
        for (int u = 1; u < 8; ++u)
            if (u < n) v += q[u];
        for (int s = 8; s < n; ++s) v += *reinterpret_cast<const fx4 *>(r + (size_t)s * ys);
        return v;
    }
};

// One wave per dispatch position pos (slot a = perm[pos], token t = a / k):
// dgw[a] = <Y(a), dout[t]> (lane-strided partial sums, then a butterfly),
// dY[pos] = gw[a] dout[t], inv[a] = pos.
__global__ __launch_bounds__(256) void slot_kernel(SlotRows Y, const float *dout,
                                                   const float *gw, const int *perm, int k, int d,
                                                   int n, float *dgw, float *dY, int *inv) {
    const int pos = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (pos >= n) return;
    const int a = perm[pos], t = a / k;
    const float w = gw[a];
    const float *go = dout + (size_t)t * d;
    float *dy = dY + (size_t)pos * d;
    float s = 0.f;
    // Four columns per step, their loads issued together.
    for (int c0 = lane; c0 < d; c0 += 256) {
        float v[4], y[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = min(c0 + 64 * u, d - 1);
            v[u] = go[c];
            y[u] = Y.at(pos, a, d, c);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (c0 + 64 * u < d) {
                s = fmaf(y[u], v[u], s);
                dy[c0 + 64 * u] = w * v[u];
            }
    }
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) {
        dgw[a] = s;
        inv[a] = pos;
    }
}

// Eight lanes per token: dlogits [T x E] from dgw through the gate
// renormalisation, the aux term and the softmax.  Every lane of a token
// loads its ids and dgw (kMaxTopK of each, clamped, masked) and the
// probabilities of its experts e = g, g + 8, ... (g = lane % 8) at once, then
// the selected probabilities; S, c and dp(e) are summed in slot order and
// the dot over the experts in expert order (through shuffles), as one thread
// per token would.
// JN experts per lane: 16 up to 128 experts, 32 up to 256.
constexpr int kRbG = 8;
template <int JN>
__global__ __launch_bounds__(256) void router_bwd_kernel(const float *probs, const int *ids,
                                                         const float *dgw,
                                                         const int *counts, int T, int E, int k,
                                                         float aux_coef, float *dlogits) {
    const int gid = blockIdx.x * 256 + threadIdx.x;
    const int t = gid / kRbG, g = gid % kRbG;
    const int tc = min(t, T - 1);
    const float *p = probs + (size_t)tc * E;
    int id[kMaxTopK];
    float dg[kMaxTopK], ps[kMaxTopK];
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) {
        const size_t q = (size_t)tc * k + min(s, k - 1);
        id[s] = ids[q];
        dg[s] = dgw[q];
    }
    // The aux term's counts enter as differences from a fixed count (the
    // softmax gradient p (dp - sum p dp) does not change when every dp moves
    // by one constant): near-uniform loads then give small exact values, so
    // the subtraction below does not cancel the large common part in fp32.
    const int cref = (int)(((long long)T * k) / E);
    float pv[JN], cn[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j)
        if (kRbG * j < E) {
            const int e = min(g + kRbG * j, E - 1);
            pv[j] = p[e];
            cn[j] = (float)(counts[e] - cref);
        }
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) ps[s] = p[id[s]];
    // c = sum over slots of dgw * (p / S), the renormalised weights taken
    // as p / S here: at top-1 that is exactly 1, so the slot term (dgw - c)
    // / S vanishes exactly as its derivative does (the stored gate weight,
    // p * (1 / S), can sit an ulp below 1).
    float S = 0.f, c = 0.f;
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s)
        if (s < k) S += ps[s];
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s)
        if (s < k) c = fmaf(dg[s], ps[s] / S, c);
    const float aux_scale = aux_coef * (float)E / ((float)T * (float)T * (float)k);
    float dpv[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j)
        if (kRbG * j < E) {
            const int e = g + kRbG * j;
            float v = aux_scale * cn[j];
#pragma unroll
            for (int s = 0; s < kMaxTopK; ++s)
                if (s < k && id[s] == e) v += (dg[s] - c) / S;
            dpv[j] = v;
        }
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < JN; ++j)
        if (kRbG * j < E)
#pragma unroll
            for (int q = 0; q < kRbG; ++q)
                if (kRbG * j + q < E)
                    dot = fmaf(__shfl(dpv[j], q, kRbG), __shfl(pv[j], q, kRbG), dot);
    if (t >= T) return;
#pragma unroll
    for (int j = 0; j < JN; ++j)
        if (g + kRbG * j < E) dlogits[(size_t)t * E + g + kRbG * j] = pv[j] * (dpv[j] - dot);
}

// dx[t][c..c+3] = sum over slots (in order) of dXr(t k + s), plus
// sum_e dlogits[t][e] wr[c][e] (read from wrT [E x d]); one thread per 4
// columns (d % 4 == 0).
__global__ __launch_bounds__(256) void dx_kernel(SlotRows dXr, const int *inv,
                                                 const float *dlogits, const float *wrT, int T,
                                                 int d, int E, int k, int accumulate, float *dx) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int d4 = d / 4;
    if (i >= (size_t)T * d4) return;
    const int t = (int)(i / d4), c = 4 * (int)(i % d4);
    fx4 v = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < k; ++s) {
        const int a = t * k + s;
        v += dXr.at4(dXr.by_slot ? a : inv[a], a, d, c);
    }
    fx4 rr = {0.f, 0.f, 0.f, 0.f};
    const float *dl = dlogits + (size_t)t * E;
    // Eight experts per step, their loads issued together.
    for (int e0 = 0; e0 < E; e0 += 8) {
        float gv[8];
        fx4 wv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = min(e0 + u, E - 1);
            gv[u] = dl[e];
            wv[u] = *reinterpret_cast<const fx4 *>(wrT + (size_t)e * d + c);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (e0 + u < E)
#pragma unroll
                for (int j = 0; j < 4; ++j) rr[j] = fmaf(gv[u], wv[u][j], rr[j]);
    }
    v += rr;
    fx4 *o = reinterpret_cast<fx4 *>(dx + (size_t)t * d + c);
    *o = accumulate ? *o + v : v;
}

unsigned blocks_for(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256, 16384); }

#define BWD_TRY(x)                               \
    do {                                         \
        hipError_t e_ = (x);                     \
        if (e_ != hipSuccess) return e_;         \
    } while (0)

}  // namespace

bool backward_engine_ok(int d, int F) { return d % 64 == 0 && F % 64 == 0; }

size_t backward_dh_floats(size_t n, int d, int F, int E) {
    return std::max(n * (size_t)F, (size_t)d * E + E);
}

size_t backward_tail_floats(int d, int F, int max_mtiles) {
    if (!backward_engine_ok(d, F)) return 0;
    const int g = std::max(gateup_tail_groups(2 * F, d, max_mtiles), gateup_tail_groups(F, d, max_mtiles));
    return (size_t)g * kGemmBM * 256;
}

int backward_slot_splits(int d, int F, int max_mtiles, size_t n) {
    if (!backward_engine_ok(d, F)) return 1;
    return std::max(down_plan(d, F, max_mtiles, n).slots, down_plan(d, 2 * F, max_mtiles, n).slots);
}

hipError_t launch_moe_backward(const BackwardArgs &b, hipStream_t s) {
    const int d = b.d, F = b.F, E = b.E, k = b.k, T = b.T;
    const size_t n = (size_t)T * k;
    if (T <= 0) return hipSuccess;
    if (d % 16 || F % 16) return hipErrorInvalidValue;   // (dx_kernel: d % 4)
    auto rows = [&](auto gather, auto bt, const float *A, int lda, const float *B, size_t b_e,
                    int ldb, float *C, int K, int N, int accumulate) {
        RowsGemm g{A, lda, b.perm, k, B, b_e, ldb, C, N, b.offsets, b.tile_off, b.tile_expert,
                   E, K, N, b.max_mtiles, accumulate};
        const unsigned grid = (unsigned)(b.max_mtiles * ((N + kRN - 1) / kRN));
        if (K % kMK == 0)
            hipLaunchKernelGGL((rows_mfma_kernel<decltype(gather)::value, decltype(bt)::value>),
                               dim3(grid), dim3(128), 0, s, g);
        else
            hipLaunchKernelGGL((rows_gemm_kernel<decltype(gather)::value, decltype(bt)::value>),
                               dim3(grid), dim3(256), 0, s, g);
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    const size_t nd = n * d;
    const unsigned slot_grid = (unsigned)((n + 3) / 4);
    SlotRows dXr{b.Y, 0, 1, 0};
    if (b.wgu) {
        // The forward's tile engine on the packed weights and their unit
        // transposes; G and U adjacent as GU [n x 2F] in packed column order.
        float *GU = b.G;
        BWD_TRY(launch_transpose_units(b.wdT, b.wdTT, d, F, E, s));
        BWD_TRY(launch_transpose_units(b.wgu, b.wguT, 2 * F, d, E, s));
        GemmArgs g{};
        g.perm = b.perm; g.topk = k; g.offsets = b.offsets; g.tile_off = b.tile_off;
        g.tile_expert = b.tile_expert; g.E = E; g.max_mtiles = b.max_mtiles;
        // Recompute GU and H, then Y by slot (split partials).
        GemmArgs gu = g;
        gu.a = b.x; gu.b = b.wgu; gu.c = GU; gu.K = d; gu.N = 2 * F; gu.ldc = 2 * F;
        gu.c2 = b.H; gu.ldc2 = F;
        if (b.tail_part) {
            gu.tail_groups = gateup_tail_groups(2 * F, d, b.max_mtiles);
            gu.tail_part = b.tail_part;
        }
        BWD_TRY(launch_gemm_bwd(gu, 2, s));
        BWD_TRY(launch_tail_fixup(gu, 2, s));
        // (Y and dX: down-projection shapes, by slot with split partials or
        // stream-K pieces, moe::down_plan; one piece-count table serves both
        // in turn.)
        const DownPlan py = down_plan(d, F, b.max_mtiles, n);
        GemmArgs gy = g;
        gy.a = b.H; gy.b = b.wdT; gy.c = b.Y; gy.K = F; gy.N = d; gy.ldc = d;
        gy.ksplit = py.slots; gy.split_stride = nd;
        gy.streamk = py.streamk; gy.sk_groups = py.groups; gy.pieces = b.pieces;
        BWD_TRY(launch_gemm_down(gy, s));
        hipLaunchKernelGGL(slot_kernel, dim3(slot_grid), dim3(256), 0, s,
                           SlotRows{b.Y, 1, py.slots, nd, py.streamk ? b.pieces : nullptr, 256},
                           b.dout, b.gw, b.perm, k, d, (int)n, b.dgw, b.dY, b.inv);
        // dH -> dG, dU in place over GU; dXr = dGU wgu^T by slot (over Y).
        GemmArgs gh = g;
        gh.a = b.dY; gh.b = b.wdTT; gh.c = GU; gh.K = d; gh.N = F; gh.ldc = 2 * F;
        if (b.tail_part) {
            gh.tail_groups = gateup_tail_groups(F, d, b.max_mtiles);
            gh.tail_part = b.tail_part;
        }
        BWD_TRY(launch_gemm_bwd(gh, 3, s));
        BWD_TRY(launch_tail_fixup(gh, 3, s));
        const DownPlan px = down_plan(d, 2 * F, b.max_mtiles, n);
        GemmArgs gx = g;
        gx.a = GU; gx.b = b.wguT; gx.c = b.Y; gx.K = 2 * F; gx.N = d; gx.ldc = d;
        gx.ksplit = px.slots; gx.split_stride = nd;
        gx.streamk = px.streamk; gx.sk_groups = px.groups; gx.pieces = b.pieces;
        BWD_TRY(launch_gemm_down(gx, s));
        dXr = SlotRows{b.Y, 1, px.slots, nd, px.streamk ? b.pieces : nullptr, 256};
    } else {
        // Recompute: G, U (gathered x rows), H, Y.
        rows(T_{}, F_{}, b.x, d, b.wg, (size_t)d * F, F, b.G, d, F, 0);
        rows(T_{}, F_{}, b.x, d, b.wu, (size_t)d * F, F, b.U, d, F, 0);
        hipLaunchKernelGGL(act_kernel, dim3(blocks_for(n * F)), dim3(256), 0, s, b.G, b.U, b.H,
                           n * F);
        rows(F_{}, F_{}, b.H, F, b.wd, (size_t)F * d, d, b.Y, F, d, 0);
        // Slots: dgw, dY, the slot -> position map.
        hipLaunchKernelGGL(slot_kernel, dim3(slot_grid), dim3(256), 0, s, SlotRows{b.Y, 0, 1, 0},
                           b.dout, b.gw, b.perm, k, d, (int)n, b.dgw, b.dY, b.inv);
        // Experts: dH, dG and dU (in place over G, U), dXr (over Y).
        rows(F_{}, T_{}, b.dY, d, b.wd, (size_t)F * d, d, b.dH, d, F, 0);
        hipLaunchKernelGGL(swiglu_bwd_kernel, dim3(blocks_for(n * F)), dim3(256), 0, s, b.G,
                           b.U, b.dH, n * F);
        rows(F_{}, T_{}, b.G, F, b.wg, (size_t)d * F, F, b.Y, F, d, 0);
        rows(F_{}, T_{}, b.U, F, b.wu, (size_t)d * F, F, b.Y, F, d, 1);
    }
    // Router and dx.
    {
        const dim3 grid((unsigned)(((size_t)T * kRbG + 255) / 256));
        if (E <= 128)
            hipLaunchKernelGGL(router_bwd_kernel<128 / kRbG>, grid, dim3(256), 0, s, b.probs, b.ids,
                               b.dgw, b.counts, T, E, k, b.aux_coef, b.dlogits);
        else
            hipLaunchKernelGGL(router_bwd_kernel<kMaxExperts / kRbG>, grid, dim3(256), 0, s, b.probs,
                               b.ids, b.dgw, b.counts, T, E, k, b.aux_coef, b.dlogits);
    }
    hipLaunchKernelGGL(dx_kernel, dim3((unsigned)(((size_t)T * (d / 4) + 255) / 256)), dim3(256),
                       0, s, dXr, b.inv,
                       b.dlogits, b.wrT, T, d, E, k, b.accumulate, b.dx);
    // Weight gradients over each expert's rows; the router's over all tokens.
    auto reduce = [&](auto gather, const float *A, int lda, const float *B, int ldb, float *C,
                      size_t c_e, int M, int N, const int *offsets, int nrows, int chunk,
                      int groups, int accumulate) {
        ReduceGemm g{A, lda, b.perm, k, B, ldb, C, c_e, N, offsets, nrows, chunk, M, N,
                     accumulate, M % 4 == 0 && lda % 4 == 0, N % 4 == 0 && ldb % 4 == 0};
        dim3 grid((unsigned)((N + kQN - 1) / kQN), (unsigned)((M + kQM - 1) / kQM),
                  (unsigned)groups);
        hipLaunchKernelGGL((reduce_gemm_kernel<decltype(gather)::value>), grid, dim3(256), 0, s,
                           g);
    };
    if (b.wgu) {
        auto mfma = [&](auto gather, const float *A, int lda, const float *B, int ldb, float *C,
                        float *C_up, int M, int N, int ldc) {
            ReduceGemm g{A, lda, b.perm, k, B, ldb, C, (size_t)M * ldc, ldc, b.offsets, 0, 0, M,
                         N, b.accumulate, 1, 1, C_up};
            // The widest tile that still gives every CU a workgroup.
            const long cus = device_cus();
            auto tiles = [&](int wm, int wn) { return (long)(M / (64 * wm)) * (N / (64 * wn)) * E; };
            // The wider tiles run 8 waves (two per SIMD): 128 x 128 as 64 x 32
            // blocks 4 % faster than 4 waves of 64 x 64, 128 x 64 as 32 x 32
            // blocks 8 % faster than 4 waves of 64 x 32.
            auto go = [&](auto wm, auto wn) {
                constexpr int WM = decltype(wm)::value, WN = decltype(wn)::value;
                constexpr int NWM = WM == 2 && WN == 1 ? 4 : 2;
                constexpr int NWN = WN == 2 ? 4 : 2;
                hipLaunchKernelGGL((reduce_mfma_kernel<decltype(gather)::value, WM, WN, NWM, NWN>),
                                   dim3((unsigned)(N / (64 * WN)), (unsigned)(M / (64 * WM)),
                                        (unsigned)E),
                                   dim3(64 * NWM * NWN), 0, s, g);
            };
            using I1 = std::integral_constant<int, 1>;
            using I2 = std::integral_constant<int, 2>;
            if (M % 128 == 0 && N % 128 == 0 && tiles(2, 2) >= cus) go(I2{}, I2{});
            else if (M % 128 == 0 && tiles(2, 1) >= cus)           go(I2{}, I1{});
            else if (N % 128 == 0 && tiles(1, 2) >= cus)           go(I1{}, I2{});
            else                                                    go(I1{}, I1{});
        };
        mfma(F_{}, b.H, F, b.dY, d, b.dwd, nullptr, F, d, d);
        // dW_g and dW_u in one launch over GU's 2F packed columns.
        mfma(T_{}, b.x, d, b.G, 2 * F, b.dwg, b.dwu, d, 2 * F, F);
    } else {
        reduce(F_{}, b.H, F, b.dY, d, b.dwd, (size_t)F * d, F, d, b.offsets, 0, 0, E,
               b.accumulate);
        reduce(T_{}, b.x, d, b.G, F, b.dwg, (size_t)d * F, d, F, b.offsets, 0, 0, E,
               b.accumulate);
        reduce(T_{}, b.x, d, b.U, F, b.dwu, (size_t)d * F, d, F, b.offsets, 0, 0, E,
               b.accumulate);
    }
    // The router's over all tokens (and the aux loss's column sums), in row
    // chunks whose partials (in dH, free by now) are then added in chunk
    // order: enough chunks for about one workgroup per CU, as many as dH
    // holds (it holds one chunk's at least: backward_dh_floats).
    const int ncb = (d + 63) / 64;
    const size_t cap = backward_dh_floats(n, d, F, E);
    int R = std::max(16, (int)((T + std::max(1, 256 / ncb) - 1) / std::max(1, 256 / ncb)));
    while (R < T && (size_t)((T + R - 1) / R) * ((size_t)d * E + E) > cap) R *= 2;
    const int nz = (T + R - 1) / R;
    float *P = b.dH, *CS = b.aux ? b.dH + (size_t)nz * d * E : nullptr;
    hipLaunchKernelGGL(router_grad_kernel, dim3((unsigned)ncb, (unsigned)nz), dim3(256), 0, s,
                       b.x, b.dlogits, b.probs, T, d, E, R, P, CS);
    const int nb = (int)((d * E + 255) / 256);
    hipLaunchKernelGGL(router_grad_final_kernel, dim3((unsigned)(nb + (b.aux ? 1 : 0))), dim3(256),
                       0, s, P, nz, d * E, b.accumulate, b.dwr, CS, b.counts, T, E, k, b.aux);
    return hipGetLastError();
}

}  // namespace moe
