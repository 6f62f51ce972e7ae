/*
 * moe_oracle.c — TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of murderface-cpu/llm.c's mixture-of-experts layer, used
 * by the tests, smoke() and the CPU-baseline leg of bench.py to check and
 * time the device results.
 * Nothing in the shipped library links, loads or calls this file.
 *
 * What it restates (reference paths relative to the reference repo root):
 *   orc_router_logits   src/matrix.c:357-400 (mat_mul, AVX2+FMA build) with
 *                       axpy_avx2fma src/matrix.c:278-303; optional bias add
 *                       as mat_mul_add src/matrix.c:418-439
 *   orc_exp_poly        exp_avx2 src/matrix.c:82-116 (one lane), under the
 *                       FTZ/DAZ mode that -ffast-math executables run with
 *   orc_expf            glibc 2.35 expf (sysdeps/ieee754/flt-32/e_expf.c, the
 *                       exp2f_data table design), which the reference calls
 *                       in scalar tails (src/matrix.c:568, :652)
 *   orc_softmax_rows    softmax_rows src/matrix.c:529-586 with hsum256
 *                       include/simd.h:110-121
 *   orc_topk            src/transformer.c:317-337 (selection, tie-break,
 *                       renormalisation)
 *   orc_dispatch        stable counting sort of expert ids; the reference has
 *                       no grouping (token-major loop src/transformer.c:312),
 *                       this is the canonical permutation the GPU must match
 *   orc_swiglu          swiglu src/matrix.c:618-655 (source semantics)
 *   orc_moe_forward     moe_forward src/transformer.c:287-366 with
 *                       ffn_forward src/transformer.c:157-165
 *   orc_moe_forward_f64 textbook fp64 MoE layer (tolerance reference)
 *   orc_rms_norm        rms_norm src/matrix.c:666-711 (AVX2+FMA build) as
 *                       the reference build compiles it, except 1/sqrt:
 *                       see the function
 *   orc_attn_decode     the attention half of inference_step
 *                       src/inference.c:252-308 (source semantics) for B
 *                       sequences, each with its own K/V cache and position
 *
 * Numerics: compile with -ffp-contract=off; every fused multiply-add the
 * reference performs is an explicit fmaf()/fma() here.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <stdio.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <xmmintrin.h>
#endif

#include "../llm.c_amd/csrc/synth.h"

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* Flush a float result that is subnormal to a signed zero (FTZ). */
static inline float ftz(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7f800000u) == 0) return u2f(u & 0x80000000u);
    return x;
}

/* ------------------------------------------------------------------------
 * FTZ/DAZ switch for the calling thread: -ffast-math executables start with
 * both bits set (crtfastmath), so the compiled reference is called under it.
 * ---------------------------------------------------------------------- */
int orc_set_ftz_daz(int on) {
#if defined(__x86_64__)
    unsigned int csr = _mm_getcsr();
    unsigned int old = csr;
    if (on) csr |= 0x8040u; else csr &= ~0x8040u;
    _mm_setcsr(csr);
    return (int)((old & 0x8040u) == 0x8040u);
#else
    (void)on; return 0;
#endif
}

/* Every entry point runs under FTZ/DAZ, as the reference executables do. */
static inline unsigned int fpenv_enter(void) {
#if defined(__x86_64__)
    unsigned int csr = _mm_getcsr();
    _mm_setcsr(csr | 0x8040u);
    return csr;
#else
    return 0;
#endif
}
static inline void fpenv_leave(unsigned int csr) {
#if defined(__x86_64__)
    _mm_setcsr(csr);
#else
    (void)csr;
#endif
}

/* ------------------------------------------------------------------------
 * Router logits: out[t][e] = sum_k x[t][k] * Wr[k][e] as ONE fused-multiply-
 * add chain per element, k ascending from +0.0f, skipping x == 0
 * (src/matrix.c:381-400 zeroes out, then for each k with a_ik != 0 calls
 * axpy_avx2fma, src/matrix.c:278-303, whose every lane is an FMA).
 * Optional bias: out[t][e] += b[e] afterwards (mat_mul_add, :418-439).
 * ---------------------------------------------------------------------- */
void orc_router_logits(const float *x, const float *wr, const float *bias,
                       int T, int d, int E, float *out) {
    unsigned int csr = fpenv_enter();
    for (int t = 0; t < T; ++t) {
        float *o = out + (size_t)t * E;
        for (int e = 0; e < E; ++e) o[e] = 0.0f;
        for (int k = 0; k < d; ++k) {
            float a = x[(size_t)t * d + k];
            if (a == 0.0f) continue;
            const float *b = wr + (size_t)k * E;
            for (int e = 0; e < E; ++e) o[e] = fmaf(a, b[e], o[e]);
        }
        if (bias)
            for (int e = 0; e < E; ++e) o[e] = o[e] + bias[e];
    }
    fpenv_leave(csr);
}

/* Generic chain matmul (same recipe), used for the expert FFN products. */
static void chain_matmul(const float *A, const float *B, float *C,
                         int M, int K, int N) {
    for (int i = 0; i < M; ++i) {
        float *c = C + (size_t)i * N;
        for (int j = 0; j < N; ++j) c[j] = 0.0f;
        for (int k = 0; k < K; ++k) {
            float a = A[(size_t)i * K + k];
            if (a == 0.0f) continue;
            const float *b = B + (size_t)k * N;
            for (int j = 0; j < N; ++j) c[j] = fmaf(a, b[j], c[j]);
        }
    }
}

/* ------------------------------------------------------------------------
 * exp_avx2, one lane (src/matrix.c:82-116): clamp to [-88, 88], z = v*log2e,
 * n = floor(z), f = z - n, 2^f by a degree-6 Horner chain of FMAs, times
 * 2^n built from exponent bits.  Under DAZ the scale 2^-127 (exponent field
 * 0) reads as zero, and FTZ flushes a subnormal product.
 * ---------------------------------------------------------------------- */
float orc_exp_poly(float v) {
    v = fminf(fmaxf(ftz(v), -88.0f), 88.0f);   /* DAZ on the input */
    float z = ftz(v * 1.4426950408f);
    float n = floorf(z);
    float f = ftz(z - n);
    float p = 0.0001540353f;
    p = fmaf(p, f, 0.0013333558f);
    p = fmaf(p, f, 0.0096181292f);
    p = fmaf(p, f, 0.0555041086f);
    p = fmaf(p, f, 0.2402265069f);
    p = fmaf(p, f, 0.6931471806f);
    p = fmaf(p, f, 1.0000000000f);
    int ni = (int)n;
    uint32_t sb = (uint32_t)(ni + 127) << 23;
    if ((sb & 0x7f800000u) == 0) return 0.0f;   /* DAZ: 2^-127 reads as 0 */
    return ftz(p * u2f(sb));
}

/* ------------------------------------------------------------------------
 * glibc expf (glibc 2.35, sysdeps/ieee754/flt-32/e_expf.c; design from
 * ARM optimized-routines): with N = 32,
 *   z = x * N/ln2 (double); k = round-to-nearest(z) via the 1.5*2^52 shift;
 *   r = z - k; s = 2^(k/N) from a 32-entry table of 2^(i/N) with the
 *   exponent of k/N added into the bits; poly(r) = C0 r^3 + C1 r^2 + C2 r + 1
 *   evaluated as (C0 r + C1) r^2 + (C2 r + 1); result (float)(poly * s).
 * The x86-64 build selected on FMA hardware (e_expf-fma) is compiled with FMA
 * contraction: both uses of x*N/ln2 are additions, so the product is fused
 * into each of them, and the three polynomial a*b+c steps are fused too.
 * Special cases as in glibc: -inf -> 0, x < -103.97 -> 0, NaN -> x + x,
 * x > 88.72 -> inf.  Subnormal results are flushed (FTZ, as under
 * -ffast-math executables).
 * ---------------------------------------------------------------------- */
static uint64_t expf_tab[32];
static int expf_tab_ready = 0;

static void expf_init(void) {
    if (expf_tab_ready) return;
    for (int i = 0; i < 32; ++i) {
        /* 2^(i/32) correctly rounded to double via long double. */
        long double v = exp2l((long double)i / 32.0L);
        double dv = (double)v;
        expf_tab[i] = d2u(dv) - ((uint64_t)i << 47);
    }
    expf_tab_ready = 1;
}

uint64_t orc_expf_table_entry(int i) { expf_init(); return expf_tab[i & 31]; }

float orc_expf_raw(float x, int fused) {
    expf_init();
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double SHIFT = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint32_t ax = f2u(x) & 0x7fffffffu;
    if ((ax >> 20) >= (f2u(88.0f) >> 20)) {
        if (f2u(x) == f2u(-INFINITY)) return 0.0f;
        if (ax >= 0x7f800000u) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double xd = (double)x;
    double z, kd, r;
    uint64_t ki;
    if (fused) {
        /* Both uses of InvLn2N*xd are additions, so the FMA build fuses the
         * product into each of them. */
        kd = fma(InvLn2N, xd, SHIFT);
        ki = d2u(kd);
        kd -= SHIFT;
        r = fma(InvLn2N, xd, -kd);
    } else {
        z = InvLn2N * xd;
        kd = z + SHIFT;
        ki = d2u(kd);
        kd -= SHIFT;
        r = z - kd;
    }
    uint64_t t = expf_tab[ki % 32];
    t += ki << (52 - 5);
    double s = u2d(t);
    double y;
    if (fused) {
        double zz = fma(C0, r, C1);
        double r2 = r * r;
        double yy = fma(C2, r, 1.0);
        yy = fma(zz, r2, yy);
        y = yy * s;
    } else {
        double zz = C0 * r + C1;
        double r2 = r * r;
        double yy = C2 * r + 1.0;
        yy = zz * r2 + yy;
        y = yy * s;
    }
    return (float)y;
}

float orc_expf(float x) { return ftz(orc_expf_raw(x, 1)); }

void orc_expf_array(const float *x, float *y, long long n) {
    expf_init();
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}

void orc_exp_poly_array(const float *x, float *y, long long n) {
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; ++i) y[i] = orc_exp_poly(x[i]);
}

/* Exhaustive check helper: compare orc_expf_raw against the host libm expf
 * for every float whose bit pattern is in [lo, hi]; returns the mismatch
 * count and the first mismatching pattern. */
long long orc_expf_compare_libm(uint32_t lo, uint32_t hi, int fused,
                                uint32_t *first_bad) {
    expf_init();
    long long bad = 0;
    uint32_t first = 0;
    #pragma omp parallel for schedule(static) reduction(+:bad)
    for (long long b = (long long)lo; b <= (long long)hi; ++b) {
        float x = u2f((uint32_t)b);
        float a = orc_expf_raw(x, fused);
        float c = expf(x);
        if (f2u(a) != f2u(c) && !(a != a && c != c)) {
            ++bad;
            #pragma omp critical
            { if (first == 0 || (uint32_t)b < first) first = (uint32_t)b; }
        }
    }
    if (first_bad) *first_bad = first;
    return bad;
}

/* ------------------------------------------------------------------------
 * softmax_rows (src/matrix.c:529-586), AVX2+FMA build:
 *   max:  8-wide max from -1e38 over full blocks, lane tree, then scalar
 *         tail compares (:541-550);
 *   exp:  exp_avx2(x - max) on full blocks, lane-wise sums, hsum256 order
 *         ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)) (include/simd.h:110-121),
 *         then tail: libm expf and a sequential sum (:558-568);
 *   norm: blocks times (1/sum); tail divided by sum (:575-580).
 * `tail_recip` selects the tail form the compiled reference uses
 * (-freciprocal-math may turn the tail division into a multiply by 1/sum).
 * ---------------------------------------------------------------------- */
static int softmax_tail_recip = 0;
void orc_set_softmax_tail_recip(int on) { softmax_tail_recip = on; }

void orc_softmax_row(float *row, int cols) {
    int nb = cols / 8;
    float lane[8];
    for (int l = 0; l < 8; ++l) lane[l] = -1e38f;
    for (int b = 0; b < nb; ++b)
        for (int l = 0; l < 8; ++l) lane[l] = fmaxf(lane[l], row[8 * b + l]);
    /* _mm_max over hi/lo halves, then pairs: any order gives the same max. */
    float row_max = lane[0];
    for (int l = 1; l < 8; ++l) row_max = fmaxf(row_max, lane[l]);
    for (int j = nb * 8; j < cols; ++j) if (row[j] > row_max) row_max = row[j];

    float vs[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < nb; ++b)
        for (int l = 0; l < 8; ++l) {
            float ex = orc_exp_poly(row[8 * b + l] - row_max);
            row[8 * b + l] = ex;
            vs[l] = vs[l] + ex;
        }
    float sum = ((vs[0] + vs[4]) + (vs[1] + vs[5])) + ((vs[2] + vs[6]) + (vs[3] + vs[7]));
    for (int j = nb * 8; j < cols; ++j) {
        row[j] = orc_expf(row[j] - row_max);
        sum = sum + row[j];
    }
    float inv = 1.0f / sum;
    for (int j = 0; j < nb * 8; ++j) row[j] = row[j] * inv;
    for (int j = nb * 8; j < cols; ++j)
        row[j] = softmax_tail_recip ? row[j] * inv : row[j] / sum;
}

void orc_softmax_rows(float *m, int rows, int cols) {
    unsigned int csr = fpenv_enter();
    for (int i = 0; i < rows; ++i) orc_softmax_row(m + (size_t)i * cols, cols);
    fpenv_leave(csr);
}

/* ------------------------------------------------------------------------
 * Top-k (src/transformer.c:317-332): k rounds of argmax over experts not yet
 * chosen, best = -1.0f, best_e = 0, strict '>' (descending probability, ties
 * to the lowest index).  Gate weights (:334-337, :350): s = sum of chosen
 * probabilities in slot order; inv = s > 1e-9 ? 1/s : 0; w = p * inv.
 * ---------------------------------------------------------------------- */
void orc_topk(const float *probs, int T, int E, int k, int *ids, float *w) {
    unsigned int csr = fpenv_enter();
    for (int t = 0; t < T; ++t) {
        const float *p = probs + (size_t)t * E;
        int *id = ids + (size_t)t * k;
        for (int ki = 0; ki < k; ++ki) {
            float best = -1.0f;
            int best_e = 0;
            for (int e = 0; e < E; ++e) {
                int already = 0;
                for (int kj = 0; kj < ki; ++kj)
                    if (id[kj] == e) { already = 1; break; }
                if (!already && p[e] > best) { best = p[e]; best_e = e; }
            }
            id[ki] = best_e;
        }
        if (w) {
            float s = 0.0f;
            for (int ki = 0; ki < k; ++ki) s = s + p[id[ki]];
            float inv = (s > 1e-9f) ? 1.0f / s : 0.0f;
            for (int ki = 0; ki < k; ++ki) w[(size_t)t * k + ki] = p[id[ki]] * inv;
        }
    }
    fpenv_leave(csr);
}

/* ------------------------------------------------------------------------
 * Canonical dispatch: flatten a = t*k + ki; counts[e] = #{a : ids[a] == e};
 * offsets = exclusive scan (offsets[E] = T*k); pos[a] = offsets[e] +
 * #{a' < a : ids[a'] == e}; perm[pos[a]] = a.  A stable counting sort by
 * expert (tokens ascending, then slots ascending, within each expert).
 * ---------------------------------------------------------------------- */
void orc_dispatch(const int *ids, int T, int k, int E,
                  int *counts, int *offsets, int *perm) {
    long long n = (long long)T * k;
    for (int e = 0; e < E; ++e) counts[e] = 0;
    for (long long a = 0; a < n; ++a) counts[ids[a]]++;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int *cur = (int *)malloc(sizeof(int) * (size_t)(E > 0 ? E : 1));
    for (int e = 0; e < E; ++e) cur[e] = offsets[e];
    for (long long a = 0; a < n; ++a) perm[cur[ids[a]]++] = (int)a;
    free(cur);
}

/* ------------------------------------------------------------------------
 * swiglu (src/matrix.c:618-655), source semantics: on 8-element blocks
 * h = (g * 1/(1 + exp_avx2(-g))) * u (sigmoid_avx2/silu_avx2 :118-127), on
 * the scalar tail h = (g / (1 + expf(-g))) * u.
 * ---------------------------------------------------------------------- */
static void swiglu_impl(const float *g, const float *u, float *h, int n) {
    int nb = (n / 8) * 8;
    for (int i = 0; i < nb; ++i) {
        float x = g[i];
        float den = 1.0f + orc_exp_poly(-x);
        float sig = 1.0f / den;
        h[i] = (x * sig) * u[i];
    }
    for (int i = nb; i < n; ++i) {
        float x = g[i];
        h[i] = (x / (1.0f + orc_expf(-x))) * u[i];
    }
}

void orc_swiglu(const float *g, const float *u, float *h, int n) {
    unsigned int csr = fpenv_enter();
    swiglu_impl(g, u, h, n);
    fpenv_leave(csr);
}

/* ------------------------------------------------------------------------
 * rms_norm (src/matrix.c:666-711), AVX2+FMA build, per row:
 *   ss: lanes l < 8 of two 8-wide FMA accumulators over 16-column blocks
 *       (v0 takes columns 16b + l, v1 columns 16b + 8 + l), v0 += v1
 *       lane-wise, one more 8-column block into v0 if present, hsum256 fold
 *       ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)), then the scalar tail as FMAs;
 *   inv_rms = 1 / sqrt(ss / cols + eps), which the compiled reference (GCC
 *       -ffast-math, our build of matrix.c) evaluates as fma(ss, 1/cols, eps)
 *       followed by RSQRTSS and one Newton-Raphson step.  RSQRTSS's table is
 *       the x86 vendor's, so here (and on the GPU) 1/sqrt is correctly
 *       rounded instead: the two agree to an ulp or two, not bit for bit;
 *   y = (x * inv_rms) * w.
 * Columns not a multiple of 8 take a scalar tail here; the compiled
 * reference vectorises that tail loop (another summation order).
 * ---------------------------------------------------------------------- */
void orc_rms_norm(const float *x, const float *w, float eps, int rows, int cols, float *y) {
    unsigned int csr = fpenv_enter();
    const float rcp_cols = 1.0f / (float)cols;
    for (int i = 0; i < rows; ++i) {
        const float *xr = x + (size_t)i * cols;
        float *yr = y + (size_t)i * cols;
        float v0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, v1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int j = 0;
        for (; j + 16 <= cols; j += 16)
            for (int l = 0; l < 8; ++l) {
                v0[l] = fmaf(xr[j + l], xr[j + l], v0[l]);
                v1[l] = fmaf(xr[j + 8 + l], xr[j + 8 + l], v1[l]);
            }
        for (int l = 0; l < 8; ++l) v0[l] = v0[l] + v1[l];
        for (; j + 8 <= cols; j += 8)
            for (int l = 0; l < 8; ++l) v0[l] = fmaf(xr[j + l], xr[j + l], v0[l]);
        float ss = ((v0[0] + v0[4]) + (v0[1] + v0[5])) + ((v0[2] + v0[6]) + (v0[3] + v0[7]));
        for (; j < cols; ++j) ss = fmaf(xr[j], xr[j], ss);
        const float inv = 1.0f / sqrtf(fmaf(ss, rcp_cols, eps));
        for (int k = 0; k < cols; ++k) yr[k] = (xr[k] * inv) * w[k];
    }
    fpenv_leave(csr);
}

/* ------------------------------------------------------------------------
 * Decode attention (src/inference.c:252-308, source semantics) for sequence
 * b of B, in place on x[b] [d]; its caches K, V [max_seq x kd] get row pos.
 *   xn = rmsnorm_vec (:209-215): sequential sum of squares (FMA),
 *        inv = 1 / sqrtf(ss / d + eps), y = x * inv * w;
 *   q, k, v = matvec (:174-182): per output one FMA chain over the input
 *        index, ascending, inputs equal to zero skipped;
 *   RoPE at pos (:187-203) on q (nh heads) and k (nkv heads), tables given;
 *   K[pos] = k, V[pos] = v;
 *   head h (kv head h / gqa): s_j = vec_dot(q_h, K[j]) * scale, j <= pos
 *        (:133-155: lanes l < 8 of two 8-wide FMA accumulators over 16-blocks,
 *        added lane-wise, an 8-block, hsum256 fold, FMA tail);
 *        softmax_vec (:218-225): max, expf(s - max), sequential sum,
 *        times 1/sum; o_h = axpy over j ascending (FMA);
 *   x += matvec(W_O, o) element by element.
 * The reference's GCC build auto-vectorises rmsnorm_vec's loop for the
 * build machine, so its summation order is not fixed by the source.
 * ---------------------------------------------------------------------- */
static void matvec_chain(const float *mat, const float *vec, float *out, int M, int N) {
    for (int n = 0; n < N; ++n) out[n] = 0.0f;
    for (int i = 0; i < M; ++i) {
        const float vi = vec[i];
        if (vi == 0.0f) continue;
        for (int n = 0; n < N; ++n) out[n] = fmaf(vi, mat[(size_t)i * N + n], out[n]);
    }
}

static float dot_avx2(const float *a, const float *b, int n) {
    float v0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, v1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 8; ++l) {
            v0[l] = fmaf(a[i + l], b[i + l], v0[l]);
            v1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], v1[l]);
        }
    for (int l = 0; l < 8; ++l) v0[l] = v0[l] + v1[l];
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) v0[l] = fmaf(a[i + l], b[i + l], v0[l]);
    float r = ((v0[0] + v0[4]) + (v0[1] + v0[5])) + ((v0[2] + v0[6]) + (v0[3] + v0[7]));
    for (; i < n; ++i) r = fmaf(a[i], b[i], r);
    return r;
}

static void rope_pos(float *v, const float *cos_row, const float *sin_row, int heads, int hd) {
    const int half = hd / 2;
    for (int h = 0; h < heads; ++h) {
        float *w = v + (size_t)h * hd;
        for (int i = 0; i < half; ++i) {
            const float a = w[2 * i], b = w[2 * i + 1];
            w[2 * i] = a * cos_row[i] - b * sin_row[i];
            w[2 * i + 1] = a * sin_row[i] + b * cos_row[i];
        }
    }
}

void orc_attn_decode(float *x, int B, int d, int nh, int nkv, int hd, const float *rms_w,
                     float eps, const float *wq, const float *wk, const float *wv,
                     const float *wo, const float *cos_t, const float *sin_t, float *kc,
                     float *vc, int max_seq, const int *pos) {
    unsigned int csr = fpenv_enter();
    const int qd = nh * hd, kd = nkv * hd, gqa = nh / nkv, half = hd / 2;
    const float scale = 1.0f / sqrtf((float)hd);
    float *xn = malloc(sizeof(float) * d), *q = malloc(sizeof(float) * qd);
    float *kk = malloc(sizeof(float) * kd), *vv = malloc(sizeof(float) * kd);
    float *ho = malloc(sizeof(float) * qd), *ao = malloc(sizeof(float) * d);
    float *att = malloc(sizeof(float) * max_seq);
    for (int b = 0; b < B; ++b) {
        float *xb = x + (size_t)b * d;
        float *K = kc + (size_t)b * max_seq * kd, *V = vc + (size_t)b * max_seq * kd;
        const int p = pos[b];
        float ss = 0.0f;
        for (int i = 0; i < d; ++i) ss = fmaf(xb[i], xb[i], ss);
        const float inv = 1.0f / sqrtf(ss / (float)d + eps);
        for (int i = 0; i < d; ++i) xn[i] = xb[i] * inv * rms_w[i];
        matvec_chain(wq, xn, q, d, qd);
        matvec_chain(wk, xn, kk, d, kd);
        matvec_chain(wv, xn, vv, d, kd);
        rope_pos(q, cos_t + (size_t)p * half, sin_t + (size_t)p * half, nh, hd);
        rope_pos(kk, cos_t + (size_t)p * half, sin_t + (size_t)p * half, nkv, hd);
        memcpy(K + (size_t)p * kd, kk, sizeof(float) * kd);
        memcpy(V + (size_t)p * kd, vv, sizeof(float) * kd);
        for (int i = 0; i < qd; ++i) ho[i] = 0.0f;
        for (int h = 0; h < nh; ++h) {
            const int kvh = h / gqa;
            for (int j = 0; j <= p; ++j)
                att[j] = dot_avx2(q + (size_t)h * hd, K + (size_t)j * kd + kvh * hd, hd) * scale;
            float vmax = att[0];
            for (int j = 1; j <= p; ++j) if (att[j] > vmax) vmax = att[j];
            float sum = 0.0f;
            for (int j = 0; j <= p; ++j) { att[j] = expf(att[j] - vmax); sum = sum + att[j]; }
            const float rs = 1.0f / sum;
            for (int j = 0; j <= p; ++j) att[j] = att[j] * rs;
            float *oh = ho + (size_t)h * hd;
            for (int j = 0; j <= p; ++j)
                for (int t = 0; t < hd; ++t)
                    oh[t] = fmaf(att[j], V[(size_t)j * kd + kvh * hd + t], oh[t]);
        }
        matvec_chain(wo, ho, ao, qd, d);
        for (int i = 0; i < d; ++i) xb[i] = xb[i] + ao[i];
    }
    free(xn); free(q); free(kk); free(vv); free(ho); free(ao); free(att);
    fpenv_leave(csr);
}

/* RoPE tables as rope_buffer_init builds them (src/attention.c:151-167):
 * angle = pos / powf(theta, 2i/hd), cos and sin of it (host libm). */
void orc_rope_tables(int max_seq, int hd, float theta, float *cos_t, float *sin_t) {
    const int half = hd / 2;
    for (int p = 0; p < max_seq; ++p)
        for (int i = 0; i < half; ++i) {
            const float angle = (float)p / powf(theta, 2.f * (float)i / (float)hd);
            cos_t[(size_t)p * half + i] = cosf(angle);
            sin_t[(size_t)p * half + i] = sinf(angle);
        }
}

/* ------------------------------------------------------------------------
 * moe_forward (src/transformer.c:287-366):
 *   logits = x . W_router (+ bias), probs = softmax_rows(logits) -> probs_out,
 *   per token: top-k ids -> ids_out, gate weights, and for each slot
 *   y = ffn_forward(x_t) (gate/up chain products, swiglu, down chain
 *   product; src/transformer.c:157-165), out[t] += w * y as an FMA (the
 *   compiled `out_row[j] += w * y[j]` is contracted).
 * Experts are given as arrays of pointers to row-major [d x F] gate/up and
 * [F x d] down matrices.  Tokens are independent, so nthreads > 1 splits
 * the token loop without changing any result bit.
 * ---------------------------------------------------------------------- */
void orc_moe_forward(const float *x, int T, int d, int F, int E, int k,
                     const float *wr, const float *bias,
                     const float *const *wg, const float *const *wu,
                     const float *const *wd,
                     float *out, float *probs_out, int *ids_out, int nthreads) {
    float *probs = (float *)malloc(sizeof(float) * (size_t)T * E + 4);
    orc_router_logits(x, wr, bias, T, d, E, probs);
    orc_softmax_rows(probs, T, E);
    if (probs_out) memcpy(probs_out, probs, sizeof(float) * (size_t)T * E);
    int *ids = ids_out ? ids_out : (int *)malloc(sizeof(int) * (size_t)T * k + 4);
    float *w = (float *)malloc(sizeof(float) * (size_t)T * k + 4);
    orc_topk(probs, T, E, k, ids, w);
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
    #pragma omp parallel num_threads(nthreads)
#endif
    {
        unsigned int tcsr = fpenv_enter();
        float *g = (float *)malloc(sizeof(float) * (size_t)F);
        float *u = (float *)malloc(sizeof(float) * (size_t)F);
        float *y = (float *)malloc(sizeof(float) * (size_t)d);
#ifdef _OPENMP
        #pragma omp for schedule(dynamic, 1)
#endif
        for (int t = 0; t < T; ++t) {
            const float *xt = x + (size_t)t * d;
            float *o = out + (size_t)t * d;
            for (int j = 0; j < d; ++j) o[j] = 0.0f;
            for (int ki = 0; ki < k; ++ki) {
                int e = ids[(size_t)t * k + ki];
                chain_matmul(xt, wg[e], g, 1, d, F);
                chain_matmul(xt, wu[e], u, 1, d, F);
                swiglu_impl(g, u, g, F);
                chain_matmul(g, wd[e], y, 1, F, d);
                float wt = w[(size_t)t * k + ki];
                for (int j = 0; j < d; ++j) o[j] = fmaf(wt, y[j], o[j]);
            }
        }
        free(g); free(u); free(y);
        fpenv_leave(tcsr);
    }
    free(w);
    if (!ids_out) free(ids);
    free(probs);
}

/* Textbook fp64 layer for the tolerance analysis: same routing (ids given),
 * gate weights renormalised in double, silu(g) = g / (1 + exp(-g)). */
void orc_moe_forward_f64(const float *x, int T, int d, int F, int k,
                         const int *ids, const float *probs, int E,
                         const float *const *wg, const float *const *wu,
                         const float *const *wd, double *out) {
    double *g = (double *)malloc(sizeof(double) * (size_t)F);
    double *u = (double *)malloc(sizeof(double) * (size_t)F);
    for (int t = 0; t < T; ++t) {
        const float *xt = x + (size_t)t * d;
        double *o = out + (size_t)t * d;
        for (int j = 0; j < d; ++j) o[j] = 0.0;
        double s = 0.0;
        for (int ki = 0; ki < k; ++ki) s += probs[(size_t)t * E + ids[(size_t)t * k + ki]];
        for (int ki = 0; ki < k; ++ki) {
            int e = ids[(size_t)t * k + ki];
            double wt = probs[(size_t)t * E + e] / s;
            for (int f = 0; f < F; ++f) { g[f] = 0.0; u[f] = 0.0; }
            for (int c = 0; c < d; ++c) {
                double a = xt[c];
                const float *bg = wg[e] + (size_t)c * F;
                const float *bu = wu[e] + (size_t)c * F;
                for (int f = 0; f < F; ++f) { g[f] += a * bg[f]; u[f] += a * bu[f]; }
            }
            for (int f = 0; f < F; ++f) g[f] = g[f] / (1.0 + exp(-g[f])) * u[f];
            for (int f = 0; f < F; ++f) {
                double a = g[f];
                const float *bd = wd[e] + (size_t)f * d;
                for (int j = 0; j < d; ++j) o[j] += wt * a * bd[j];
            }
        }
    }
    free(g); free(u);
}

/* Synthetic tensors (same generator the GPU library uses on the device). */
void orc_synth_normal(float *out, long long n, unsigned long long seed,
                      unsigned long long stream, float mean, float std) {
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; ++i)
        out[i] = synth_normal(seed, stream, (uint64_t)i, mean, std);
}
