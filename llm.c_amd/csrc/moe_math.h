// moe_math.h — scalar device functions whose bits must match the reference's
// CPU arithmetic.  Contraction is off for everything after this include:
// every fused multiply-add is an explicit fmaf()/fma().
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace moe {

// v where in, else zeros, component by component (a select between whole
// float4 structs is lowered through private memory, with flat loads that
// wait one by one).
__device__ inline float4 masked4(bool in, float4 v) {
    return make_float4(in ? v.x : 0.0f, in ? v.y : 0.0f, in ? v.z : 0.0f, in ? v.w : 0.0f);
}

__device__ inline float ftz_f(float x) {
    uint32_t u = __float_as_uint(x);
    return ((u & 0x7f800000u) == 0u) ? __uint_as_float(u & 0x80000000u) : x;
}

// exp_avx2 lane (src/matrix.c:82-116) under DAZ/FTZ.
__device__ inline float exp_poly(float v) {
    v = fminf(fmaxf(ftz_f(v), -88.0f), 88.0f);
    float z = ftz_f(v * 1.4426950408f);
    float n = floorf(z);
    float f = ftz_f(z - n);
    float p = 0.0001540353f;
    p = fmaf(p, f, 0.0013333558f);
    p = fmaf(p, f, 0.0096181292f);
    p = fmaf(p, f, 0.0555041086f);
    p = fmaf(p, f, 0.2402265069f);
    p = fmaf(p, f, 0.6931471806f);
    p = fmaf(p, f, 1.0000000000f);
    int ni = (int)n;
    uint32_t sb = (uint32_t)(ni + 127) << 23;
    if ((sb & 0x7f800000u) == 0u) return 0.0f;
    return ftz_f(p * __uint_as_float(sb));
}

// 2^(i/32) as doubles with i<<47 subtracted from the bits (the table layout
// of glibc's expf, glibc 2.35 sysdeps/ieee754/flt-32/e_expf.c).
static __constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

// glibc expf as the FMA build of x86-64 computes it: z = x*32/ln2 fused
// into both of its additions, k by the 1.5*2^52 shift, cubic in r, scaled by
// the table entry with k/32's exponent added; subnormal results flushed.
__device__ inline float glibc_expf(float x) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double SHIFT = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint32_t ux = __float_as_uint(x);
    uint32_t ax = ux & 0x7fffffffu;
    if ((ax >> 20) >= (0x42b00000u >> 20)) {
        if (ux == 0xff800000u) return 0.0f;
        if (ax >= 0x7f800000u) return x + x;
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double xd = (double)x;
    double kd = fma(InvLn2N, xd, SHIFT);
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= SHIFT;
    double r = fma(InvLn2N, xd, -kd);
    uint64_t t = kExp2Tab[ki % 32];
    t += ki << (52 - 5);
    double s = __longlong_as_double((long long)t);
    double zz = fma(C0, r, C1);
    double r2 = r * r;
    double yy = fma(C2, r, 1.0);
    yy = fma(zz, r2, yy);
    double y = yy * s;
    return ftz_f((float)y);
}

// silu(g) * u (swiglu, src/matrix.c:618-655) for the expert epilogues, with
// the hardware exp2 and reciprocal (about 1 ulp each).  The expert outputs
// are held to a tolerance, not bits (the compiled reference itself divides
// with an rcpps estimate here), so the fast forms cost nothing in parity.
// rms_norm (src/matrix.c:666-711) of one row of cols = 16 * nb floats by the
// 16 lanes of a lane group (lane l = the reference's accumulator lane l:
// columns 16b + l, b ascending, fused multiply-adds), folded as
// v_l = acc_l + acc_(l+8), s_i = v_i + v_(i+4), ((s_0 + s_1) + (s_2 + s_3)),
// then y = (x * inv) * w with inv = 1 / sqrt(fma(ss, rcp_cols, eps))
// correctly rounded.  ld(i) returns x[i] of the row; every lane of the group
// calls this (a dead row passes any valid row and store = false).  ys: an
// optional second copy of the row (e.g. in LDS), written even when !store,
// flushed to zero if FTZ.
// Within each 16-lane row: lane l reads lane l + N (DPP row_shl; the top N
// lanes keep their own value, which the folds below never read), and lane
// 0's value to every lane of the row (row_newbcast).  The same moves as
// width-16 shuffles, without an LDS permute round trip.
template <int N> __device__ inline float row_down(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                      0x100 + N, 0xF, 0xF, false));
}
__device__ inline float row_lane0(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                      0x150, 0xF, 0xF, false));
}

template <class LD>
__device__ inline void rms_row16(const LD &ld, const float *w, int nb, float eps, float rcp_cols,
                                 float *y, bool store, float *ys = nullptr, bool ftz = false) {
    const int l = threadIdx.x & 15;
    constexpr int kHeld = 32;   // rows up to 512 wide stay in registers
    float v[kHeld], wv[kHeld];
    float acc = 0.0f;
    if (nb <= kHeld) {
#pragma unroll
        for (int b = 0; b < kHeld; ++b) v[b] = ld(16 * (b < nb ? b : 0) + l);
#pragma unroll
        for (int b = 0; b < kHeld; ++b) wv[b] = w[16 * (b < nb ? b : 0) + l];
#pragma unroll
        for (int b = 0; b < kHeld; ++b)
            if (b < nb) acc = fmaf(v[b], v[b], acc);
    } else {
        for (int b0 = 0; b0 < nb; b0 += 8) {
            float u8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) u8[u] = ld(16 * (b0 + u < nb ? b0 + u : 0) + l);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (b0 + u < nb) acc = fmaf(u8[u], u8[u], acc);
        }
    }
    acc = acc + row_down<8>(acc);
    acc = acc + row_down<4>(acc);
    acc = acc + row_down<1>(acc);
    acc = acc + row_down<2>(acc);
    const float inv = row_lane0(1.0f / sqrtf(fmaf(acc, rcp_cols, eps)));
    if (!store && !ys) return;
    auto put = [&](int i, float o) {
        if (store) y[i] = o;
        if (ys) ys[i] = ftz ? ftz_f(o) : o;
    };
    if (nb <= kHeld) {
#pragma unroll
        for (int b = 0; b < kHeld; ++b)
            if (b < nb) put(16 * b + l, (v[b] * inv) * wv[b]);
    } else {
        for (int b = 0; b < nb; ++b) put(16 * b + l, (ld(16 * b + l) * inv) * w[16 * b + l]);
    }
}

__device__ inline float swiglu_fast(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504f);
    const float sig = __builtin_amdgcn_rcpf(1.0f + e);
    return (g * sig) * u;
}

}  // namespace moe
