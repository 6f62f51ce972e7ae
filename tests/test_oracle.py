"""CPU tests of the oracle (oracle/moe_oracle.c), which the GPU parity tests
trust.  Every oracle function is pinned by at least one of:
  * the golden vectors written by the reference's own code compiled from
    source (tests/golden/make_golden.py) — bitwise for routing;
  * the host libm (the glibc expf restatement, exhaustively);
  * closed forms / brute force / textbook fp64 on small inputs;
  * the compiled reference itself, live, where oracle/_ref was built.
Sensitivity checks plant plausible mistakes in the oracle's options and show
the pins catch them.
"""
import ctypes as C
import math
import os
import sys

import numpy as np
import pytest

import orc
from abi_types import HostMoE, make_cache, matrix
from conftest import CONFIGS, GOLDEN

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
import make_golden as mg  # noqa: E402  (input builders only; the reference is not run)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def host_layer(d, F, E, k, seed, std_router, std_expert):
    wr, ex = orc.synth_layer_host(d, F, E, k, seed, std_router, std_expert)
    return HostMoE(wr, np.stack([ex[e][0] for e in range(E)]),
                   np.stack([ex[e][1] for e in range(E)]),
                   np.stack([ex[e][2] for e in range(E)]), k)


def load(name):
    return np.load(os.path.join(GOLDEN, name))


# ------------------------------------------------------------------ exp
def test_glibc_expf_restatement_exhaustive():
    """orc_expf (the restated glibc 2.35 expf) equals the host libm expf on
    every float in [-inf, 0] and [0, +inf] (NaN payloads aside)."""
    bad = C.c_uint32()
    n1 = orc.orc().orc_expf_compare_libm(0x80000000, 0xFFFFFFFF, 1, C.byref(bad))
    n2 = orc.orc().orc_expf_compare_libm(0x00000000, 0x7FFFFFFF, 1, C.byref(bad))
    assert n1 == 0 and n2 == 0, f"{n1 + n2} mismatches, first {hex(bad.value)}"


def test_glibc_expf_unfused_variant_is_caught():
    """Sensitivity: the same algorithm without FMA contraction differs from
    libm somewhere in [-104, 0] — the exhaustive check can tell them apart."""
    bad = C.c_uint32()
    n = orc.orc().orc_expf_compare_libm(0x80000000, 0xC2D00000, 0, C.byref(bad))
    assert n > 0


def test_expf_table_is_2_pow_i_over_32():
    from decimal import Decimal, getcontext
    import struct
    getcontext().prec = 50
    for i in range(32):
        v = float(format(Decimal(2) ** (Decimal(i) / Decimal(32)), ".40e"))
        b = struct.unpack("<Q", struct.pack("<d", v))[0]
        assert orc.orc().orc_expf_table_entry(i) == (b - (i << 47)) & (2**64 - 1)


def test_exp_poly_closed_form():
    o = orc.orc()
    assert o.orc_exp_poly(0.0) == 1.0
    xs = np.linspace(-87.0, 88.0, 20001).astype(np.float32)
    ys = orc.exp_poly_array(xs).astype(np.float64)
    ref = np.exp(xs.astype(np.float64))
    rel = np.abs(ys - ref) / ref
    # The polynomial is the degree-6 Taylor series of 2^f = e^(f ln 2) (its
    # coefficients are (ln 2)^n / n!), so its error is the remainder
    # ~ (f ln 2)^7 / 7! (up to 1.5e-5 as f -> 1, not the 1.9e-7 the source
    # comment claims), plus float roundings of z = x log2(e) (~|z| 2^-24 ln 2)
    # and of the Horner steps.
    z = xs.astype(np.float64) * math.log2(math.e)
    f = z - np.floor(z)
    bound = (f * math.log(2)) ** 7 / 5040 * 1.1 + 4e-7 + 6e-8 * np.abs(z)
    assert (rel <= bound).all()
    assert rel.max() > 1e-5          # the Taylor remainder really is there
    assert (np.diff(ys) >= 0).all()              # monotone
    # Below the DAZ threshold (2^-127 scale) the lane returns exactly 0.
    assert o.orc_exp_poly(-88.0) == 0.0 and o.orc_exp_poly(-1000.0) == 0.0
    assert o.orc_exp_poly(float("nan")) == 0.0   # max/min clamp maps NaN to -88


# ------------------------------------------------------------------ softmax
@pytest.mark.parametrize("E", [1, 4, 5, 8, 12, 16, 23, 64])
def test_softmax_matches_compiled_reference(E):
    g = load("golden_softmax.npz")
    got = orc.softmax_rows(g[f"in_{E}"])
    assert np.array_equal(bits(got), bits(g[f"out_{E}"]))


def test_softmax_tail_division_variant_is_caught():
    """Sensitivity: dividing the E % 8 tail by the sum (the source text) instead
    of multiplying by 1/sum (what -freciprocal-math compiles) breaks the
    golden vectors for tails."""
    g = load("golden_softmax.npz")
    orc.orc().orc_set_softmax_tail_recip(0)
    try:
        got = orc.softmax_rows(g["in_5"])
    finally:
        orc.orc().orc_set_softmax_tail_recip(1)
    assert not np.array_equal(bits(got), bits(g["out_5"]))


def test_softmax_textbook():
    rng = np.random.default_rng(3)
    for E in (4, 8, 13, 64):
        m = (rng.standard_normal((256, E)) * 4).astype(np.float32)
        p = orc.softmax_rows(m).astype(np.float64)
        z = np.exp(m - m.max(1, keepdims=True))
        ref = z / z.sum(1, keepdims=True)
        # exp_avx2 carries up to ~1.5e-5 relative error (its Taylor remainder)
        assert (np.abs(p - ref) <= 3.2e-5 * ref + 2e-7).all()
        assert np.abs(p.sum(1) - 1).max() < 1e-6
        # order preserved
        assert (np.argsort(-m, kind="stable", axis=1)[:, 0] == np.argmax(p, 1)).all()
    # stability at large logits (the reference test_matrix.c checks 1000+)
    p = orc.softmax_rows(np.array([[1000.0, 1001.0, 1002.0] * 4], np.float32))
    assert np.isfinite(p).all() and abs(p.sum() - 1) < 1e-6


# ------------------------------------------------------------------ router
def test_router_logits_match_compiled_reference():
    g = load("golden_logits.npz")
    for i, (T, d, E) in enumerate(mg.LOGIT_CASES):
        x, w = mg.logit_inputs(i, T, d, E)
        assert mg.sha(x) == str(g[f"sha_x_{i}"]) and mg.sha(w) == str(g[f"sha_w_{i}"])
        assert np.array_equal(bits(orc.router_logits(x, w)), bits(g[f"out_{i}"]))


def test_router_logits_exact_small_integers():
    """With small integer inputs every partial sum is exact: the chain must
    equal the integer product whatever its order."""
    rng = np.random.default_rng(5)
    x = rng.integers(-8, 9, (40, 70)).astype(np.float32)
    w = rng.integers(-8, 9, (70, 12)).astype(np.float32)
    ref = (x.astype(np.int64) @ w.astype(np.int64)).astype(np.float32)
    assert np.array_equal(orc.router_logits(x, w), ref)


def test_router_chain_is_sequential_fma():
    """One fused multiply-add per term, in ascending k (a transposed operand,
    a pairwise sum or a plain multiply-add would each change these bits)."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, 50)).astype(np.float32)
    w = (rng.standard_normal((50, 4)) * 0.1).astype(np.float32)
    got = orc.router_logits(x, w)
    for t in range(3):
        for e in range(4):
            acc = np.float32(0.0)
            for kk in range(50):
                # fma in float64 then one rounding == fmaf for these magnitudes
                acc = np.float32(np.float64(x[t, kk]) * np.float64(w[kk, e]) + np.float64(acc))
            assert got[t, e] == acc


# ------------------------------------------------------------------ top-k / dispatch
def test_topk_brute_force():
    rng = np.random.default_rng(7)
    for E, k in ((4, 2), (8, 3), (16, 16), (64, 4)):
        p = rng.integers(0, 6, (300, E)).astype(np.float32) / 8   # many exact ties
        ids, w = orc.topk(p, k)
        for t in range(300):
            order = sorted(range(E), key=lambda e: (-p[t, e], e))[:k]
            assert list(ids[t]) == order
            s = np.float32(0)
            for e in order:
                s = np.float32(s + p[t, e])
            inv = np.float32(1) / s if s > np.float32(1e-9) else np.float32(0)
            assert np.array_equal(w[t], (p[t, order] * inv).astype(np.float32))


def test_topk_degenerate():
    ids, w = orc.topk(np.full((1, 6), 0.25, np.float32), 3)
    assert list(ids[0]) == [0, 1, 2]
    ids, w = orc.topk(np.zeros((1, 4), np.float32), 2)      # s = 0 -> weights 0
    assert list(ids[0]) == [0, 1] and (w == 0).all()


def test_dispatch_is_stable_counting_sort():
    rng = np.random.default_rng(9)
    for T, k, E in ((1, 1, 1), (100, 2, 8), (777, 4, 64), (50, 3, 128)):
        ids = rng.integers(0, E, (T, k)).astype(np.int32)
        counts, offsets, perm = orc.dispatch(ids, E)
        flat = ids.ravel()
        assert np.array_equal(counts, np.bincount(flat, minlength=E))
        assert offsets[0] == 0 and offsets[-1] == T * k
        assert np.array_equal(np.diff(offsets), counts)
        assert np.array_equal(perm, np.argsort(flat, kind="stable"))
        assert np.array_equal(np.sort(perm), np.arange(T * k))


# ------------------------------------------------------------------ expert FFN
def test_swiglu_textbook_and_tail():
    rng = np.random.default_rng(13)
    for n in (8, 64, 13):                         # 13: 8-block + 5-element tail
        g = (rng.standard_normal(n) * 3).astype(np.float32)
        u = rng.standard_normal(n).astype(np.float32)
        h = np.empty(n, np.float32)
        orc.orc().orc_swiglu(orc.fptr(g), orc.fptr(u), orc.fptr(h), n)
        g64, u64 = g.astype(np.float64), u.astype(np.float64)
        ref = g64 / (1 + np.exp(-g64)) * u64
        assert np.abs(h - ref).max() <= 1e-6 * np.abs(ref).max() + 1e-12
    z = np.zeros(16, np.float32)
    one = np.ones(16, np.float32)
    h = np.empty(16, np.float32)
    orc.orc().orc_swiglu(orc.fptr(z), orc.fptr(one), orc.fptr(h), 16)
    assert (h == 0).all()                         # swiglu(0) = 0 (test_matrix.c:174-196)


def test_moe_forward_vs_fp64_textbook():
    c = CONFIGS["c1"]
    hw = host_layer(c["d"], c["F"], c["E"], c["k"], 0, c["std_router"], c["std_expert"])
    x = orc.synth((c["T"], c["d"]), 0, 0, 1.0)
    out, probs, ids = orc.moe_forward(x, hw)
    o64 = orc.moe_forward_f64(x, hw, ids, probs)
    assert orc.rel_l2(out, o64) < 1e-6


def test_moe_forward_c1_matches_compiled_reference():
    g = load("golden_c1.npz")
    c = CONFIGS["c1"]
    hw = host_layer(c["d"], c["F"], c["E"], c["k"], 0, c["std_router"], c["std_expert"])
    x = orc.synth((c["T"], c["d"]), 0, 0, 1.0)
    assert mg.sha(x) == str(g["sha_x"]) and mg.sha(hw.wr) == str(g["sha_wr"])
    out, probs, ids = orc.moe_forward(x, hw)
    assert np.array_equal(bits(probs), bits(g["probs"]))
    assert np.array_equal(ids, g["ids"])
    # The compiled swiglu divides with rcpps + one Newton step
    # (-ffast-math), a CPU-model-dependent rounding; outputs agree to ~2e-7.
    assert orc.rel_l2(out, g["out"]) < 1e-6


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_routing_samples_match_compiled_reference(name):
    g = load("golden_route.npz")
    c = CONFIGS[name]
    T = min(c["T"], 256)
    x = orc.synth((T, c["d"]), 7, 0, 1.0)
    wr = orc.synth((c["d"], c["E"]), 7, 1, c["std_router"])
    assert mg.sha(x) == str(g[f"{name}_sha_x"])
    bias = np.load(os.path.join(GOLDEN, "zipf_bias_e64_k4.npy")) if name == "c5" else None
    probs, ids, _ = orc.route(x, wr, c["k"], bias)
    assert np.array_equal(bits(probs), bits(g[f"{name}_probs"]))
    assert np.array_equal(ids, g[f"{name}_ids"])


@pytest.mark.parametrize("name,T,d,E,k,std", mg.WIDE_ROUTES, ids=[c[0] for c in mg.WIDE_ROUTES])
def test_wide_routing_matches_compiled_reference(name, T, d, E, k, std):
    """Routers wider than 128 experts (the 8-lane softmax blocks, the E % 8
    tail and top-16) against the compiled reference's bits."""
    g = load("golden_route_wide.npz")
    x = orc.synth((T, d), 7, 0, 1.0)
    wr = orc.synth((d, E), 7, 1, std)
    assert mg.sha(x) == str(g[f"{name}_sha_x"]) and mg.sha(wr) == str(g[f"{name}_sha_wr"])
    probs, ids, _ = orc.route(x, wr, k)
    assert np.array_equal(bits(probs), bits(g[f"{name}_probs"]))
    assert np.array_equal(ids, g[f"{name}_ids"])


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_layer_samples_match_compiled_reference(name):
    g = load("golden_moe.npz")
    c = CONFIGS[name]
    d, F, E, k = c["d"], c["F"], c["E"], c["k"]
    ns = g[f"{name}_out"].shape[0]
    x = orc.synth((ns, d), 3, 0, 1.0)
    wr = orc.synth((d, E), 3, 1, c["std_router"])
    bias = np.load(os.path.join(GOLDEN, "zipf_bias_e64_k4.npy")) if name == "c5" else None
    ids_g = g[f"{name}_ids"]
    need = sorted(set(ids_g.ravel().tolist()))
    _, ex = orc.synth_layer_host(d, F, E, k, 3, c["std_router"], c["std_expert"], experts=need)
    out, probs, ids = orc.moe_forward_experts(x, wr, ex, d, F, E, k, bias, nthreads=8)
    assert np.array_equal(ids, ids_g)
    assert np.array_equal(bits(probs), bits(g[f"{name}_probs"]))
    assert orc.rel_l2(out, g[f"{name}_out"]) < 1e-6


# ------------------------------------------------------------------ live reference
@pytest.mark.skipif(not orc.ref_available(), reason="reference not built here (oracle/_ref)")
def test_oracle_vs_compiled_reference_live():
    orc.orc().orc_set_ftz_daz(1)
    try:
        for (T, d, F, E, k, seed) in ((96, 64, 96, 6, 2, 1), (50, 128, 256, 16, 3, 2),
                                      (40, 64, 64, 9, 9, 3)):
            hw = host_layer(d, F, E, k, seed, 0.3, 0.05)
            x = orc.synth((T, d), seed, 0, 1.0)
            fc, probs, ids = make_cache(T, E, k)
            out = np.zeros((T, d), np.float32)
            orc.ref().moe_forward(C.byref(matrix(x)), C.byref(hw.weights),
                                  C.byref(hw.config(T)), C.byref(fc), C.byref(matrix(out)))
            o2, p2, i2 = orc.moe_forward(x, hw)
            assert np.array_equal(bits(probs), bits(p2))
            assert np.array_equal(ids, i2)
            assert orc.rel_l2(o2, out) < 1e-6
    finally:
        orc.orc().orc_set_ftz_daz(0)


# ------------------------------------------------------------------ rms_norm
def ulps(a, b):
    ia = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


@pytest.mark.parametrize("cols", mg.RMS_WIDTHS)
def test_rms_norm_close_to_compiled_reference(cols):
    """Against rms_norm compiled from src/matrix.c: the reference build takes
    1/sqrt from RSQRTSS plus a Newton step (x86-vendor tables), the oracle
    correctly rounded, so the rows agree to a few ulp, not bitwise.  Rows
    span six decades; the last row is all zeros."""
    g = load("golden_rms.npz")
    x, w = mg.rms_inputs(cols)
    assert mg.sha(x) == str(g[f"sha_x_{cols}"]) and mg.sha(w) == str(g[f"sha_w_{cols}"])
    orc.orc().orc_set_ftz_daz(1)
    try:
        y = orc.rms_norm(x, w, 1e-5)
    finally:
        orc.orc().orc_set_ftz_daz(0)
    ref = g[f"out_{cols}"]
    assert int(ulps(y, ref).max()) <= 4
    assert np.array_equal(y[13], ref[13]) and not np.any(y[13])


def test_rms_norm_textbook_fp64():
    x = orc.synth((64, 300), 8, 0, 1.0) * 7.0
    w = orc.synth((300,), 8, 1, 0.2, mean=1.0)
    y = orc.rms_norm(x, w, 1e-5)
    xd = x.astype(np.float64)
    yd = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-5) * w.astype(np.float64)
    assert float(np.abs(y - yd).max() / np.abs(yd).max()) < 1e-6


def test_rms_norm_power_of_two_scaling_is_exact():
    """eps = 0: scaling a row by 2^j scales ss by 4^j and 1/sqrt by 2^-j
    exactly, so y is unchanged bit for bit (any reordering of the squares or
    a dropped term would survive this, a wrong mean would not: see below)."""
    x = orc.synth((16, 512), 9, 0, 1.0)
    w = orc.synth((512,), 9, 1, 0.1, mean=1.0)
    y = orc.rms_norm(x, w, 0.0)
    for j in (-6, -1, 3, 10):
        assert np.array_equal(bits(orc.rms_norm(x * np.float32(2.0 ** j), w, 0.0)), bits(y))
    # Constant rows c = 2^j, eps = 0: inv_rms = 1/|c| exactly, y = sign(c) * w.
    for c in (0.25, -8.0, 1.0):
        xc = np.full((1, 48), c, np.float32)
        assert np.array_equal(bits(orc.rms_norm(xc, w[:48], 0.0)[0]),
                              bits(np.float32(math.copysign(1.0, c)) * w[:48]))


def test_rms_norm_mean_uses_all_columns():
    """One large column among zeros: ss = v^2 whatever the block it falls
    in (16-blocks, the 8-block, the scalar tail), y = v / sqrt(v^2/cols)."""
    for cols in (40, 100, 7):
        for j in range(cols):
            x = np.zeros((1, cols), np.float32)
            x[0, j] = 4.0
            y = orc.rms_norm(x, np.ones(cols, np.float32), 0.0)
            assert y[0, j] == np.float32(4.0) / np.sqrt(np.float32(16.0 / cols)), (cols, j)


# ------------------------------------------------------------------ inputs
def test_synthetic_generator():
    a = orc.synth((200000,), 1, 2, 1.0)
    assert np.array_equal(bits(a), bits(orc.synth((200000,), 1, 2, 1.0)))
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1.0) < 0.01
    # tails of N(0,1): P(|z| > 3) = 0.0027
    assert 0.0020 < float((np.abs(a) > 3).mean()) < 0.0035
    b = orc.synth((200000,), 1, 3, 1.0)
    assert abs(float(np.corrcoef(a, b)[0, 1])) < 0.01
    s = orc.synth((1000,), 9, 0, 0.02, mean=1.0)
    assert abs(float(s.mean()) - 1.0) < 0.005 and abs(float(s.std()) - 0.02) < 0.002
    assert math.isfinite(float(np.abs(orc.synth((1 << 20,), 4, 4, 1.0)).max()))
