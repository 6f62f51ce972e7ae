"""GPU parity: libmoe_hip (through its C ABI) against the CPU oracle.

Bars (the layer's contract):
  * router probabilities, expert ids, gate weights, expert counts, offsets
    and the dispatch permutation: bit-exact;
  * layer output: rel-L2 <= 1e-5 and max-abs <= 1e-4 against the oracle's
    fp32 restatement of the reference on identical seeded inputs.
"""
import os

import numpy as np
import pytest

import moe_hip as mh
import orc
from abi_types import HostMoE
from conftest import CONFIGS, GOLDEN

pytestmark = pytest.mark.gpu

REL_TOL = 1e-5
ABS_TOL = 1e-4


def say(*a):
    print("[gpu-test]", *a, flush=True)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def host_layer(d, F, E, k, seed, std_router, std_expert):
    wr, ex = orc.synth_layer_host(d, F, E, k, seed, std_router, std_expert)
    wg = np.stack([ex[e][0] for e in range(E)])
    wu = np.stack([ex[e][1] for e in range(E)])
    wd = np.stack([ex[e][2] for e in range(E)])
    return HostMoE(wr, wg, wu, wd, k)


def route_on_device(layer, x):
    T = x.shape[0]
    E, k = layer.E, layer.k
    dx = mh.DeviceArray.from_host(x)
    probs = mh.DeviceArray((T, E))
    ids = mh.DeviceArray((T, k), np.int32)
    gw = mh.DeviceArray((T, k))
    counts = mh.DeviceArray((E,), np.int32)
    offsets = mh.DeviceArray((E + 1,), np.int32)
    perm = mh.DeviceArray((T * k,), np.int32)
    layer.route_dev(dx.ptr, T, probs.ptr, ids.ptr, gw.ptr, counts.ptr, offsets.ptr, perm.ptr)
    mh.synchronize()
    return (probs.to_host(), ids.to_host(), gw.to_host(), counts.to_host(), offsets.to_host(),
            perm.to_host())


def assert_route_equal(dev, x, wr, k, E, bias=None):
    probs, ids, gw, counts, offsets, perm = dev
    p_ref, i_ref, w_ref = orc.route(x, wr, k, bias)
    c_ref, o_ref, perm_ref = orc.dispatch(i_ref, E)
    n_p = int((bits(probs) != bits(p_ref)).sum())
    n_i = int((ids != i_ref).sum())
    n_w = int((bits(gw) != bits(w_ref)).sum())
    assert n_p == 0, f"{n_p} router probabilities differ in bits"
    assert n_i == 0, f"{n_i} expert ids differ"
    assert n_w == 0, f"{n_w} gate weights differ in bits"
    assert np.array_equal(counts, c_ref)
    assert np.array_equal(offsets, o_ref)
    assert np.array_equal(perm, perm_ref), "dispatch permutation differs"


def assert_close(out, ref, what):
    rel = orc.rel_l2(out, ref)
    mabs = float(np.abs(out.astype(np.float64) - ref.astype(np.float64)).max()) if out.size else 0.0
    say(f"{what}: rel-L2 {rel:.3e} max-abs {mabs:.3e}")
    assert rel <= REL_TOL, f"{what}: rel-L2 {rel:.3e} > {REL_TOL}"
    assert mabs <= ABS_TOL, f"{what}: max-abs {mabs:.3e} > {ABS_TOL}"


# --------------------------------------------------------------------- scalars
def test_device_exp_functions_bitexact():
    """The two scalar exponentials of the routing softmax: exp_avx2 lanes and
    the glibc expf restatement, on every 61st float of [-104, 0] plus
    special values, against the oracle (itself pinned to libm)."""
    lo, hi = 0x80000000, 0xC2D00000
    pats = np.arange(lo, hi, 61, dtype=np.uint64).astype(np.uint32)
    extra = np.array([0x00000000, 0x80000000, 0xFF800000, 0x7F800000, 0x7FC00000,
                      0x42B00000, 0xC2B00000, 0xC2AE0000, 0xC2CFFFFF, 0x00000001,
                      0x80000001, 0x3F800000, 0xBF800000], dtype=np.uint32)
    pats = np.concatenate([pats, extra])
    x = pats.view(np.float32)
    say(f"exp check over {x.size} inputs")
    dx = mh.DeviceArray.from_host(x)
    dy = mh.DeviceArray(x.shape)
    for which, fn in ((0, orc.exp_poly_array), (1, orc.expf_array)):
        mh.eval_exp_dev(which, dx.ptr, dy.ptr, x.size)
        mh.synchronize()
        y = dy.to_host()
        yr = fn(x)
        same = (bits(y) == bits(yr)) | (np.isnan(y) & np.isnan(yr))
        assert same.all(), f"which={which}: {int((~same).sum())} mismatches, first at " \
                           f"{hex(int(pats[np.argmin(same)]))}"


def test_device_synth_matches_host():
    for seed, stream, std in ((0, 0, 1.0), (7, 17, 0.02), (123, 1, 0.1)):
        n = 1 << 20
        d = mh.DeviceArray((n,))
        mh.fill_normal_dev(d.ptr, n, seed, stream, 0.0, std)
        mh.synchronize()
        assert np.array_equal(bits(d.to_host()), bits(orc.synth((n,), seed, stream, std)))


# --------------------------------------------------------------------- routing
ROUTE_CASES = [
    # name, T, d, E, k, std_router
    ("c1", 256, 128, 4, 2, 0.02),
    ("c2", 4096, 256, 8, 2, 0.1),
    ("c3", 4096, 512, 8, 2, 0.02),
    ("c4", 64, 512, 16, 2, 0.02),
    ("e12k3_ragged", 1000, 192, 12, 3, 0.1),
    ("e5k5_all", 33, 64, 5, 5, 0.5),
    ("e64k4", 2048, 2048, 64, 4, 0.02),
    ("e128k1", 777, 128, 128, 1, 0.2),
    ("t1", 1, 256, 8, 2, 0.1),
    ("t65_d64", 65, 64, 16, 2, 0.1),
    ("t5000", 5000, 128, 16, 2, 0.1),
    # the grouped dispatch: 128 experts over 6 workgroups; 40000 assignments
    # over 32 workgroups, two 64-entry groups per wave
    ("e128k2_g6", 3000, 64, 128, 2, 0.2),
    ("t20000_g32", 20000, 64, 16, 2, 0.1),
    ("e128k16_g32", 8192, 64, 128, 16, 0.3),   # 131072 assignments, four groups per wave
    # wider than 128 experts: 8-wave router blocks, four expert bases per lane
    ("e256k8_g24", 3000, 128, 256, 8, 0.1),
    ("e160k4", 700, 192, 160, 4, 0.2),
    ("e250k16_t40", 40, 64, 250, 16, 0.3),     # the router's fused dispatch
]

ROUTER_PATHS = [0, 1, 2]   # automatic, token x expert tiles, 16-token row blocks


@pytest.fixture
def router_path():
    yield mh.set_router_path
    mh.set_router_path(0)


@pytest.mark.parametrize("path", ROUTER_PATHS, ids=["auto", "tiles", "rows"])
@pytest.mark.parametrize("name,T,d,E,k,std_router", ROUTE_CASES, ids=[c[0] for c in ROUTE_CASES])
def test_route_bitexact(name, T, d, E, k, std_router, path, router_path):
    say(f"route {name}: T={T} d={d} E={E} k={k} path={path}")
    router_path(path)
    x = orc.synth((T, d), 11, 0, 1.0)
    layer = mh.Layer(d, 64, E, k)
    layer.fill_synthetic(11, std_router, 0.02)
    wr = layer.get_router()
    assert np.array_equal(bits(wr), bits(orc.synth((d, E), 11, 1, std_router)))
    assert_route_equal(route_on_device(layer, x), x, wr, k, E)
    layer.close()


WIDE_GOLDEN = [("e256k8", 64, 128, 256, 8, 0.1), ("e250k16", 40, 64, 250, 16, 0.3),
               # past 256 experts or top-16: the general routing kernels
               ("e264k4", 64, 64, 264, 4, 0.2), ("e300k20", 48, 64, 300, 20, 0.3),
               ("e1024k32", 32, 128, 1024, 32, 0.1), ("e40k24", 40, 64, 40, 24, 0.5)]


@pytest.mark.parametrize("name,T,d,E,k,std", WIDE_GOLDEN, ids=[c[0] for c in WIDE_GOLDEN])
def test_route_wide_matches_compiled_reference(name, T, d, E, k, std):
    """Probabilities and ids of routers wider than 128 experts against the
    compiled reference's golden bits (same seeded inputs)."""
    say(f"route wide golden {name}: T={T} d={d} E={E} k={k}")
    g = np.load(os.path.join(GOLDEN, "golden_route_wide.npz"))
    layer = mh.Layer(d, 64, E, k)
    layer.fill_synthetic(7, std, 0.02)
    x = orc.synth((T, d), 7, 0, 1.0)
    dev = route_on_device(layer, x)
    layer.close()
    probs, ids = dev[:2]
    assert np.array_equal(bits(probs), bits(g[f"{name}_probs"]))
    assert np.array_equal(ids, g[f"{name}_ids"])
    # gate weights and the dispatch (counts, offsets, stable permutation)
    assert_route_equal(dev, x, orc.synth((d, E), 7, 1, std), k, E)


@pytest.mark.parametrize("path", ROUTER_PATHS, ids=["auto", "tiles", "rows"])
def test_route_zero_skip_nonfinite_weights(path, router_path):
    """The reference skips x == 0 (DAZ: also denormal x), so an inf router
    weight facing a zero (or denormal) x leaves the logit finite."""
    T, d, E, k = 100, 128, 16, 2
    router_path(path)
    x = orc.synth((T, d), 7, 0, 1.0)
    x[:, 5] = 0.0
    x[:, 9] = -0.0
    x[:, 40] = np.float32(1e-40)            # denormal: zero under DAZ
    x[::3, 77] = 0.0                         # zero for some tokens only
    wr = orc.synth((d, E), 7, 1, 0.1)
    wr[5, :] = np.inf
    wr[9, ::2] = -np.inf
    wr[40, 3] = np.nan
    wr[77, 1] = 0.0
    hw = HostMoE(wr, np.zeros((E, d, 64), np.float32), np.zeros((E, d, 64), np.float32),
                 np.zeros((E, 64, d), np.float32), k)
    layer = mh.Layer(d, 64, E, k)
    layer.load(hw)
    dev = route_on_device(layer, x)
    assert np.isfinite(dev[0]).all()
    assert_route_equal(dev, x, wr, k, E)
    layer.close()


def test_route_ties_and_bias():
    """Exact ties go to the lowest expert; a router bias (mat_mul_add form)
    can starve experts completely (empty groups in the dispatch)."""
    T, d, E, k = 300, 64, 16, 2
    x = orc.synth((T, d), 5, 0, 1.0)
    col = orc.synth((d, 1), 5, 1, 0.1)
    wr = np.ascontiguousarray(np.repeat(col, E, axis=1))     # all logits equal per row
    hw = HostMoE(wr, np.zeros((E, d, 64), np.float32), np.zeros((E, d, 64), np.float32),
                 np.zeros((E, 64, d), np.float32), k)
    layer = mh.Layer(d, 64, E, k)
    layer.load(hw)
    dev = route_on_device(layer, x)
    assert (dev[1] == np.arange(k)).all(), "ties must pick experts 0..k-1"
    assert_route_equal(dev, x, wr, k, E)
    bias = np.zeros(E, np.float32)
    bias[[3, 9]] = 50.0
    layer.set_bias(bias)
    dev = route_on_device(layer, x)
    assert_route_equal(dev, x, wr, k, E, bias)
    assert dev[3][3] == T and dev[3][9] == T and dev[3].sum() == T * k
    layer.close()


def test_route_wide_skip_ties_bias():
    """The general routing kernels (300 experts, top-20) on the edge cases
    of the fast ones: zero, negative-zero and denormal x facing inf and NaN
    router weights (the per-step zero-skip), exact ties (lowest experts
    first) and a router bias that starves experts."""
    T, d, E, k = 100, 128, 300, 20
    x = orc.synth((T, d), 7, 0, 1.0)
    x[:, 5] = 0.0
    x[:, 9] = -0.0
    x[:, 40] = np.float32(1e-40)            # denormal: zero under DAZ
    x[::3, 77] = 0.0
    wr = orc.synth((d, E), 7, 1, 0.1)
    wr[5, :] = np.inf
    wr[9, ::2] = -np.inf
    wr[40, 3] = np.nan
    wr[77, 1] = 0.0
    z = lambda *s: np.zeros(s, np.float32)
    hw = HostMoE(wr, z(E, d, 64), z(E, d, 64), z(E, 64, d), k)
    layer = mh.Layer(d, 64, E, k)
    layer.load(hw)
    dev = route_on_device(layer, x)
    assert np.isfinite(dev[0]).all()
    assert_route_equal(dev, x, wr, k, E)
    layer.close()
    col = orc.synth((d, 1), 5, 1, 0.1)
    wr = np.ascontiguousarray(np.repeat(col, E, axis=1))     # all logits equal per row
    hw = HostMoE(wr, z(E, d, 64), z(E, d, 64), z(E, 64, d), k)
    layer = mh.Layer(d, 64, E, k)
    layer.load(hw)
    dev = route_on_device(layer, x)
    assert (dev[1] == np.arange(k)).all(), "ties must pick experts 0..k-1"
    assert_route_equal(dev, x, wr, k, E)
    bias = np.zeros(E, np.float32)
    bias[[3, 9, 260]] = 50.0
    layer.set_bias(bias)
    dev = route_on_device(layer, x)
    assert_route_equal(dev, x, wr, k, E, bias)
    assert dev[3][3] == T and dev[3][9] == T and dev[3][260] == T and dev[3].sum() == T * k
    layer.close()


# --------------------------------------------------------------------- full layer
def test_dropin_moe_forward_c1():
    """Config 1 through the host-pointer drop-in moe_forward."""
    c = CONFIGS["c1"]
    hw = host_layer(c["d"], c["F"], c["E"], c["k"], 0, c["std_router"], c["std_expert"])
    x = orc.synth((c["T"], c["d"]), 0, 0, 1.0)
    out, probs, ids = mh.moe_forward(x, hw)
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw)
    assert np.array_equal(bits(probs), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    assert_close(out, o_ref, "c1 drop-in")
    g = os.path.join(GOLDEN, "golden_c1.npz")
    if os.path.exists(g):
        gz = np.load(g)
        assert np.array_equal(bits(probs), bits(gz["probs"]))
        assert np.array_equal(ids, gz["ids"])
        assert_close(out, gz["out"], "c1 vs compiled reference")


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_forward_dev_configs(name):
    c = CONFIGS[name]
    T, d, F, E, k = c["T"], c["d"], c["F"], c["E"], c["k"]
    say(f"forward {name}: T={T} d={d} F={F} E={E} k={k}")
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(1, c["std_router"], c["std_expert"])
    hw = host_layer(d, F, E, k, 1, c["std_router"], c["std_expert"])
    x = orc.synth((T, d), 1, 0, 1.0)
    dx = mh.DeviceArray.from_host(x)
    dout = mh.DeviceArray((T, d))
    dprobs = mh.DeviceArray((T, E))
    dids = mh.DeviceArray((T, k), np.int32)
    layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
    mh.synchronize()
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw, nthreads=16)
    assert np.array_equal(bits(dprobs.to_host()), bits(p_ref))
    assert np.array_equal(dids.to_host(), i_ref)
    assert_close(dout.to_host(), o_ref, name)
    # the same rows from host memory through the pinned staging: the same bits
    oh = np.empty((T, d), np.float32)
    ph = np.empty((T, E), np.float32)
    ih = np.empty((T, k), np.int32)
    layer.forward_host(x, oh, ph, ih)
    assert np.array_equal(bits(oh), bits(dout.to_host()))
    assert np.array_equal(bits(ph), bits(dprobs.to_host()))
    assert np.array_equal(ih, dids.to_host())
    layer.close()


def test_forward_host_chunks():
    """moe_hip_forward_host on 41 MB of rows (three 16 MB staging chunks up
    and down, the last one partial): the same bits as forward_dev on the
    same rows, with and without the probs / ids outputs."""
    T, d, F, E, k = 40000, 256, 256, 8, 2
    say(f"forward_host chunks: T={T} d={d}")
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(7, 0.1, 0.02)
    x = orc.synth((T, d), 7, 0, 1.0)
    dx = mh.DeviceArray.from_host(x)
    dout = mh.DeviceArray((T, d))
    dprobs = mh.DeviceArray((T, E))
    dids = mh.DeviceArray((T, k), np.int32)
    layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
    mh.synchronize()
    oh = np.full((T, d), np.nan, np.float32)
    ph = np.empty((T, E), np.float32)
    ih = np.empty((T, k), np.int32)
    layer.forward_host(x, oh, ph, ih)
    assert np.array_equal(bits(oh), bits(dout.to_host()))
    assert np.array_equal(bits(ph), bits(dprobs.to_host()))
    assert np.array_equal(ih, dids.to_host())
    oh2 = np.full((T, d), np.nan, np.float32)
    layer.forward_host(x, oh2)
    assert np.array_equal(bits(oh2), bits(oh))
    layer.close()


def gateup_tail(ids, E, ntiles, nks, groups=256):
    """The gate/up launch's split tail for these routes: (live tiles, tail
    tiles R, pieces per tail tile S); R = S = 0 when it is not split."""
    counts = np.bincount(ids.ravel(), minlength=E)
    live = int(((counts + 127) // 128).sum()) * ntiles
    r = live % groups
    s = min(nks, 4, groups // r) if r else 0
    return (live, r, s) if s >= 2 else (live, 0, 0)


@pytest.mark.parametrize("T", [1500, 2000, 2500, 2600, 4096])
def test_gateup_split_tail(T):
    """Small layers (256-column tiles in fewer than 4 rounds of the CUs):
    the tiles past the last whole round are split along d into 2-4 pieces
    whose sums a second kernel adds in order.  Every tail layout the token
    counts give (also none) matches the oracle."""
    d, F, E, k = 256, 1024, 8, 2
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(17, 0.1, 0.02)
    hw = host_layer(d, F, E, k, 17, 0.1, 0.02)
    x = orc.synth((T, d), 17, 0, 1.0)
    dx = mh.DeviceArray.from_host(x)
    dout = mh.DeviceArray((T, d))
    dprobs = mh.DeviceArray((T, E))
    dids = mh.DeviceArray((T, k), np.int32)
    layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
    mh.synchronize()
    ids = dids.to_host()
    say(f"split tail T={T}: (live tiles, tail tiles, pieces) = {gateup_tail(ids, E, 2 * F // 256, d // 32)}")
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw, nthreads=16)
    assert np.array_equal(bits(dprobs.to_host()), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    assert_close(dout.to_host(), o_ref, f"split tail T={T}")
    layer.close()


def test_gateup_split_tail_layouts_covered():
    """The token counts of test_gateup_split_tail's cases (routes from the
    oracle, no GPU work) give tails of 2, 3 and 4 pieces and one unsplit."""
    d, F, E, k = 256, 1024, 8, 2
    wr, _ = orc.synth_layer_host(d, F, E, k, 17, 0.1, 0.02)
    seen = set()
    for T in (1500, 2000, 2500, 2600, 4096):
        _, ids, _ = orc.route(orc.synth((T, d), 17, 0, 1.0), wr, k)
        seen.add(gateup_tail(ids, E, 2 * F // 256, d // 32)[2])
    say(f"split tail piece counts seen: {sorted(seen)}")
    assert {0, 2, 3, 4} <= seen


TINY = [
    # name, T, d, F, E, k (steps of at most 8 assignments with the routing
    # inside, at most 4 after a router launch)
    ("t1_c4", 1, 512, 2048, 16, 2),
    ("t4_c4", 4, 512, 2048, 16, 2),
    ("t8_k1", 8, 256, 512, 16, 1),
    ("t1_k8", 1, 512, 256, 16, 8),
    ("t2_k4_e5", 2, 256, 128, 5, 4),
    ("t1_k1", 1, 256, 256, 8, 1),
    ("t2_c4", 2, 512, 2048, 16, 2),
    ("t2_d1024", 2, 1024, 512, 8, 2),
    ("t1_k4_e64", 1, 512, 128, 64, 4),
    ("t3_k1_f192", 3, 256, 192, 4, 1),
    ("t2_e2", 2, 256, 64, 2, 2),      # both experts take every token
    ("t4_k1_e32", 4, 512, 1024, 32, 1),
]


@pytest.mark.parametrize("name,T,d,F,E,k", TINY, ids=[c[0] for c in TINY])
def test_decode_tiny(name, T, d, F, E, k):
    """Decode steps of at most four assignments: the few-row kernel (the used
    experts' 16-feature groups over the CUs; path 6 routes inside it for up to
    16 experts at d 256 or 512, path 5 after a router launch) within the bars
    of the oracle, routing bit-exact, and as x += MoE through
    moe_decode_batch.  Where the routing runs inside, the router launch
    (router path 2) gives the same bits."""
    say(f"tiny decode {name}: T={T} d={d} F={F} E={E} k={k}")
    inside = E <= 16 and d in (256, 512)
    assert inside or T * k <= 4
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(31, 0.1, 0.02)
    hw = host_layer(d, F, E, k, 31, 0.1, 0.02)
    x = orc.synth((T, d), 31, 0, 1.0)
    try:
        dx = mh.DeviceArray.from_host(x)
        dout = mh.DeviceArray((T, d))
        dprobs = mh.DeviceArray((T, E))
        dids = mh.DeviceArray((T, k), np.int32)
        layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
        mh.synchronize()
        assert mh.last_forward_path() == (6 if inside else 5)
        o_ref, p_ref, i_ref = orc.moe_forward(x, hw, nthreads=8)
        assert np.array_equal(bits(dprobs.to_host()), bits(p_ref))
        assert np.array_equal(dids.to_host(), i_ref)
        assert_close(dout.to_host(), o_ref, f"tiny {name}")
        if inside and T * k <= 4:
            mh.set_router_path(2)
            try:
                dout2 = mh.DeviceArray((T, d))
                layer.forward_dev(dx.ptr, T, dout2.ptr)
                mh.synchronize()
                assert mh.last_forward_path() == 5
            finally:
                mh.set_router_path(0)
            assert np.array_equal(bits(dout2.to_host()), bits(dout.to_host()))
        base = orc.synth((T, d), 31, 5, 1.0)
        assert_close(mh.decode_batch(x, base, hw), base + o_ref, f"tiny {name} decode_batch")
        # A router bias (mat_mul_add form) strong enough to move the choices.
        bias = (0.3 * np.random.default_rng(E + T).standard_normal(E)).astype(np.float32)
        layer.set_bias(bias)
        layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
        mh.synchronize()
        assert mh.last_forward_path() == (6 if inside else 5)
        o_b, p_b, i_b = orc.moe_forward(x, hw, bias, nthreads=8)
        assert np.array_equal(bits(dprobs.to_host()), bits(p_b))
        assert np.array_equal(dids.to_host(), i_b)
        assert_close(dout.to_host(), o_b, f"tiny {name} with bias")
    finally:
        layer.close()


@pytest.mark.parametrize("k", [1, 2])
def test_decode_tiny_guess_differs(k):
    """A step whose logits' top-k differs from the probabilities': logits 0
    and 2^-30 round to the same probability, and the reference takes the
    lower index (expert 0) where the larger logit is expert 1 (k = 1:
    another expert; k = 2: the same experts in another order).  The few-row
    kernel with the routing inside chooses on the rounded probabilities as
    the reference does: routing bit-exact, outputs within the bars."""
    T, d, F, E = 1, 256, 256, 4
    wr = np.zeros((d, E), np.float32)
    wr[0] = [0.0, 2.0 ** -30, -1.0, -1.0]     # only x[0] reaches the logits
    rng = np.random.default_rng(3)
    g = (0.05 * rng.standard_normal((E, d, F))).astype(np.float32)
    u = (0.05 * rng.standard_normal((E, d, F))).astype(np.float32)
    dn = (0.05 * rng.standard_normal((E, F, d))).astype(np.float32)
    hw = HostMoE(wr, g, u, dn, k)
    x = rng.standard_normal((T, d)).astype(np.float32)
    x[0, 0] = 1.0
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw)
    assert bits(p_ref)[0, 0] == bits(p_ref)[0, 1] and i_ref[0, 0] == 0   # the tie this case needs
    layer = mh.Layer(d, F, E, k)
    try:
        layer.load(hw)
        dx = mh.DeviceArray.from_host(x)
        dout = mh.DeviceArray((T, d))
        dprobs = mh.DeviceArray((T, E))
        dids = mh.DeviceArray((T, k), np.int32)
        layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
        mh.synchronize()
        assert mh.last_forward_path() == 6
        assert np.array_equal(bits(dprobs.to_host()), bits(p_ref))
        assert np.array_equal(dids.to_host(), i_ref)
        assert_close(dout.to_host(), o_ref, f"guess differs k={k}")
    finally:
        layer.close()


def test_down_short_first():
    """A down projection of at least 4 rounds of 256-column tiles (d 2048,
    64 experts, a skewed router bias) runs the experts' short last m-tiles
    first: every token against the oracle, and the routes do give short
    m-tiles (97 rows or fewer) to reorder."""
    T, d, F, E, k = 2048, 2048, 64, 64, 4
    say(f"down short-first: T={T} d={d} F={F} E={E} k={k}")
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(23, 0.02, 0.05)
    bias = (np.linspace(1.5, -1.5, E) ** 3 * 0.5).astype(np.float32)
    layer.set_bias(bias)
    hw = host_layer(d, F, E, k, 23, 0.02, 0.05)
    x = orc.synth((T, d), 23, 0, 1.0)
    dx = mh.DeviceArray.from_host(x)
    dout = mh.DeviceArray((T, d))
    dprobs = mh.DeviceArray((T, E))
    dids = mh.DeviceArray((T, k), np.int32)
    layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
    mh.synchronize()
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw, bias, nthreads=16)
    ids = dids.to_host()
    assert np.array_equal(bits(dprobs.to_host()), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    counts = np.bincount(ids.ravel(), minlength=E)
    m = (counts + 127) // 128
    short = int(((m > 0) & (counts - 128 * (m - 1) <= 96)).sum())
    say(f"down short-first: m-tiles {int(m.sum())}, short {short}")
    # (the library takes the order when its m-tile bound, ceil(T k / 128) + E,
    # makes at least 4 rounds of 256 workgroups)
    assert short > 0 and ((T * k + 127) // 128 + E) * (d // 256) >= 4 * 256
    assert_close(dout.to_host(), o_ref, "down short-first")
    layer.close()


@pytest.mark.parametrize("accumulate", [0, 1])
def test_forward_large_skewed(accumulate):
    """A large layer (T k = 32768 routed rows), every token against the
    oracle.  A skewed router bias gives one expert nearly every token and
    others a few dozen to a few hundred rows (short last m-tiles);
    accumulate = 1 adds the layer into out."""
    T, d, F, E, k = 8192, 256, 512, 8, 4
    say(f"large skewed layer: T={T} d={d} F={F} E={E} k={k} accumulate={accumulate}")
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(9, 0.1, 0.05)
    bias = np.array([3.0, 1.5, 0.5, 0.0, -1.0, -2.0, -3.5, -5.0], np.float32)
    layer.set_bias(bias)
    hw = host_layer(d, F, E, k, 9, 0.1, 0.05)
    x = orc.synth((T, d), 9, 0, 1.0)
    base = orc.synth((T, d), 9, 1, 1.0)
    dx = mh.DeviceArray.from_host(x)
    dout = mh.DeviceArray.from_host(base)
    dprobs = mh.DeviceArray((T, E))
    dids = mh.DeviceArray((T, k), np.int32)
    layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr, accumulate=accumulate)
    mh.synchronize()
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw, bias, nthreads=16)
    ids = dids.to_host()
    assert np.array_equal(bits(dprobs.to_host()), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    counts = np.bincount(ids.ravel(), minlength=E)
    say(f"large skewed layer: rows per expert {counts.tolist()}")
    assert counts.min() < 256 and counts.max() > 4 * 256
    expect = o_ref + base if accumulate else o_ref
    assert_close(dout.to_host(), expect, "large skewed layer")
    layer.close()


def test_forward_c5_sampled():
    """Config 5 at full size on the device (12.9 GB of experts, Zipf-skewed
    router bias when its fixture exists); routing compared for all tokens,
    the layer output for a sample of tokens: for every expert the first and
    the last token routed to it (so every expert's first and last 128-row
    m-tile of both grouped GEMMs is checked), plus a few random tokens."""
    c = CONFIGS["c5"]
    T, d, F, E, k = c["T"], c["d"], c["F"], c["E"], c["k"]
    say("c5: filling 12.9 GB of synthetic experts on the device")
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(5, c["std_router"], c["std_expert"])
    bias = None
    bpath = os.path.join(GOLDEN, "zipf_bias_e64_k4.npy")
    if os.path.exists(bpath):
        bias = np.load(bpath).astype(np.float32)
        layer.set_bias(bias)
    x = orc.synth((T, d), 5, 0, 1.0)
    dx = mh.DeviceArray.from_host(x)
    dout = mh.DeviceArray((T, d))
    dprobs = mh.DeviceArray((T, E))
    dids = mh.DeviceArray((T, k), np.int32)
    say("c5: forward")
    layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
    mh.synchronize()
    wr = layer.get_router()
    p_ref, i_ref, _ = orc.route(x, wr, k, bias)
    ids = dids.to_host()
    assert np.array_equal(bits(dprobs.to_host()), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    counts = np.bincount(ids.ravel(), minlength=E)
    say(f"c5: expert load max/mean {counts.max() / counts.mean():.2f}")
    rng = np.random.default_rng(0)
    sample = [rng.choice(T, 6, replace=False), [0, T - 1]]
    for e in range(E):
        # the dispatch orders an expert's rows by token: its first token sits
        # in its first m-tile, its last token in its last one
        toks = np.nonzero((ids == e).any(1))[0]
        if toks.size:
            sample.append([toks[0], toks[-1]])
    sample = np.unique(np.concatenate(sample))
    need = sorted(set(ids[sample].ravel().tolist()))
    say(f"c5: reading {len(need)} experts back for {sample.size} sampled tokens")
    out = dout.to_host()
    o_ref = np.empty((sample.size, d), np.float32)
    # the oracle in token batches whose experts fit comfortably in host memory
    for lo in range(0, sample.size, 32):
        part = sample[lo:lo + 32]
        ex = {e: layer.get_expert(e) for e in sorted(set(ids[part].ravel().tolist()))}
        o_ref[lo:lo + 32], _, _ = orc.moe_forward_experts(x[part], wr, ex, d, F, E, k, bias,
                                                          nthreads=16)
        del ex
    assert_close(out[sample], o_ref, f"c5 sampled ({sample.size} tokens, every expert's first "
                                     "and last m-tile)")
    layer.close()


def test_decode_batch_c4():
    """moe_decode_batch: x += MoE(x_norm) for 64 rows (host pointers)."""
    c = CONFIGS["c4"]
    T, d, F, E, k = c["T"], c["d"], c["F"], c["E"], c["k"]
    hw = host_layer(d, F, E, k, 4, c["std_router"], c["std_expert"])
    xn = orc.synth((T, d), 4, 0, 1.0)
    x0 = orc.synth((T, d), 4, 2, 1.0)
    x1 = mh.decode_batch(xn, x0, hw)
    o_ref, _, _ = orc.moe_forward(xn, hw, nthreads=16)
    assert_close(x1 - x0, o_ref, "c4 decode increment")
    # Single-row entry (the inference_step slot).
    x_one = x0[:1].copy()
    mh.lib().moe_decode_step(hw.weights, hw.config(1), mh.fptr(np.ascontiguousarray(xn[:1])),
                             mh.fptr(x_one))
    assert mh.last_forward_path() == 6   # the few-row kernel with the routing inside
    o1, _, _ = orc.moe_forward(xn[:1].copy(), hw)
    assert_close(x_one - x0[:1], o1, "c4 decode step")


# --------------------------------------------------------------------- rms_norm + FFN sublayer
@pytest.mark.parametrize("cols", [128, 256, 512, 1024, 2048, 24, 8, 100, 7, 16, 48])
def test_rms_norm_device_bitexact(cols):
    """Device rms_norm against the oracle, bit for bit: the reference's
    accumulator lanes and fold, fused multiply-adds, a correctly rounded
    1/sqrt; 300 rows over six decades, one all-zero row."""
    rows = 300
    scale = (10.0 ** np.linspace(-3, 3, rows)).astype(np.float32)[:, None]
    x = np.ascontiguousarray(orc.synth((rows, cols), 21, cols, 1.0) * scale)
    x[7] = 0.0
    w = orc.synth((cols,), 21, 500 + cols, 0.1, mean=1.0)
    dx, dw = mh.DeviceArray.from_host(x), mh.DeviceArray.from_host(w)
    dy = mh.DeviceArray((rows, cols))
    mh.rms_norm_dev(dx.ptr, dw.ptr, 1e-5, rows, cols, dy.ptr)
    mh.synchronize()
    ref = orc.rms_norm(x, w, 1e-5)
    nd = int((bits(dy.to_host()) != bits(ref)).sum())
    assert nd == 0, f"{nd} of {ref.size} normalised values differ in bits"


@pytest.mark.parametrize("name,T", [("c4", 64), ("c2", 512), ("c4", 1), ("c4", 2)],
                         ids=["c4", "c2", "c4_t1", "c4_t2"])
def test_ffn_sublayer_dev(name, T):
    """x += MoE(rms_norm(x)) in place on a device-resident residual stream:
    x_norm bit-exact, routing bit-exact, x within the layer tolerance.  One
    or two tokens take the few-row kernel with the norm and the routing
    inside (path 6)."""
    c = CONFIGS[name]
    d, F, E, k = c["d"], c["F"], c["E"], c["k"]
    say(f"ffn sublayer {name}: T={T} d={d} F={F} E={E} k={k}")
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(11, c["std_router"], c["std_expert"])
    hw = host_layer(d, F, E, k, 11, c["std_router"], c["std_expert"])
    x = np.ascontiguousarray(orc.synth((T, d), 11, 0, 1.0) * np.float32(3.0))
    w = orc.synth((d,), 11, 9, 0.1, mean=1.0)
    dx, dw = mh.DeviceArray.from_host(x), mh.DeviceArray.from_host(w)
    dxn = mh.DeviceArray((T, d))
    dprobs = mh.DeviceArray((T, E))
    dids = mh.DeviceArray((T, k), np.int32)
    layer.ffn_sublayer_dev(dx.ptr, dw.ptr, 1e-5, T, dxn.ptr, dprobs.ptr, dids.ptr)
    mh.synchronize()
    if T * k <= 4:
        assert mh.last_forward_path() == 6
    xn_ref = orc.rms_norm(x, w, 1e-5)
    assert np.array_equal(bits(dxn.to_host()), bits(xn_ref))
    o_ref, p_ref, i_ref = orc.moe_forward(xn_ref, hw, nthreads=16)
    assert np.array_equal(bits(dprobs.to_host()), bits(p_ref))
    assert np.array_equal(dids.to_host(), i_ref)
    assert_close(dx.to_host(), x + o_ref, f"{name} sublayer")
    # The workspace form (x_norm not returned) gives the same bits.
    dx2 = mh.DeviceArray.from_host(x)
    layer.ffn_sublayer_dev(dx2.ptr, dw.ptr, 1e-5, T)
    mh.synchronize()
    assert np.array_equal(bits(dx2.to_host()), bits(dx.to_host()))
    layer.close()


def test_block_ffn_dropin_c1():
    """moe_block_ffn (host pointers): the FFN half of a MoE block_forward."""
    c = CONFIGS["c1"]
    hw = host_layer(c["d"], c["F"], c["E"], c["k"], 0, c["std_router"], c["std_expert"])
    x = orc.synth((c["T"], c["d"]), 0, 5, 1.0)
    w = orc.synth((c["d"],), 0, 6, 0.1, mean=1.0)
    x1, xn, fo, probs, ids = mh.block_ffn(x, w, hw)
    xn_ref = orc.rms_norm(x, w, 1e-5)
    assert np.array_equal(bits(xn), bits(xn_ref))
    o_ref, p_ref, i_ref = orc.moe_forward(xn_ref, hw)
    assert np.array_equal(bits(probs), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    assert_close(fo, o_ref, "c1 block ffn_out")
    assert np.array_equal(bits(x1), bits(x + fo))


@pytest.mark.parametrize("path,rpath,T", [(2, 0, 64), (2, 2, 64), (3, 0, 64), (1, 0, 64),
                                          (0, 0, 2), (0, 2, 2)],
                         ids=["gemv_routed", "gemv", "gemv2", "gemm", "tiny_routed", "tiny"])
def test_graph_replay(path, rpath, T):
    """A captured forward (two layers, accumulating) replays to the same bits
    as the eager calls, replay after replay, with eager work and
    synchronisations in between."""
    d, F, E, k = 512, 2048, 16, 2
    mh.set_expert_path(path)
    mh.set_router_path(rpath)
    layers = [mh.Layer(d, F, E, k) for _ in range(2)]
    try:
        for i, L in enumerate(layers):
            L.fill_synthetic(40 + i, 0.02, 0.02)
        xn = mh.DeviceArray((T, d))
        mh.fill_normal_dev(xn.ptr, T * d, 41, 0, 0.0, 1.0)
        x0 = orc.synth((T, d), 41, 2, 1.0)
        out = mh.DeviceArray.from_host(x0)
        ids = [mh.DeviceArray((T, k), np.int32) for _ in layers]

        def step():
            for L, i in zip(layers, ids):
                L.forward_dev(xn.ptr, T, out.ptr, None, i.ptr, accumulate=1)

        step()                       # eager; also sizes the workspace
        mh.synchronize()
        if path == 0:
            assert mh.last_forward_path() == (6 if rpath == 0 else 5)
        ref = out.to_host()
        ref_ids = [i.to_host() for i in ids]
        with mh.Graph() as g:
            step()
        other = mh.DeviceArray((T, d))
        for rep in range(3):
            out.upload(x0)
            for i in ids:
                i.zero()
            g.launch()
            assert np.array_equal(bits(out.to_host()), bits(ref)), f"replay {rep}: output differs"
            for i, r in zip(ids, ref_ids):
                assert np.array_equal(i.to_host(), r), f"replay {rep}: expert ids differ"
            # Eager work on other data between replays.
            layers[0].forward_dev(out.ptr, T, other.ptr)
            mh.synchronize()
        g.close()
    finally:
        mh.set_expert_path(0)
        mh.set_router_path(0)
        for L in layers:
            L.close()


def test_workspace_does_not_move_under_a_live_graph():
    """A graph keeps the workspace addresses it recorded.  While one is alive,
    a call that would grow the workspace (here the staging buffer of a
    larger layer's synthetic fill) is refused with MOE_HIP_ERR_ARG instead of
    freeing memory the graph still uses; the graph still replays correctly,
    and once it is destroyed the same call succeeds."""
    T, d, F, E, k = 16, 128, 256, 4, 2
    layer = mh.Layer(d, F, E, k)
    big = mh.Layer(4096, 16384, 1, 1)   # its fill stages 805 MB, more than any other test
    try:
        layer.fill_synthetic(3, 0.02, 0.02)
        x = mh.DeviceArray((T, d))
        mh.fill_normal_dev(x.ptr, T * d, 3, 0, 0.0, 1.0)
        out = mh.DeviceArray((T, d))
        layer.forward_dev(x.ptr, T, out.ptr)      # eager; sizes the workspace
        mh.synchronize()
        ref = out.to_host()
        with mh.Graph() as g:
            layer.forward_dev(x.ptr, T, out.ptr)
        try:
            rc = mh.lib().moe_hip_layer_fill_synthetic(big.h, 1, 0.02, 0.02)
            assert rc == 1, rc
            assert b"captured graph" in mh.lib().moe_hip_last_error_message()
            out.zero()
            g.launch()
            mh.synchronize()
            assert np.array_equal(bits(out.to_host()), bits(ref))
        finally:
            g.close()
        big.fill_synthetic(1, 0.02, 0.02)        # no live graph: it may grow now
        mh.synchronize()
    finally:
        layer.close()
        big.close()


EDGE_CASES = [
    # name, T, d, F, E, k
    ("t1", 1, 128, 256, 8, 2),
    ("t31_k1", 31, 64, 96, 4, 1),
    ("t129", 129, 192, 160, 6, 2),
    ("k_eq_e", 70, 64, 64, 4, 4),
    ("e3", 200, 128, 128, 3, 2),
    ("e256_k8", 300, 64, 64, 256, 8),
    ("e130", 90, 128, 96, 130, 2),
]


@pytest.mark.parametrize("name,T,d,F,E,k", EDGE_CASES, ids=[c[0] for c in EDGE_CASES])
def test_forward_edge_shapes(name, T, d, F, E, k):
    hw = host_layer(d, F, E, k, 9, 0.3, 0.05)
    x = orc.synth((T, d), 9, 0, 1.0)
    out, probs, ids = mh.moe_forward(x, hw)
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw)
    assert np.array_equal(bits(probs), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    assert_close(out, o_ref, name)


def test_repeatable_and_residency():
    """Two calls give identical bits; changing weights in place needs
    moe_hip_invalidate, after which the new weights are used."""
    c = CONFIGS["c1"]
    hw = host_layer(c["d"], c["F"], c["E"], c["k"], 3, 0.1, 0.02)
    x = orc.synth((c["T"], c["d"]), 3, 0, 1.0)
    a = mh.moe_forward(x, hw)
    b = mh.moe_forward(x, hw)
    for u, v in zip(a, b):
        assert np.array_equal(np.ascontiguousarray(u).view(np.uint8),
                              np.ascontiguousarray(v).view(np.uint8))
    hw.wd *= 2.0                        # in place: same pointers
    mh.check(mh.lib().moe_hip_invalidate(hw.weights))
    out2, _, _ = mh.moe_forward(x, hw)
    o_ref, _, _ = orc.moe_forward(x, hw)
    assert_close(out2, o_ref, "after invalidate")


def test_error_paths():
    hw = host_layer(128, 512, 4, 2, 0, 0.02, 0.02)
    bad = HostMoE(hw.wr, hw.wg, hw.wu, hw.wd, 5)        # top_k > n_experts
    x = orc.synth((4, 128), 0, 0, 1.0)
    with pytest.raises(mh.MoeHipError):
        mh.moe_forward(x, bad)
    many = host_layer(64, 32, 300, 257, 0, 0.02, 0.02)  # top_k above the supported 256
    with pytest.raises(mh.MoeHipError):
        mh.moe_forward(orc.synth((4, 64), 0, 0, 1.0), many)


# Layers past the fast routing kernels' tables (more than 256 experts or
# top-k above 16) route through the general kernels and then run the same
# expert products: the decode kernels for small batches, the grouped GEMMs
# for large ones.
WIDE_LAYERS = [
    # name, T, d, F, E, k, expert path (2 fused decode, 1 grouped GEMMs)
    ("e300k20_decode", 24, 64, 128, 300, 20, 2),
    ("e300k20_gemm", 400, 64, 128, 300, 20, 1),
    ("e40k24_gemm", 256, 128, 64, 40, 24, 1),
    ("e520k2_decode", 96, 64, 64, 520, 2, 2),
    ("e520k2_gemm", 3000, 64, 64, 520, 2, 1),
]


@pytest.mark.parametrize("name,T,d,F,E,k,path", WIDE_LAYERS, ids=[c[0] for c in WIDE_LAYERS])
def test_wide_layers(name, T, d, F, E, k, path):
    """The layer (device rows and the host drop-in) and the in-place FFN
    sublayer at wide routing shapes: routing and dispatch bit-exact with
    the oracle, outputs within the bars."""
    say(f"wide layer {name}: T={T} d={d} F={F} E={E} k={k}")
    hw = host_layer(d, F, E, k, 23, 0.3, 0.05)
    x = orc.synth((T, d), 23, 0, 1.0)
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw, nthreads=16)
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(23, 0.3, 0.05)
    try:
        dx = mh.DeviceArray.from_host(x)
        dout = mh.DeviceArray((T, d))
        dprobs = mh.DeviceArray((T, E))
        dids = mh.DeviceArray((T, k), np.int32)
        layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
        mh.synchronize()
        assert mh.last_forward_path() == path
        assert np.array_equal(bits(dprobs.to_host()), bits(p_ref))
        assert np.array_equal(dids.to_host(), i_ref)
        assert_close(dout.to_host(), o_ref, f"{name} forward_dev")
        # without probs / ids outputs (the logits then go to library scratch)
        dout2 = mh.DeviceArray((T, d))
        layer.forward_dev(dx.ptr, T, dout2.ptr, None, None)
        mh.synchronize()
        assert np.array_equal(bits(dout2.to_host()), bits(dout.to_host()))
        dev = route_on_device(layer, x)
        assert_route_equal(dev, x, hw.wr, k, E)
        # x += MoE(rms_norm(x)) in place (the rows are normalised by a
        # separate launch first)
        w = orc.synth((d,), 23, 9, 0.1, mean=1.0)
        dw = mh.DeviceArray.from_host(w)
        layer.ffn_sublayer_dev(dx.ptr, dw.ptr, 1e-5, T)
        mh.synchronize()
        xn_ref = orc.rms_norm(x, w, 1e-5)
        o2, _, i2 = orc.moe_forward(xn_ref, hw, nthreads=16)
        assert_close(dx.to_host(), x + o2, f"{name} ffn sublayer")
    finally:
        layer.close()
    out, probs, ids = mh.moe_forward(x, hw)
    assert np.array_equal(bits(probs), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    assert_close(out, o_ref, f"{name} moe_forward")


# Widths the kernels do not tile, which the host drop-ins take by padding
# (zeros in x and in every weight past d_model / ffn_hidden).
ODD_WIDTHS = [
    # name, T, d, F, E, k
    ("d100_f70", 33, 100, 70, 5, 2),
    ("d96", 64, 96, 512, 4, 2),         # d_model % 64 only
    ("d130_k3", 7, 130, 96, 8, 3),      # ffn_hidden a multiple of 32: d only
    ("f40_k1", 200, 64, 40, 6, 1),      # ffn_hidden only
    ("d1_f1", 5, 1, 1, 3, 2),           # the narrowest layer
]


@pytest.mark.parametrize("name,T,d,F,E,k", ODD_WIDTHS, ids=[c[0] for c in ODD_WIDTHS])
def test_dropins_odd_widths(name, T, d, F, E, k):
    """moe_forward, moe_decode_batch and moe_block_ffn on widths the kernels do
    not tile: routing bit-exact and the layer within the bars, like every
    other shape."""
    say(f"odd widths {name}: T={T} d={d} F={F} E={E} k={k}")
    hw = host_layer(d, F, E, k, 17, 0.3, 0.05)
    x = orc.synth((T, d), 17, 0, 1.0)
    out, probs, ids = mh.moe_forward(x, hw)
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw)
    assert np.array_equal(bits(probs), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    assert_close(out, o_ref, f"{name} moe_forward")
    base = orc.synth((T, d), 17, 3, 1.0)
    assert_close(mh.decode_batch(x, base, hw), base + o_ref, f"{name} moe_decode_batch")
    w = orc.synth((d,), 17, 9, 0.1, mean=1.0)
    x1, xn, fo, probs, ids = mh.block_ffn(x, w, hw)
    xn_ref = orc.rms_norm(x, w, 1e-5)
    assert np.array_equal(bits(xn), bits(xn_ref))
    o2, p2, i2 = orc.moe_forward(xn_ref, hw)
    assert np.array_equal(bits(probs), bits(p2))
    assert np.array_equal(ids, i2)
    assert_close(fo, o2, f"{name} moe_block_ffn")


FORCED_PATH_CASES = [
    # name, T, d, F, E, k, path (1 = grouped GEMMs, 2 = fused decode GEMVs,
    # 3 = decode GEMVs as two launches)
    ("c4_gemv", 64, 512, 2048, 16, 2, 2),
    ("c4_gemv2", 64, 512, 2048, 16, 2, 3),
    ("e64_gemv", 48, 256, 256, 64, 4, 2),            # 64 experts, 8-wave items
    ("many_rows_gemv", 1500, 128, 128, 8, 2, 2),     # ~375 rows per expert: 12 passes
    ("c4_gemm", 64, 512, 2048, 16, 2, 1),
    ("multipass_gemv", 200, 128, 256, 4, 2, 2),     # ~100 rows per expert: 4 passes
    ("multipass_gemv2", 200, 128, 256, 4, 2, 3),
    ("kchunks_gemv", 48, 1024, 512, 16, 2, 2),      # d = 1024: two K chunks
    ("kchunks_gemv2", 48, 1024, 512, 16, 2, 3),
    ("oddblocks_gemv", 40, 192, 128, 8, 2, 2),      # d / 64 = 3 column blocks per wave
    ("tiny_gemv", 5, 64, 64, 8, 3, 2),
    ("tiny_gemv2", 5, 64, 64, 8, 3, 3),
    ("wide_gemm", 300, 256, 1024, 8, 2, 1),
]


@pytest.mark.parametrize("name,T,d,F,E,k,path", FORCED_PATH_CASES,
                         ids=[c[0] for c in FORCED_PATH_CASES])
def test_forced_expert_paths(name, T, d, F, E, k, path):
    """Both expert-product paths (grouped MFMA GEMMs and the skinny decode
    GEMVs) against the oracle, whatever the automatic choice would be."""
    hw = host_layer(d, F, E, k, 21, 0.1, 0.02)
    x = orc.synth((T, d), 21, 0, 1.0)
    mh.set_expert_path(path)
    try:
        out, probs, ids = mh.moe_forward(x, hw)
    finally:
        mh.set_expert_path(0)
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw)
    assert np.array_equal(bits(probs), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    assert_close(out, o_ref, name)


def test_weight_pack_roundtrip():
    """Upload packs the reference-layout matrices into 16 x 16 units; reading
    an expert back must return the same bits (device synth and host synth
    agree as well)."""
    d, F, E, k = 128, 96, 3, 2
    hw = host_layer(d, F, E, k, 31, 0.1, 0.02)
    layer = mh.Layer(d, F, E, k)
    layer.load(hw)
    for e in range(E):
        wg, wu, wd = layer.get_expert(e)
        assert np.array_equal(bits(wg), bits(hw.wg[e]))
        assert np.array_equal(bits(wu), bits(hw.wu[e]))
        assert np.array_equal(bits(wd), bits(hw.wd[e]))
    layer.fill_synthetic(31, 0.1, 0.02)
    wg, wu, wd = layer.get_expert(2)
    assert np.array_equal(bits(wd), bits(hw.wd[2]))
    layer.close()
