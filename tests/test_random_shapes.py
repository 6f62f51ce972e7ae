"""A seeded sweep of random layer shapes through the device layer, each
checked against the oracle: routing bit-exact (probabilities, expert ids),
the layer output within rel-L2 1e-5 / max-abs 1e-4 (src/transformer.c:
287-366).  The shapes range over what the entry points take: one token to a
few hundred, 1 to 40 experts and a 300-expert layer (the general routing
kernels), top-1 to top-20 (k <= E), the kernels' widths, router scales from
near-ties to peaked; so every expert path (routed decode, fused decode,
grouped GEMMs) and router path is reached by some case.  A second sweep
forces each router path and expert path in turn on shapes up to 300
experts and top-24."""
import numpy as np
import pytest

import moe_hip as mh
import orc
from test_gpu_parity import assert_close, bits, host_layer

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu-test]", *a, flush=True)


def draw(i):
    rng = np.random.default_rng(1000 + i)
    d = int(rng.choice([64, 128, 256, 512]))
    F = int(rng.choice([64, 128, 256]))
    E = int(rng.choice([1, 2, 3, 5, 8, 13, 16, 24, 40])) if i % 7 else 300
    if E == 300:
        d, F = 64, 64   # (the 300-expert layer kept small on the host)
    k = int(rng.integers(1, min(E, 20) + 1))
    T = int(rng.choice([1, 2, 7, 33, 64, 65, 150, 300]))
    std = float(rng.choice([1e-3, 0.02, 0.3]))
    return T, d, F, E, k, std


CASES = [draw(i) for i in range(24)]


@pytest.mark.parametrize("i", range(len(CASES)), ids=[f"T{c[0]}_d{c[1]}_F{c[2]}_E{c[3]}_k{c[4]}" for c in CASES])
def test_random_shape(i):
    T, d, F, E, k, std = CASES[i]
    say(f"random shape {i}: T={T} d={d} F={F} E={E} k={k} std={std}")
    hw = host_layer(d, F, E, k, 50 + i, std, 0.05)
    x = orc.synth((T, d), 50 + i, 0, 1.0)
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw, nthreads=8)
    layer = mh.Layer(d, F, E, k)
    try:
        layer.fill_synthetic(50 + i, std, 0.05)
        dx = mh.DeviceArray.from_host(x)
        dout = mh.DeviceArray((T, d))
        dprobs = mh.DeviceArray((T, E))
        dids = mh.DeviceArray((T, k), np.int32)
        layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
        mh.synchronize()
        say(f"  expert path {mh.last_forward_path()}")
        assert np.array_equal(bits(dprobs.to_host()), bits(p_ref)), "router probabilities differ"
        assert np.array_equal(dids.to_host(), i_ref), "expert ids differ"
        assert_close(dout.to_host(), o_ref, f"random shape {i}")
    finally:
        layer.close()


def draw_paths(i):
    """Shapes as draw() (wider: up to 300 experts and top-24), each with a
    router path (automatic, token x expert tiles, row blocks) and an expert
    path (automatic, grouped GEMMs forced, fused decode forced, two-launch
    decode forced)."""
    rng = np.random.default_rng(5000 + i)
    d = int(rng.choice([64, 128, 192, 256, 512]))
    F = int(rng.choice([64, 128, 192, 256, 320]))
    E = int(rng.choice([1, 2, 4, 7, 8, 16, 33, 64, 130, 257, 300]))
    k = int(rng.integers(1, min(E, 24) + 1))
    T = int(rng.choice([1, 3, 16, 64, 65, 100, 257, 513, 1024, 2100]))
    if E > 256 or k > 16:
        d, F, T = min(d, 128), min(F, 128), min(T, 300)
    std = float(rng.choice([1e-3, 0.02, 0.3, 2.0]))
    rpath = int(rng.integers(0, 3))
    epath = int(rng.choice([0, 0, 1, 2, 3]))
    return T, d, F, E, k, std, rpath, epath


PATH_CASES = [draw_paths(i) for i in range(48)]


@pytest.fixture
def paths_reset():
    yield
    mh.set_router_path(0)
    mh.set_expert_path(0)


@pytest.mark.parametrize("i", range(len(PATH_CASES)),
                         ids=[f"T{c[0]}_E{c[3]}_k{c[4]}_r{c[6]}_e{c[7]}" for c in PATH_CASES])
def test_random_shape_paths(i, paths_reset):
    """Random shapes through every router and expert path.  A forced decode
    path refuses T*k above its slot limit with MOE_HIP_ERR_UNSUPPORTED (and
    nothing else); every accepted case matches the oracle to the same bars."""
    T, d, F, E, k, std, rpath, epath = PATH_CASES[i]
    say(f"random shape/path {i}: T={T} d={d} F={F} E={E} k={k} std={std} router={rpath} experts={epath}")
    hw = host_layer(d, F, E, k, 70 + i, std, 0.05)
    x = orc.synth((T, d), 70 + i, 0, 1.0)
    mh.set_router_path(rpath)
    mh.set_expert_path(epath)
    layer = mh.Layer(d, F, E, k)
    try:
        layer.fill_synthetic(70 + i, std, 0.05)
        dx = mh.DeviceArray.from_host(x)
        dout = mh.DeviceArray((T, d))
        dprobs = mh.DeviceArray((T, E))
        dids = mh.DeviceArray((T, k), np.int32)
        if epath >= 2 and T * k > 4096:
            with pytest.raises(mh.MoeHipError, match="unsupported shape"):
                layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
            return
        layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr)
        mh.synchronize()
        say(f"  expert path {mh.last_forward_path()}")
        o_ref, p_ref, i_ref = orc.moe_forward(x, hw, nthreads=8)
        assert np.array_equal(bits(dprobs.to_host()), bits(p_ref)), "router probabilities differ"
        assert np.array_equal(dids.to_host(), i_ref), "expert ids differ"
        assert_close(dout.to_host(), o_ref, f"random shape/path {i}")
    finally:
        layer.close()
