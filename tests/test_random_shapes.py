"""A seeded sweep of random layer shapes through the device layer, each
checked against the oracle: routing bit-exact (probabilities, expert ids),
the layer output within rel-L2 1e-5 / max-abs 1e-4 (src/transformer.c:
287-366).  The shapes range over what the entry points take: one token to a
few hundred, 1 to 40 experts and a 300-expert layer (the general routing
kernels), top-1 to top-20 (k <= E), the kernels' widths, router scales from
near-ties to peaked; so every expert path (routed decode, fused decode,
grouped GEMMs) and router path is reached by some case."""
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
