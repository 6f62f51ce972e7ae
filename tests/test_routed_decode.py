"""The fused decode kernel with the routing inside (router path 0, decode steps
of up to 64 tokens over up to 16 experts, d_model 256 or 512) against the
same layer with the row-block router in its own launch (router path 2), and
both against the oracle.

Bars: the two arrangements give the same bits (routing, layer output and,
for the rms_norm sublayer, x_norm and x); routing is bit-exact against the
oracle and the layer output within rel-L2 1e-5 / max-abs 1e-4.
"""
import numpy as np
import pytest

import moe_hip as mh
import orc
from abi_types import HostMoE

pytestmark = pytest.mark.gpu

REL_TOL = 1e-5
ABS_TOL = 1e-4


def say(*a):
    print("[gpu-test]", *a, flush=True)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def assert_close(out, ref, what):
    rel = orc.rel_l2(out, ref)
    mabs = float(np.abs(out.astype(np.float64) - ref.astype(np.float64)).max())
    say(f"{what}: rel-L2 {rel:.3e} max-abs {mabs:.3e}")
    assert rel <= REL_TOL, f"{what}: rel-L2 {rel:.3e} > {REL_TOL}"
    assert mabs <= ABS_TOL, f"{what}: max-abs {mabs:.3e} > {ABS_TOL}"


def host_layer(d, F, E, k, seed, std_router, std_expert):
    wr, ex = orc.synth_layer_host(d, F, E, k, seed, std_router, std_expert)
    return HostMoE(wr, np.stack([ex[e][0] for e in range(E)]), np.stack([ex[e][1] for e in range(E)]),
                   np.stack([ex[e][2] for e in range(E)]), k)


CASES = [
    # name, T, d, F, E, k, bias, std_router, routed (the routing runs inside
    # the fused kernel; otherwise the rows, results and slot lists exceed
    # its 160 KB of LDS and the router launch runs first)
    ("c4", 64, 512, 2048, 16, 2, False, 0.02, True),
    ("t1", 1, 512, 256, 16, 2, False, 0.1, True),
    ("t7_e8_k1", 7, 256, 256, 8, 1, False, 0.1, True),          # one expert per token, RE = 1
    ("t33_e12_k3_bias", 33, 512, 384, 12, 3, True, 0.1, True),  # E % 8 tail, ragged last block
    ("t64_e3_k3", 64, 256, 256, 3, 3, False, 0.5, True),        # k == E: every expert per token
    ("t48_e16_k4_bias", 48, 512, 256, 16, 4, True, 0.1, True),
    ("t17_e16_k16", 17, 256, 128, 16, 16, False, 0.1, True),    # all 16 experts, 272 slots
    ("t64_e16_k2_hot", 64, 512, 256, 16, 2, True, 0.1, True),   # biased: one expert takes > 32 rows
    # more slots than the workgroup's 512 threads: the slot lists take
    # several ballot rounds (576 and 1024 slots)
    ("t64_e16_k9", 64, 256, 256, 16, 9, False, 0.1, True),
    ("t64_e16_k16", 64, 256, 128, 16, 16, False, 0.1, True),
    ("t64_d512_e16_k9", 64, 512, 256, 16, 9, False, 0.1, True),    # 159 KB of LDS
    ("t64_d512_e16_k16", 64, 512, 128, 16, 16, False, 0.1, False),  # 166 KB: router launch
]


@pytest.fixture
def paths():
    yield
    mh.set_router_path(0)
    mh.set_expert_path(0)


def bias_of(name, E):
    if not name.endswith("bias") and not name.endswith("hot"):
        return None
    b = np.zeros(E, np.float32)
    if name.endswith("hot"):
        b[5] = 30.0            # every token picks expert 5: two 32-row passes of its items
    else:
        b[1] = 0.5
        b[E - 1] = -0.75
    return b


@pytest.mark.parametrize("name,T,d,F,E,k,bias,std_router,routed", CASES,
                         ids=[c[0] for c in CASES])
def test_routed_matches_router_launch_and_oracle(name, T, d, F, E, k, bias, std_router, routed,
                                                 paths):
    say(f"routed decode {name}: T={T} d={d} F={F} E={E} k={k}")
    mh.set_expert_path(2)      # the fused decode kernel
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(23, std_router, 0.02)
    b = bias_of(name, E)
    if b is not None:
        layer.set_bias(b)
    hw = host_layer(d, F, E, k, 23, std_router, 0.02)
    x = orc.synth((T, d), 23, 0, 1.0)
    base = orc.synth((T, d), 23, 4, 1.0)
    dx = mh.DeviceArray.from_host(x)
    res = {}
    for rp in (0, 2):
        mh.set_router_path(rp)
        dout = mh.DeviceArray.from_host(base)
        dprobs = mh.DeviceArray((T, E))
        dids = mh.DeviceArray((T, k), np.int32)
        layer.forward_dev(dx.ptr, T, dout.ptr, dprobs.ptr, dids.ptr, accumulate=1)
        mh.synchronize()
        # path 0 must be the routed kernel (4) where it fits, path 2 the
        # router launch before the fused kernel (2)
        assert mh.last_forward_path() == (4 if rp == 0 and routed else 2), mh.last_forward_path()
        res[rp] = (dout.to_host(), dprobs.to_host(), dids.to_host())
    for a, c in zip(res[0], res[2]):
        assert np.array_equal(bits(a), bits(c)), "routing inside the kernel changed the bits"
    out, probs, ids = res[0]
    o_ref, p_ref, i_ref = orc.moe_forward(x, hw, bias=b, nthreads=16)
    assert np.array_equal(bits(probs), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    if name.endswith("hot"):
        assert int((ids == 5).sum()) == T
    assert_close(out, base + o_ref, name)
    layer.close()


@pytest.mark.parametrize("T,d,F,E,k", [(64, 512, 2048, 16, 2), (20, 256, 256, 8, 2)],
                         ids=["c4", "t20_d256"])
def test_routed_ffn_sublayer(T, d, F, E, k, paths):
    """x += MoE(rms_norm(x)) with the normalisation inside the routed kernel:
    x_norm, routing and x the same bits as with the router launch (which
    normalises), x_norm and routing bit-exact against the oracle."""
    say(f"routed sublayer: T={T} d={d} F={F} E={E} k={k}")
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(31, 0.1, 0.02)
    hw = host_layer(d, F, E, k, 31, 0.1, 0.02)
    x = np.ascontiguousarray(orc.synth((T, d), 31, 0, 1.0) * np.float32(3.0))
    w = orc.synth((d,), 31, 9, 0.1, mean=1.0)
    dw = mh.DeviceArray.from_host(w)
    res = {}
    for rp in (0, 2):
        mh.set_router_path(rp)
        dx = mh.DeviceArray.from_host(x)
        dxn = mh.DeviceArray((T, d))
        dprobs = mh.DeviceArray((T, E))
        dids = mh.DeviceArray((T, k), np.int32)
        layer.ffn_sublayer_dev(dx.ptr, dw.ptr, 1e-5, T, dxn.ptr, dprobs.ptr, dids.ptr)
        mh.synchronize()
        assert mh.last_forward_path() == (4 if rp == 0 else 2), mh.last_forward_path()
        res[rp] = (dx.to_host(), dxn.to_host(), dprobs.to_host(), dids.to_host())
    for a, c in zip(res[0], res[2]):
        assert np.array_equal(bits(a), bits(c)), "routing inside the kernel changed the bits"
    x1, xn, probs, ids = res[0]
    xn_ref = orc.rms_norm(x, w, 1e-5)
    assert np.array_equal(bits(xn), bits(xn_ref))
    o_ref, p_ref, i_ref = orc.moe_forward(xn_ref, hw, nthreads=16)
    assert np.array_equal(bits(probs), bits(p_ref))
    assert np.array_equal(ids, i_ref)
    assert_close(x1, x + o_ref, "routed sublayer")
    layer.close()
