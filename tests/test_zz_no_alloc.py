"""GPU checks of moe_hip_forward_dev_noalloc, the allocation-free variant of
moe_hip_forward_dev: called through the C ABI, it must give the same routing
and the same layer output as the workspace entry point, on two calls in a
row with the second one smaller (the fixed scratch array keeps the first
call's contents), when recorded in a HIP graph and replayed, and it must
refuse a call whose temporaries exceed its fixed array."""
import numpy as np
import pytest

import moe_hip as mh
import orc
from conftest import CONFIGS

pytestmark = pytest.mark.gpu

REL_TOL = 1e-5
ABS_TOL = 1e-4


def say(*a):
    print("[gpu-test]", *a, flush=True)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def make_layer(T, d, F, E, k, std_router, std_expert, seed):
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(seed, std_router, std_expert)
    x = mh.DeviceArray((T, d))
    mh.fill_normal_dev(x.ptr, T * d, seed, 0, 0.0, 1.0)
    return layer, x


def run(layer, fn, x, T, accumulate=0, base=None):
    """One forward of the first T rows of x through fn (forward_dev or
    forward_dev_noalloc); returns out, probs, ids on the host."""
    out = mh.DeviceArray((T, layer.d))
    if base is not None:
        out.upload(base[:T])
    probs = mh.DeviceArray((T, layer.E))
    ids = mh.DeviceArray((T, layer.k), np.int32)
    fn(x.ptr, T, out.ptr, probs.ptr, ids.ptr, accumulate)
    mh.synchronize()
    return out.to_host(), probs.to_host(), ids.to_host()


def assert_same(a, b, what):
    """The two entry points run the same kernels on the same plan: routing
    and outputs agree bit for bit."""
    for name, u, v in zip(("out", "probs", "ids"), a, b):
        assert np.array_equal(bits(u) if u.dtype == np.float32 else u,
                              bits(v) if v.dtype == np.float32 else v), f"{what}: {name} differs"


# (config, first T, second smaller T): the decode layer (skinny fused
# GEMVs), the small prefill layer (grouped GEMMs), the batch-8x512 layer
# (grouped GEMMs with a split down projection) and the decode layer at
# four and one sequences (the few-row kernel with the routing inside).
CASES = [("c4", 64, 23), ("c1", 256, 97), ("c2", 4096, 1000), ("c4", 4, 1)]


@pytest.mark.parametrize("cfg,t1,t2", CASES, ids=[f"{c[0]}_t{c[1]}" for c in CASES])
def test_noalloc_matches_forward_dev(cfg, t1, t2):
    c = CONFIGS[cfg]
    d, F, E, k = c["d"], c["F"], c["E"], c["k"]
    say(f"noalloc {cfg}: T={t1} then T={t2}, d={d} F={F} E={E} k={k}")
    layer, x = make_layer(t1, d, F, E, k, c["std_router"], c["std_expert"], 11)
    try:
        for T in (t1, t2):
            ref = run(layer, layer.forward_dev, x, T)
            got = run(layer, layer.forward_dev_noalloc, x, T)
            assert_same(got, ref, f"{cfg} T={T}")
            # and the oracle's routing (bit-exact) and output (tolerance)
            xh = x.to_host()[:T]
            wr = layer.get_router()
            ex = {e: layer.get_expert(e) for e in range(E)}
            o_ref, p_ref, i_ref = orc.moe_forward_experts(np.ascontiguousarray(xh), wr, ex, d, F,
                                                          E, k, None, nthreads=8)
            assert np.array_equal(bits(got[1]), bits(p_ref)), "router probabilities differ"
            assert np.array_equal(got[2], i_ref), "expert ids differ"
            rel = orc.rel_l2(got[0], o_ref)
            mabs = float(np.abs(got[0].astype(np.float64) - o_ref).max())
            say(f"{cfg} T={T}: rel-L2 {rel:.2e} max-abs {mabs:.2e}")
            assert rel <= REL_TOL and mabs <= ABS_TOL, (rel, mabs)
        # the decode form: out += MoE(x), twice in a row
        base = np.random.default_rng(5).standard_normal((t1, d)).astype(np.float32)
        for T in (t1, t2):
            ref = run(layer, layer.forward_dev, x, T, accumulate=1, base=base)
            got = run(layer, layer.forward_dev_noalloc, x, T, accumulate=1, base=base)
            assert_same(got, ref, f"{cfg} accumulate T={T}")
    finally:
        layer.close()


def test_noalloc_wide_routing():
    """A layer past the fast routing kernels' tables (300 experts, top-20):
    the general routing kernels' logits and dispatch scratch come from the
    fixed array too; the grouped GEMMs at T = 400, then the decode kernels
    at T = 24, each bit-identical to forward_dev."""
    d, F, E, k = 64, 128, 300, 20
    say(f"noalloc wide: T=400 then T=24, d={d} F={F} E={E} k={k}")
    layer, x = make_layer(400, d, F, E, k, 0.3, 0.05, 13)
    try:
        for T in (400, 24):
            ref = run(layer, layer.forward_dev, x, T)
            got = run(layer, layer.forward_dev_noalloc, x, T)
            assert_same(got, ref, f"wide T={T}")
    finally:
        layer.close()


def test_noalloc_in_graph_replays():
    """Recorded in a HIP graph (no allocation happens during capture) and
    replayed several times with eager work and synchronisations between the
    replays: every replay equals the eager result."""
    c = CONFIGS["c4"]
    T, d, F, E, k = c["T"], c["d"], c["F"], c["E"], c["k"]
    layer, x = make_layer(T, d, F, E, k, c["std_router"], c["std_expert"], 12)
    other, xo = make_layer(T, d, F, E, k, c["std_router"], c["std_expert"], 13)
    try:
        eager = run(layer, layer.forward_dev_noalloc, x, T)
        out = mh.DeviceArray((T, d))
        probs = mh.DeviceArray((T, E))
        ids = mh.DeviceArray((T, k), np.int32)
        with mh.Graph() as g:
            layer.forward_dev_noalloc(x.ptr, T, out.ptr, probs.ptr, ids.ptr)
        try:
            for rep in range(4):
                out.zero()
                g.launch()
                mh.synchronize()
                got = (out.to_host(), probs.to_host(), ids.to_host())
                assert_same(got, eager, f"replay {rep}")
                # eager work on the same scratch between replays
                run(other, other.forward_dev_noalloc, xo, T - 7 * rep)
        finally:
            g.close()
    finally:
        layer.close()
        other.close()


def test_noalloc_refuses_oversized_call():
    """Temporaries above the fixed array: MOE_HIP_ERR_UNSUPPORTED, before any
    kernel runs."""
    d, F, E, k, T = 256, 1024, 8, 2, 16384   # H alone fills the 128 MiB array
    layer = mh.Layer(d, F, E, k)
    try:
        x = mh.DeviceArray((T, d))
        out = mh.DeviceArray((T, d))
        rc = mh.lib().moe_hip_forward_dev_noalloc(layer.h, x.ptr, T, out.ptr, None, None, 0,
                                                  None)
        assert rc == 2
        assert b"scratch" in mh.lib().moe_hip_last_error_message()
        # the bad call left the library usable
        mh.synchronize()
    finally:
        layer.close()


CHILD = r"""
import ctypes as C, os, sys
import numpy as np
sys.path[:0] = sys.argv[1:3]
import moe_hip as mh
hip = C.CDLL(os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so"))
mh.check(mh.lib().moe_hip_init(0))
T, d, F, E, k = 64, 512, 2048, 16, 2
small = mh.Layer(d, F, E, k)
small.fill_synthetic(14, 0.02, 0.02)
x = mh.DeviceArray((T, d))
mh.fill_normal_dev(x.ptr, T * d, 14, 0, 0.0, 1.0)
out, ref = mh.DeviceArray((T, d)), mh.DeviceArray((T, d))
small.forward_dev_noalloc(x.ptr, T, ref.ptr)
mh.synchronize()
s, g, ge = C.c_void_p(), C.c_void_p(), C.c_void_p()
assert hip.hipStreamCreate(C.byref(s)) == 0
assert hip.hipStreamBeginCapture(s, 1) == 0          # thread-local mode
small.forward_dev_noalloc(x.ptr, T, out.ptr, stream=s)
assert hip.hipStreamEndCapture(s, C.byref(g)) == 0
assert hip.hipGraphInstantiate(C.byref(ge), g, None, None, 0) == 0
assert hip.hipGraphLaunch(ge, s) == 0
assert hip.hipStreamSynchronize(s) == 0
assert np.array_equal(out.to_host().view(np.uint32), ref.to_host().view(np.uint32))
assert hip.hipGraphExecDestroy(ge) == 0 and hip.hipGraphDestroy(g) == 0
assert hip.hipStreamDestroy(s) == 0
# The capture recorded no workspace address, so the workspace may grow:
# a wider layer's synthetic fill stages more than the first one did, and a
# forward of it through the workspace entry point sizes new buffers.
big = mh.Layer(d, 2 * F, E, k)
big.fill_synthetic(15, 0.02, 0.02)
big.forward_dev(x.ptr, T, out.ptr)
mh.synchronize()
print("child ok", flush=True)
"""


def test_noalloc_captured_on_caller_stream_leaves_workspace_growable():
    """A capture the caller begins on its own stream, with only the
    allocation-free entry point recorded into it, must not pin the
    workspace: afterwards calls that grow it still succeed (in a fresh
    process, so that the first sizing is known to be the small layer's)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    say("noalloc captured on a caller stream, then a workspace-growing call (child process)")
    r = subprocess.run([sys.executable, "-c", CHILD, os.path.join(root, "llm.c_amd"),
                        os.path.join(root, "oracle")], capture_output=True, text=True,
                       timeout=180)
    say(r.stdout.strip(), r.stderr.strip()[-2000:])
    assert r.returncode == 0 and "child ok" in r.stdout
