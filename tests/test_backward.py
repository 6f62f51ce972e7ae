"""Backward pass of the MoE layer and its load-balancing loss
(moe_hip_backward_dev).  The reference has no backward for this layer and no
code for the loss its comment defines (src/transformer.c:280-282), so there
is no golden: the fp64 restatement oracle/moe_backward.py is pinned by
central finite differences of its own fp64 forward (every gradient, with and
without the loss), by closed forms (uniform routing: aux = 1 and the loss
adds nothing to the router gradient; softmax gradients sum to zero per
token), and the device is checked against it within the layer tolerance,
with the routing the fp32 forward (bit-exact with the reference) decides."""
import os
import sys

import numpy as np
import pytest

import moe_hip as mh
import orc

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "oracle"))
import moe_backward as mb  # noqa: E402


def small_case(seed, T=6, d=8, F=5, E=4, k=2):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, d))
    wr = rng.standard_normal((d, E)) * 0.5
    wg = rng.standard_normal((E, d, F)) * 0.3
    wu = rng.standard_normal((E, d, F)) * 0.3
    wd = rng.standard_normal((E, F, d)) * 0.3
    _, p = mb.moe_forward64(x, wr, wg, wu, wd, np.zeros((T, k), int))
    ids = np.argsort(-p, axis=1, kind="stable")[:, :k]
    dout = rng.standard_normal((T, d))
    return x, wr, wg, wu, wd, ids, dout


@pytest.mark.parametrize("seed,aux_coef,k", [(0, 0.0, 2), (1, 0.7, 2), (2, 1.5, 1), (3, 0.3, 3)])
def test_oracle_vs_finite_differences(seed, aux_coef, k):
    x, wr, wg, wu, wd, ids, dout = small_case(seed, k=k)
    E = wr.shape[1]
    g = mb.moe_backward64(x, wr, wg, wu, wd, ids, dout, aux_coef)

    def loss(args):
        out, p = mb.moe_forward64(*args, ids)
        return float(np.sum(dout * out)) + aux_coef * mb.aux_loss64(p, ids, E)[0]

    rng = np.random.default_rng(100 + seed)
    base = [x, wr, wg, wu, wd]
    eps = 1e-6
    for i, name in enumerate(("dx", "dwr", "dwg", "dwu", "dwd")):
        for _ in range(6):
            idx = tuple(int(rng.integers(0, n)) for n in base[i].shape)
            plus = [a.copy() for a in base]
            minus = [a.copy() for a in base]
            plus[i][idx] += eps
            minus[i][idx] -= eps
            fd = (loss(plus) - loss(minus)) / (2 * eps)
            assert abs(fd - g[name][idx]) <= 1e-7 + 1e-6 * abs(fd), (name, idx, fd, g[name][idx])


def test_oracle_closed_forms():
    """Uniform router (W_r = 0, every p = 1/E) and round-robin ids: f_e =
    1/E, so aux = 1 exactly and its gradient on the logits vanishes; the
    logit gradient of any case sums to zero per token."""
    T, d, F, E, k = 8, 6, 4, 4, 1
    x, _, wg, wu, wd, _, dout = small_case(7, T, d, F, E, k)
    ids = (np.arange(T) % E)[:, None]
    g = mb.moe_backward64(x, np.zeros((d, E)), wg, wu, wd, ids, np.zeros_like(dout), 2.0)
    assert abs(g["aux"] - 1.0) < 1e-15
    assert np.abs(g["dlogits"]).max() < 1e-15
    x, wr, wg, wu, wd, ids, dout = small_case(8)
    g = mb.moe_backward64(x, wr, wg, wu, wd, ids, dout, 0.5)
    assert np.abs(g["dlogits"].sum(axis=1)).max() < 1e-12


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_oracle_forward64_matches_compiled_reference(name):
    """moe_forward64, the forward whose finite differences pin the backward,
    against the outputs of the reference's own moe_forward
    (src/transformer.c:287-366, compiled from source): its probabilities, its
    top-k under the reference's tie rule, and the layer output with the
    reference's gate renormalisation all agree with the golden fixtures
    (fp32 reference against fp64 restatement: 1e-6 relative).  A mistake
    shared by the backward and this forward (the renormalisation, the slot
    weights, the SwiGLU side) would show here."""
    from conftest import CONFIGS
    c = CONFIGS[name]
    d, F, E, k = c["d"], c["F"], c["E"], c["k"]
    bias = None
    if name == "c1":
        g = np.load(os.path.join(GOLDEN, "golden_c1.npz"))
        out_g, probs_g, ids_g = g["out"], g["probs"], g["ids"]
        x = orc.synth((c["T"], d), 0, 0, 1.0)
        seed = 0
    else:
        g = np.load(os.path.join(GOLDEN, "golden_moe.npz"))
        out_g, probs_g, ids_g = g[f"{name}_out"], g[f"{name}_probs"], g[f"{name}_ids"]
        x = orc.synth((out_g.shape[0], d), 3, 0, 1.0)
        seed = 3
        if name == "c5":
            bias = np.load(os.path.join(GOLDEN, "zipf_bias_e64_k4.npy")).astype(np.float64)
    need = sorted(set(ids_g.ravel().tolist()))
    wr, ex = orc.synth_layer_host(d, F, E, k, seed, c["std_router"], c["std_expert"],
                                  experts=need)
    wg = {e: ex[e][0] for e in need}
    wu = {e: ex[e][1] for e in need}
    wd = {e: ex[e][2] for e in need}
    out, p = mb.moe_forward64(x, wr, wg, wu, wd, ids_g, bias)
    # E < 8: the reference's softmax is all scalar tail (libm expf, correctly
    # rounded to ~1 ulp); E >= 8 takes exp_avx2 (src/matrix.c:82-116), a
    # degree-6 Taylor polynomial whose relative error reaches 1.5e-5, which
    # the fp64 exp does not share: the bar follows that error.
    rel_p = 1e-6 if E < 8 else 2e-5
    assert np.all(np.abs(p - probs_g) <= rel_p * probs_g + 1e-12)
    # the reference's top-k of its probabilities: descending, ties to the
    # lower expert id, equal to the ids it chose
    order = np.lexsort((np.broadcast_to(np.arange(E), probs_g.shape), -probs_g), axis=1)[:, :k]
    assert np.array_equal(order, ids_g)
    # Renormalised gate weights carry the probabilities' relative error; a
    # missing renormalisation or a wrong slot weight is off by 10 % or more.
    rel = orc.rel_l2(out, out_g)
    assert rel < (1e-6 if E < 8 else 1e-5), rel


# ---------------------------------------------------------------- GPU
def run_device_backward(d, F, E, k, T, seed, aux_coef, accumulate_twice=False):
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(seed, 0.1, 0.05)
    wr, ex = orc.synth_layer_host(d, F, E, k, seed, 0.1, 0.05)
    x = orc.synth((T, d), seed, 77, 1.0)
    dout = orc.synth((T, d), seed, 78, 1.0)
    dxd, dod = mh.DeviceArray.from_host(x), mh.DeviceArray.from_host(dout)
    outs = dict(dx=mh.DeviceArray((T, d)), dwr=mh.DeviceArray((d, E)),
                dwg=mh.DeviceArray((E, d, F)), dwu=mh.DeviceArray((E, d, F)),
                dwd=mh.DeviceArray((E, F, d)))
    aux = mh.DeviceArray((1,))
    args = [outs[n].ptr for n in ("dx", "dwr", "dwg", "dwu", "dwd")]
    layer.backward_dev(dxd.ptr, T, dod.ptr, aux_coef, *args, aux.ptr)
    if accumulate_twice:
        layer.backward_dev(dxd.ptr, T, dod.ptr, aux_coef, *args, aux.ptr, accumulate=1)
    mh.synchronize()
    res = {n: a.to_host() for n, a in outs.items()}
    res["aux"] = float(aux.to_host()[0])
    layer.close()
    wg = np.stack([ex[e][0] for e in range(E)])
    wu = np.stack([ex[e][1] for e in range(E)])
    wd = np.stack([ex[e][2] for e in range(E)])
    return res, x, dout, wr, wg, wu, wd


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(128, 512, 4, 2, 256), (256, 1024, 8, 2, 384),
                                   (128, 256, 16, 4, 100), (64, 96, 4, 2, 150),
                                   (192, 1024, 8, 2, 600), (64, 128, 256, 8, 400),
                                   (128, 96, 3, 1, 64), (64, 64, 4, 1, 700)],
                         ids=["c1", "c2-rows", "e16-k4", "untiled", "d192", "e256-k8",
                              "top1-e3", "top1-e4"])
@pytest.mark.parametrize("aux_coef", [0.0, 0.5])
def test_backward_device_vs_oracle(shape, aux_coef):
    """The tile-engine path (d, F multiples of 64; split partials by slot at
    c2-rows) and the untiled row products (F = 96).  At top-1 the router's
    gradient is the aux term alone, small against its parts when the loads
    are near-uniform (a cancellation the kernel avoids by counting loads
    from a fixed count).  The weight-gradient
    tiles: 64 x 64 at the small shapes, 64 x 128 for dW_g/dW_u at d192 (d
    not a multiple of 128), 128 x 128 and 128 x 64 at the batch-8x512 shape
    (test_backward_device_split_tail)."""
    d, F, E, k, T = shape
    print(f"[gpu-test] backward d={d} F={F} E={E} k={k} T={T} aux={aux_coef}", flush=True)
    res, x, dout, wr, wg, wu, wd = run_device_backward(d, F, E, k, T, 31, aux_coef)
    hw_ids = orc.route(x, wr, k)[1]   # the fp32 forward's routing (bit-exact on the device)
    g = mb.moe_backward64(x, wr, wg, wu, wd, hw_ids, dout, aux_coef)
    for name in ("dx", "dwr", "dwg", "dwu", "dwd"):
        rel = orc.rel_l2(res[name], g[name])
        print(f"[gpu-test]   {name}: rel-L2 {rel:.3e}", flush=True)
        assert rel <= 1e-5, name
    assert abs(res["aux"] - g["aux"]) <= 1e-5 * max(1.0, abs(g["aux"]))


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(192, 96, 3, 1, 1), (128, 128, 16, 1, 1), (64, 64, 256, 2, 3),
                                   (256, 64, 64, 4, 5)],
                         ids=["untiled-t1", "engine-t1", "e256-t3", "e64-t5"])
def test_backward_tiny_layers(shape):
    """A few tokens against a wide router: the router gradient's row-chunk
    partials (d E + E floats for one chunk) exceed the T k F floats of dH,
    which they reuse; the workspace holds one chunk at least."""
    d, F, E, k, T = shape
    print(f"[gpu-test] backward tiny d={d} F={F} E={E} k={k} T={T}", flush=True)
    res, x, dout, wr, wg, wu, wd = run_device_backward(d, F, E, k, T, 51, 0.5)
    hw_ids = orc.route(x, wr, k)[1]
    g = mb.moe_backward64(x, wr, wg, wu, wd, hw_ids, dout, 0.5)
    for name in ("dx", "dwr", "dwg", "dwu", "dwd"):
        rel = orc.rel_l2(res[name], g[name])
        print(f"[gpu-test]   {name}: rel-L2 {rel:.3e}", flush=True)
        assert rel <= 1e-5, name
    assert abs(res["aux"] - g["aux"]) <= 1e-5 * max(1.0, abs(g["aux"]))


@pytest.mark.gpu
@pytest.mark.parametrize("T", [4096, 2500], ids=["t4096", "t2500"])
def test_backward_device_split_tail(T):
    """The batch-8x512 shape (256-column tiles in fewer than 4 rounds): the
    GU recompute and the dH product split their last tiles along d into
    pieces a fixup adds (GU, H, then dG, dU in place)."""
    d, F, E, k = 256, 1024, 8, 2
    print(f"[gpu-test] backward split tail d={d} F={F} E={E} k={k} T={T}", flush=True)
    res, x, dout, wr, wg, wu, wd = run_device_backward(d, F, E, k, T, 41, 0.5)
    hw_ids = orc.route(x, wr, k)[1]
    g = mb.moe_backward64(x, wr, wg, wu, wd, hw_ids, dout, 0.5)
    for name in ("dx", "dwr", "dwg", "dwu", "dwd"):
        rel = orc.rel_l2(res[name], g[name])
        print(f"[gpu-test]   {name}: rel-L2 {rel:.3e}", flush=True)
        assert rel <= 1e-5, name
    assert abs(res["aux"] - g["aux"]) <= 1e-5 * max(1.0, abs(g["aux"]))


@pytest.mark.gpu
def test_backward_deterministic_and_accumulates():
    """Same bits on a repeat; accumulate = 1 adds a second pass exactly."""
    a, *_ = run_device_backward(128, 256, 4, 2, 200, 5, 0.3)
    b, *_ = run_device_backward(128, 256, 4, 2, 200, 5, 0.3)
    c, *_ = run_device_backward(128, 256, 4, 2, 200, 5, 0.3, accumulate_twice=True)
    for name in ("dx", "dwr", "dwg", "dwu", "dwd"):
        assert np.array_equal(a[name], b[name]), name
        assert np.array_equal(c[name], a[name] + a[name]), name


def draw_backward(i):
    rng = np.random.default_rng(9000 + i)
    d = int(rng.choice([64, 128, 192, 256]))
    F = int(rng.choice([64, 96, 128, 256, 320, 512]))
    E = int(rng.choice([1, 2, 3, 4, 8, 16, 64, 256]))
    k = int(rng.integers(1, min(E, 16) + 1))
    T = int(rng.choice([1, 5, 64, 129, 300, 700]))
    aux = float(rng.choice([0.0, 0.5]))
    return d, F, E, k, T, aux


BWD_RANDOM = [draw_backward(i) for i in range(32)]


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(len(BWD_RANDOM)),
                         ids=[f"d{c[0]}_F{c[1]}_E{c[2]}_k{c[3]}_T{c[4]}_a{c[5]}" for c in BWD_RANDOM])
def test_backward_random_shapes(i):
    """Seeded random layers (1 to 700 tokens, 1 to 256 experts, top-1 to
    top-16, tiled and untiled widths, with and without the aux loss): every
    gradient within rel-L2 1e-5 of the fp64 oracle."""
    d, F, E, k, T, aux = BWD_RANDOM[i]
    print(f"[gpu-test] backward random {i}: d={d} F={F} E={E} k={k} T={T} aux={aux}", flush=True)
    res, x, dout, wr, wg, wu, wd = run_device_backward(d, F, E, k, T, 100 + i, aux)
    hw_ids = orc.route(x, wr, k)[1]
    g = mb.moe_backward64(x, wr, wg, wu, wd, hw_ids, dout, aux)
    for name in ("dx", "dwr", "dwg", "dwu", "dwd"):
        if not np.abs(g[name]).max() > 0:   # (top-1 without the loss: no router gradient)
            assert np.abs(res[name]).max() <= 1e-6, name
            continue
        rel = orc.rel_l2(res[name], g[name])
        assert rel <= 1e-5, (name, rel)
    assert abs(res["aux"] - g["aux"]) <= 1e-5 * max(1.0, abs(g["aux"]))
