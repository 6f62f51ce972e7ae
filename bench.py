"""Benchmark of the MI355X MoE layer (libmoe_hip) — one JSON line on stdout.

Headline workload: the large imbalanced prefill layer — T=16384 tokens,
d_model=2048, d_ff=8192, E=64 experts, top-4, Zipf-skewed router bias,
inputs N(0,1), weights N(0,0.02), all fp32, synthetic and resident in HBM
before the timed region.  A "step" is one full layer forward (route,
dispatch, gate/up GEMM, down GEMM, combine).  K steps are issued back to back
on the library stream with device marks between them and nothing waiting
inside the loop (the loop is synchronised on both sides); the per-step
figure is the median of the K marked intervals.  The phase breakdown comes
from a separate pass with per-phase events.

Also measured in the same run (each a median of K marked steps unless said):
  * prefill_host_io: the headline layer with x read from and out, probs,
    ids written to pageable host memory, as the moe_forward drop-in does
    (PCIe included; wall time per synchronous call);
  * decode: 64 sequences x 1 token through 8 MoE layers of d=512, d_ff=2048,
    E=16, top-2 (8 layers' weights, 1.6 GB, so the 256 MB last-level cache
    cannot hold them), reported as MoE decode tokens/s and HBM GB/s;
  * decode_host_dropin: the same 8 layers through moe_decode_batch with
    host x_norm and x (the inference_step slot, batched; wall time);
  * prefill_batch8x512: the T=4096 (batch 8 x seq 512) layer, d=256,
    d_ff=1024, E=8, top-2, plus its host-pointer moe_forward drop-in and its
    backward pass (every gradient and the load-balancing loss);
  * moe_layer_c3 / moe_stack_c3: one MoE layer of the 8-block decoder
    (T=4096, d=512, d_ff=2048, E=8, top-2), and its 8 MoE FFN sublayers
    x += MoE(rms_norm(x)) in place through moe_hip_ffn_sublayer_dev;
  * decode_step: the whole block stack of that decode step (GQA attention
    over a 1024-position KV cache, then the MoE FFN sublayer, per block) with
    the residual stream on the device;
  * cpu_baseline: the reference's own moe_forward, compiled from its
    sources (oracle/_ref), on a bounded token sample of the same prefill
    layer, on one host thread as that build runs it (its 1-row expert
    products are not parallelised): one warm-up pass, then the median of 5
    passes; cpu_port_all_threads: the oracle port on every host thread,
    parallel over tokens, for context.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode]
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llm.c_amd"))

METRIC = "MoE layer tokens/s + % fp32 MFMA peak (prefill); decode tok/s + HBM GB/s"
PEAK_FP32_MFMA_TFLOPS = 157.3      # MI355X dense fp32 matrix
PEAK_HBM_GBS = 8000.0              # MI355X HBM3E
# How oracle/Makefile builds the CPU oracle timed as the baseline.
ORACLE_BUILD = "gcc -O3 -mavx2 -mfma -ffp-contract=off -fopenmp (oracle/Makefile)"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def stats(ms):
    a = np.asarray(ms, np.float64)
    return dict(median=float(np.median(a)), mean=float(a.mean()), min=float(a.min()),
                max=float(a.max()), n=int(a.size))


def layer_flops(T, d, F, E, k):
    return 6.0 * T * k * d * F + 2.0 * T * d * E


def prefill(mh, steps, warmup, T=16384, d=2048, F=8192, E=64, k=4, seed=5):
    layer = mh.Layer(d, F, E, k)
    t0 = time.time()
    layer.fill_synthetic(seed, 0.02, 0.02)
    bias_path = os.path.join(ROOT, "tests", "golden", "zipf_bias_e64_k4.npy")
    bias = None
    if os.path.exists(bias_path):
        bias = np.load(bias_path).astype(np.float32)
        layer.set_bias(bias)
    x = mh.DeviceArray((T, d))
    mh.fill_normal_dev(x.ptr, T * d, seed, 0, 0.0, 1.0)
    out = mh.DeviceArray((T, d))
    probs = mh.DeviceArray((T, E))
    ids = mh.DeviceArray((T, k), np.int32)
    mh.synchronize()
    log(f"prefill setup {time.time() - t0:.1f}s (weights {3 * E * d * F * 4 / 1e9:.2f} GB)")

    step = lambda: layer.forward_dev(x.ptr, T, out.ptr, probs.ptr, ids.ptr)
    t0 = time.perf_counter()
    per = mh.timed_steps(step, steps, warmup)
    wall = time.perf_counter() - t0
    st = stats(per)
    # Phase breakdown (separate pass; per-phase events and a wait per step).
    mh.set_timing(True)
    phase = np.zeros(5)
    nph = 5
    for _ in range(nph):
        step()
        phase += np.array(mh.last_timings())
    mh.set_timing(False)
    phase /= nph
    counts = np.bincount(ids.to_host().ravel(), minlength=E)
    flops_gu = 4.0 * T * k * d * F
    flops_dn = 2.0 * T * k * d * F
    ms = st["median"]
    res = dict(T=T, d=d, F=F, E=E, k=k, ms=ms, step_ms=st, wall_s=wall, phase_ms=phase.tolist(),
               counts_max_over_mean=float(counts.max() / counts.mean()),
               gateup_tflops=flops_gu / (phase[2] * 1e-3) / 1e12,
               down_tflops=flops_dn / (phase[3] * 1e-3) / 1e12,
               layer_tflops=layer_flops(T, d, F, E, k) / (ms * 1e-3) / 1e12,
               bias=bias is not None)
    state = dict(layer=layer, x=x, out=out, probs=probs, ids_dev=ids, bias=bias,
                 ids=ids.to_host(), seed=seed)
    return res, state


def prefill_host_io(mh, st, steps=5):
    """The headline layer with its activations in pageable host memory
    (moe_hip_forward_host: x up, out / probs / ids back through the pinned
    staging, as the moe_forward drop-in moves them; same router-biased
    layer, weights resident), wall time of the synchronous call."""
    layer, x, probs, ids = st["layer"], st["x"], st["probs"], st["ids_dev"]
    T, d = x.shape
    xh = x.to_host()
    oh = np.empty_like(xh)
    ph = np.empty(probs.shape, np.float32)
    ih = np.empty(ids.shape, np.int32)
    call = lambda: layer.forward_host(xh, oh, ph, ih)
    call()
    per = []
    for _ in range(steps):
        t0 = time.perf_counter()
        call()
        per.append((time.perf_counter() - t0) * 1e3)
    s = stats(per)
    pcie = float(xh.nbytes + oh.nbytes + ph.nbytes + ih.nbytes)
    return dict(T=T, ms=s["median"], step_ms=s, tokens_per_s=T / (s["median"] * 1e-3),
                pcie_bytes=pcie, up_bytes=float(xh.nbytes), down_bytes=float(oh.nbytes),
                overlapped_bytes=float(ph.nbytes + ih.nbytes))


def layer_bench(mh, steps, warmup, T, d, F, E, k, std_router, seed):
    """One layer forward on device rows (median of marked steps)."""
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(seed, std_router, 0.02)
    x = mh.DeviceArray((T, d))
    mh.fill_normal_dev(x.ptr, T * d, seed, 0, 0.0, 1.0)
    out = mh.DeviceArray((T, d))
    mh.synchronize()
    s = stats(mh.timed_steps(lambda: layer.forward_dev(x.ptr, T, out.ptr), steps, warmup))
    layer.close()
    ms = s["median"]
    return dict(T=T, d=d, F=F, E=E, k=k, ms=ms, step_ms=s, tokens_per_s=T / (ms * 1e-3),
                mfma_frac=layer_flops(T, d, F, E, k) / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS)


def ffn_stack(mh, steps, warmup, n_layers=8, T=4096, d=512, F=2048, E=8, k=2, eps=1e-5):
    """The MoE FFN half of every block of the 8-block decoder at batch 8 x
    seq 512: x += MoE(rms_norm(x; rms_ffn)) in place, block after block
    (src/transformer.c:760-767), through moe_hip_ffn_sublayer_dev.  Weights
    N(0, 0.02), rms_ffn = 1 (src/transformer.c:429-433), x ~ N(0, 1)."""
    layers = []
    for li in range(n_layers):
        L = mh.Layer(d, F, E, k)
        L.fill_synthetic(200 + li, 0.02, 0.02)
        layers.append(L)
    rms = mh.DeviceArray.from_host(np.ones(d, np.float32))
    x = mh.DeviceArray((T, d))
    mh.fill_normal_dev(x.ptr, T * d, 201, 0, 0.0, 1.0)
    mh.synchronize()

    def step():
        for L in layers:
            L.ffn_sublayer_dev(x.ptr, rms.ptr, eps, T)

    s = stats(mh.timed_steps(step, steps, warmup))
    for L in layers:
        L.close()
    ms = s["median"]
    return dict(layers=n_layers, T=T, d=d, F=F, E=E, k=k, ms_per_step=ms, step_ms=s,
                tokens_per_s=T / (ms * 1e-3), ms_per_layer=ms / n_layers,
                mfma_frac=n_layers * layer_flops(T, d, F, E, k) / (ms * 1e-3) / 1e12
                / PEAK_FP32_MFMA_TFLOPS)


def dropin_small(mh, steps, warmup, T=4096, d=256, F=1024, E=8, k=2):
    """The host-pointer drop-in moe_forward (x in host memory, out, probs and
    ids back to host memory) on the batch-8 x seq-512 layer: the
    PCIe-inclusive rate.  Weights become device-resident on the first call."""
    import abi_types
    rng = np.random.default_rng(4)
    f = lambda *sh, sd: (sd * rng.standard_normal(sh)).astype(np.float32)
    hw = abi_types.HostMoE(f(d, E, sd=0.1), f(E, d, F, sd=0.02), f(E, d, F, sd=0.02),
                           f(E, F, d, sd=0.02), k)
    x = f(T, d, sd=1.0)
    for _ in range(max(warmup, 1)):
        mh.moe_forward(x, hw)
    per = []
    for _ in range(steps):
        t0 = time.perf_counter()
        mh.moe_forward(x, hw)
        per.append((time.perf_counter() - t0) * 1e3)
    s = stats(per)
    pcie_bytes = 4.0 * T * (2 * d + E + k)
    return dict(T=T, ms=s["median"], step_ms=s, tokens_per_s=T / (s["median"] * 1e-3),
                pcie_bytes=pcie_bytes)


def backward_small(mh, steps, warmup, T=4096, d=256, F=1024, E=8, k=2, aux_coef=0.01):
    """moe_hip_backward_dev on the batch-8 x seq-512 layer: the routing and
    expert products recomputed, then every gradient and the aux loss.
    Flops: 18 T k d F (G, U, Y, dH, dX and the three weight gradients)."""
    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(2, 0.1, 0.02)
    x = mh.DeviceArray((T, d))
    mh.fill_normal_dev(x.ptr, T * d, 2, 0, 0.0, 1.0)
    dout = mh.DeviceArray((T, d))
    mh.fill_normal_dev(dout.ptr, T * d, 2, 1, 0.0, 1.0)
    bufs = [mh.DeviceArray(sh) for sh in ((T, d), (d, E), (E, d, F), (E, d, F), (E, F, d))]
    aux = mh.DeviceArray((1,))
    run = lambda: layer.backward_dev(x.ptr, T, dout.ptr, aux_coef, *[b.ptr for b in bufs], aux.ptr)
    s = stats(mh.timed_steps(run, steps, max(warmup, 1)))
    layer.close()
    ms = s["median"]
    tflops = 18.0 * T * k * d * F / (ms * 1e-3) / 1e12
    return dict(T=T, d=d, F=F, E=E, k=k, ms=ms, step_ms=s, tokens_per_s=T / (ms * 1e-3),
                tflops=tflops, mfma_frac=tflops / PEAK_FP32_MFMA_TFLOPS)


def decode(mh, steps, warmup, n_layers=8, T=64, d=512, F=2048, E=16, k=2):
    layers = []
    for li in range(n_layers):
        L = mh.Layer(d, F, E, k)
        L.fill_synthetic(100 + li, 0.02, 0.02)
        layers.append(L)
    xn = mh.DeviceArray((T, d))
    mh.fill_normal_dev(xn.ptr, T * d, 99, 0, 0.0, 1.0)
    x = mh.DeviceArray((T, d))
    mh.fill_normal_dev(x.ptr, T * d, 99, 2, 0.0, 1.0)
    ids = [mh.DeviceArray((T, k), np.int32) for _ in range(n_layers)]
    mh.synchronize()

    def step():
        for li, L in enumerate(layers):
            L.forward_dev(xn.ptr, T, x.ptr, None, ids[li].ptr, accumulate=1)

    # Headline: K decode steps issued back to back on the library stream.
    t0 = time.perf_counter()
    s = stats(mh.timed_steps(step, steps, max(warmup, 1)))
    wall = time.perf_counter() - t0
    # The same step replayed from a captured HIP graph (informational).
    with mh.Graph() as graph:
        step()
    graph_s = stats(mh.timed_steps(graph.launch, steps, 1))
    graph.close()
    # Breakdown (informational): one more pass with per-phase events, which
    # themselves add a few microseconds each.
    mh.set_timing(True)
    phase = np.zeros(5)
    for li, L in enumerate(layers):
        L.forward_dev(xn.ptr, T, x.ptr, None, ids[li].ptr, accumulate=1)
        phase += np.array(mh.last_timings())
    mh.set_timing(False)
    phase /= n_layers
    ms_step = s["median"]
    used = [int((np.bincount(i.to_host().ravel(), minlength=E) > 0).sum()) for i in ids]
    bytes_layer = [4.0 * (3 * d * F * u + d * E + 2 * T * d) for u in used]
    bytes_experts = [4.0 * 3 * d * F * u for u in used]
    dev_ms_layer = ms_step / n_layers
    # Events: [route, (dispatch: none in decode), gate/up (the fused kernel
    # does gate/up and down), down (only in the two-launch mode), combine].
    experts_ms = phase[2] + phase[3]
    res = dict(layers=n_layers, T=T, d=d, F=F, E=E, k=k, ms_per_step=ms_step, step_ms=s,
               wall_ms_per_step=wall * 1e3 / (steps + max(warmup, 1)),
               graph_ms_per_step=graph_s["median"],
               tokens_per_s=T / (ms_step * 1e-3),
               device_ms_per_layer=dev_ms_layer,
               phase_ms={"route": phase[0], "experts": experts_ms, "combine": phase[4]},
               experts_used=used,
               hbm_gbs_layer=float(np.mean(bytes_layer)) / (dev_ms_layer * 1e-3) / 1e9,
               experts_gbs=float(np.mean(bytes_experts)) / (experts_ms * 1e-3) / 1e9)
    state = dict(layers=layers, xn=xn, x=x)
    return res, state


def decode_host_dropin(mh, st, steps=10, T=64):
    """moe_decode_batch (host x_norm and x, synchronous) through the same 8
    layers' weights: the inference_step slot batched over 64 sequences, with
    its PCIe transfers; weights become resident on the first call."""
    import abi_types
    hws = []
    for L in st["layers"]:
        wg = np.empty((L.E, L.d, L.F), np.float32)
        wu = np.empty((L.E, L.d, L.F), np.float32)
        wd = np.empty((L.E, L.F, L.d), np.float32)
        for e in range(L.E):
            mh.check(mh.lib().moe_hip_layer_get_expert(L.h, e, mh.fptr(wg[e]), mh.fptr(wu[e]),
                                                       mh.fptr(wd[e])))
        hws.append(abi_types.HostMoE(L.get_router(), wg, wu, wd, L.k))
    xn = st["xn"].to_host()
    x = st["x"].to_host()
    # As a C caller makes the calls: the structs built once, x updated in
    # place by each layer (x += MoE(x_norm)).
    cfgs = [hw.config(T) for hw in hws]
    fn = mh.lib().moe_decode_batch
    pxn, px = mh.fptr(xn), mh.fptr(x)
    calls = [(C.byref(hw.weights), C.byref(cfg)) for hw, cfg in zip(hws, cfgs)]

    def step():
        for w, cfg in calls:
            mh.check(fn(w, cfg, pxn, T, px))

    step()
    per = []
    for _ in range(steps):
        t0 = time.perf_counter()
        step()
        per.append((time.perf_counter() - t0) * 1e3)
    s = stats(per)
    return dict(T=T, layers=len(hws), ms_per_step=s["median"], step_ms=s,
                tokens_per_s=T / (s["median"] * 1e-3),
                pcie_bytes_per_layer=4.0 * 3 * T * hws[0].d)


def decode_step(mh, steps, warmup, n_layers=8, B=64, ctx=1024, d=512, nh=8, nkv=2, F=2048,
                E=16, k=2, eps=1e-5):
    """The whole block stack of one KV-cache decode step, device resident,
    one moe_hip_decode_block_dev per block: x += Attn(rms_norm(x)) at
    position ctx over caches holding ctx earlier positions
    (src/inference.c:252-308), then x += MoE(rms_norm(x)) (:311-343).
    Caches, weights and x are synthetic N(0, 1) / N(0, 0.02)."""
    hd = d // nh
    kd, max_seq = nkv * hd, ctx + 1
    rng = np.random.default_rng(7)
    i = np.arange(hd // 2, dtype=np.float64)
    ang = np.arange(max_seq)[:, None] / 10000.0 ** (2 * i / hd)[None, :]
    cos_t, sin_t = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    attn, layers, caches = [], [], []
    rms = mh.DeviceArray.from_host(np.ones(d, np.float32))
    for li in range(n_layers):
        a = mh.Attn(d, nh, nkv, hd, max_seq)
        w = lambda r, c: (0.02 * rng.standard_normal((r, c))).astype(np.float32)
        a.load(w(d, nh * hd), w(d, kd), w(d, kd), w(nh * hd, d), np.ones(d, np.float32))
        a.set_rope(cos_t, sin_t)
        attn.append(a)
        L = mh.Layer(d, F, E, k)
        L.fill_synthetic(100 + li, 0.02, 0.02)
        layers.append(L)
        kc, vc = mh.DeviceArray((B, max_seq, kd)), mh.DeviceArray((B, max_seq, kd))
        mh.fill_normal_dev(kc.ptr, kc.nbytes // 4, 300 + li, 0, 0.0, 1.0)
        mh.fill_normal_dev(vc.ptr, vc.nbytes // 4, 300 + li, 1, 0.0, 1.0)
        caches.append((kc, vc))
    x = mh.DeviceArray((B, d))
    pos = mh.DeviceArray.from_host(np.full(B, ctx, np.int32))
    mh.synchronize()

    def attn_only():
        for li in range(n_layers):
            attn[li].decode_dev(x.ptr, B, pos.ptr, caches[li][0].ptr, caches[li][1].ptr, eps)

    def step():
        for li in range(n_layers):
            attn[li].decode_block_dev(layers[li], rms.ptr, x.ptr, B, pos.ptr, caches[li][0].ptr,
                                      caches[li][1].ptr, eps)

    # (the residual updates are small enough that x stays near N(0, 1))
    mh.fill_normal_dev(x.ptr, B * d, 99, 2, 0.0, 1.0)
    step_s = stats(mh.timed_steps(step, steps, max(warmup, 1)))
    attn_s = stats(mh.timed_steps(attn_only, steps, max(warmup, 1)))
    # The same step replayed from a captured HIP graph (informational).
    with mh.Graph() as graph:
        step()
    graph_s = stats(mh.timed_steps(graph.launch, steps, 1))
    graph.close()
    # Algorithmic bytes of one block's attention: K and V rows 0..ctx of each
    # sequence read once (the new row written once), plus W_Q, W_K, W_V, W_O.
    kv_bytes = 4.0 * 2 * B * (ctx + 1) * kd
    w_bytes = 4.0 * (2 * d * nh * hd + 2 * d * kd)
    step_ms, attn_ms = step_s["median"], attn_s["median"]
    attn_layer = attn_ms / n_layers
    res = dict(layers=n_layers, B=B, ctx=ctx, d=d, nh=nh, nkv=nkv, hd=hd, F=F, E=E, k=k,
               ms_per_step=step_ms, step_ms=step_s, tokens_per_s=B / (step_ms * 1e-3),
               graph_ms_per_step=graph_s["median"],
               graph_tokens_per_s=B / (graph_s["median"] * 1e-3),
               attn_ms_per_layer=attn_layer,
               attn_gbs=(kv_bytes + w_bytes) / (attn_layer * 1e-3) / 1e9,
               moe_ms_per_layer=(step_ms - attn_ms) / n_layers)
    for o in attn + layers:
        o.close()
    return res


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# How oracle/Makefile builds the reference's own MoE path (oracle/_ref).
REF_BUILD = ("gcc -O3 -march=native -ffast-math -funroll-loops -flto -fopenmp, the reference's "
             "release flags minus -DUSE_OPENBLAS (its AVX2+FMA mat_mul; oracle/Makefile)")


def _sized_passes(run, n0, n_max, pass_s):
    """Calibrate a sample size n so one pass of run(n) takes about pass_s
    seconds, run one warm-up pass at that size, then time 5 passes; returns
    (n, median seconds)."""
    n = n0
    for _ in range(2):   # calibration (small samples run slower per token)
        secs = run(n)
        n = int(min(n_max, max(n, n * pass_s / max(secs, 1e-6))))
    run(n)
    return n, float(np.median([run(n) for _ in range(5)]))


def cpu_baseline(mh, st, T=16384, d=2048, F=8192, E=64, k=4, pass_s=2.5):
    """The CPU baseline of the prefill layer: the reference's own moe_forward
    (src/transformer.c:287-366, compiled from its sources into oracle/_ref)
    on the first tokens of the same layer's rows and weights, on one host
    thread, which is how that build runs the layer: its expert products are
    1-row mat_muls, and mat_mul only parallelises blocks of 128+ rows
    (src/matrix.c:385).  The reference has no router bias, so it routes
    without one; its per-token work (k experts, three 1-row products each)
    is the same either way.  Tokens/s extrapolates linearly: tokens are
    independent in its loop (src/transformer.c:312).  Falls back to the
    oracle port (one thread) where oracle/_ref was not built."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import orc
    layer = st["layer"]
    wr = layer.get_router()
    xh = st["x"].to_host()
    ex = st.setdefault("host_experts", {})
    kind = "reference" if orc.ref_available() else "port"

    def run(n):
        xs = np.ascontiguousarray(xh[:n])
        _, ids, _ = orc.route(xs, wr, k)
        for e in sorted(set(ids.ravel().tolist()) - set(ex)):
            ex[e] = layer.get_expert(e)
        t0 = time.perf_counter()
        if kind == "reference":
            orc.ref_moe_forward_experts(xs, wr, ex, d, F, E, k, threads=1)
        else:
            orc.moe_forward_experts(xs, wr, ex, d, F, E, k, None, nthreads=1)
        return time.perf_counter() - t0

    n, med = _sized_passes(run, 4, T, pass_s)
    what = (f"the reference's moe_forward built from its sources ({REF_BUILD})"
            if kind == "reference" else "the oracle port (oracle/Makefile)")
    return dict(value=n / med, unit="tokens/s", cores=1, kind=kind,
                sample=f"first {n} of {T} tokens of the same layer (router bias off: the "
                       f"reference has none), warm-up then median of 5 passes ({med:.2f} s "
                       f"each), 1 thread, as that build runs each token's expert products; "
                       f"{cpu_model()}; {what}")


def cpu_port_threads(mh, st, T=16384, d=2048, F=8192, E=64, k=4, pass_s=2.5, threads=None):
    """Context for the baseline above: the oracle port of the same layer
    (bias included) on every host thread, parallelised over tokens, which
    the reference's build does not do."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import orc
    layer, ids = st["layer"], st["ids"]
    wr = layer.get_router()
    xh = st["x"].to_host()
    threads = threads or os.cpu_count() or 1
    ex = st.setdefault("host_experts", {})

    def run(n):
        for e in sorted(set(ids[:n].ravel().tolist()) - set(ex)):
            ex[e] = layer.get_expert(e)
        xs = np.ascontiguousarray(xh[:n])
        t0 = time.perf_counter()
        orc.moe_forward_experts(xs, wr, ex, d, F, E, k, st["bias"], nthreads=threads)
        return time.perf_counter() - t0

    n, med = _sized_passes(run, max(4 * threads, 8), T, pass_s)
    return dict(value=n / med, unit="tokens/s", cores=threads, kind="port",
                sample=f"first {n} of {T} tokens of the same prefill layer, warm-up then median "
                       f"of 5 passes ({med:.2f} s each), {threads} threads each taking whole "
                       f"tokens (the reference runs a token's experts on one thread, "
                       f"src/matrix.c:385); {cpu_model()}; oracle built with {ORACLE_BUILD}")


def cpu_decode_baseline(mh, T=64, d=512, F=2048, E=16, k=2, n_layers=8):
    """The reference's moe_forward (oracle/_ref; the oracle port where it
    was not built) on the T decode rows of one layer, one thread as that
    build runs it, warm-up then the median of 5; decode tokens/s = T / (8
    layers x that time)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import orc
    L = mh.Layer(d, F, E, k)
    L.fill_synthetic(100, 0.02, 0.02)
    ex = {e: L.get_expert(e) for e in range(E)}
    wr = L.get_router()
    L.close()
    x = np.random.default_rng(3).standard_normal((T, d)).astype(np.float32)
    kind = "reference" if orc.ref_available() else "port"

    def run():
        t0 = time.perf_counter()
        if kind == "reference":
            orc.ref_moe_forward_experts(x, wr, ex, d, F, E, k, threads=1)
        else:
            orc.moe_forward_experts(x, wr, ex, d, F, E, k, None, nthreads=1)
        return time.perf_counter() - t0

    run()
    layer_s = float(np.median([run() for _ in range(5)]))
    what = (f"the reference's moe_forward built from its sources ({REF_BUILD})"
            if kind == "reference" else "the oracle port (oracle/Makefile)")
    return dict(value=T / (n_layers * layer_s), unit="tokens/s", cores=1, kind=kind,
                sample=f"one MoE layer on the {T} decode row{'s' if T > 1 else ''}, x{n_layers} "
                       f"layers, warm-up then "
                       f"median of 5 ({layer_s * 1e3:.1f} ms per layer), 1 thread; "
                       f"{cpu_model()}; {what}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--only", choices=["prefill", "prefill_small", "backward", "decode",
                                       "decode_step", "decode_single", "c3", "copy"],
                    default=None,
                    help="run one section only (for profiling); prints its JSON to stderr")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are not part "
                                   "of it (see the sharding design notes)", "n_gpus": args.gpus}))
        sys.exit(2)
    import moe_hip as mh
    mh.check(mh.lib().moe_hip_init(0))

    if args.only == "copy":
        # Calibration for the HBM traffic counters: one 1 GiB device-to-device
        # copy (1 GiB read + 1 GiB written), then 1 GiB read through each load
        # path of the kernels (LDS DMA, vector loads, non-temporal vector
        # loads; moe_hip_read_probe), each from a buffer not read before.
        n = 1 << 28
        a, b = mh.DeviceArray((n,)), mh.DeviceArray((n,))
        mh.fill_normal_dev(a.ptr, n, 1, 0, 0.0, 1.0)
        mh.synchronize()
        mh.check(mh.lib().moe_hip_memcpy(b.ptr, a.ptr, 4 * n, 3))
        out = mh.DeviceArray((1024,))
        for mode in range(3):
            src = mh.DeviceArray((n,))
            mh.fill_normal_dev(src.ptr, n, 2 + mode, 0, 0.0, 1.0)
            mh.synchronize()
            mh.check(mh.lib().moe_hip_read_probe(src.ptr, 4 * n, mode, out.ptr, None))
            mh.synchronize()
            src.free()
        log("copy", json.dumps({"bytes": 4 * n, "probes": ["lds_dma", "vector", "vector_nt"]}))
        return
    small_shape = dict(T=4096, d=256, F=1024, E=8, k=2, std_router=0.1, seed=2)
    c3_shape = dict(T=4096, d=512, F=2048, E=8, k=2, std_router=0.02, seed=3)
    if args.only == "decode":
        log("decode", json.dumps(decode(mh, args.steps, args.warmup)[0]))
        return
    if args.only == "prefill_small":
        log("prefill_small", json.dumps(layer_bench(mh, args.steps, args.warmup, **small_shape)))
        return
    if args.only == "backward":
        log("backward", json.dumps(backward_small(mh, args.steps, args.warmup)))
        return
    if args.only == "decode_step":
        log("decode_step", json.dumps(decode_step(mh, args.steps, args.warmup)))
        return
    if args.only == "decode_single":
        log("decode T=1", json.dumps(decode(mh, args.steps, args.warmup, T=1)[0]))
        log("decode_step B=1", json.dumps(decode_step(mh, args.steps, args.warmup, B=1)))
        return
    if args.only == "c3":
        log("c3_layer", json.dumps(layer_bench(mh, args.steps, args.warmup, **c3_shape)))
        log("c3_stack", json.dumps(ffn_stack(mh, args.steps, args.warmup)))
        return
    pre, st = prefill(mh, args.steps, args.warmup)
    log("prefill", json.dumps(pre))
    if args.only == "prefill":
        return
    h2d, d2h = mh.link_rate()
    log("link", json.dumps({"h2d_gbs": h2d, "d2h_gbs": d2h}))
    hio = prefill_host_io(mh, st)
    log("prefill_host_io", json.dumps(hio))
    small = layer_bench(mh, args.steps, args.warmup, **small_shape)
    log("prefill_small", json.dumps(small))
    bwd = backward_small(mh, args.steps, args.warmup)
    log("backward", json.dumps(bwd))
    dropin = dropin_small(mh, args.steps, args.warmup)
    log("dropin", json.dumps(dropin))
    c3 = layer_bench(mh, args.steps, args.warmup, **c3_shape)
    log("c3_layer", json.dumps(c3))
    c3s = ffn_stack(mh, args.steps, args.warmup)
    log("c3_stack", json.dumps(c3s))
    dec = dech = stp = dec1 = dech1 = stp1 = None
    if not args.no_decode:
        dec, dst = decode(mh, args.steps, args.warmup)
        log("decode", json.dumps(dec))
        dech = decode_host_dropin(mh, dst)
        log("decode_host_dropin", json.dumps(dech))
        for L in dst["layers"]:
            L.close()
        stp = decode_step(mh, args.steps, args.warmup)
        log("decode_step", json.dumps(stp))
        # One sequence (the reference's inference_step shape): the same 8
        # MoE layers at T=1, then the whole block stack at B=1.
        dec1, dst1 = decode(mh, args.steps, args.warmup, T=1)
        log("decode T=1", json.dumps(dec1))
        dech1 = decode_host_dropin(mh, dst1, T=1)
        log("decode_host_dropin T=1", json.dumps(dech1))
        for L in dst1["layers"]:
            L.close()
        stp1 = decode_step(mh, args.steps, args.warmup, B=1)
        log("decode_step B=1", json.dumps(stp1))
    cpu = cpu_all = cpu_dec = cpu_dec1 = None
    if not args.no_cpu:
        cpu = cpu_baseline(mh, st)
        log("cpu", json.dumps(cpu))
        cpu_all = cpu_port_threads(mh, st)
        log("cpu port, all threads", json.dumps(cpu_all))
        cpu_dec = cpu_decode_baseline(mh)
        log("cpu decode", json.dumps(cpu_dec))
        if not args.no_decode:
            cpu_dec1 = cpu_decode_baseline(mh, T=1)
            log("cpu decode T=1", json.dumps(cpu_dec1))

    ms = pre["ms"]
    gu_tflops = pre["gateup_tflops"]
    # HBM bytes per gate/up launch come from the rocprofv3 FETCH_SIZE /
    # WRITE_SIZE passes summarised in profiles/ (counters cannot be read from
    # inside this process); null when that summary is absent.
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "moe_prefill_gateup_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
    line = {
        "metric": METRIC,
        "value": pre["T"] / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "ms_per_step_stats": pre["step_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "moe prefill layer T=16384 d=2048 d_ff=8192 E=64 top-4 "
                               "Zipf(1.1)-biased router", "T": pre["T"], "d_model": pre["d"],
                   "d_ff": pre["F"], "n_experts": pre["E"], "top_k": pre["k"]},
        "roofline": {"bound": "mfma", "kernel": "grouped gate/up GEMM",
                     "achieved": gu_tflops, "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": gu_tflops / PEAK_FP32_MFMA_TFLOPS, "traffic": traffic},
        "layer_mfma_frac": pre["layer_tflops"] / PEAK_FP32_MFMA_TFLOPS,
        "prefill_phase_ms": dict(zip(["route", "dispatch", "gate_up", "down", "combine"],
                                     pre["phase_ms"])),
        "expert_load_max_over_mean": pre["counts_max_over_mean"],
        "cpu_baseline": cpu,
        "cpu_port_all_threads": cpu_all,
    }
    line["host_link_gbs"] = {"h2d": h2d, "d2h": d2h,
                             "how": "one 256 MiB pinned copy each way (moe_hip_link_rate)"}
    line["prefill_host_io"] = {
        "workload": "the headline layer with x from and out / probs / ids to pageable host "
                    "memory through the pinned staging (moe_hip_forward_host, synchronous)",
        "tokens_per_s": hio["tokens_per_s"], "ms_per_step": hio["ms"],
        "pcie_bytes_per_call": hio["pcie_bytes"],
        # device time plus x up and out down at the link rate (probs and ids
        # travel under the expert products)
        "bound_ms": ms + hio["up_bytes"] / (h2d * 1e6) + hio["down_bytes"] / (d2h * 1e6)}
    line["prefill_batch8x512"] = {
        "workload": "moe prefill layer T=4096 (8 x 512) d=256 d_ff=1024 E=8 top-2",
        "tokens_per_s": small["tokens_per_s"], "ms_per_step": small["ms"],
        "layer_mfma_frac": small["mfma_frac"]}
    line["prefill_batch8x512_host_dropin"] = {
        "workload": "moe_forward with host x / out / probs / ids (PCIe included), same layer",
        "tokens_per_s": dropin["tokens_per_s"], "ms_per_step": dropin["ms"],
        "pcie_bytes_per_call": dropin["pcie_bytes"]}
    line["backward_batch8x512"] = {
        "workload": "moe layer backward + aux loss, T=4096 d=256 d_ff=1024 E=8 top-2 "
                    "(routing and expert products recomputed)",
        "ms_per_step": bwd["ms"], "tokens_per_s": bwd["tokens_per_s"],
        "tflops": bwd["tflops"], "fp32_peak_frac": bwd["mfma_frac"]}
    line["moe_layer_c3"] = {
        "workload": "one MoE layer of the 8-block decoder at batch 8 x seq 512: T=4096 d=512 "
                    "d_ff=2048 E=8 top-2",
        "tokens_per_s": c3["tokens_per_s"], "ms_per_step": c3["ms"],
        "layer_mfma_frac": c3["mfma_frac"]}
    line["moe_stack_c3"] = {
        "workload": "the 8 MoE FFN sublayers of that decoder, x += MoE(rms_norm(x)) in place "
                    "(moe_hip_ffn_sublayer_dev)",
        "tokens_per_s": c3s["tokens_per_s"], "ms_per_step": c3s["ms_per_step"],
        "ms_per_layer": c3s["ms_per_layer"], "mfma_frac": c3s["mfma_frac"]}
    if dec:
        line["decode"] = {
            "workload": "64 seqs x 1 token, 8 MoE layers d=512 d_ff=2048 E=16 top-2",
            "tokens_per_s": dec["tokens_per_s"], "ms_per_step": dec["ms_per_step"],
            "graph_ms_per_step": dec["graph_ms_per_step"],
            "device_ms_per_layer": dec["device_ms_per_layer"],
            "hbm_gbs": dec["hbm_gbs_layer"], "hbm_frac": dec["hbm_gbs_layer"] / PEAK_HBM_GBS,
            "experts_gbs": dec["experts_gbs"],
            # (per-phase HIP events add a few microseconds to each phase)
            "phase_ms_per_layer": dec["phase_ms"],
            "cpu_baseline": cpu_dec,
        }
        line["decode_host_dropin"] = {
            "workload": "the same 8 layers through moe_decode_batch, host x_norm and x "
                        "(synchronous calls from a C-style loop, x updated in place; transfers "
                        "by copy kernels across the bus)",
            "tokens_per_s": dech["tokens_per_s"], "ms_per_step": dech["ms_per_step"],
            "bound_ms": dec["ms_per_step"] + dech["layers"] * dech["pcie_bytes_per_layer"]
                        * (2 / (h2d * 1e6) + 1 / (d2h * 1e6)) / 3}
    if stp:
        line["decode_step"] = {
            "workload": "64 seqs x 1 token at context 1024, 8 blocks of GQA 8/2 attention "
                        "(hd 64) + MoE E=16 top-2, d=512 d_ff=2048, device-resident x",
            "tokens_per_s": stp["tokens_per_s"], "ms_per_step": stp["ms_per_step"],
            "graph_ms_per_step": stp["graph_ms_per_step"],
            "attn_ms_per_layer": stp["attn_ms_per_layer"], "attn_gbs": stp["attn_gbs"],
            "attn_hbm_frac": stp["attn_gbs"] / PEAK_HBM_GBS,
            "moe_ms_per_layer": stp["moe_ms_per_layer"],
        }
    if dec1:
        line["decode_single_seq"] = {
            "workload": "1 seq x 1 token, the same 8 MoE layers (d=512 d_ff=2048 E=16 top-2): "
                        "the few-row expert kernel with the routing inside",
            "tokens_per_s": dec1["tokens_per_s"], "ms_per_step": dec1["ms_per_step"],
            "graph_ms_per_step": dec1["graph_ms_per_step"],
            "device_ms_per_layer": dec1["device_ms_per_layer"],
            "hbm_gbs": dec1["hbm_gbs_layer"], "hbm_frac": dec1["hbm_gbs_layer"] / PEAK_HBM_GBS,
            "cpu_baseline": cpu_dec1,
        }
    if dech1:
        line["decode_single_seq_host_dropin"] = {
            "workload": "the same 8 layers through moe_decode_batch with one row (moe_decode_step, "
                        "the inference_step slot), host x_norm and x, synchronous calls",
            "tokens_per_s": dech1["tokens_per_s"], "ms_per_step": dech1["ms_per_step"],
            "us_per_call": dech1["ms_per_step"] * 1e3 / dech1["layers"],
        }
    if stp1:
        line["decode_step_single_seq"] = {
            "workload": "1 seq x 1 token at context 1024, the same 8 blocks (GQA 8/2 attention "
                        "+ MoE), device-resident x",
            "tokens_per_s": stp1["tokens_per_s"], "ms_per_step": stp1["ms_per_step"],
            "graph_ms_per_step": stp1["graph_ms_per_step"],
            "attn_ms_per_layer": stp1["attn_ms_per_layer"],
            "moe_ms_per_layer": stp1["moe_ms_per_layer"],
        }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
