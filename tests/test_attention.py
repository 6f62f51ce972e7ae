"""The attention half of the KV-cache decode step (src/inference.c:252-308).

CPU: the oracle restatement (orc_attn_decode) pinned against the compiled
reference's own decode step (golden_attn.npz: inference_step of
src/inference.c, built from source, on a one-block MoE model whose decode
FFN is the identity), by an fp64 textbook evaluation and by closed forms
(position 0 attends only the new token, so W_Q and W_K drop out; RoPE at
position 0 is the identity).
GPU: moe_hip_attn_decode_dev against the oracle within the layer tolerance
(chunked softmax and V sums reorder the reference's sequential ones)."""
import numpy as np
import pytest

import moe_hip as mh
import orc

import os, sys  # noqa: E401
sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden as mg  # noqa: E402  (input builders only; the reference is not run)

D, NH, NKV, HD = 128, 8, 2, 16


def make_case(B, max_seq, pos, seed, d=D, nh=NH, nkv=NKV, hd=HD):
    rng = np.random.default_rng(seed)
    qd, kd = nh * hd, nkv * hd
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    w = dict(wq=f(d, qd) / np.sqrt(d), wk=f(d, kd) / np.sqrt(d), wv=f(d, kd) / np.sqrt(d),
             wo=f(qd, d) / np.sqrt(qd), rms=(1.0 + 0.1 * f(d)).astype(np.float32))
    w = {k: v.astype(np.float32) for k, v in w.items()}
    x = f(B, d)
    kc, vc = f(B, max_seq, kd), f(B, max_seq, kd)
    cos_t, sin_t = orc.rope_tables(max_seq, hd, 10000.0)
    return x, w, kc, vc, np.asarray(pos, np.int32), cos_t, sin_t


def run_oracle(x, w, kc, vc, pos, cos_t, sin_t, nh=NH, nkv=NKV, hd=HD):
    return orc.attn_decode(x, w["rms"], 1e-5, w["wq"], w["wk"], w["wv"], w["wo"], cos_t, sin_t,
                           kc, vc, pos, nh, nkv, hd)


def textbook(x, w, kc, vc, pos, cos_t, sin_t, nh=NH, nkv=NKV, hd=HD):
    """fp64 attention step with the reference's definitions."""
    x = x.astype(np.float64)
    out = x.copy()
    B, d = x.shape
    gqa, half = nh // nkv, hd // 2
    for b in range(B):
        p = int(pos[b])
        xn = x[b] / np.sqrt((x[b] ** 2).mean() + 1e-5) * w["rms"]
        q, k, v = xn @ w["wq"], xn @ w["wk"], xn @ w["wv"]
        def rope(t, heads):
            t = t.reshape(heads, hd).copy()
            c, s = cos_t[p].astype(np.float64), sin_t[p].astype(np.float64)
            a, bb = t[:, 0::2].copy(), t[:, 1::2].copy()
            t[:, 0::2], t[:, 1::2] = a * c - bb * s, a * s + bb * c
            return t
        q, k = rope(q, nh), rope(k, nkv).reshape(-1)
        K = kc[b].astype(np.float64).copy()
        V = vc[b].astype(np.float64).copy()
        K[p], V[p] = k, v
        ho = np.zeros((nh, hd))
        for h in range(nh):
            kv = h // gqa
            sc = K[: p + 1, kv * hd:(kv + 1) * hd] @ q[h] / np.sqrt(hd)
            e = np.exp(sc - sc.max())
            ho[h] = (e / e.sum()) @ V[: p + 1, kv * hd:(kv + 1) * hd]
        out[b] = x[b] + ho.reshape(-1) @ w["wo"]
    return out


@pytest.mark.parametrize("case", range(len(mg.ATTN_CASES)))
def test_oracle_vs_reference_decode_step(case):
    """The oracle against the compiled reference's inference_step, position
    by position: x within 2e-6 relative (the reference's -ffast-math build
    reassociates rmsnorm_vec's sum and vectorises expf), the k and v rows it
    appends within 1e-6."""
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "golden_attn.npz"))
    d, nh, nkv, hd, ms, _ = mg.ATTN_CASES[case]
    x, w, kc, vc, pos, cos_t, sin_t = mg.attn_inputs(case)
    B = len(pos)
    kcb = np.ascontiguousarray(np.broadcast_to(kc, (B,) + kc.shape))
    vcb = np.ascontiguousarray(np.broadcast_to(vc, (B,) + vc.shape))
    xo, ko, vo = run_oracle(x, w, kcb, vcb, pos, cos_t, sin_t, nh, nkv, hd)
    assert orc.rel_l2(xo, g[f"x_{case}"]) < 2e-6
    assert float(np.abs(xo - g[f"x_{case}"]).max()) < 2e-5
    for b, p in enumerate(pos):
        assert orc.rel_l2(ko[b, p], g[f"k_{case}"][b]) < 1e-6
        assert orc.rel_l2(vo[b, p], g[f"v_{case}"][b]) < 1e-6


def test_oracle_vs_fp64_textbook():
    pos = [0, 1, 5, 30, 63, 17]
    x, w, kc, vc, pos, c, s = make_case(len(pos), 64, pos, 1)
    xo, kco, vco = run_oracle(x, w, kc, vc, pos, c, s)
    ref = textbook(x, w, kc, vc, pos, c, s)
    assert float(np.abs(xo - ref).max() / np.abs(ref).max()) < 2e-6
    # Cache rows other than pos are untouched, row pos holds the new k and v.
    for b, p in enumerate(pos):
        keep = np.arange(64) != p
        assert np.array_equal(kco[b, keep], kc[b, keep]) and np.array_equal(vco[b, keep], vc[b, keep])
        assert not np.array_equal(kco[b, p], kc[b, p])


def test_position_zero_ignores_query_and_key():
    """At position 0 the softmax has one entry (weight 1), so the output is
    x + W_O . repeat(v): W_Q and W_K drop out exactly."""
    x, w, kc, vc, pos, c, s = make_case(3, 8, [0, 0, 0], 2)
    a, _, _ = run_oracle(x, w, kc, vc, pos, c, s)
    w2 = dict(w, wq=w["wq"] * 3.0 + 1.0, wk=-w["wk"])
    b, _, _ = run_oracle(x, w2, kc, vc, pos, c, s)
    assert np.array_equal(a, b)
    # and the cache contents past row 0 do not matter
    _, _, _ = run_oracle(x, w, kc * 0 + 7, vc * 0 - 3, pos, c, s)
    d2, _, _ = run_oracle(x, w, kc * 0 + 7, vc * 0 - 3, pos, c, s)
    assert np.array_equal(a, d2)


def test_rope_table_identity_at_position_zero():
    c, s = orc.rope_tables(16, HD, 10000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    # angle of pair 0 is the position itself
    assert np.allclose(c[:, 0], np.cos(np.arange(16)), atol=1e-6)


# ---------------------------------------------------------------- GPU
def run_device(x, w, kc, vc, pos, c, s, nh=NH, nkv=NKV, hd=HD):
    B, d = x.shape
    max_seq = kc.shape[1]
    at = mh.Attn(d, nh, nkv, hd, max_seq)
    try:
        at.load(w["wq"], w["wk"], w["wv"], w["wo"], w["rms"])
        at.set_rope(c, s)
        dx, dk, dv = (mh.DeviceArray.from_host(np.ascontiguousarray(a)) for a in (x, kc, vc))
        dp = mh.DeviceArray.from_host(np.ascontiguousarray(pos, np.int32))
        at.decode_dev(dx.ptr, B, dp.ptr, dk.ptr, dv.ptr, 1e-5)
        return dx.to_host(), dk.to_host(), dv.to_host()
    finally:
        at.close()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(128, 8, 2, 16, 600), (512, 8, 2, 64, 1100),
                                   (256, 8, 1, 32, 300), (64, 4, 4, 16, 300),
                                   (64, 2, 1, 8, 300)],
                         ids=["small", "config4", "g8", "mha-generic", "hd8-unpacked"])
def test_attn_decode_device(shape):
    """Outputs within the layer tolerance of the oracle; the new k, v rows
    within it too, every other cache row bit-for-bit unchanged.  mha-generic
    (one query head per kv head) runs the generic chunk kernels."""
    d, nh, nkv, hd, max_seq = shape
    pos = [0, 1, 2, 127, 128, 129, 255, 256, max_seq - 1, 100, min(300, max_seq - 2), 37]
    x, w, kc, vc, pos, c, s = make_case(len(pos), max_seq, pos, 5, d, nh, nkv, hd)
    print(f"[gpu-test] attention {shape}", flush=True)
    xg, kg, vg = run_device(x, w, kc, vc, pos, c, s, nh, nkv, hd)
    xo, ko, vo = run_oracle(x, w, kc, vc, pos, c, s, nh, nkv, hd)
    rel = orc.rel_l2(xg, xo)
    mabs = float(np.abs(xg - xo).max())
    print(f"[gpu-test]   rel-L2 {rel:.3e} max-abs {mabs:.3e}", flush=True)
    assert rel <= 1e-5 and mabs <= 1e-4
    for b, p in enumerate(pos):
        keep = np.arange(max_seq) != p
        assert np.array_equal(kg[b, keep], kc[b, keep]) and np.array_equal(vg[b, keep], vc[b, keep])
        assert orc.rel_l2(kg[b, p], ko[b, p]) < 1e-5 and orc.rel_l2(vg[b, p], vo[b, p]) < 1e-5


@pytest.mark.gpu
def test_attn_decode_repeatable_and_batch_sizes():
    """The same bits on a repeat (the merge counters are back at zero) and at
    other batch sizes (ragged row tiles; up to 4 rows, the projections take
    one workgroup per output column quad)."""
    for B in (1, 2, 4, 5, 33, 64, 70):
        pos = np.arange(B, dtype=np.int32) * 7 % 200
        x, w, kc, vc, pos, c, s = make_case(B, 200, pos, 8)
        a1 = run_device(x, w, kc, vc, pos, c, s)
        a2 = run_device(x, w, kc, vc, pos, c, s)
        for u, v in zip(a1, a2):
            assert np.array_equal(u, v)
        xo, _, _ = run_oracle(x, w, kc, vc, pos, c, s)
        assert orc.rel_l2(a1[0], xo) <= 1e-5, B


@pytest.mark.gpu
def test_attn_decode_position_out_of_range():
    """A position outside [0, max_seq) leaves that sequence untouched."""
    x, w, kc, vc, _, c, s = make_case(3, 64, [0, 0, 0], 6)
    pos = np.array([5, 64, -1], np.int32)
    xg, kg, vg = run_device(x, w, kc, vc, pos, c, s)
    for b in (1, 2):
        assert np.array_equal(xg[b], x[b])
        assert np.array_equal(kg[b], kc[b]) and np.array_equal(vg[b], vc[b])
    xo, _, _ = run_oracle(x[:1], w, kc[:1], vc[:1], pos[:1], c, s)
    assert orc.rel_l2(xg[:1], xo) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("B", [40, 1, 2])
def test_decode_block_device(B):
    """moe_hip_decode_block_dev: x += Attn(rms_norm(x)), then x += MoE(
    rms_norm(x; rms_ffn)).  The FFN's normalised rows (made by the MoE
    router's first step) are bit-identical to rms_norm of the attention
    output, routing on them is bit-exact, and x is within the layer
    tolerance of that output plus the oracle's MoE.  One or two sequences
    (the single-sequence inference step) take the few-row expert kernel."""
    from conftest import CONFIGS
    from test_gpu_parity import assert_close, bits, host_layer
    c = CONFIGS["c4"]
    d, F, E, k = c["d"], c["F"], c["E"], c["k"]
    nh, nkv, hd, max_seq = 8, 2, d // 8, 300
    pos = np.random.default_rng(12).integers(0, max_seq, B).astype(np.int32)
    if B > 3:
        pos[3] = max_seq      # out of range: attention skipped, FFN still applied
    x, w, kc, vc, pos, cs, sn = make_case(B, max_seq, pos, 12, d, nh, nkv, hd)
    rms_ffn = (1.0 + 0.1 * np.random.default_rng(13).standard_normal(d)).astype(np.float32)
    x_attn, _, _ = run_device(x, w, kc, vc, pos, cs, sn, nh, nkv, hd)

    layer = mh.Layer(d, F, E, k)
    layer.fill_synthetic(11, c["std_router"], c["std_expert"])
    hw = host_layer(d, F, E, k, 11, c["std_router"], c["std_expert"])
    at = mh.Attn(d, nh, nkv, hd, max_seq)
    try:
        at.load(w["wq"], w["wk"], w["wv"], w["wo"], w["rms"])
        at.set_rope(cs, sn)
        dx, dk, dv = (mh.DeviceArray.from_host(np.ascontiguousarray(a)) for a in (x, kc, vc))
        dp = mh.DeviceArray.from_host(pos)
        dw = mh.DeviceArray.from_host(rms_ffn)
        dxn = mh.DeviceArray((B, d))
        dids = mh.DeviceArray((B, k), np.int32)
        print(f"[gpu-test] decode block B={B}", flush=True)
        at.decode_block_dev(layer, dw.ptr, dx.ptr, B, dp.ptr, dk.ptr, dv.ptr, 1e-5, dxn.ptr,
                            dids.ptr)
        xn_ref = orc.rms_norm(x_attn, rms_ffn, 1e-5)
        assert np.array_equal(bits(dxn.to_host()), bits(xn_ref))
        o_ref, _, i_ref = orc.moe_forward(xn_ref, hw, nthreads=16)
        assert np.array_equal(dids.to_host(), i_ref)
        assert_close(dx.to_host(), x_attn + o_ref, "decode block")
        if B * k <= 4:
            assert mh.last_forward_path() == 6
    finally:
        at.close()
        layer.close()


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(mg.ATTN_CASES)))
def test_attn_decode_device_vs_reference(case):
    """The device sublayer on the golden inputs against the compiled
    reference's inference_step outputs (golden_attn.npz), within the layer
    tolerance."""
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "golden_attn.npz"))
    d, nh, nkv, hd, ms, _ = mg.ATTN_CASES[case]
    x, w, kc, vc, pos, cos_t, sin_t = mg.attn_inputs(case)
    B = len(pos)
    kcb = np.ascontiguousarray(np.broadcast_to(kc, (B,) + kc.shape))
    vcb = np.ascontiguousarray(np.broadcast_to(vc, (B,) + vc.shape))
    print(f"[gpu-test] attention vs reference case {case}", flush=True)
    xg, kg, vg = run_device(x, w, kcb, vcb, pos, cos_t, sin_t, nh, nkv, hd)
    rel, mabs = orc.rel_l2(xg, g[f"x_{case}"]), float(np.abs(xg - g[f"x_{case}"]).max())
    print(f"[gpu-test]   rel-L2 {rel:.3e} max-abs {mabs:.3e}", flush=True)
    assert rel <= 1e-5 and mabs <= 1e-4
    for b, p in enumerate(pos):
        assert orc.rel_l2(kg[b, p], g[f"k_{case}"][b]) < 1e-5
        assert orc.rel_l2(vg[b, p], g[f"v_{case}"][b]) < 1e-5


def draw_attn(i):
    rng = np.random.default_rng(7000 + i)
    hd = int(rng.choice([8, 16, 32, 64]))
    nkv = int(rng.choice([1, 2, 4]))
    nh = nkv * int(rng.choice([1, 2, 4, 8]))
    d = int(rng.choice([64, 128, 256, 512]))
    B = int(rng.choice([1, 3, 17, 64]))
    max_seq = int(rng.choice([1, 2, 100, 129, 700, 1100]))
    return d, nh, nkv, hd, B, max_seq, rng.integers(0, max_seq, B)


ATTN_RANDOM = [draw_attn(i) for i in range(24)]


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(len(ATTN_RANDOM)),
                         ids=[f"d{c[0]}_h{c[1]}_kv{c[2]}_hd{c[3]}_B{c[4]}_S{c[5]}" for c in ATTN_RANDOM])
def test_attn_decode_random_shapes(i):
    """Seeded random head shapes (hd 8-64, one to eight query heads per kv
    head, 1-64 sequences at random positions, caches of 1-1100 positions):
    x within the layer tolerance of the oracle, the new cache rows too,
    every other cache row unchanged bit for bit."""
    d, nh, nkv, hd, B, max_seq, pos = ATTN_RANDOM[i]
    x, w, kc, vc, pos, c, s = make_case(B, max_seq, pos, 200 + i, d, nh, nkv, hd)
    print(f"[gpu-test] attention random {i}: d={d} nh={nh} nkv={nkv} hd={hd} B={B} S={max_seq}",
          flush=True)
    xg, kg, vg = run_device(x, w, kc, vc, pos, c, s, nh, nkv, hd)
    xo, ko, vo = run_oracle(x, w, kc, vc, pos, c, s, nh, nkv, hd)
    assert orc.rel_l2(xg, xo) <= 1e-5 and float(np.abs(xg - xo).max()) <= 1e-4
    for b, p in enumerate(pos):
        keep = np.arange(max_seq) != p
        assert np.array_equal(kg[b, keep], kc[b, keep]) and np.array_equal(vg[b, keep], vc[b, keep])
        assert orc.rel_l2(kg[b, p], ko[b, p]) < 1e-5 and orc.rel_l2(vg[b, p], vo[b, p]) < 1e-5
