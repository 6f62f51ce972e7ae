"""Golden vectors from the reference's own MoE code, compiled from source.

Runs oracle/_ref/libref_moe.so (src/matrix.c + src/transformer.c of the
reference built by `make -C oracle ref` with its release flags, AVX2+FMA
path) under FTZ/DAZ, the floating-point mode its -ffast-math executables
start in, on the synthetic inputs the tests use, and stores the outputs as
small .npz fixtures next to this script:

  golden_c1.npz        full config 1 layer (T=256 d=128 F=512 E=4 k=2):
                       probs, ids, out
  golden_softmax.npz   softmax_rows on crafted rows (ties, clamps, tails)
  golden_logits.npz    mat_mul router products incl. exact zeros in x
  golden_route.npz     probs/ids of token samples at every config's router
                       shape (config 5 with its Zipf bias)
  golden_moe.npz       layer outputs of token samples at configs 2-5
  golden_route_wide.npz probs/ids of routers wider than 128 experts (256
                       experts top-8; 250 experts top-16, an E % 8 tail) and
                       past 256 experts or top-16 (264 top-4, 300 top-20,
                       1024 top-32, 40 top-24)
  golden_rms.npz       rms_norm (src/matrix.c:666-711) rows at the configs'
                       widths and at widths with 8-column and scalar tails
  golden_attn.npz      the decode step's attention sublayer, x after
                       inference_step (src/inference.c:231-363) of a one-block
                       MoE model (whose decode FFN is the identity) and the
                       cache rows it writes, at several head shapes and
                       positions (oracle/_ref/libref_attn.so, run by
                       oracle/ref_attn_harness.c)

The reference MoE has no router bias (src/transformer.c:299-300).  Config 5
is run through the reference's own moe_forward with x extended by a column of
ones and W_router by the bias row: the FMA chain's last term is then 1*b[e],
i.e. logits + b rounded once — the mat_mul_add form the library implements.

Run (where the reference sources are present): python tests/golden/make_golden.py
(`... make_golden.py rms` / `... attn` / `... wide` write golden_rms.npz /
golden_attn.npz / golden_route_wide.npz only)
"""
import ctypes as C
import hashlib
import os
import sys

# One thread: the reference's OpenMP regions then run on the thread whose
# FP mode is set below (set before libgomp initialises).
os.environ["OMP_NUM_THREADS"] = "1"

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "llm.c_amd"))
import orc  # noqa: E402
from abi_types import FFNWeights, HostMoE, make_cache, matrix  # noqa: E402

CONFIGS = {
    "c1": dict(T=256, d=128, F=512, E=4, k=2, std_router=0.02, std_expert=0.02),
    "c2": dict(T=4096, d=256, F=1024, E=8, k=2, std_router=0.1, std_expert=0.02),
    "c3": dict(T=4096, d=512, F=2048, E=8, k=2, std_router=0.02, std_expert=0.02),
    "c4": dict(T=64, d=512, F=2048, E=16, k=2, std_router=0.02, std_expert=0.02),
    "c5": dict(T=16384, d=2048, F=8192, E=64, k=4, std_router=0.02, std_expert=0.02),
}


LOGIT_CASES = ((33, 100, 5), (64, 128, 16), (17, 2048, 64))


def logit_inputs(i, T, d, E):
    """Router-product inputs of golden_logits case i: exact zeros every 7th
    column of x and negative zeros in column 3 of every 5th row."""
    x = orc.synth((T, d), 77, i, 1.0)
    x[:, ::7] = 0.0
    x[::5, 3] = -0.0
    w = orc.synth((d, E), 77, 10 + i, 0.05)
    return x, w


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def ref_moe(x, hw):
    """The reference moe_forward on x with HostMoE weights."""
    T = x.shape[0]
    fc, probs, ids = make_cache(T, hw.E, hw.k)
    out = np.zeros((T, hw.d), np.float32)
    cfg = hw.config(T)
    orc.ref().moe_forward(C.byref(matrix(x)), C.byref(hw.weights), C.byref(cfg), C.byref(fc),
                          C.byref(matrix(out)))
    return out, probs, ids


def sparse_host(wr, experts, d, F, E, k):
    """HostMoE-like struct set where missing experts are tiny zero matrices
    the reference never touches (only routed experts are evaluated)."""
    class Sparse:
        pass
    s = Sparse()
    s.d, s.F, s.E, s.k = d, F, E, k
    s.wr = np.ascontiguousarray(wr)
    s.keep = []
    arr = (FFNWeights * E)()
    for e in range(E):
        if e in experts:
            wg, wu, wd = experts[e]
        else:
            wg = np.zeros((d, F), np.float32) if F * d <= (1 << 16) else np.zeros((1, 1), np.float32)
            wu, wd = wg, wg
        s.keep += [wg, wu, wd]
        arr[e] = FFNWeights(matrix(wg), matrix(wu), matrix(wd))
    s.arr = arr
    from abi_types import MoEWeights
    s.weights = MoEWeights(C.cast(arr, C.POINTER(FFNWeights)), matrix(s.wr), E, k)
    s.config = lambda T: HostMoE.config(s, T)
    return s


def route_with_bias(x, wr, bias, k, F=32):
    """Reference routing with a bias row (see module docstring)."""
    T, d = x.shape
    E = wr.shape[1]
    xb = np.ascontiguousarray(np.concatenate([x, np.ones((T, 1), np.float32)], axis=1))
    wb = np.ascontiguousarray(np.concatenate([wr, bias[None, :]], axis=0))
    z = np.zeros((E, d + 1, F), np.float32)
    zd = np.zeros((E, F, d + 1), np.float32)
    hw = HostMoE(wb, z, z, zd, k)
    _, probs, ids = ref_moe(xb, hw)
    return probs, ids


def main():
    if not orc.ref_available():
        sys.exit("oracle/_ref/libref_moe.so missing: run `make -C oracle ref` first")
    orc.orc().orc_set_ftz_daz(1)          # the calling thread now runs under FTZ/DAZ

    # ---- config 1, full layer
    c = CONFIGS["c1"]
    wr, ex = orc.synth_layer_host(c["d"], c["F"], c["E"], c["k"], 0, c["std_router"],
                                  c["std_expert"])
    hw = HostMoE(wr, np.stack([ex[e][0] for e in range(c["E"])]),
                 np.stack([ex[e][1] for e in range(c["E"])]),
                 np.stack([ex[e][2] for e in range(c["E"])]), c["k"])
    x = orc.synth((c["T"], c["d"]), 0, 0, 1.0)
    out, probs, ids = ref_moe(x, hw)
    np.savez_compressed(os.path.join(HERE, "golden_c1.npz"), probs=probs, ids=ids, out=out,
                        sha_x=sha(x), sha_wr=sha(wr), sha_wg0=sha(hw.wg[0]))
    print("c1:", np.bincount(ids.ravel(), minlength=c["E"]))

    # ---- softmax rows
    rng = np.random.default_rng(1234)
    rows = {}
    for E in (1, 4, 5, 8, 12, 16, 23, 64):
        m = [rng.standard_normal((64, E)) * 3,
             np.full((4, E), 0.25),                                   # all ties
             rng.uniform(-120, 0, (16, E)),                           # exp clamps / FTZ
             rng.uniform(-90, 90, (16, E)),
             np.round(rng.standard_normal((16, E)) * 2) / 4]          # many duplicates
        inp = np.concatenate(m).astype(np.float32)
        got = inp.copy()
        orc.ref().softmax_rows(C.byref(matrix(got)))
        rows[f"in_{E}"] = inp
        rows[f"out_{E}"] = got
    np.savez_compressed(os.path.join(HERE, "golden_softmax.npz"), **rows)

    # ---- router products (mat_mul) with exact zeros and negative zeros in x
    lg = {}
    for i, (T, d, E) in enumerate(LOGIT_CASES):
        x, w = logit_inputs(i, T, d, E)
        o = np.zeros((T, E), np.float32)
        orc.ref().mat_mul(C.byref(matrix(x)), C.byref(matrix(w)), C.byref(matrix(o)))
        lg[f"out_{i}"], lg[f"sha_x_{i}"], lg[f"sha_w_{i}"] = o, sha(x), sha(w)
    np.savez_compressed(os.path.join(HERE, "golden_logits.npz"), **lg)

    # ---- routing samples at every config's router shape
    zipf = np.load(os.path.join(HERE, "zipf_bias_e64_k4.npy")).astype(np.float32)
    rt = {}
    for name in ("c2", "c3", "c4", "c5"):
        c = CONFIGS[name]
        T = min(c["T"], 256)
        x = orc.synth((T, c["d"]), 7, 0, 1.0)
        wr = orc.synth((c["d"], c["E"]), 7, 1, c["std_router"])
        if name == "c5":
            probs, ids = route_with_bias(x, wr, zipf, c["k"])
        else:
            z = np.zeros((c["E"], c["d"], 32), np.float32)
            zd = np.zeros((c["E"], 32, c["d"]), np.float32)
            _, probs, ids = ref_moe(x, HostMoE(wr, z, z, zd, c["k"]))
        rt[f"{name}_probs"], rt[f"{name}_ids"] = probs, ids
        rt[f"{name}_sha_x"], rt[f"{name}_sha_wr"] = sha(x), sha(wr)
    np.savez_compressed(os.path.join(HERE, "golden_route.npz"), **rt)

    # ---- layer outputs on token samples (seed 3)
    mo = {}
    for name, ns in (("c2", 64), ("c3", 32), ("c4", 64), ("c5", 6)):
        c = CONFIGS[name]
        d, F, E, k = c["d"], c["F"], c["E"], c["k"]
        x = orc.synth((ns, d), 3, 0, 1.0)
        wr = orc.synth((d, E), 3, 1, c["std_router"])
        if name == "c5":
            probs, ids = route_with_bias(x, wr, zipf, k)
            need = sorted(set(ids.ravel().tolist()))
            _, ex = orc.synth_layer_host(d, F, E, k, 3, c["std_router"], c["std_expert"],
                                         experts=need)
            # Fold the bias into x/W_router exactly as route_with_bias does.
            xb = np.ascontiguousarray(np.concatenate([x, np.ones((ns, 1), np.float32)], 1))
            wb = np.ascontiguousarray(np.concatenate([wr, zipf[None, :]], 0))
            exb = {e: (np.ascontiguousarray(np.concatenate([g, np.zeros((1, F), np.float32)], 0)),
                       np.ascontiguousarray(np.concatenate([u, np.zeros((1, F), np.float32)], 0)),
                       np.ascontiguousarray(np.concatenate([dn, np.zeros((F, 1), np.float32)], 1)))
                   for e, (g, u, dn) in ex.items()}
            sp = sparse_host(wb, exb, d + 1, F, E, k)
            out, probs2, ids2 = ref_moe(xb, sp)
            assert np.array_equal(ids2, ids)
            out = np.ascontiguousarray(out[:, :d])
        else:
            _, ex = orc.synth_layer_host(d, F, E, k, 3, c["std_router"], c["std_expert"])
            hw = HostMoE(wr, np.stack([ex[e][0] for e in range(E)]),
                         np.stack([ex[e][1] for e in range(E)]),
                         np.stack([ex[e][2] for e in range(E)]), k)
            out, probs, ids = ref_moe(x, hw)
        mo[f"{name}_out"], mo[f"{name}_probs"], mo[f"{name}_ids"] = out, probs, ids
        print(name, "sample done")
    np.savez_compressed(os.path.join(HERE, "golden_moe.npz"), **mo)


RMS_WIDTHS = (128, 256, 512, 2048, 24, 8, 100, 7)


def rms_inputs(cols):
    """rms_norm golden inputs: 12 rows of N(0, 1) scaled per row over six
    decades, one all-zero row (ss = 0), weights N(1, 0.1); eps 1e-5."""
    x = orc.synth((14, cols), 55, cols, 1.0)
    x *= (10.0 ** np.linspace(-3, 3, 14, dtype=np.float32))[:, None]
    x[13] = 0.0
    w = orc.synth((cols,), 55, 1000 + cols, 0.1, mean=1.0)
    return np.ascontiguousarray(x), w


def main_rms():
    if not orc.ref_available():
        sys.exit("oracle/_ref/libref_moe.so missing: run `make -C oracle ref` first")
    orc.orc().orc_set_ftz_daz(1)
    ref = orc.ref()
    ref.rms_norm.argtypes = [C.c_void_p, C.c_void_p, C.c_float, C.c_void_p]
    rs = {}
    for cols in RMS_WIDTHS:
        x, w = rms_inputs(cols)
        y = np.zeros_like(x)
        ref.rms_norm(C.byref(matrix(x)), w.ctypes.data, C.c_float(1e-5), C.byref(matrix(y)))
        rs[f"out_{cols}"], rs[f"sha_x_{cols}"], rs[f"sha_w_{cols}"] = y, sha(x), sha(w)
    np.savez_compressed(os.path.join(HERE, "golden_rms.npz"), **rs)


# (d, nh, nkv, hd, max_seq, positions): GQA 4, the decode config's heads
# (d 512, hd 64), 8 query heads on one kv head, and one query head per kv head.
ATTN_CASES = (
    (128, 8, 2, 16, 40, (0, 1, 17, 39)),
    (512, 8, 2, 64, 160, (0, 5, 127, 128, 159)),
    (256, 8, 1, 32, 70, (0, 33, 69)),
    (64, 4, 4, 16, 24, (0, 2, 23)),
)


def attn_inputs(i):
    """Inputs of attention case i: x N(0, 3^2) rows (one per position), W_Q,
    W_K, W_V N(0, 1/d), W_O N(0, 1/qd), rms_attn N(1, 0.1), caches N(0, 1);
    RoPE tables from orc.rope_tables(max_seq, hd, 10000)."""
    d, nh, nkv, hd, ms, pos = ATTN_CASES[i]
    qd, kd, sd = nh * hd, nkv * hd, 900 + 10 * i
    f = lambda shape, st, std, mean=0.0: orc.synth(shape, sd, st, std, mean=mean)
    w = dict(wq=f((d, qd), 1, d ** -0.5), wk=f((d, kd), 2, d ** -0.5), wv=f((d, kd), 3, d ** -0.5),
             wo=f((qd, d), 4, qd ** -0.5), rms=f((d,), 5, 0.1, mean=1.0))
    x = f((len(pos), d), 6, 3.0)
    kc, vc = f((ms, kd), 7, 1.0), f((ms, kd), 8, 1.0)
    cos_t, sin_t = orc.rope_tables(ms, hd, 10000.0)
    return x, w, kc, vc, np.asarray(pos, np.int32), cos_t, sin_t


def main_attn():
    lib_path = os.path.join(ROOT, "oracle", "_ref", "libref_attn.so")
    if not os.path.exists(lib_path):
        sys.exit("oracle/_ref/libref_attn.so missing: run `make -C oracle ref` first")
    orc.orc().orc_set_ftz_daz(1)
    ref = C.CDLL(lib_path)
    P, I, F = C.c_void_p, C.c_int, C.c_float
    ref.ref_attn_step.argtypes = [I, I, I, I, I, F] + [P] * 9 + [I, P]
    ref.ref_attn_step.restype = I
    gs = {}
    for i, (d, nh, nkv, hd, ms, pos) in enumerate(ATTN_CASES):
        x, w, kc, vc, pos, cos_t, sin_t = attn_inputs(i)
        outs, krows, vrows = [], [], []
        for j, p in enumerate(pos):
            xo, k2, v2 = x[j].copy(), kc.copy(), vc.copy()
            ptr = lambda a: a.ctypes.data
            rc = ref.ref_attn_step(d, nh, nkv, hd, ms, F(1e-5), ptr(w["wq"]), ptr(w["wk"]),
                                   ptr(w["wv"]), ptr(w["wo"]), ptr(w["rms"]), ptr(cos_t),
                                   ptr(sin_t), ptr(k2), ptr(v2), int(p), ptr(xo))
            assert rc == 0
            keep = np.arange(ms) != p
            assert np.array_equal(k2[keep], kc[keep]) and np.array_equal(v2[keep], vc[keep])
            outs.append(xo); krows.append(k2[p]); vrows.append(v2[p])
        gs[f"x_{i}"], gs[f"k_{i}"], gs[f"v_{i}"] = np.stack(outs), np.stack(krows), np.stack(vrows)
        gs[f"sha_x_{i}"], gs[f"sha_kc_{i}"], gs[f"sha_wq_{i}"] = sha(x), sha(kc), sha(w["wq"])
        print("attention case", i, "done")
    np.savez_compressed(os.path.join(HERE, "golden_attn.npz"), **gs)


# Routing samples of layers wider than 128 experts (one with an E % 8 tail).
WIDE_ROUTES = [
    # name, T, d, E, k, std_router
    ("e256k8", 64, 128, 256, 8, 0.1),
    ("e250k16", 40, 64, 250, 16, 0.3),
    # past the fast routing kernels' tables (the general kernels)
    ("e264k4", 64, 64, 264, 4, 0.2),
    ("e300k20", 48, 64, 300, 20, 0.3),
    ("e1024k32", 32, 128, 1024, 32, 0.1),
    ("e40k24", 40, 64, 40, 24, 0.5),
]


def main_wide():
    if not orc.ref_available():
        sys.exit("oracle/_ref/libref_moe.so missing: run `make -C oracle ref` first")
    orc.orc().orc_set_ftz_daz(1)
    rt = {}
    for name, T, d, E, k, std in WIDE_ROUTES:
        x = orc.synth((T, d), 7, 0, 1.0)
        wr = orc.synth((d, E), 7, 1, std)
        z = np.zeros((E, d, 32), np.float32)
        zd = np.zeros((E, 32, d), np.float32)
        _, probs, ids = ref_moe(x, HostMoE(wr, z, z, zd, k))
        rt[f"{name}_probs"], rt[f"{name}_ids"] = probs, ids
        rt[f"{name}_sha_x"], rt[f"{name}_sha_wr"] = sha(x), sha(wr)
    np.savez_compressed(os.path.join(HERE, "golden_route_wide.npz"), **rt)


if __name__ == "__main__":
    if sys.argv[1:] == ["rms"]:
        main_rms()
    elif sys.argv[1:] == ["attn"]:
        main_attn()
    elif sys.argv[1:] == ["wide"]:
        main_wide()
    else:
        main()
        main_rms()
        main_attn()
        main_wide()
