"""TEST INFRASTRUCTURE: ctypes wrapper of the CPU oracle (oracle/liborc_moe.so)
and of the reference compiled from source (oracle/_ref/libref_moe.so, only
present where the reference sources were available at build time).

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use this.
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "llm.c_amd"))
from abi_types import fptr, iptr  # noqa: E402

ORC_PATH = os.path.join(HERE, "liborc_moe.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_moe.so")

_F = C.POINTER(C.c_float)
_I = C.POINTER(C.c_int)
_FP = C.POINTER(_F)

_orc = None
_ref = None


def orc():
    global _orc
    if _orc is None:
        if not os.path.exists(ORC_PATH):
            raise FileNotFoundError(f"{ORC_PATH} missing: run `make -C oracle`")
        L = C.CDLL(ORC_PATH)
        L.orc_set_ftz_daz.restype = C.c_int
        L.orc_set_ftz_daz.argtypes = [C.c_int]
        L.orc_router_logits.argtypes = [_F, _F, _F, C.c_int, C.c_int, C.c_int, _F]
        L.orc_exp_poly.restype = C.c_float
        L.orc_exp_poly.argtypes = [C.c_float]
        L.orc_expf.restype = C.c_float
        L.orc_expf.argtypes = [C.c_float]
        L.orc_expf_raw.restype = C.c_float
        L.orc_expf_raw.argtypes = [C.c_float, C.c_int]
        L.orc_expf_table_entry.restype = C.c_uint64
        L.orc_expf_table_entry.argtypes = [C.c_int]
        L.orc_expf_compare_libm.restype = C.c_longlong
        L.orc_expf_compare_libm.argtypes = [C.c_uint32, C.c_uint32, C.c_int,
                                            C.POINTER(C.c_uint32)]
        L.orc_expf_array.argtypes = [_F, _F, C.c_longlong]
        L.orc_exp_poly_array.argtypes = [_F, _F, C.c_longlong]
        L.orc_set_softmax_tail_recip.argtypes = [C.c_int]
        L.orc_rms_norm.argtypes = [_F, _F, C.c_float, C.c_int, C.c_int, _F]
        L.orc_attn_decode.argtypes = [_F, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _F,
                                      C.c_float, _F, _F, _F, _F, _F, _F, _F, _F, C.c_int, _I]
        L.orc_rope_tables.argtypes = [C.c_int, C.c_int, C.c_float, _F, _F]
        L.orc_softmax_rows.argtypes = [_F, C.c_int, C.c_int]
        L.orc_topk.argtypes = [_F, C.c_int, C.c_int, C.c_int, _I, _F]
        L.orc_dispatch.argtypes = [_I, C.c_int, C.c_int, C.c_int, _I, _I, _I]
        L.orc_swiglu.argtypes = [_F, _F, _F, C.c_int]
        L.orc_moe_forward.argtypes = [_F, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _F, _F,
                                      _FP, _FP, _FP, _F, _F, _I, C.c_int]
        L.orc_moe_forward_f64.argtypes = [_F, C.c_int, C.c_int, C.c_int, C.c_int, _I, _F,
                                          C.c_int, _FP, _FP, _FP, C.POINTER(C.c_double)]
        L.orc_synth_normal.argtypes = [_F, C.c_longlong, C.c_ulonglong, C.c_ulonglong,
                                       C.c_float, C.c_float]
        # The compiled reference computes the softmax tail as x * (1/sum)
        # (-freciprocal-math); the oracle defaults to that form.
        L.orc_set_softmax_tail_recip(1)
        _orc = L
    return _orc


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    global _ref
    if _ref is None:
        _ref = C.CDLL(REF_PATH)
    return _ref


# ---------------------------------------------------------------- helpers
def synth(shape, seed, stream, std, mean=0.0):
    a = np.empty(shape, np.float32)
    orc().orc_synth_normal(fptr(a), a.size, seed, stream, mean, std)
    return a


def rms_norm(x, w, eps):
    """rms_norm (src/matrix.c:666-711) rows of x with weight w; see
    orc_rms_norm for the one deliberate difference (correctly rounded
    1/sqrt instead of the x86 RSQRTSS estimate)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    orc().orc_rms_norm(fptr(x), fptr(np.ascontiguousarray(w, np.float32)), eps, x.shape[0],
                       x.shape[1], fptr(y))
    return y


def rope_tables(max_seq, hd, theta):
    """cos, sin [max_seq x hd/2] as rope_buffer_init (src/attention.c:151-167)
    computes them (host libm)."""
    c = np.empty((max_seq, hd // 2), np.float32)
    s = np.empty((max_seq, hd // 2), np.float32)
    orc().orc_rope_tables(max_seq, hd, theta, fptr(c), fptr(s))
    return c, s


def attn_decode(x, rms_w, eps, wq, wk, wv, wo, cos_t, sin_t, kc, vc, pos, nh, nkv, hd):
    """The attention half of inference_step (src/inference.c:252-308) for
    rows x [B x d]; returns (x', kc', vc') (inputs untouched).  kc, vc
    [B x max_seq x nkv*hd]; pos [B]."""
    x = np.array(x, np.float32, copy=True, order="C")
    kc = np.array(kc, np.float32, copy=True, order="C")
    vc = np.array(vc, np.float32, copy=True, order="C")
    pos = np.ascontiguousarray(pos, np.int32)
    B, d = x.shape
    # The restatement, like inference_step, needs pos < max_seq (it writes
    # cache row pos and scores 0 .. pos); refuse rather than overrun.
    if pos.shape != (B,) or kc.shape[0] != B or (pos < 0).any() or (pos >= kc.shape[1]).any():
        raise ValueError("attn_decode: every position must lie in [0, max_seq)")
    ar = [np.ascontiguousarray(a, np.float32) for a in (rms_w, wq, wk, wv, wo, cos_t, sin_t)]
    orc().orc_attn_decode(fptr(x), B, d, nh, nkv, hd, fptr(ar[0]), eps, fptr(ar[1]), fptr(ar[2]),
                          fptr(ar[3]), fptr(ar[4]), fptr(ar[5]), fptr(ar[6]), fptr(kc), fptr(vc),
                          kc.shape[1], iptr(pos))
    return x, kc, vc


def router_logits(x, wr, bias=None):
    T, d = x.shape
    E = wr.shape[1]
    out = np.empty((T, E), np.float32)
    orc().orc_router_logits(fptr(x), fptr(wr), fptr(bias) if bias is not None else None,
                            T, d, E, fptr(out))
    return out


def softmax_rows(m):
    m = np.array(m, np.float32, copy=True, order="C")
    orc().orc_softmax_rows(fptr(m), m.shape[0], m.shape[1])
    return m


def topk(probs, k):
    T, E = probs.shape
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    orc().orc_topk(fptr(probs), T, E, k, iptr(ids), fptr(w))
    return ids, w


def dispatch(ids, E):
    T, k = ids.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    perm = np.empty(T * k, np.int32)
    orc().orc_dispatch(iptr(np.ascontiguousarray(ids)), T, k, E, iptr(counts), iptr(offsets),
                       iptr(perm))
    return counts, offsets, perm


def route(x, wr, k, bias=None):
    """(probs, ids, gate_weights) as the reference computes them."""
    probs = softmax_rows(router_logits(x, wr, bias))
    ids, w = topk(probs, k)
    return probs, ids, w


def moe_forward(x, hw, bias=None, nthreads=1):
    """Oracle layer output for x [T x d] with HostMoE weights hw."""
    T = x.shape[0]
    out = np.empty((T, hw.d), np.float32)
    probs = np.empty((T, hw.E), np.float32)
    ids = np.empty((T, hw.k), np.int32)
    g, u, dn = hw.expert_ptr_arrays()
    orc().orc_moe_forward(fptr(x), T, hw.d, hw.F, hw.E, hw.k, fptr(hw.wr),
                          fptr(bias) if bias is not None else None, g, u, dn, fptr(out),
                          fptr(probs), iptr(ids), nthreads)
    return out, probs, ids


def moe_forward_experts(x, wr, experts, d, F, E, k, bias=None, nthreads=1):
    """Oracle layer output when only some experts' weights are materialised:
    `experts` maps expert id -> (wg [d x F], wu [d x F], wd [F x d]); every
    expert chosen by the rows of x must be present."""
    T = x.shape[0]
    out = np.empty((T, d), np.float32)
    probs = np.empty((T, E), np.float32)
    ids = np.empty((T, k), np.int32)
    P = _F * E
    null = C.cast(None, _F)
    g = P(*[fptr(experts[e][0]) if e in experts else null for e in range(E)])
    u = P(*[fptr(experts[e][1]) if e in experts else null for e in range(E)])
    dn = P(*[fptr(experts[e][2]) if e in experts else null for e in range(E)])
    orc().orc_moe_forward(fptr(x), T, d, F, E, k, fptr(wr),
                          fptr(bias) if bias is not None else None, g, u, dn, fptr(out),
                          fptr(probs), iptr(ids), nthreads)
    return out, probs, ids


def ref_moe_forward_experts(x, wr, experts, d, F, E, k, threads=1):
    """The compiled reference's own moe_forward (oracle/_ref/libref_moe.so,
    src/transformer.c:287-366 built with the release flags) on x [T x d],
    with OpenMP limited to `threads`; FTZ/DAZ on, as its executables run.
    `experts` maps expert id -> (wg, wu, wd) and must hold every expert the
    rows choose (the reference has no router bias; `route` gives its ids).
    Returns (out, probs, ids)."""
    from abi_types import FFNWeights, Matrix, MoEWeights, ModelConfig, make_cache, matrix
    T = x.shape[0]
    _, need, _ = route(x, wr, k)
    missing = set(need.ravel().tolist()) - set(experts)
    if missing:
        raise ValueError(f"experts {sorted(missing)} are chosen but not materialised")
    arr = (FFNWeights * E)()
    empty = Matrix(None, None, 0, 0)
    for e in range(E):
        arr[e] = (FFNWeights(matrix(experts[e][0]), matrix(experts[e][1]), matrix(experts[e][2]))
                  if e in experts else FFNWeights(empty, empty, empty))
    w = MoEWeights(C.cast(arr, C.POINTER(FFNWeights)), matrix(wr), E, k)
    cfg = ModelConfig(vocab_size=0, max_seq_len=T, d_model=d, n_layers=1, n_heads=1,
                      n_kv_heads=1, head_dim=d, window_size=0, ffn_hidden=F, n_experts=E,
                      top_k_experts=k, rms_norm_eps=1e-5, rope_theta=10000.0)
    fc, probs, ids = make_cache(T, E, k)
    out = np.zeros((T, d), np.float32)
    gomp = C.CDLL("libgomp.so.1")
    prev = gomp.omp_get_max_threads()
    gomp.omp_set_num_threads(threads)
    orc().orc_set_ftz_daz(1)
    try:
        ref().moe_forward(C.byref(matrix(x)), C.byref(w), C.byref(cfg), C.byref(fc),
                          C.byref(matrix(out)))
    finally:
        orc().orc_set_ftz_daz(0)
        gomp.omp_set_num_threads(prev)
    return out, probs, ids


def moe_forward_f64(x, hw, ids, probs):
    T = x.shape[0]
    out = np.empty((T, hw.d), np.float64)
    g, u, dn = hw.expert_ptr_arrays()
    orc().orc_moe_forward_f64(fptr(x), T, hw.d, hw.F, hw.k, iptr(ids), fptr(probs), hw.E,
                              g, u, dn, out.ctypes.data_as(C.POINTER(C.c_double)))
    return out


def synth_layer_host(d, F, E, k, seed, std_router, std_expert, experts=None):
    """Host copy of the weights moe_hip_layer_fill_synthetic generates: router
    stream 1; expert e gate 16+3e, up 17+3e, down 18+3e.  `experts` limits
    which experts are generated (dict id -> (wg, wu, wd))."""
    wr = synth((d, E), seed, 1, std_router)
    ex = {}
    for e in (range(E) if experts is None else experts):
        ex[e] = (synth((d, F), seed, 16 + 3 * e, std_expert),
                 synth((d, F), seed, 17 + 3 * e, std_expert),
                 synth((F, d), seed, 18 + 3 * e, std_expert))
    return wr, ex


def expf_array(x):
    y = np.empty_like(x)
    orc().orc_expf_array(fptr(x), fptr(y), x.size)
    return y


def exp_poly_array(x):
    y = np.empty_like(x)
    orc().orc_exp_poly_array(fptr(x), fptr(y), x.size)
    return y


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / den) if den > 0 else float(np.linalg.norm(a - b))
