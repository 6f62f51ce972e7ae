"""Python binding of libmoe_hip (ctypes), mirroring the reference interface.

`moe_forward(x, layer, cfg, cache, out)` keeps the argument meaning of the
reference's moe_forward (include/transformer.h:270-272): x and out are
[T x d_model] matrices, cache receives router_probs [T x E] and expert_ids
[T x top_k].  The device-resident API works on raw device addresses
(DeviceArray below allocates them through the library itself).

The library is the native code in llm.c_amd/libmoe_hip.so; importing this
module raises if it has not been built.
"""
import ctypes as C
import os

import numpy as np

from abi_types import (FFNWeights, ForwardCache, HostMoE, Matrix, MoEWeights,  # noqa: F401
                       ModelConfig, fptr, iptr, make_cache, matrix)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmoe_hip.so")

OK = 0
ERRORS = {1: "invalid argument", 2: "unsupported shape", 3: "HIP runtime error",
          4: "device out of memory", 5: "no GPU"}

_P = C.c_void_p
_F = C.POINTER(C.c_float)
_I = C.POINTER(C.c_int)

# name -> (restype, argtypes); one entry per function of include/moe_hip.h.
SIGNATURES = {
    "moe_forward": (None, [C.POINTER(Matrix), C.POINTER(MoEWeights), C.POINTER(ModelConfig),
                           C.POINTER(ForwardCache), C.POINTER(Matrix)]),
    "moe_hip_forward": (C.c_int, [C.POINTER(Matrix), C.POINTER(MoEWeights),
                                  C.POINTER(ModelConfig), C.POINTER(ForwardCache),
                                  C.POINTER(Matrix)]),
    "moe_decode_step": (None, [C.POINTER(MoEWeights), C.POINTER(ModelConfig), _F, _F]),
    "moe_decode_batch": (C.c_int, [C.POINTER(MoEWeights), C.POINTER(ModelConfig), _F,
                                   C.c_int, _F]),
    "moe_block_ffn": (None, [C.POINTER(Matrix), _F, C.POINTER(MoEWeights),
                             C.POINTER(ModelConfig), C.POINTER(ForwardCache)]),
    "moe_hip_block_ffn": (C.c_int, [C.POINTER(Matrix), _F, C.POINTER(MoEWeights),
                                    C.POINTER(ModelConfig), C.POINTER(ForwardCache)]),
    "moe_hip_init": (C.c_int, [C.c_int]),
    "moe_hip_shutdown": (None, []),
    "moe_hip_invalidate": (C.c_int, [C.POINTER(MoEWeights)]),
    "moe_hip_last_error": (C.c_int, []),
    "moe_hip_error_string": (C.c_char_p, [C.c_int]),
    "moe_hip_last_error_message": (C.c_char_p, []),
    "moe_hip_layer_create": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(_P)]),
    "moe_hip_layer_destroy": (C.c_int, [_P]),
    "moe_hip_layer_load": (C.c_int, [_P, C.POINTER(MoEWeights)]),
    "moe_hip_layer_set_router_bias": (C.c_int, [_P, _F]),
    "moe_hip_layer_fill_synthetic": (C.c_int, [_P, C.c_uint64, C.c_float, C.c_float]),
    "moe_hip_layer_get_expert": (C.c_int, [_P, C.c_int, _F, _F, _F]),
    "moe_hip_layer_get_router": (C.c_int, [_P, _F]),
    "moe_hip_forward_dev": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, C.c_int, _P]),
    "moe_hip_forward_dev_noalloc": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, C.c_int, _P]),
    "moe_hip_forward_host": (C.c_int, [_P, _F, C.c_int, _F, _F, _I]),
    "moe_hip_route_dev": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, _P, _P, _P, _P]),
    "moe_hip_rms_norm_dev": (C.c_int, [_P, _P, C.c_float, C.c_int, C.c_int, _P, _P]),
    "moe_hip_attn_create": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.POINTER(_P)]),
    "moe_hip_attn_destroy": (C.c_int, [_P]),
    "moe_hip_attn_load": (C.c_int, [_P, _F, _F, _F, _F, _F]),
    "moe_hip_attn_set_rope": (C.c_int, [_P, _F, _F]),
    "moe_hip_attn_decode_dev": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, C.c_float, _P]),
    "moe_hip_model_load": (C.c_int, [C.c_char_p, C.POINTER(_P)]),
    "moe_hip_model_free": (C.c_int, [_P]),
    "moe_hip_model_config": (C.c_int, [_P, C.POINTER(ModelConfig)]),
    "moe_hip_model_layer": (_P, [_P, C.c_int]),
    "moe_hip_model_rms_ffn": (_P, [_P, C.c_int]),
    "moe_hip_ffn_sublayer_dev": (C.c_int, [_P, _P, _P, C.c_float, C.c_int, _P, _P, _P, _P]),
    "moe_hip_fill_normal_dev": (C.c_int, [_P, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float,
                                          C.c_float, _P]),
    "moe_hip_eval_exp": (C.c_int, [C.c_int, _P, _P, C.c_size_t, _P]),
    "moe_hip_read_probe": (C.c_int, [_P, C.c_size_t, C.c_int, _P, _P]),
    "moe_hip_link_rate": (C.c_int, [C.c_size_t, _F, _F]),
    "moe_hip_last_timings": (C.c_int, [_F]),
    "moe_hip_set_timing": (C.c_int, [C.c_int]),
    "moe_hip_set_expert_path": (C.c_int, [C.c_int]),
    "moe_hip_set_router_path": (C.c_int, [C.c_int]),
    "moe_hip_last_forward_path": (C.c_int, []),
    "moe_hip_backward_dev": (C.c_int, [_P, _P, C.c_int, _P, C.c_float, _P, _P, _P, _P, _P, _P,
                                       C.c_int, _P]),
    "moe_hip_decode_block_dev": (C.c_int, [_P, _P, _P, _P, C.c_int, _P, _P, _P, C.c_float, _P,
                                           _P, _P]),
    "moe_hip_timer_start": (C.c_int, []),
    "moe_hip_timer_stop": (C.c_int, [_F]),
    "moe_hip_timer_mark": (C.c_int, [C.c_int]),
    "moe_hip_timer_between": (C.c_int, [C.c_int, C.c_int, _F]),
    "moe_hip_dev_alloc": (C.c_int, [C.POINTER(_P), C.c_size_t]),
    "moe_hip_dev_free": (C.c_int, [_P]),
    "moe_hip_memcpy": (C.c_int, [_P, _P, C.c_size_t, C.c_int]),
    "moe_hip_memset": (C.c_int, [_P, C.c_int, C.c_size_t]),
    "moe_hip_synchronize": (C.c_int, []),
    "moe_hip_graph_begin": (C.c_int, [_P]),
    "moe_hip_graph_end": (C.c_int, [_P, C.POINTER(_P)]),
    "moe_hip_graph_launch": (C.c_int, [_P, _P]),
    "moe_hip_graph_destroy": (C.c_int, [_P]),
}

_lib = None


def lib():
    """Load libmoe_hip.so once; raises FileNotFoundError if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `make -C llm.c_amd` "
                "(or __graft_entry__.build()); there is no fallback path")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class MoeHipError(RuntimeError):
    pass


def check(rc):
    if rc != OK:
        msg = lib().moe_hip_last_error_message().decode(errors="replace")
        raise MoeHipError(f"libmoe_hip error {rc} ({ERRORS.get(rc, '?')}): {msg}")


def moe_forward(x, hw, cache_probs=None, cache_ids=None):
    """Host-pointer drop-in: returns (out, probs, ids) for x [T x d] (numpy)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    out = np.zeros((T, hw.d), np.float32)
    fc, probs, ids = make_cache(T, hw.E, hw.k)
    cfg = hw.config(T)
    check(lib().moe_hip_forward(C.byref(matrix(x)), C.byref(hw.weights), C.byref(cfg),
                                C.byref(fc), C.byref(matrix(out))))
    return out, probs, ids


def decode_batch(x_norm, x, hw):
    """x[r] += MoE(x_norm[r]) through moe_decode_batch; returns the new x."""
    xn = np.ascontiguousarray(x_norm, dtype=np.float32)
    xo = np.array(x, dtype=np.float32, copy=True, order="C")
    cfg = hw.config(xn.shape[0])
    check(lib().moe_decode_batch(C.byref(hw.weights), C.byref(cfg), fptr(xn), xn.shape[0],
                                 fptr(xo)))
    return xo


def block_ffn(x, rms_w, hw):
    """The FFN half of a MoE block_forward through moe_hip_block_ffn: returns
    (x + ffn_out, x_norm_ffn, ffn_out, probs, ids) for x [T x d] (numpy)."""
    xo = np.array(x, dtype=np.float32, copy=True, order="C")
    T = xo.shape[0]
    xn = np.zeros((T, hw.d), np.float32)
    fo = np.zeros((T, hw.d), np.float32)
    fc, probs, ids = make_cache(T, hw.E, hw.k)
    fc.x_norm_ffn = matrix(xn)
    fc.ffn_out = matrix(fo)
    w = np.ascontiguousarray(rms_w, dtype=np.float32)
    cfg = hw.config(T)
    check(lib().moe_hip_block_ffn(C.byref(matrix(xo)), fptr(w), C.byref(hw.weights),
                                  C.byref(cfg), C.byref(fc)))
    return xo, xn, fo, probs, ids


def rms_norm_dev(x_ptr, w_ptr, eps, rows, cols, y_ptr, stream=None):
    check(lib().moe_hip_rms_norm_dev(x_ptr, w_ptr, eps, rows, cols, y_ptr, stream))


class Layer:
    """Device-resident MoE layer (packed weights in HBM)."""

    def __init__(self, d, F, E, k, handle=None):
        """A new layer, or (handle set) a view of one owned elsewhere."""
        self.d, self.F, self.E, self.k = d, F, E, k
        self.owned = handle is None
        if handle is None:
            handle = _P()
            check(lib().moe_hip_layer_create(d, F, E, k, C.byref(handle)))
        self.h = handle

    def close(self):
        if self.h and self.owned:
            lib().moe_hip_layer_destroy(self.h)
        self.h = _P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def load(self, hw):
        check(lib().moe_hip_layer_load(self.h, C.byref(hw.weights)))

    def set_bias(self, bias):
        if bias is None:
            check(lib().moe_hip_layer_set_router_bias(self.h, None))
        else:
            b = np.ascontiguousarray(bias, dtype=np.float32)
            assert b.shape == (self.E,)
            check(lib().moe_hip_layer_set_router_bias(self.h, fptr(b)))

    def fill_synthetic(self, seed, std_router, std_expert):
        check(lib().moe_hip_layer_fill_synthetic(self.h, seed, std_router, std_expert))

    def get_expert(self, e):
        wg = np.empty((self.d, self.F), np.float32)
        wu = np.empty((self.d, self.F), np.float32)
        wd = np.empty((self.F, self.d), np.float32)
        check(lib().moe_hip_layer_get_expert(self.h, e, fptr(wg), fptr(wu), fptr(wd)))
        return wg, wu, wd

    def get_router(self):
        wr = np.empty((self.d, self.E), np.float32)
        check(lib().moe_hip_layer_get_router(self.h, fptr(wr)))
        return wr

    def forward_dev(self, x_ptr, T, out_ptr, probs_ptr=None, ids_ptr=None, accumulate=0,
                    stream=None):
        check(lib().moe_hip_forward_dev(self.h, x_ptr, T, out_ptr, probs_ptr, ids_ptr,
                                        accumulate, stream))

    def forward_dev_noalloc(self, x_ptr, T, out_ptr, probs_ptr=None, ids_ptr=None,
                            accumulate=0, stream=None):
        """forward_dev on the library's fixed scratch array (no device
        allocation; moe_hip_forward_dev_noalloc)."""
        check(lib().moe_hip_forward_dev_noalloc(self.h, x_ptr, T, out_ptr, probs_ptr, ids_ptr,
                                                accumulate, stream))

    def forward_host(self, x, out, probs=None, ids=None):
        """moe_hip_forward_host: x, out [T x d] (and probs [T x E], ids
        [T x k] when given) numpy arrays in host memory."""
        assert x.dtype == np.float32 and out.dtype == np.float32 and x.flags["C_CONTIGUOUS"]
        check(lib().moe_hip_forward_host(self.h, fptr(x), x.shape[0], fptr(out),
                                         fptr(probs) if probs is not None else None,
                                         iptr(ids) if ids is not None else None))

    def ffn_sublayer_dev(self, x_ptr, rms_w_ptr, eps, T, x_norm_ptr=None, probs_ptr=None,
                         ids_ptr=None, stream=None):
        """x += MoE(rms_norm(x)) in place on device rows x [T x d]."""
        check(lib().moe_hip_ffn_sublayer_dev(self.h, x_ptr, rms_w_ptr, eps, T, x_norm_ptr,
                                             probs_ptr, ids_ptr, stream))

    def backward_dev(self, x_ptr, T, dout_ptr, aux_coef, dx_ptr, dwr_ptr, dwg_ptr, dwu_ptr,
                     dwd_ptr, aux_ptr=None, accumulate=0, stream=None):
        """Gradients of sum(dout * out) + aux_coef * aux (moe_hip_backward_dev)."""
        check(lib().moe_hip_backward_dev(self.h, x_ptr, T, dout_ptr, aux_coef, dx_ptr, dwr_ptr,
                                         dwg_ptr, dwu_ptr, dwd_ptr, aux_ptr, accumulate, stream))

    def route_dev(self, x_ptr, T, probs=None, ids=None, gw=None, counts=None, offsets=None,
                  perm=None, stream=None):
        check(lib().moe_hip_route_dev(self.h, x_ptr, T, probs, ids, gw, counts, offsets, perm,
                                      stream))


class Attn:
    """One block's decode attention on the device (moe_hip_attn_*)."""

    def __init__(self, d, nh, nkv, hd, max_seq):
        self.d, self.nh, self.nkv, self.hd, self.max_seq = d, nh, nkv, hd, max_seq
        h = _P()
        check(lib().moe_hip_attn_create(d, nh, nkv, hd, max_seq, C.byref(h)))
        self.h = h

    def load(self, wq, wk, wv, wo, rms_attn):
        arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (wq, wk, wv, wo, rms_attn)]
        check(lib().moe_hip_attn_load(self.h, *[fptr(a) for a in arrs]))

    def set_rope(self, cos_t, sin_t):
        c = np.ascontiguousarray(cos_t, dtype=np.float32)
        s = np.ascontiguousarray(sin_t, dtype=np.float32)
        check(lib().moe_hip_attn_set_rope(self.h, fptr(c), fptr(s)))

    def decode_dev(self, x_ptr, B, pos_ptr, k_cache_ptr, v_cache_ptr, eps, stream=None):
        check(lib().moe_hip_attn_decode_dev(self.h, x_ptr, B, pos_ptr, k_cache_ptr, v_cache_ptr,
                                            eps, stream))

    def decode_block_dev(self, layer, rms_ffn_ptr, x_ptr, B, pos_ptr, k_cache_ptr, v_cache_ptr,
                         eps, x_norm_ptr=None, ids_ptr=None, stream=None):
        """One decoder block: x += Attn(rms_norm(x)), then x += MoE(rms_norm(x))
        with the MoE layer `layer` (moe_hip_decode_block_dev)."""
        check(lib().moe_hip_decode_block_dev(self.h, layer.h, rms_ffn_ptr, x_ptr, B, pos_ptr,
                                             k_cache_ptr, v_cache_ptr, eps, x_norm_ptr, ids_ptr,
                                             stream))

    def close(self):
        if self.h:
            lib().moe_hip_attn_destroy(self.h)
            self.h = _P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """The MoE blocks of a model_save checkpoint, loaded into packed device
    layers (moe_hip_model_load)."""

    def __init__(self, path):
        h = _P()
        check(lib().moe_hip_model_load(path.encode(), C.byref(h)))
        self.h = h
        cfg = ModelConfig()
        check(lib().moe_hip_model_config(h, C.byref(cfg)))
        self.cfg = cfg

    def config(self):
        return {f: getattr(self.cfg, f) for f, _ in ModelConfig._fields_}

    def layer(self, l):
        """Block l's MoE layer (a view owned by the model) or None."""
        h = lib().moe_hip_model_layer(self.h, l)
        if not h:
            return None
        c = self.cfg
        return Layer(c.d_model, c.ffn_hidden, c.n_experts, c.top_k_experts, handle=_P(h))

    def rms_ffn_ptr(self, l):
        return lib().moe_hip_model_rms_ffn(self.h, l)

    def close(self):
        if self.h:
            lib().moe_hip_model_free(self.h)
            self.h = _P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def fill_normal_dev(ptr, n, seed, stream_id, mean, std, stream=None):
    check(lib().moe_hip_fill_normal_dev(ptr, n, seed, stream_id, mean, std, stream))


def eval_exp_dev(which, x_ptr, y_ptr, n, stream=None):
    check(lib().moe_hip_eval_exp(which, x_ptr, y_ptr, n, stream))


class DeviceArray:
    """A device buffer owned through libmoe_hip (numpy dtype + shape)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in np.atleast_1d(np.asarray(shape)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = _P()
        check(lib().moe_hip_dev_alloc(C.byref(p), self.nbytes))
        self.ptr = p

    @classmethod
    def from_host(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        check(lib().moe_hip_memcpy(d.ptr, a.ctypes.data_as(_P), d.nbytes, 1))
        return d

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        check(lib().moe_hip_memcpy(self.ptr, a.ctypes.data_as(_P), self.nbytes, 1))

    def to_host(self):
        a = np.empty(self.shape, self.dtype)
        check(lib().moe_hip_memcpy(a.ctypes.data_as(_P), self.ptr, self.nbytes, 2))
        return a

    def zero(self):
        check(lib().moe_hip_memset(self.ptr, 0, self.nbytes))

    def free(self):
        if self.ptr:
            lib().moe_hip_dev_free(self.ptr)
            self.ptr = _P()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize():
    check(lib().moe_hip_synchronize())


class Graph:
    """Records the library calls made inside ``with Graph() as g:`` (on the
    library stream) into a HIP graph; ``g.launch()`` replays them."""

    def __init__(self):
        self.h = None

    def __enter__(self):
        check(lib().moe_hip_graph_begin(None))
        return self

    def __exit__(self, exc_type, exc, tb):
        h = C.c_void_p()
        rc = lib().moe_hip_graph_end(None, C.byref(h))
        if exc_type is None:
            check(rc)
            self.h = h
        return False

    def launch(self):
        check(lib().moe_hip_graph_launch(self.h, None))

    def close(self):
        if self.h is not None:
            lib().moe_hip_graph_destroy(self.h)
            self.h = None


def set_expert_path(mode):
    """0 automatic, 1 grouped GEMMs, 2 decode GEMVs (gate/up fused with a
    split-K down projection), 3 decode GEMVs as two launches."""
    check(lib().moe_hip_set_expert_path(int(mode)))


def set_router_path(mode):
    """0 automatic, 1 token x expert tiles, 2 16-token row blocks."""
    check(lib().moe_hip_set_router_path(int(mode)))


def last_forward_path():
    """Kernels of the last layer forward: 1 router + grouped GEMMs, 2 router +
    fused decode kernel, 3 router + two-launch decode, 4 fused decode kernel
    with the routing inside."""
    return int(lib().moe_hip_last_forward_path())


def link_rate(nbytes=256 << 20):
    """(host-to-device, device-to-host) GB/s of pinned copies of nbytes."""
    a, b = C.c_float(), C.c_float()
    check(lib().moe_hip_link_rate(nbytes, C.byref(a), C.byref(b)))
    return a.value, b.value


def set_timing(on):
    check(lib().moe_hip_set_timing(1 if on else 0))


def timer_start():
    check(lib().moe_hip_timer_start())


def timer_stop():
    """Milliseconds of device time since timer_start (waits for the stream)."""
    ms = C.c_float()
    check(lib().moe_hip_timer_stop(C.byref(ms)))
    return ms.value


def timed_steps(fn, steps, warmup):
    """Device milliseconds of each of `steps` calls of fn() on the library
    stream, read from marks recorded between the calls (nothing inside the
    loop waits); warmup untimed calls first.  Returns the per-call list."""
    for _ in range(warmup):
        fn()
    synchronize()
    out = []
    done = 0
    while done < steps:
        n = min(steps - done, 63)
        check(lib().moe_hip_timer_mark(0))
        for i in range(n):
            fn()
            check(lib().moe_hip_timer_mark(i + 1))
        ms = C.c_float()
        for i in range(n):
            check(lib().moe_hip_timer_between(i, i + 1, C.byref(ms)))
            out.append(ms.value)
        done += n
    synchronize()
    return out


def last_timings():
    """[route, dispatch, gate_up, down, combine] in ms for the last forward_dev."""
    a = (C.c_float * 5)()
    check(lib().moe_hip_last_timings(a))
    return list(a)
