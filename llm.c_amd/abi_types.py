"""ctypes mirrors of the reference's C structs on the MoE path.

Byte-compatible with murderface-cpu/llm.c:
  Matrix        include/matrix.h:33-38
  FFNWeights    include/transformer.h:35-39
  MoEWeights    include/transformer.h:53-58
  ModelConfig   include/config.h:23-48
  ForwardCache  include/transformer.h:108-124
The same definitions drive both libmoe_hip.so (include/moe_hip.h declares the
identical layouts) and, in the tests, the reference compiled from source, so
an ABI mismatch shows up as a parity failure.
"""
import ctypes as C

import numpy as np


class Matrix(C.Structure):
    _fields_ = [("data", C.POINTER(C.c_float)),
                ("grad", C.POINTER(C.c_float)),
                ("rows", C.c_int),
                ("cols", C.c_int)]


class FFNWeights(C.Structure):
    _fields_ = [("W_gate", Matrix), ("W_up", Matrix), ("W_down", Matrix)]


class MoEWeights(C.Structure):
    _fields_ = [("experts", C.POINTER(FFNWeights)),
                ("W_router", Matrix),
                ("n_experts", C.c_int),
                ("top_k", C.c_int)]


class ModelConfig(C.Structure):
    _fields_ = [("vocab_size", C.c_int), ("max_seq_len", C.c_int),
                ("d_model", C.c_int), ("n_layers", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int),
                ("head_dim", C.c_int), ("window_size", C.c_int),
                ("ffn_hidden", C.c_int), ("n_experts", C.c_int),
                ("top_k_experts", C.c_int),
                ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float)]


class ForwardCache(C.Structure):
    _fields_ = [("x_norm_attn", Matrix), ("x_norm_ffn", Matrix),
                ("attn_out", Matrix), ("ffn_out", Matrix),
                ("Q", Matrix), ("K", Matrix), ("V", Matrix),
                ("attn_scores", Matrix), ("attn_weighted", Matrix),
                ("gate_buf", Matrix), ("up_buf", Matrix),
                ("router_probs", C.POINTER(C.c_float)),
                ("expert_ids", C.POINTER(C.c_int))]


def fptr(a):
    """float* to a C-contiguous float32 numpy array."""
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_float))


def iptr(a):
    """int* to a C-contiguous int32 numpy array."""
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_int))


def matrix(a):
    """Matrix view of a 2-D float32 numpy array (no copy, no grad)."""
    assert a.ndim == 2
    return Matrix(fptr(a), None, a.shape[0], a.shape[1])


class HostMoE:
    """Owns numpy buffers for one MoE layer and the C structs that view them.

    wr: [d, E]; wg, wu: [E, d, F]; wd: [E, F, d] (each expert row-major, the
    reference layout).  Keep this object alive while the structs are in use.
    """

    def __init__(self, wr, wg, wu, wd, top_k):
        self.wr = np.ascontiguousarray(wr, dtype=np.float32)
        self.wg = np.ascontiguousarray(wg, dtype=np.float32)
        self.wu = np.ascontiguousarray(wu, dtype=np.float32)
        self.wd = np.ascontiguousarray(wd, dtype=np.float32)
        self.E, self.d, self.F = self.wg.shape
        self.k = int(top_k)
        arr = (FFNWeights * self.E)()
        for e in range(self.E):
            arr[e] = FFNWeights(matrix(self.wg[e]), matrix(self.wu[e]), matrix(self.wd[e]))
        self._experts = arr
        self.weights = MoEWeights(C.cast(arr, C.POINTER(FFNWeights)),
                                  matrix(self.wr), self.E, self.k)

    def config(self, max_seq_len=0):
        return ModelConfig(vocab_size=0, max_seq_len=max_seq_len,
                           d_model=self.d, n_layers=1, n_heads=1, n_kv_heads=1,
                           head_dim=self.d, window_size=0, ffn_hidden=self.F,
                           n_experts=self.E, top_k_experts=self.k,
                           rms_norm_eps=1e-5, rope_theta=10000.0)

    def expert_ptr_arrays(self):
        """(gate, up, down) arrays of float* per expert, for the oracle."""
        P = C.POINTER(C.c_float) * self.E
        g = P(*[fptr(self.wg[e]) for e in range(self.E)])
        u = P(*[fptr(self.wu[e]) for e in range(self.E)])
        dn = P(*[fptr(self.wd[e]) for e in range(self.E)])
        return g, u, dn


def make_cache(T, E, k):
    """A ForwardCache whose router_probs/expert_ids point at fresh arrays."""
    probs = np.zeros((T, E), np.float32)
    ids = np.zeros((T, k), np.int32)
    fc = ForwardCache()
    fc.router_probs = fptr(probs)
    fc.expert_ids = iptr(ids)
    return fc, probs, ids
