"""Checkpoint format of model_save / model_load (src/transformer.c:573-700),
restated for the tests: the byte layout of every section and a writer for
synthetic checkpoints.  Test infrastructure only.

Layout: uint32 magic 0x4C4C4D43, ModelConfig (include/config.h:23-48, 11
ints + 2 floats), embed [vocab x d], then per block rms_attn [d], W_Q
[d x nh*hd], W_K and W_V [d x nkv*hd], W_O [nh*hd x d] (src/attention.c:
133-144), rms_ffn [d], and either W_gate, W_up [d x F], W_down [F x d]
(dense) or W_router [d x E] and each expert's W_gate, W_up, W_down (every
block is MoE when n_experts > 1, src/transformer.c:437); then rms_final [d]
and lm_head [d x vocab].  fp32, row-major, no padding.
"""
import struct
import zlib

import numpy as np

MAGIC = 0x4C4C4D43
CFG_FIELDS = ("vocab_size", "max_seq_len", "d_model", "n_layers", "n_heads", "n_kv_heads",
              "head_dim", "window_size", "ffn_hidden", "n_experts", "top_k_experts",
              "rms_norm_eps", "rope_theta")
HEADER = 4 + 11 * 4 + 2 * 4


def pack_config(cfg):
    return struct.pack("<I11i2f", MAGIC, *[cfg[f] for f in CFG_FIELDS])


def read_config(blob):
    vals = struct.unpack("<I11i2f", blob[:HEADER])
    assert vals[0] == MAGIC, hex(vals[0])
    return dict(zip(CFG_FIELDS, vals[1:]))


def layout(cfg):
    """[(name, shape)] in file order."""
    d, F, E, V = cfg["d_model"], cfg["ffn_hidden"], cfg["n_experts"], cfg["vocab_size"]
    qd, kd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    out = [("embed", (V, d))]
    for l in range(cfg["n_layers"]):
        out += [(f"{l}.rms_attn", (d,)), (f"{l}.W_Q", (d, qd)), (f"{l}.W_K", (d, kd)),
                (f"{l}.W_V", (d, kd)), (f"{l}.W_O", (qd, d)), (f"{l}.rms_ffn", (d,))]
        if E > 1:
            out.append((f"{l}.W_router", (d, E)))
            for e in range(E):
                out += [(f"{l}.{e}.W_gate", (d, F)), (f"{l}.{e}.W_up", (d, F)),
                        (f"{l}.{e}.W_down", (F, d))]
        else:
            out += [(f"{l}.W_gate", (d, F)), (f"{l}.W_up", (d, F)), (f"{l}.W_down", (F, d))]
    out += [("rms_final", (d,)), ("lm_head", (d, V))]
    return out


def offsets(cfg):
    """{name: (byte offset, shape)} and the total file size."""
    at, res = HEADER, {}
    for name, shape in layout(cfg):
        res[name] = (at, shape)
        at += 4 * int(np.prod(shape))
    return res, at


def write(path, cfg, seed=0):
    """A checkpoint of cfg with N(0, 1/sqrt(d)) matrices and N(1, 0.1) norm
    scales from numpy's generator `seed`; returns {name: array} as written."""
    rng = np.random.default_rng(seed)
    arrays = {}
    with open(path, "wb") as f:
        f.write(pack_config(cfg))
        for name, shape in layout(cfg):
            if name.split(".")[-1].startswith("rms"):
                a = (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
            else:
                a = (rng.standard_normal(shape) / np.sqrt(cfg["d_model"])).astype(np.float32)
            arrays[name] = a
            f.write(np.ascontiguousarray(a).tobytes())
    return arrays


# The small MoE model whose checkpoint tests/golden/ckpt_moe_ref.bin was
# written by the reference's own model_save (tests/golden/make_moe_ckpt.py).
REF_MOE_CFG = dict(vocab_size=16, max_seq_len=8, d_model=64, n_layers=2, n_heads=2,
                   n_kv_heads=1, head_dim=32, window_size=0, ffn_hidden=32, n_experts=3,
                   top_k_experts=2, rms_norm_eps=1e-5, rope_theta=10000.0)


def named_arrays(cfg, seed):
    """{name: array} for every tensor of cfg, each from its own stream of
    numpy's generator (seed, crc32 of the name), so a tensor's values do not
    depend on where any file layout puts it.  Norm scales N(1, 0.1), the rest
    N(0, 1/sqrt(d))."""
    out = {}
    for name, shape in layout(cfg):
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
        if name.split(".")[-1].startswith("rms"):
            out[name] = (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
        else:
            out[name] = (rng.standard_normal(shape) / np.sqrt(cfg["d_model"])).astype(np.float32)
    return out
