"""Writes tests/golden/ckpt_moe_ref.bin with the reference's own model_save
(src/transformer.c:573-616), compiled from its sources into
oracle/_ref/libref_ckpt.so (make -C oracle ref).  The tensors are
ckpt_format.named_arrays(REF_MOE_CFG, seed 11), handed to the reference's
Model struct by field (oracle/ref_ckpt_harness.c); the file layout is the
reference's.  Run from the repo root:  python tests/golden/make_moe_ckpt.py
"""
import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "tests"), os.path.join(ROOT, "llm.c_amd")]
import ckpt_format as cf  # noqa: E402
from abi_types import ModelConfig  # noqa: E402

SEED = 11
OUT = os.path.join(ROOT, "tests", "golden", "ckpt_moe_ref.bin")


def main():
    lib = C.CDLL(os.path.join(ROOT, "oracle", "_ref", "libref_ckpt.so"))
    cfg = cf.REF_MOE_CFG
    a = cf.named_arrays(cfg, SEED)
    L, E = cfg["n_layers"], cfg["n_experts"]
    F = C.POINTER(C.c_float)
    p = lambda arr: arr.ctypes.data_as(F)
    per = lambda key: (F * L)(*[p(a[f"{l}.{key}"]) for l in range(L)])
    ex = lambda key: (F * (L * E))(*[p(a[f"{l}.{e}.{key}"]) for l in range(L) for e in range(E)])
    mc = ModelConfig(**cfg)
    rc = lib.ref_ckpt_save(OUT.encode(), C.byref(mc), p(a["embed"]), per("rms_attn"), per("W_Q"),
                           per("W_K"), per("W_V"), per("W_O"), per("rms_ffn"), per("W_router"),
                           ex("W_gate"), ex("W_up"), ex("W_down"), p(a["rms_final"]),
                           p(a["lm_head"]))
    assert rc == 0, rc
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
