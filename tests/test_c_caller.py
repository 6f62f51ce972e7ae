"""The library from C: tests/c_caller/caller.c, built against
include/moe_hip.h alone and linked to libmoe_hip.so, calls moe_forward,
moe_block_ffn and moe_decode_step with the reference's structs as the patched
block_forward and inference_step would (src/transformer.c:760-767,
src/inference.c:342-343).  Its outputs are compared with the compiled
reference's golden outputs of the same layer and with the oracle."""
import os
import subprocess

import numpy as np
import pytest

import orc
from abi_types import HostMoE
from conftest import CONFIGS, GOLDEN, ROOT

SRC = os.path.join(ROOT, "tests", "c_caller", "caller.c")
LIBDIR = os.path.join(ROOT, "llm.c_amd")


def build(tmp_path):
    exe = tmp_path / "caller"
    subprocess.run(["gcc", "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror",
                    "-I" + os.path.join(ROOT, "include"), SRC, "-o", str(exe),
                    "-L" + LIBDIR, "-lmoe_hip", "-Wl,-rpath," + LIBDIR], check=True)
    return exe


def test_c_caller_builds_against_the_header_alone(tmp_path):
    """Compiles as C11 with warnings as errors and links every entry point it
    uses (no GPU needed)."""
    assert build(tmp_path).exists()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.gpu
def test_c_caller_matches_reference(tmp_path):
    exe = build(tmp_path)
    c = CONFIGS["c1"]
    T, d, F, E, k = c["T"], c["d"], c["F"], c["E"], c["k"]
    wr, ex = orc.synth_layer_host(d, F, E, k, 0, c["std_router"], c["std_expert"])
    x = orc.synth((T, d), 0, 0, 1.0)
    wg = np.stack([ex[e][0] for e in range(E)])
    wu = np.stack([ex[e][1] for e in range(E)])
    wd = np.stack([ex[e][2] for e in range(E)])
    rms = (1.0 + 0.1 * orc.synth((d,), 0, 5, 1.0)).astype(np.float32)
    xd = orc.synth((1, d), 0, 6, 1.0)
    xnd = orc.synth((1, d), 0, 7, 1.0)
    io = tmp_path / "io"
    io.mkdir()
    np.array([T, d, F, E, k], np.int32).tofile(io / "shape.i32")
    for name, a in (("x", x), ("wr", wr), ("wg", wg), ("wu", wu), ("wd", wd), ("rms", rms),
                    ("xd", xd), ("xnd", xnd)):
        np.ascontiguousarray(a, np.float32).tofile(io / f"{name}.f32")
    print(f"[gpu-test] C caller: T={T} d={d} F={F} E={E} k={k}", flush=True)
    r = subprocess.run([str(exe), str(io)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    rd = lambda n, dt, sh: np.fromfile(io / n, dt).reshape(sh)
    out, probs, ids = rd("out.f32", np.float32, (T, d)), rd("probs.f32", np.float32, (T, E)), \
        rd("ids.i32", np.int32, (T, k))
    # moe_forward against the compiled reference's own outputs for this layer
    g = np.load(os.path.join(GOLDEN, "golden_c1.npz"))
    assert np.array_equal(bits(probs), bits(g["probs"]))
    assert np.array_equal(ids, g["ids"])
    assert orc.rel_l2(out, g["out"]) <= 1e-5
    assert float(np.abs(out - g["out"]).max()) <= 1e-4
    # moe_block_ffn: x_norm_ffn = rms_norm(x), ffn_out = MoE(x_norm), x += ffn_out
    hw = HostMoE(wr, wg, wu, wd, k)
    xn_ref = orc.rms_norm(x, rms, 1e-5)
    bxn = rd("blk_xn.f32", np.float32, (T, d))
    assert np.array_equal(bits(bxn), bits(xn_ref))
    o_ref, p_ref, i_ref = orc.moe_forward(bxn, hw)
    assert np.array_equal(bits(rd("blk_probs.f32", np.float32, (T, E))), bits(p_ref))
    assert np.array_equal(rd("blk_ids.i32", np.int32, (T, k)), i_ref)
    bfo = rd("blk_fo.f32", np.float32, (T, d))
    assert orc.rel_l2(bfo, o_ref) <= 1e-5
    assert np.array_equal(bits(rd("blk_x.f32", np.float32, (T, d))), bits(x + bfo))
    # moe_decode_step: x += MoE(x_norm) for one row
    o1, _, _ = orc.moe_forward(xnd, hw)
    dx = rd("dec_x.f32", np.float32, (1, d))
    assert float(np.abs(dx.astype(np.float64) - (xd + o1)).max()) <= 1e-5
