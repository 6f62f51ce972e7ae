"""Checkpoint format (model_save, src/transformer.c:573-616): the layout
restated in tests/ckpt_format.py against a dense checkpoint the reference
ships and a MoE checkpoint the reference's own model_save wrote
(tests/golden/ckpt_moe_ref.bin), and the library's loader
(moe_hip_model_load) against that file and synthetic MoE and dense
checkpoints written in the restated layout."""
import os

import numpy as np
import pytest

import ckpt_format as cf
import moe_hip as mh
import orc
from abi_types import HostMoE
from conftest import GOLDEN

REF_CKPT = "/root/reference/checkpoints/ckpt_00500.bin"


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_layout_size_matches_reference_checkpoint():
    """The section arithmetic gives the exact size of a checkpoint the
    reference wrote (dense blocks, GQA 4/2, d=128, F=384, 4 blocks)."""
    g = np.load(os.path.join(GOLDEN, "ckpt_reference_header.npz"))
    cfg = cf.read_config(g["header"].tobytes())
    assert cfg["n_experts"] == 1 and cfg["n_kv_heads"] < cfg["n_heads"]
    _, total = cf.offsets(cfg)
    assert total == int(g["size"])


@pytest.mark.skipif(not os.path.exists(REF_CKPT), reason="reference checkpoints not present")
def test_layout_offsets_on_reference_checkpoint():
    """Every norm-scale section of the reference's checkpoint (never trained:
    all exactly 1.0) sits at the computed offset; the matrices around them
    are not 1.0, so an offset off by any amount would show."""
    blob = open(REF_CKPT, "rb").read()
    cfg = cf.read_config(blob)
    offs, total = cf.offsets(cfg)
    assert total == len(blob)
    d = cfg["d_model"]
    for name, (at, shape) in offs.items():
        v = np.frombuffer(blob, np.float32, count=int(np.prod(shape)), offset=at)
        if name.split(".")[-1].startswith("rms"):
            assert np.all(v == 1.0), name
            before = np.frombuffer(blob, np.float32, count=1, offset=at - 4)[0]
            after = np.frombuffer(blob, np.float32, count=1, offset=at + 4 * d)[0]
            assert before != 1.0 and after != 1.0, name
        else:
            assert np.count_nonzero(v == 1.0) < v.size // 100, name


def test_writer_roundtrip(tmp_path):
    cfg = dict(vocab_size=40, max_seq_len=16, d_model=32, n_layers=2, n_heads=2, n_kv_heads=1,
               head_dim=16, window_size=0, ffn_hidden=64, n_experts=3, top_k_experts=2,
               rms_norm_eps=1e-5, rope_theta=10000.0)
    p = tmp_path / "moe.bin"
    arrays = cf.write(p, cfg, seed=3)
    blob = p.read_bytes()
    offs, total = cf.offsets(cfg)
    assert len(blob) == total and cf.read_config(blob) == {**cfg, "rms_norm_eps": np.float32(1e-5).item()}
    for name, (at, shape) in offs.items():
        got = np.frombuffer(blob, np.float32, count=int(np.prod(shape)), offset=at).reshape(shape)
        assert np.array_equal(got, arrays[name]), name


REF_MOE_CKPT = os.path.join(GOLDEN, "ckpt_moe_ref.bin")


def test_layout_matches_reference_written_moe_checkpoint():
    """tests/golden/ckpt_moe_ref.bin was written by the reference's own
    model_save (tests/golden/make_moe_ckpt.py) from named tensors: its
    config, its size and every section (each block's router and every
    expert's gate, up and down matrices included) sit where the restated
    layout puts them, holding the tensor of that name."""
    blob = open(REF_MOE_CKPT, "rb").read()
    cfg = cf.read_config(blob)
    assert cfg == {**cf.REF_MOE_CFG, "rms_norm_eps": np.float32(1e-5).item()}
    offs, total = cf.offsets(cf.REF_MOE_CFG)
    assert total == len(blob)
    arrays = cf.named_arrays(cf.REF_MOE_CFG, 11)
    for name, (at, shape) in offs.items():
        got = np.frombuffer(blob, np.float32, count=int(np.prod(shape)), offset=at).reshape(shape)
        assert np.array_equal(got, arrays[name]), name


@pytest.mark.gpu
def test_model_load_reference_written_moe_checkpoint():
    """moe_hip_model_load on the checkpoint the reference's model_save wrote:
    every block's router, experts and rms_ffn come back bit for bit."""
    cfg = cf.REF_MOE_CFG
    arrays = cf.named_arrays(cfg, 11)
    m = mh.Model(REF_MOE_CKPT)
    try:
        assert m.config()["n_experts"] == cfg["n_experts"]
        d, E = cfg["d_model"], cfg["n_experts"]
        for l in range(cfg["n_layers"]):
            L = m.layer(l)
            assert np.array_equal(bits(L.get_router()), bits(arrays[f"{l}.W_router"]))
            for e in range(E):
                g, u, dn = L.get_expert(e)
                assert np.array_equal(bits(g), bits(arrays[f"{l}.{e}.W_gate"]))
                assert np.array_equal(bits(u), bits(arrays[f"{l}.{e}.W_up"]))
                assert np.array_equal(bits(dn), bits(arrays[f"{l}.{e}.W_down"]))
            rw = mh.DeviceArray((d,))
            mh.check(mh.lib().moe_hip_memcpy(rw.ptr, m.rms_ffn_ptr(l), 4 * d, 3))
            assert np.array_equal(bits(rw.to_host()), bits(arrays[f"{l}.rms_ffn"]))
    finally:
        m.close()


# ---------------------------------------------------------------- the loader (GPU)
MOE_CFG = dict(vocab_size=48, max_seq_len=32, d_model=128, n_layers=3, n_heads=4, n_kv_heads=2,
               head_dim=32, window_size=0, ffn_hidden=256, n_experts=4, top_k_experts=2,
               rms_norm_eps=1e-5, rope_theta=10000.0)


@pytest.mark.gpu
def test_model_load_moe(tmp_path):
    """Every MoE block's router, experts and rms_ffn come back bit for bit,
    and a loaded block computes the layer the oracle computes."""
    p = tmp_path / "moe.bin"
    arrays = cf.write(p, MOE_CFG, seed=7)
    m = mh.Model(str(p))
    try:
        assert m.config()["n_experts"] == 4 and m.config()["n_layers"] == 3
        d, F, E = MOE_CFG["d_model"], MOE_CFG["ffn_hidden"], MOE_CFG["n_experts"]
        for l in range(MOE_CFG["n_layers"]):
            L = m.layer(l)
            assert L is not None
            assert np.array_equal(bits(L.get_router()), bits(arrays[f"{l}.W_router"]))
            for e in range(E):
                g, u, dn = L.get_expert(e)
                assert np.array_equal(bits(g), bits(arrays[f"{l}.{e}.W_gate"]))
                assert np.array_equal(bits(u), bits(arrays[f"{l}.{e}.W_up"]))
                assert np.array_equal(bits(dn), bits(arrays[f"{l}.{e}.W_down"]))
            rw = mh.DeviceArray((d,))
            mh.check(mh.lib().moe_hip_memcpy(rw.ptr, m.rms_ffn_ptr(l), 4 * d, 3))
            assert np.array_equal(bits(rw.to_host()), bits(arrays[f"{l}.rms_ffn"]))
        # Block 1 as a layer: x += MoE(rms_norm(x)) against the oracle.
        T, l = 40, 1
        hw = HostMoE(arrays[f"{l}.W_router"], np.stack([arrays[f"{l}.{e}.W_gate"] for e in range(E)]),
                     np.stack([arrays[f"{l}.{e}.W_up"] for e in range(E)]),
                     np.stack([arrays[f"{l}.{e}.W_down"] for e in range(E)]), 2)
        x = orc.synth((T, d), 7, 1, 1.0)
        dx = mh.DeviceArray.from_host(x)
        dids = mh.DeviceArray((T, 2), np.int32)
        m.layer(l).ffn_sublayer_dev(dx.ptr, m.rms_ffn_ptr(l), 1e-5, T, None, None, dids.ptr)
        mh.synchronize()
        xn = orc.rms_norm(x, arrays[f"{l}.rms_ffn"], 1e-5)
        o_ref, _, i_ref = orc.moe_forward(xn, hw)
        assert np.array_equal(dids.to_host(), i_ref)
        assert orc.rel_l2(dx.to_host(), x + o_ref) < 1e-5
    finally:
        m.close()


@pytest.mark.gpu
def test_model_load_dense_and_errors(tmp_path):
    dense = dict(MOE_CFG, n_experts=1, top_k_experts=1)
    p = tmp_path / "dense.bin"
    arrays = cf.write(p, dense, seed=8)
    m = mh.Model(str(p))
    try:
        assert all(m.layer(l) is None for l in range(dense["n_layers"]))
        rw = mh.DeviceArray((dense["d_model"],))
        mh.check(mh.lib().moe_hip_memcpy(rw.ptr, m.rms_ffn_ptr(2), 4 * dense["d_model"], 3))
        assert np.array_equal(bits(rw.to_host()), bits(arrays["2.rms_ffn"]))
    finally:
        m.close()
    # Truncated by one float, and a wrong magic: both rejected.
    q = tmp_path / "cut.bin"
    cf.write(q, MOE_CFG, seed=9)
    q.write_bytes(q.read_bytes()[:-4])
    with pytest.raises(mh.MoeHipError):
        mh.Model(str(q))
    r = tmp_path / "bad.bin"
    r.write_bytes(b"\x00" * 4096)
    with pytest.raises(mh.MoeHipError):
        mh.Model(str(r))
