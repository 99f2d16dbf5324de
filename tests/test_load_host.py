"""The native checkpoint loader's host side (qw_checkpoint_open and its
table), on the CPU: the committed trimmed toy checkpoints read back tensor
for tensor against an independent Python reader; the small-matrix dequant
pinned against the golden layer fixtures; the reference's error cases
(qwasar.c:700-775, :892-903, :1426-1495).  Device uploads are GPU tests."""
import ctypes as C
import json
import os
import shutil
import struct

import numpy as np
import pytest

from qwasar_amd import gpu
from tests import ckpt_util as cu

GOLD = cu.GOLD


def open_ck(d):
    err = C.create_string_buffer(512)
    ck = gpu.qw_checkpoint_open(d.encode(), err, 512)
    return ck, err.value.decode()


def tensor(ck, name):
    data, nb, nd = C.c_void_p(), C.c_size_t(), C.c_int32()
    shape, dt = (C.c_int64 * 8)(), C.create_string_buffer(16)
    if not gpu.qw_checkpoint_tensor(ck, name.encode(), C.byref(data), C.byref(nb), C.byref(nd), shape, dt):
        return None
    return dt.value.decode(), [shape[i] for i in range(nd.value)], C.string_at(data, nb.value)


@pytest.mark.parametrize("tag", ["q4", "mlx"])
def test_table_matches_python_reader(tag):
    ck, err = open_ck(cu.CKPTS[tag])
    assert ck, err
    try:
        assert gpu.qw_checkpoint_layers(ck) == cu.config(cu.CKPTS[tag])["num_hidden_layers"]
        want = cu.entries(cu.CKPTS[tag])
        assert len(want) > 20
        for name, e in want.items():
            assert tensor(ck, name) == (e[0], list(e[1]), e[2]), name
        assert tensor(ck, "language_model.model.layers.0.mlp.nope.weight") is None
    finally:
        gpu.qw_checkpoint_close(ck)


@pytest.mark.parametrize("tag", ["q4", "mlx"])
def test_small_dequant_matches_golden(tag):
    """The Python restatement of the 8-bit router dequant (used by the GPU
    test to check the loader's) against the committed layer fixtures."""
    g = np.load(os.path.join(GOLD, f"tiny_{tag}_layer0.npz"), allow_pickle=False)
    L = cu.layer(tag, 0)
    assert np.array_equal(L.router, g["router"])
    assert np.array_equal(L.sh_gate_w, g["sh_gate_vec"])
    assert L.group == int(g["group"]) and L.split == bool(int(g["split"]))


def copy_ckpt(tmp_path, tag):
    d = tmp_path / f"{tag}{len(list(tmp_path.iterdir()))}"
    shutil.copytree(cu.CKPTS[tag], d)
    return d


def write_st(path, hdr, body=b""):
    h = json.dumps(hdr).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + body)


def test_errors(tmp_path):
    ck, err = open_ck(str(tmp_path / "missing"))
    assert not ck and "config.json" in err

    d = copy_ckpt(tmp_path, "q4")
    cfg = json.loads((d / "config.json").read_text())
    cfg["model_type"] = "qwen4_exp"                     # flat fields need qwen4_exp_text
    (d / "config.json").write_text(json.dumps(cfg))
    ck, err = open_ck(str(d))
    assert not ck and "no text_config" in err

    d = copy_ckpt(tmp_path, "mlx")
    shutil.copy(d / "model.safetensors", d / "model-copy.safetensors")
    ck, err = open_ck(str(d))
    assert not ck and "appears twice" in err

    d = copy_ckpt(tmp_path, "q4")
    write_st(d / "extra.safetensors", {"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 12]}}, b"\0" * 16)
    ck, err = open_ck(str(d))
    assert not ck and "do not hold its shape" in err

    d = copy_ckpt(tmp_path, "q4")
    write_st(d / "extra.safetensors", {"t": {"dtype": "Q3", "shape": [4], "data_offsets": [0, 4]}}, b"\0" * 4)
    ck, err = open_ck(str(d))
    assert not ck and "unknown dtype" in err

    d = copy_ckpt(tmp_path, "q4")
    (d / "extra.safetensors").write_bytes(struct.pack("<Q", 1 << 20) + b"{}")
    ck, err = open_ck(str(d))
    assert not ck and "overruns" in err

    # dims whose product wraps 64 bits to the data's length (2^62 * 4 bytes = 2^64 == 0
    # mod 2^64, against an empty range), and a negative dim
    for shape in ([1 << 62], [-4], [1 << 40, 1 << 40]):
        d = copy_ckpt(tmp_path, "q4")
        write_st(d / "extra.safetensors", {"t": {"dtype": "F32", "shape": shape, "data_offsets": [0, 0]}}, b"")
        ck, err = open_ck(str(d))
        assert not ck and "negative or oversized shape" in err, (shape, err)

    d = copy_ckpt(tmp_path, "q4")
    for f in d.glob("*.safetensors"):
        f.unlink()
    ck, err = open_ck(str(d))
    assert not ck and "no .safetensors" in err


def test_layer_errors_before_upload():
    """Out-of-range and absent layers fail before any device call."""
    ck, err = open_ck(cu.CKPTS["q4"])
    assert ck, err
    try:
        m = gpu.qw_moe_layer()
        e = C.create_string_buffer(512)
        assert not gpu.qw_moe_layer_load(ck, 8, C.byref(m), e, 512)
        assert "outside 0..7" in e.value.decode()
        assert not gpu.qw_moe_layer_load(ck, 5, C.byref(m), e, 512)    # not in the trimmed copy
        assert "layers.5.mlp.gate" in e.value.decode()
    finally:
        gpu.qw_checkpoint_close(ck)


def _rewrite_header(path, edit):
    raw = path.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + n])
    edit(hdr)
    write_st(path, hdr, raw[8 + n:])


def _file_holding(d, name):
    for f in sorted(d.glob("*.safetensors")):
        raw = f.read_bytes()
        n = struct.unpack("<Q", raw[:8])[0]
        if name in json.loads(raw[8:8 + n]):
            return f
    raise KeyError(name)


@pytest.mark.parametrize("tag", ["q4", "mlx"])
def test_layer_shape_errors_before_upload(tmp_path, tag):
    """A router stored with the right bytes but the wrong dims, and one that
    is missing, are refused with the tensor's name before any device call."""
    name = "language_model.model.layers.0.mlp.gate.weight"
    d = copy_ckpt(tmp_path, tag)
    f = _file_holding(d, name)

    def reshape(h):
        r, c = h[name]["shape"]
        h[name]["shape"] = [r * 2, c // 2]
    _rewrite_header(f, reshape)
    ck, err = open_ck(str(d))
    assert ck, err
    try:
        m = gpu.qw_moe_layer()
        e = C.create_string_buffer(512)
        assert not gpu.qw_moe_layer_load(ck, 0, C.byref(m), e, 512)
        msg = e.value.decode()
        assert name in msg and "this layer needs" in msg, msg
    finally:
        gpu.qw_checkpoint_close(ck)

    d = copy_ckpt(tmp_path, tag)
    f = _file_holding(d, name)
    _rewrite_header(f, lambda h: h.__setitem__("renamed", h.pop(name)))
    ck, err = open_ck(str(d))
    assert ck, err
    try:
        m = gpu.qw_moe_layer()
        e = C.create_string_buffer(512)
        assert not gpu.qw_moe_layer_load(ck, 0, C.byref(m), e, 512)
        assert f"checkpoint has no tensor {name}" in e.value.decode()
    finally:
        gpu.qw_checkpoint_close(ck)
