"""The native loader end to end on the GPU: qw_moe_layer_load's device
buffers byte for byte against the checkpoint (and, for the 8-bit router and
shared-expert gate of the MLX export, against the Python dequant that the
golden layer fixtures pin), then qw_op_moe_layer on the loaded layer against
the committed golden outputs (layer 0) and the oracle (layer 1).  Routing
bit-exact; outputs within the decode path's rel-L2 bar."""
import ctypes as C

import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth
from tests import ckpt_util as cu
from tests.test_gpu_layer import DECODE_REL, GOLD, check

pytestmark = pytest.mark.gpu


class Loaded:
    def __init__(self, gpu, tag, li):
        e = C.create_string_buffer(512)
        self.gpu = gpu
        self.ck = gpu.qw_checkpoint_open(cu.CKPTS[tag].encode(), e, 512)
        assert self.ck, e.value
        self.m = gpu.qw_moe_layer()
        ok = gpu.qw_moe_layer_load(self.ck, li, C.byref(self.m), e, 512)
        gpu.qw_checkpoint_close(self.ck)          # the device copies outlive the mapping
        assert ok, e.value

    def bytes_of(self, r):
        n = self.gpu.qw_buf_length(r.buf)
        return C.string_at(self.gpu.qw_buf_contents(r.buf), n)

    def free(self):
        self.gpu.qw_moe_layer_free(C.byref(self.m))
        assert not self.m.router.buf and not self.m.down.w.buf


def run(gpu, m, x):
    rows = x.shape[0]
    B = gpu.Buf
    xb, ob, ib, wb = B.of(x), B(rows * m.H * 4), B(rows * m.K * 4), B(rows * m.K * 4)
    c = gpu.qw_cmd_begin()
    assert gpu.qw_op_moe_layer(c, ob.ref(), ib.ref(), wb.ref(), xb.ref(), C.byref(m), rows)
    gpu.run(c, f"loaded moe_layer rows={rows}")
    return ob.read(np.float32, (rows, m.H)), ib.read(np.int32, (rows, m.K)), wb.read(np.float32, (rows, m.K))


@pytest.mark.parametrize("tag", ["q4", "mlx"])
def test_loaded_buffers(gpu, tag):
    print(f"loader buffers {tag}", flush=True)
    L = cu.layer(tag, 0)
    ld = Loaded(gpu, tag, 0)
    m = ld.m
    assert (m.H, m.E, m.K, m.I, m.SI, m.split, m.norm) == (L.H, L.E, L.K, L.I, L.SI, L.split, L.norm)
    assert ld.bytes_of(m.router) == L.router.tobytes()
    assert ld.bytes_of(m.sh_gate_w) == L.sh_gate_w.tobytes()
    pairs = [("down", L.down), ("sh_gate", L.sh_gate), ("sh_up", L.sh_up), ("sh_down", L.sh_down)]
    pairs += [("gate", L.gate), ("up", L.up)] if L.split else [("gate_up", L.gate_up)]
    for name, q in pairs:
        r = getattr(m, name)
        assert r.group == q.group, name
        assert ld.bytes_of(r.w) == q.w.tobytes(), name
        assert ld.bytes_of(r.scales) == q.s.tobytes(), name
        assert ld.bytes_of(r.biases) == q.b.tobytes(), name
    ld.free()


@pytest.mark.parametrize("tag", ["q4", "mlx"])
def test_loaded_layer0_golden(gpu, tag):
    print(f"loaded layer 0 {tag} vs golden", flush=True)
    g = np.load(GOLD + "/c0_golden.npz", allow_pickle=False)
    ld = Loaded(gpu, tag, 0)
    check(run(gpu, ld.m, g[f"{tag}_x"]), (g[f"{tag}_out"], g[f"{tag}_idx"], g[f"{tag}_w"]), DECODE_REL)
    ld.free()


@pytest.mark.parametrize("tag,rows", [("q4", 3), ("mlx", 3), ("q4", 40), ("mlx", 40)])
def test_loaded_layer1_oracle(gpu, tag, rows):
    print(f"loaded layer 1 {tag} rows={rows} vs oracle", flush=True)
    L = cu.layer(tag, 1)
    x = synth.make_x(91, rows, L.H, name=f"ckpt_{tag}.x1")
    ld = Loaded(gpu, tag, 1)
    check(run(gpu, ld.m, x), ref.moe_forward(L, x), DECODE_REL if rows <= 8 else 1e-3)
    ld.free()
