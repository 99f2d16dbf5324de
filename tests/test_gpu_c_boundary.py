"""The boundary driven from C: tests/c_boundary/encode_moe (C99, built by
gcc -std=c99 -pedantic against include/qwasar_gpu.h and linked to
libqwasar_hip.so) runs the reference graph builder's op-by-op MoE chain
(qwasar_flash_graph.c:517-632) -- router, route, shared expert, the decode
bank matvecs or the grouped gather products, combine -- and its outputs are
held to the oracle: routing ids and weights bit-exact, outputs to the bar
(rel-L2 1e-3, max-abs 2e-2).

Shapes: config 0 (H 256: qmv_q4_multi and qmv_q4_bank2 decline, so the
caller's fallbacks run) and an H 2048 layer (both accepted), each at 1 and 3
rows (the decode chain) and 12 or 24 rows (the grouped chain), split and
fused banks."""
import os
import subprocess

import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_boundary", "encode_moe")


def _write(d, L, x):
    def raw(name, a):
        np.ascontiguousarray(a).tofile(os.path.join(d, name))

    raw("router.bin", L.router)
    raw("sh_gate_w.bin", L.sh_gate_w)
    raw("x.bin", x.astype(np.float32))
    names = ["down", "sh_gate", "sh_up", "sh_down"] + (["gate", "up"] if L.split else ["gate_up"])
    for n in names:
        q = getattr(L, n)
        raw(n + ".w", q.w)
        raw(n + ".s", q.s)
        raw(n + ".b", q.b)
    with open(os.path.join(d, "meta.txt"), "w") as f:
        f.write(f"{L.H} {L.E} {L.K} {L.I} {L.SI} {int(L.split)} {int(L.norm)} {L.group} {x.shape[0]}\n")


@pytest.mark.parametrize("shape,rows", [("c0", 1), ("c0", 3), ("c0", 24), ("h2048", 1), ("h2048", 3), ("h2048", 12)])
@pytest.mark.parametrize("split", [True, False])
def test_c_caller_encode_moe_chain(gpu, tmp_path, shape, rows, split):
    assert os.path.exists(EXE), "tests/c_boundary/encode_moe is not built (__graft_entry__.build())"
    if shape == "c0":
        L, x = synth.make_config(0, split=split, rows=rows, seed=600 + rows)
    else:
        L = synth.make_layer(610 + rows, H=2048, E=32, K=4, I=128, SI=128, group=64, split=split, tag="cb.")
        x = synth.make_x(620 + rows, rows, L.H, name="cb.x")
    _write(str(tmp_path), L, x)
    print(f"encode_moe {shape} rows={rows} split={split}", flush=True)
    r = subprocess.run([EXE, str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    out = np.fromfile(tmp_path / "out.bin", np.float32).reshape(rows, L.H)
    idx = np.fromfile(tmp_path / "idx.bin", np.int32).reshape(rows, L.K)
    w = np.fromfile(tmp_path / "w.bin", np.float32).reshape(rows, L.K)
    wout, widx, ww = ref.moe_forward(L, x)
    assert np.array_equal(idx, widx), "routing ids differ"
    assert np.array_equal(w.view(np.uint32), ww.view(np.uint32)), "routing weights not bit-exact"
    e = float(np.sqrt(((out - wout) ** 2).sum() / (wout ** 2).sum()))
    m = float(np.abs(out - wout).max())
    print(f"rel-L2 {e:.3g} max-abs {m:.3g}")
    assert e < 1e-3 and m < 2e-2
