"""Routing inside the one-token decode launch, on the cases that stress it.

The one-token launch routes in its gatherer workgroups (qw_route_block: the
exponentials spread over the waves, then one wave's sum, threshold,
survivor ranking, or the K-round tournament when more than 64 experts
survive).  The standalone routing op has its own edge-case tests; these run
the same cases through qw_op_moe_layer at one row, with router rows built so
that the logits tie, underflow or flatten, and hold ids and weights bit-exact
to the oracle (the CPU restatement of qwasar_flash_cpu.c's routing) and the
output to the decode tolerance.

Shape: H 256, E 512 (eight logits a lane), K 10, I = SI = 128, group 64.
Tied rows are c * sign(x) in bf16, so their order-R dots with the token are
the same float."""
import dataclasses

import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth

pytestmark = pytest.mark.gpu

H, E, K, I = 256, 512, 10, 128


def _run(gpu, L, x):
    lb = gpu.LayerBufs(L)
    B = gpu.Buf
    xb, ob = B.of(x), B(L.H * 4)
    ib, wb = B(L.K * 4), B(L.K * 4)
    c = gpu.qw_cmd_begin()
    assert gpu.qw_op_moe_layer(c, ob.ref(), ib.ref(), wb.ref(), xb.ref(), lb.desc, 1)
    gpu.run(c, "moe_layer decode routing case")
    got = (ob.read(np.float32, (1, L.H)), ib.read(np.int32, (1, L.K)), wb.read(np.float32, (1, L.K)))
    lb.free()
    return got


def _case_router(base, sx, case, g, xabs):
    """The case's router (bf16 bits); xabs = sum |x|, the dot of sign(x) with x."""
    r = base.copy()
    if case == "three_tied_top":
        r[[3, 5, 7]] = 0.05 * sx
    elif case == "64_tied":
        r[g.choice(E, 64, replace=False)] = 0.05 * sx
    elif case == "65_tied":                      # more survivors than a wave: the tournament
        r[g.choice(E, 65, replace=False)] = 0.05 * sx
    elif case == "one_lane_slots":               # 5, 69, 133, 197, 261 share lane 5
        r[[261, 197, 133, 69, 5, 2, 1]] = 0.05 * sx
    elif case == "flat":                         # every logit 0: p = 1/E each
        r[:] = 0.0
    elif case == "one_certain":                  # p = 1 for one expert, 0 for the rest
        r[300] = 1.0 * sx
    elif case == "subnormal_tail":               # the rest's exponentials subnormal (e^-95)
        r[300] = (95.0 / xabs) * sx
    return synth.to_bf16(r)


CASES = ["three_tied_top", "64_tied", "65_tied", "one_lane_slots", "flat", "one_certain", "subnormal_tail"]


@pytest.mark.parametrize("case", CASES)
def test_decode_routing_edge_cases(gpu, case):
    L0 = synth.make_layer(5150, H=H, E=E, K=K, I=I, SI=I, group=64, tag="droute.")
    x = synth.make_x(5151, 1, H)
    sx = np.where(x[0] >= 0, 1.0, -1.0).astype(np.float32)
    base = synth.bf16_to_f32(L0.router).reshape(E, H)
    g = np.random.default_rng(5152 + CASES.index(case))
    L = dataclasses.replace(L0, router=_case_router(base, sx, case, g, float(np.abs(x).sum())))
    out, idx, w = _run(gpu, L, x)
    wout, widx, ww = ref.moe_forward(L, x)
    assert np.array_equal(idx, widx), f"{case}: ids {idx} != oracle {widx}"
    assert np.array_equal(w.view(np.uint32), ww.view(np.uint32)), f"{case}: weights not bit-exact"
    e = float(np.sqrt(((out - wout) ** 2).sum() / (wout ** 2).sum()))
    m = float(np.abs(out - wout).max())
    print(f"{case}: ids {idx[0].tolist()} rel-L2 {e:.3g} max-abs {m:.3g}")
    assert e < 5e-4 and m < 2e-2
    # the cases' own answers, independent of the oracle
    if case == "three_tied_top":
        assert idx[0, :3].tolist() == [3, 5, 7]
    elif case == "one_lane_slots":
        assert idx[0, :7].tolist() == [1, 2, 5, 69, 133, 197, 261]
    elif case == "flat":
        assert idx[0].tolist() == list(range(K))
        assert np.all(w[0] == np.float32(0.1))
    elif case == "one_certain":
        assert idx[0].tolist() == [300] + list(range(K - 1))
        assert w[0, 0] == 1.0 and np.all(w[0, 1:] == 0.0)
