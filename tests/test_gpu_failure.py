"""The decode launch's failure path, forced from the host.

The decode launch hands data between workgroups through bounded waits; a
wait that gives up records its launch's epoch in the hand-off error word,
every later wait gives up at once, and each kernel still runs to its end.
qw_debug_decode_handoff_fail sets that word before a launch, so every wait
of the next decode launch gives up without any kernel spinning or faulting.
The host must then fail exactly the commands that launched at or after the
failing epoch -- whichever command waits first -- zero the state, and let the
next launch route oracle-exact again."""
import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth

pytestmark = pytest.mark.gpu


def _encode(gpu, lb, x):
    rows, L = x.shape[0], lb.L
    B = gpu.Buf
    bufs = (B.of(x), B(rows * L.H * 4), B(rows * L.K * 4), B(rows * L.K * 4))
    c = gpu.qw_cmd_begin()
    assert gpu.qw_op_moe_layer(c, bufs[1].ref(), bufs[2].ref(), bufs[3].ref(), bufs[0].ref(), lb.desc, rows)
    return c, bufs


def _finish(gpu, c):
    gpu.qw_cmd_wait(c)
    e = gpu.qw_cmd_error(c)
    gpu.qw_cmd_free(c)
    return e


def _exact(L, x, bufs):
    rows = x.shape[0]
    out, idx, w = (bufs[1].read(np.float32, (rows, L.H)), bufs[2].read(np.int32, (rows, L.K)),
                   bufs[3].read(np.float32, (rows, L.K)))
    wout, widx, ww = ref.moe_forward(L, x)
    assert np.array_equal(idx, widx)
    assert np.array_equal(w.view(np.uint32), ww.view(np.uint32))
    e = np.sqrt(((out - wout) ** 2).sum() / (wout ** 2).sum())
    assert e < 5e-4


@pytest.mark.parametrize("rows", [1, 3])
def test_handoff_give_up_is_reported_and_recovered(gpu, rows):
    """One token (the one launch) and three (the batch path's router-and-route
    launch, whose routing workgroup waits for the logits' tagged words)."""
    if rows == 1:
        L, _ = synth.make_config(0, rows=rows, seed=4101)
    else:   # the shared expert as wide as the routed ones: the matrix-core batch path
        L = synth.make_layer(4103, H=256, E=16, K=4, I=128, SI=128, group=64, tag="handoff3.")
    lb = gpu.LayerBufs(L)
    xs = [synth.make_x(4200 + rows + i, rows, L.H) for i in range(3)]
    # A launches normally; the word is then raised for the next launch, B's.
    cA, bA = _encode(gpu, lb, xs[0])
    assert gpu.qw_debug_decode_handoff_fail()
    cB, bB = _encode(gpu, lb, xs[1])
    # A waits first: its launch came before the failing one, so it succeeds,
    # and B, whose launch gave up, is failed by that same check.
    assert _finish(gpu, cA) is None
    _exact(L, xs[0], bA)
    e = _finish(gpu, cB)
    assert e is not None and b"hand-off wait gave up" in e
    # the state was zeroed: the next launch runs normally
    cC, bC = _encode(gpu, lb, xs[2])
    assert _finish(gpu, cC) is None
    _exact(L, xs[2], bC)
    lb.free()


def test_batch_decode_without_matrix_core_has_no_handoff(gpu):
    """A batch whose shared expert is wider than the routed experts runs its
    gate / up as q16 dots, with the router and the routing as launches of
    their own (no waits between workgroups): a raised error word does not
    touch it, and stays for the next one-token launch, which fails and
    recovers as above."""
    L = synth.make_layer(4150, H=256, E=32, K=4, I=64, SI=128, group=64, tag="nohandoff.")
    lb = gpu.LayerBufs(L)
    x3, x1 = synth.make_x(4151, 3, L.H), synth.make_x(4152, 1, L.H)
    assert gpu.qw_debug_decode_handoff_fail()
    c, b = _encode(gpu, lb, x3)
    assert _finish(gpu, c) is None
    _exact(L, x3, b)
    c, _ = _encode(gpu, lb, x1)
    e = _finish(gpu, c)
    assert e is not None and b"hand-off wait gave up" in e
    c, b = _encode(gpu, lb, x1)
    assert _finish(gpu, c) is None
    _exact(L, x1, b)
    lb.free()


def test_give_up_fails_the_waiting_command_itself(gpu):
    L, x = synth.make_config(0, rows=1, seed=4300)
    lb = gpu.LayerBufs(L)
    assert gpu.qw_debug_decode_handoff_fail()
    c, _ = _encode(gpu, lb, x)
    e = _finish(gpu, c)
    assert e is not None and b"hand-off wait gave up" in e
    c, b = _encode(gpu, lb, x)
    assert _finish(gpu, c) is None
    _exact(L, x, b)
    lb.free()


def test_qmv_multi_refuses_short_inputs(gpu):
    """The reference's contract: k < 2048 is refused with nothing encoded
    (qwasar_gpu.h:105-107); the command stays clean."""
    c = gpu.qw_cmd_begin()
    r = gpu.NULL_REF
    parts = (gpu.qw_qmv_part * 1)(gpu.qw_qmv_part(r, r, r, r, 8))
    assert not gpu.qw_op_qmv_q4_multi(c, r, 1024, 64, 1, parts)
    assert _finish(gpu, c) is None
