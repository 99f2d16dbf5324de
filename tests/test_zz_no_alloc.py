"""qw_op_moe_layer_noalloc (the decode path with its scratch in a static
device array, no allocation) against qw_op_moe_layer, through the C ABI:
the same bits on two calls in a row, the second with fewer rows (the array
keeps the first call's contents), at config 1's and config 0's shapes; and
the refusal of a layer whose staging does not fit the array."""
import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth

pytestmark = pytest.mark.gpu


def _run(gpu, op, lb, x):
    rows, L = x.shape[0], lb.L
    B = gpu.Buf
    xb, ob, ib, wb = B.of(x), B(rows * L.H * 4), B(rows * L.K * 4), B(rows * L.K * 4)
    c = gpu.qw_cmd_begin()
    assert op(c, ob.ref(), ib.ref(), wb.ref(), xb.ref(), lb.desc, rows)
    gpu.run(c, f"{op.__name__} rows={rows}")
    return ob.read(np.float32, (rows, L.H)), ib.read(np.int32, (rows, L.K)), wb.read(np.float32, (rows, L.K))


@pytest.mark.parametrize("cfg,rows", [(1, (8, 3)), (0, (5, 1))])
def test_noalloc_matches_moe_layer(gpu, cfg, rows):
    L, _ = synth.make_config(cfg)
    lb = gpu.LayerBufs(L)
    for i, r in enumerate(rows):
        x = synth.make_x(7100 + 10 * cfg + i, r, L.H)
        print(f"noalloc config {cfg} call {i}: rows {r}", flush=True)
        got = _run(gpu, gpu.qw_op_moe_layer_noalloc, lb, x)
        want = _run(gpu, gpu.qw_op_moe_layer, lb, x)
        for g, w in zip(got, want):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"call {i}: differs from qw_op_moe_layer"
        # and the routing against the oracle, as for the entry it mirrors
        widx, ww = ref.route(ref.dmat_bf16(x, L.router, L.H, L.E, r), r, L.E, L.K, norm=L.norm)
        assert np.array_equal(got[1], widx)
    lb.free()


def test_noalloc_refuses_oversized_staging(gpu):
    """Staging past the static array is refused with nothing encoded (no
    command is needed to ask); a fitting shape is accepted.  Several tokens
    take the batch path, whose staging (logits, the unique-expert table, the
    f16 token rows, the pairs and tiles of the grouped products, their fp32
    activations and, where the products stream, every pair's down row) must
    fit the 1,772,800 bytes past the hand-off state.  The banks are one small
    aligned buffer: only the shapes and the alignment are looked at."""
    r = gpu.NULL_REF
    buf = gpu.Buf(4096)
    q = gpu.qw_q4_ref(buf.ref(), buf.ref(), buf.ref(), 64)
    # H 3072, K 15, I 512: 2,101,504 bytes at 8 rows do not fit, 1,577,216 at 6 do
    big = gpu.qw_moe_layer(3072, 512, 15, 512, 512, True, True, buf.ref(), q, q, q, q, q, q, q, buf.ref())
    assert gpu.qw_op_moe_layer(None, r, r, r, r, big, 8)
    assert not gpu.qw_op_moe_layer_noalloc(None, r, r, r, r, big, 8)
    assert gpu.qw_op_moe_layer_noalloc(None, r, r, r, r, big, 6)
    assert gpu.qw_op_moe_layer_noalloc(None, r, r, r, r, big, 1)
    # config 1's shape: 1,466,624 bytes at 8 rows
    small = gpu.qw_moe_layer(3072, 512, 10, 512, 512, True, True, buf.ref(), q, q, q, q, q, q, q, buf.ref())
    assert gpu.qw_op_moe_layer_noalloc(None, r, r, r, r, small, 8)
    assert not gpu.qw_op_moe_layer_noalloc(None, r, r, r, r, small, 9)   # past the decode path
    buf.free()


def test_noalloc_refreshes_caller_mirrors(gpu):
    """The outputs' host mirrors are current after qw_cmd_wait without another
    qw_buf_contents: caller memory wrapped by qw_buf_wrap, and a view taken
    before the call."""
    L, _ = synth.make_config(1)
    lb = gpu.LayerBufs(L)
    x = synth.make_x(7300, 3, L.H)
    want = _run(gpu, gpu.qw_op_moe_layer, lb, x)
    B = gpu.Buf
    out = np.zeros((3, L.H), np.float32)
    ob = B(wrap=out)                   # the caller's own array is the mirror
    ib = B(3 * L.K * 4)
    iv = ib.view(np.int32, (3, L.K))   # a view kept from before the call
    wb, xb = B(3 * L.K * 4), B.of(x)
    c = gpu.qw_cmd_begin()
    assert gpu.qw_op_moe_layer_noalloc(c, ob.ref(), ib.ref(), wb.ref(), xb.ref(), lb.desc, 3)
    gpu.run(c, "noalloc into wrapped outputs")
    assert np.array_equal(ob._keep.view(np.uint32), want[0].view(np.uint32)), "wrapped output not refreshed"
    assert np.array_equal(iv, want[1]), "a view from before the call is stale"
    lb.free()


def test_noalloc_after_reinit(gpu):
    """qw_gpu_shutdown then qw_gpu_init zeroes the static hand-off state (the
    epochs restart at 1), so the calls after re-init give qw_op_moe_layer's
    bits, not words left by the earlier session."""
    L, _ = synth.make_config(1)
    lb = gpu.LayerBufs(L)
    xs = [synth.make_x(7400 + i, 1, L.H) for i in range(6)]
    for x in xs:
        _run(gpu, gpu.qw_op_moe_layer_noalloc, lb, x)
    gpu.qw_gpu_shutdown()
    gpu.init()
    for i, x in enumerate(reversed(xs)):
        got = _run(gpu, gpu.qw_op_moe_layer_noalloc, lb, x)
        want = _run(gpu, gpu.qw_op_moe_layer, lb, x)
        for g, w in zip(got, want):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"call {i} after re-init differs"
    lb.free()
