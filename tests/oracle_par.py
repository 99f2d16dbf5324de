"""The oracle over many rows, split across host threads.

The oracle's C functions run with the GIL released (ctypes), so row chunks
run in parallel; each chunk's result is the same bits as the whole, since
the oracle's arithmetic is per row.  Used where a GPU test checks a full-size
configuration (2048-row prefill chunks)."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from oracle import ref

THREADS = 16


def _chunks(n, parts):
    step = max(1, -(-n // parts))
    return [(i, min(n, i + step)) for i in range(0, n, step)]


def route_rows(L, x, threads=THREADS):
    """Router logits (order R) and routing for every row of x."""
    x = np.ascontiguousarray(x, np.float32)
    rows = x.shape[0]

    def one(ab):
        a, b = ab
        lg = ref.dmat_bf16(x[a:b], L.router, L.H, L.E, b - a)
        return ref.route(lg, b - a, L.E, L.K, norm=L.norm)

    with ThreadPoolExecutor(threads) as ex:
        res = list(ex.map(one, _chunks(rows, threads)))
    return np.concatenate([r[0] for r in res]), np.concatenate([r[1] for r in res])


def moe_rows(L, x, threads=THREADS):
    """The whole MoE block on every row of x: (out, idx, w)."""
    x = np.ascontiguousarray(x, np.float32)

    def one(ab):
        a, b = ab
        return ref.moe_forward(L, np.ascontiguousarray(x[a:b]))

    with ThreadPoolExecutor(threads) as ex:
        res = list(ex.map(one, _chunks(x.shape[0], threads)))
    return tuple(np.concatenate([r[i] for r in res]) for i in range(3))
