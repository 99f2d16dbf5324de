"""Builds qwasar_amd.synth.MoeLayer objects from the golden .npz fixtures."""
from __future__ import annotations

import numpy as np

from qwasar_amd.synth import MoeLayer, Q4


def layer_from_npz(path: str) -> MoeLayer:
    d = np.load(path, allow_pickle=False)
    H, E, K, I, SI, G = (int(d[k]) for k in ("H", "E", "K", "I", "SI", "group"))
    split = bool(int(d["split"]))

    def q(name, rows, cols):
        if name + "_w" not in d:
            return None
        return Q4(np.ascontiguousarray(d[name + "_w"]), np.ascontiguousarray(d[name + "_s"]),
                  np.ascontiguousarray(d[name + "_b"]), G, rows, cols)

    return MoeLayer(H, E, K, I, SI, G, bool(int(d["norm"])), split,
                    np.ascontiguousarray(d["router"]),
                    q("gate_up", E * 2 * I, H), q("gate", E * I, H), q("up", E * I, H),
                    q("down", E * H, I), q("sh_gate", SI, H), q("sh_up", SI, H), q("sh_down", H, SI),
                    np.ascontiguousarray(d["sh_gate_vec"]))
