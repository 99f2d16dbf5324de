"""A stack of MoE layers joined by the residual bf16 RMS norm (BASELINE
config 4), driven through the C ABI the way the reference's layer loop
drives its ops:

    x = rms_norm(h)
    for each layer:  y = MoE(x);  h = bf16(h + y);  x = rms_norm(h)

h is carried in bf16 between layers; each norm is unit-weight, eps 1e-6, in
the form of qwasar_cpu.c:68-82 (the residual add of qw_op_add_inplace and
the norm of qw_op_rms_norm, qwasar_gpu.h:269-276 and :384, with the bf16
carry between them, as one op).

Layer weights are written on the device by qw_op_synth (per-tensor
SplitMix64 streams keyed by seed, layer and name, with the distributions of
the benchmark configs: nibbles uniform, scales bf16 U(0.001, 0.02), biases
-8 * scale, router and shared gate bf16 N(0, 0.02)), so 48 layers need no
host copy; DeviceLayer.host() downloads one for the oracle.
"""
from __future__ import annotations

import numpy as np

from . import gpu, synth

EPS = 1e-6


class _Q4Dev:
    def __init__(self, rows: int, cols: int, group: int):
        self.rows, self.cols, self.group = rows, cols, group
        self.w = gpu.Buf(rows * cols // 2)
        self.s = gpu.Buf(rows * cols // group * 2)
        self.b = gpu.Buf(rows * cols // group * 2)

    def fill(self, c, seed: int, name: str) -> None:
        nw, ng = self.rows * self.cols // 8, self.rows * self.cols // self.group
        gpu.qw_op_synth(c, self.w.ref(), synth.SYNTH_U32, nw, synth.sm_key(seed, name + ".weight"), 0.0, 0.0)
        k = synth.sm_key(seed, name + ".scales")
        gpu.qw_op_synth(c, self.s.ref(), synth.SYNTH_BF16_UNIFORM, ng, k, 0.001, 0.02)
        gpu.qw_op_synth(c, self.b.ref(), synth.SYNTH_BF16_NEG8, ng, k, 0.001, 0.02)

    def ref(self) -> gpu.qw_q4_ref:
        return gpu.qw_q4_ref(self.w.ref(), self.s.ref(), self.b.ref(), self.group)

    def host(self) -> synth.Q4:
        w = self.w.read(np.uint32, (self.rows, self.cols // 8))
        s = self.s.read(np.uint16, (self.rows, self.cols // self.group))
        b = self.b.read(np.uint16, (self.rows, self.cols // self.group))
        return synth.Q4(w, s, b, self.group, self.rows, self.cols)

    def free(self) -> None:
        for t in (self.w, self.s, self.b):
            t.free()


class DeviceLayer:
    """One MoE layer's tensors, generated on the device."""

    def __init__(self, seed: int, index: int, H: int, E: int, K: int, I: int, SI: int,
                 group: int = 64, split: bool = True, norm: bool = True):
        self.H, self.E, self.K, self.I, self.SI, self.group = H, E, K, I, SI, group
        self.split, self.norm = split, norm
        p = f"stack.L{index}."
        self.router = gpu.Buf(E * H * 2)
        self.sh_gate_w = gpu.Buf(H * 2)
        self.q = {}
        if split:
            self.q["gate"] = _Q4Dev(E * I, H, group)
            self.q["up"] = _Q4Dev(E * I, H, group)
        else:
            self.q["gate_up"] = _Q4Dev(E * 2 * I, H, group)
        self.q["down"] = _Q4Dev(E * H, I, group)
        self.q["sh_gate"] = _Q4Dev(SI, H, group)
        self.q["sh_up"] = _Q4Dev(SI, H, group)
        self.q["sh_down"] = _Q4Dev(H, SI, group)
        c = gpu.qw_cmd_begin()
        gpu.qw_op_synth(c, self.router.ref(), synth.SYNTH_BF16_NORMAL, E * H, synth.sm_key(seed, p + "router"),
                        0.02, 0.0)
        gpu.qw_op_synth(c, self.sh_gate_w.ref(), synth.SYNTH_BF16_NORMAL, H,
                        synth.sm_key(seed, p + "sh_gate_w"), 0.02, 0.0)
        for name, t in self.q.items():
            t.fill(c, seed, p + name)
        gpu.run(c, f"stack layer {index}: synth")
        empty = gpu.qw_q4_ref(gpu.NULL_REF, gpu.NULL_REF, gpu.NULL_REF, 0)
        self.desc = gpu.qw_moe_layer(
            H, E, K, I, SI, bool(norm), bool(split), self.router.ref(),
            *[self.q[n].ref() if n in self.q else empty
              for n in ("gate_up", "gate", "up", "down", "sh_gate", "sh_up", "sh_down")],
            self.sh_gate_w.ref())

    def weight_bytes(self) -> int:
        return self.router.nbytes + self.sh_gate_w.nbytes + sum(
            t.w.nbytes + t.s.nbytes + t.b.nbytes for t in self.q.values())

    def host(self) -> synth.MoeLayer:
        """The same tensors on the host, as the oracle takes them."""
        g = {n: self.q[n].host() if n in self.q else None
             for n in ("gate_up", "gate", "up", "down", "sh_gate", "sh_up", "sh_down")}
        return synth.MoeLayer(self.H, self.E, self.K, self.I, self.SI, self.group, self.norm, self.split,
                              self.router.read(np.uint16, (self.E, self.H)), g["gate_up"], g["gate"], g["up"],
                              g["down"], g["sh_gate"], g["sh_up"], g["sh_down"],
                              self.sh_gate_w.read(np.uint16, (self.H,)))

    def free(self) -> None:
        self.router.free()
        self.sh_gate_w.free()
        for t in self.q.values():
            t.free()


class Stack:
    """Working buffers for running `layers` over up to `rows_max` rows."""

    def __init__(self, layers, rows_max: int):
        self.layers = layers
        H, K = layers[0].H, layers[0].K
        self.H, self.K, self.rows_max = H, K, rows_max
        self.h = gpu.Buf(rows_max * H * 2)       # bf16 carry
        self.x = gpu.Buf(rows_max * H * 4)       # the normalised input of the next layer
        self.y = gpu.Buf(rows_max * H * 4)       # a layer's output
        self.h2 = gpu.Buf(rows_max * H * 2)      # the fused form's second h and y
        self.y2 = gpu.Buf(rows_max * H * 4)
        self.h_final = self.h
        self.idx = gpu.Buf(rows_max * K * 4)
        self.w = gpu.Buf(rows_max * K * 4)

    def encode(self, c, rows: int, first: int = 0, count: int | None = None, start: bool = True) -> None:
        """Encodes layers first .. first+count-1 over h[:rows] (and the
        opening norm when `start`)."""
        count = len(self.layers) - first if count is None else count
        if start:
            gpu.qw_op_residual_rms_norm_bf16(c, self.h.ref(), self.x.ref(), gpu.NULL_REF, self.H, rows, EPS)
        for l in range(first, first + count):
            if not gpu.qw_op_moe_layer(c, self.y.ref(), self.idx.ref(), self.w.ref(), self.x.ref(),
                                       self.layers[l].desc, rows):
                raise RuntimeError(f"qw_op_moe_layer refused layer {l} at {rows} rows")
            gpu.qw_op_residual_rms_norm_bf16(c, self.h.ref(), self.x.ref(), self.y.ref(), self.H, rows, EPS)

    def encode_fused(self, c, rows: int) -> None:
        """The whole stack over h[:rows] with each residual step folded into
        the next layer's op (qw_op_moe_layer_residual; at decode sizes inside
        its one launch): layer l reads h from one of two buffers and writes
        the other, y alternates the same way, and a last residual step
        finishes h, which ends in self.h_final.  Same arithmetic, in the same
        order, as encode()."""
        hb, yb = (self.h, self.h2), (self.y, self.y2)
        n = len(self.layers)
        for l in range(n):
            y_prev = yb[(l - 1) % 2].ref() if l else gpu.NULL_REF
            if not gpu.qw_op_moe_layer_residual(c, yb[l % 2].ref(), self.idx.ref(), self.w.ref(),
                                                hb[l % 2].ref(), y_prev, hb[(l + 1) % 2].ref(), self.x.ref(),
                                                self.layers[l].desc, rows, EPS):
                raise RuntimeError(f"qw_op_moe_layer_residual refused layer {l} at {rows} rows")
        gpu.qw_op_residual_rms_norm_bf16(c, hb[n % 2].ref(), self.x.ref(), yb[(n - 1) % 2].ref(), self.H, rows, EPS)
        self.h_final = hb[n % 2]

    def free(self) -> None:
        for t in (self.h, self.x, self.y, self.h2, self.y2, self.idx, self.w):
            t.free()
