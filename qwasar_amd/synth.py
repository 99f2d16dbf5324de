"""Seeded synthetic tensors for the MoE layer's benchmark and test configs.

Every tensor comes from its own Philox stream, keyed by (master seed, tensor
name), read as raw 64-bit words, so the values do not depend on numpy's
distribution algorithms.  Normals are Box-Muller on two 53-bit uniforms.

Layouts are the reference's MLX affine 4-bit banks (qwasar_model.h:87-153):

    weight  uint32 [rows, in/8]   element i at bit 4*(i%8) of word i/8
    scales  bf16   [rows, in/G]
    biases  bf16   [rows, in/G]   w = scale * nibble + bias

Nibbles are uniform in 0..15 (raw random bits), scales bf16 U(0.001, 0.02),
bias = -8 * scale (exact in bf16).  The router and the shared gate are bf16
N(0, 0.02); inputs are bf16-exact N(0, 1) values carried as fp32.

Router skew (configs 2 and 3) enters through the data, not the op: column 0
of every input row is 1.0 and column 0 of router row e holds the expert's
logit bias, so logit_e = bias_e + (the rest of the dot).  The layer's
arithmetic is untouched.
"""
from __future__ import annotations

import dataclasses
import hashlib
from typing import Optional

import numpy as np


def _key(seed: int, name: str) -> int:
    h = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    return int.from_bytes(h[:16], "little")


def raw64(seed: int, name: str, n: int) -> np.ndarray:
    bg = np.random.Philox(key=_key(seed, name))
    return bg.random_raw(n).astype(np.uint64, copy=False)


def raw32(seed: int, name: str, n: int) -> np.ndarray:
    r = raw64(seed, name, (n + 1) // 2)
    return r.view(np.uint32)[:n].copy()


def uniform(seed: int, name: str, n: int, lo: float, hi: float) -> np.ndarray:
    r = raw64(seed, name, n)
    u = (r >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return lo + (hi - lo) * u


def normal(seed: int, name: str, n: int, std: float = 1.0) -> np.ndarray:
    r = raw64(seed, name, 2 * n).reshape(n, 2)
    u1 = ((r[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (r[:, 1] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return std * np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def to_bf16(a) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(a) -> np.ndarray:
    return bf16_to_f32(to_bf16(a))


@dataclasses.dataclass
class Q4:
    """One MLX affine 4-bit matrix or bank: `rows` output rows of `cols` inputs."""
    w: np.ndarray   # uint32 [rows, cols/8]
    s: np.ndarray   # uint16 (bf16) [rows, cols/G]
    b: np.ndarray   # uint16 (bf16) [rows, cols/G]
    group: int
    rows: int
    cols: int

    def dequant(self, row0: int = 0, nrows: Optional[int] = None) -> np.ndarray:
        """fp32 [nrows, cols] dequantised rows (fp64-free, exact per element)."""
        nrows = self.rows - row0 if nrows is None else nrows
        w = self.w[row0:row0 + nrows]
        sh = (np.arange(8, dtype=np.uint32) * 4)
        q = ((w[:, :, None] >> sh) & 0xF).reshape(nrows, self.cols).astype(np.float32)
        s = np.repeat(bf16_to_f32(self.s[row0:row0 + nrows]), self.group, axis=1)
        b = np.repeat(bf16_to_f32(self.b[row0:row0 + nrows]), self.group, axis=1)
        return s * q + b


def make_q4(seed: int, name: str, rows: int, cols: int, group: int) -> Q4:
    assert cols % 8 == 0 and cols % group == 0
    w = raw32(seed, name + ".weight", rows * cols // 8).reshape(rows, cols // 8)
    ng = rows * cols // group
    sc = to_bf16(uniform(seed, name + ".scales", ng, 0.001, 0.02).astype(np.float32))
    bi = to_bf16(-8.0 * bf16_to_f32(sc))
    return Q4(w, sc.reshape(rows, cols // group), bi.reshape(rows, cols // group), group, rows, cols)


@dataclasses.dataclass
class MoeLayer:
    H: int
    E: int
    K: int
    I: int
    SI: int
    group: int
    norm: bool
    split: bool
    router: np.ndarray        # bf16 [E, H]
    gate_up: Optional[Q4]     # [E*2I, H] when not split (gate rows first per expert)
    gate: Optional[Q4]        # [E*I, H] when split
    up: Optional[Q4]
    down: Q4                  # [E*H, I]
    sh_gate: Q4               # [SI, H]
    sh_up: Q4
    sh_down: Q4               # [H, SI]
    sh_gate_w: np.ndarray     # bf16 [H]

    def weight_bytes(self) -> int:
        n = self.router.nbytes + self.sh_gate_w.nbytes
        for q in (self.gate_up, self.gate, self.up, self.down, self.sh_gate, self.sh_up, self.sh_down):
            if q is not None:
                n += q.w.nbytes + q.s.nbytes + q.b.nbytes
        return n

    def expert_bytes(self) -> int:
        """Bytes of one routed expert's gate, up and down (nibbles + scales + biases)."""
        per = 3 * self.I * self.H
        return per // 2 + (per // self.group) * 4


def make_router(seed: int, E: int, H: int, logit_bias: Optional[np.ndarray] = None,
                tag: str = "") -> np.ndarray:
    """bf16 [E, H] router, N(0, 0.02); column 0 holds the logit bias if given."""
    router = normal(seed, f"{tag}moe.router", E * H, 0.02).astype(np.float32).reshape(E, H)
    if logit_bias is not None:
        router[:, 0] = np.asarray(logit_bias, np.float32)
    return to_bf16(router)


def make_layer(seed: int, H: int, E: int, K: int, I: int, SI: int, group: int = 64,
               norm: bool = True, split: bool = True,
               logit_bias: Optional[np.ndarray] = None, tag: str = "") -> MoeLayer:
    p = f"{tag}moe."
    router = make_router(seed, E, H, logit_bias, tag)
    if split:
        gate = make_q4(seed, p + "gate", E * I, H, group)
        up = make_q4(seed, p + "up", E * I, H, group)
        gate_up = None
    else:
        gate = up = None
        gate_up = make_q4(seed, p + "gate_up", E * 2 * I, H, group)
    down = make_q4(seed, p + "down", E * H, I, group)
    sh_gate = make_q4(seed, p + "sh_gate", SI, H, group)
    sh_up = make_q4(seed, p + "sh_up", SI, H, group)
    sh_down = make_q4(seed, p + "sh_down", H, SI, group)
    sgw = to_bf16(normal(seed, p + "sh_gate_w", H, 0.02).astype(np.float32))
    return MoeLayer(H, E, K, I, SI, group, norm, split, router, gate_up, gate, up, down,
                    sh_gate, sh_up, sh_down, sgw)


def make_x(seed: int, rows: int, H: int, name: str = "x", const_col0: bool = False) -> np.ndarray:
    x = bf16_round(normal(seed, name, rows * H, 1.0).astype(np.float32)).reshape(rows, H)
    if const_col0:
        x[:, 0] = 1.0
    return np.ascontiguousarray(x)


# ---- the BASELINE configs ------------------------------------------------------

CONFIGS = {
    0: dict(H=256, E=16, K=4, I=128, SI=256, group=64, rows=1),
    1: dict(H=3072, E=512, K=10, I=512, SI=512, group=64, rows=1),
    2: dict(H=3072, E=512, K=10, I=512, SI=512, group=64, rows=8),
    3: dict(H=3072, E=512, K=10, I=512, SI=512, group=64, rows=512),
}

# Config 2: three experts every token picks.  With router N(0, 0.02) over
# H = 3072 inputs a logit has std ~1.1, so +8 clears every other expert.
C2_HOT = (7, 200, 411)
C2_BIAS = 8.0
ZIPF_S = 1.1


def zipf_bias(seed: int, E: int, s: float = ZIPF_S) -> np.ndarray:
    """log p_e with p_e ~ rank(e)^-s over a seeded permutation of ranks."""
    r = raw64(seed, "zipf.perm", E)
    ranks = np.argsort(r, kind="stable").argsort(kind="stable") + 1
    p = ranks.astype(np.float64) ** (-s)
    p /= p.sum()
    return np.log(p).astype(np.float32)


def make_config(cfg: int, seed: int = 1234, split: bool = True, rows: Optional[int] = None,
                tag: str = ""):
    """(layer, x) for BASELINE config `cfg` (0..3)."""
    c = dict(CONFIGS[cfg])
    rows = c.pop("rows") if rows is None else rows
    c.pop("rows", None)
    bias = None
    const0 = False
    if cfg == 2:
        bias = np.zeros(c["E"], np.float32)
        bias[list(C2_HOT)] = C2_BIAS
        const0 = True
    elif cfg == 3:
        bias = zipf_bias(seed, c["E"])
        const0 = True
    layer = make_layer(seed, split=split, logit_bias=bias, tag=tag, **c)
    x = make_x(seed, rows, c["H"], name=f"{tag}x", const_col0=const0)
    return layer, x


# ---- device-generated tensors (the layer stack) ---------------------------------
#
# The stack's weights (config 4: 48 layers, ~65 GB) are written on the device
# by qw_op_synth; these functions restate its arithmetic on the host so tests
# can check the device's output element by element.  Value i of the stream
# keyed k is the i-th output of SplitMix64 seeded with k.

SM_GOLDEN = 0x9E3779B97F4A7C15
SYNTH_U32, SYNTH_BF16_UNIFORM, SYNTH_BF16_NEG8, SYNTH_BF16_NORMAL, SYNTH_F32_BF16_NORMAL = range(5)


def sm_key(seed: int, name: str) -> int:
    h = hashlib.sha256(f"sm:{seed}:{name}".encode()).digest()
    return int.from_bytes(h[:8], "little")


def sm_raw(key: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start .. start+n-1 of SplitMix64 seeded with `key` (uint64)."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(key) + i * np.uint64(SM_GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def sm_values(kind: int, n: int, key: int, a: float = 0.0, b: float = 0.0) -> np.ndarray:
    """The host restatement of qw_op_synth's output."""
    if kind == SYNTH_U32:
        return (sm_raw(key, n) >> np.uint64(32)).astype(np.uint32)
    fa, fb = np.float64(np.float32(a)), np.float64(np.float32(b))
    if kind in (SYNTH_BF16_UNIFORM, SYNTH_BF16_NEG8):
        u = (sm_raw(key, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        s = to_bf16((fa + (fb - fa) * u).astype(np.float32))
        return s if kind == SYNTH_BF16_UNIFORM else to_bf16(np.float32(-8.0) * bf16_to_f32(s))
    r = sm_raw(key, 2 * n).reshape(n, 2)
    u1 = ((r[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (r[:, 1] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    v = (fa * np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)).astype(np.float32)
    return to_bf16(v) if kind == SYNTH_BF16_NORMAL else bf16_to_f32(to_bf16(v))
