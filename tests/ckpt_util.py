"""Reading the committed trimmed checkpoints (tests/golden/ckpt_*) in Python,
independently of the native loader: safetensors as a JSON header plus raw
bytes, the small quantised matrices dequantised to bf16 as the reference's
loader does (qwasar.c:1426-1461)."""
from __future__ import annotations

import json
import os
import struct

import numpy as np

from qwasar_amd.synth import MoeLayer, Q4

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CKPTS = {"q4": os.path.join(GOLD, "ckpt_tiny_q4"), "mlx": os.path.join(GOLD, "ckpt_tiny_mlx")}
NP = {"BF16": np.uint16, "U32": np.uint32, "I32": np.int32, "F32": np.float32}


def entries(d):
    """{name: (dtype, shape, bytes)} over every .safetensors file of d."""
    out = {}
    for fn in sorted(os.listdir(d)):
        if not fn.endswith(".safetensors"):
            continue
        raw = open(os.path.join(d, fn), "rb").read()
        n = struct.unpack("<Q", raw[:8])[0]
        hdr = json.loads(raw[8:8 + n])
        hdr.pop("__metadata__", None)
        for k, v in hdr.items():
            a, b = v["data_offsets"]
            out[k] = (v["dtype"], v["shape"], raw[8 + n + a:8 + n + b])
    return out


def arr(e):
    dt, shape, data = e
    return np.frombuffer(data, NP[dt]).reshape(shape)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def small_bf16(t, prefix, rows, cols):
    """bf16 [rows, cols]: as stored, or w = scale * q + bias per group."""
    w = t[prefix + ".weight"]
    if w[0] == "BF16":
        return arr(w).reshape(rows, cols)
    q, s, b = arr(w).view(np.uint32), arr(t[prefix + ".scales"]), arr(t[prefix + ".biases"])
    bits = q.shape[1] * 32 // cols
    per, group = 32 // bits, cols // s.shape[1]
    j = np.arange(cols)
    v = (q[:, j // per] >> (bits * (j % per)).astype(np.uint32)) & ((1 << bits) - 1)
    f = bf16_to_f32(s)[:, j // group] * v.astype(np.float32) + bf16_to_f32(b)[:, j // group]
    return f32_to_bf16(f.astype(np.float32))


def config(d):
    c = json.load(open(os.path.join(d, "config.json")))
    return c.get("text_config", c)


def layer(tag, li):
    """The MoeLayer of layer li of a trimmed checkpoint, for the oracle."""
    d = CKPTS[tag]
    t, c = entries(d), config(d)
    H, E, K, I, SI = (c[k] for k in ("hidden_size", "num_experts", "num_experts_per_tok",
                                      "moe_intermediate_size", "shared_expert_intermediate_size"))
    p = f"language_model.model.layers.{li}.mlp."
    split = p + "switch_mlp.gate_proj.weight" in t
    G = None

    def q(key, rows, cols):
        nonlocal G
        s = arr(t[p + key + ".scales"]).reshape(rows, -1)
        G = cols // s.shape[1]
        return Q4(np.ascontiguousarray(arr(t[p + key + ".weight"]).view(np.uint32).reshape(rows, -1)),
                  np.ascontiguousarray(s), np.ascontiguousarray(arr(t[p + key + ".biases"]).reshape(rows, -1)),
                  G, rows, cols)

    if split:
        gu, g, u = None, q("switch_mlp.gate_proj", E * I, H), q("switch_mlp.up_proj", E * I, H)
        dn = q("switch_mlp.down_proj", E * H, I)
    else:
        gu, g, u = q("experts.gate_up_proj", E * 2 * I, H), None, None
        dn = q("experts.down_proj", E * H, I)
    return MoeLayer(H, E, K, I, SI, G, bool(c.get("norm_topk_prob", True)), split,
                    np.ascontiguousarray(small_bf16(t, p + "gate", E, H)),
                    gu, g, u, dn, q("shared_expert.gate_proj", SI, H), q("shared_expert.up_proj", SI, H),
                    q("shared_expert.down_proj", H, SI),
                    np.ascontiguousarray(small_bf16(t, p + "shared_expert_gate", 1, H)).reshape(H))
