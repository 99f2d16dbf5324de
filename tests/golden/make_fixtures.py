"""Writes the golden fixtures under tests/golden/.  Run in the build container:

    python tests/golden/make_fixtures.py

1. tiny_q4_layer0.npz, tiny_mlx_layer0.npz -- layer 0's MoE tensors from the
   reference's own toy checkpoints (tests/fixtures/flashnext-tiny-q4: fused
   gate_up bank, group 64, bf16 router; flashnext-tiny-mlx: split switch_mlp
   banks, group 32, 8-bit router and shared gate).  Safetensors are parsed
   here as a JSON header plus raw little-endian bytes; nothing is executed.
   The 8-bit matrices are dequantised to bf16 as the reference's loader does
   (qwasar.c:1426-1461: w = scale * q + bias per group, rounded to bf16).
2. c0_golden.npz -- BASELINE config 0 (seeded synthetic tensors) with the
   oracle's routing and output for one token, and the tiny-q4 layer on
   seeded inputs with the oracle's routing and outputs: regression vectors.
3. ckpt_tiny_q4/, ckpt_tiny_mlx/ -- trimmed copies of the two toy
   checkpoints for the native loader (qw_checkpoint_open /
   qw_moe_layer_load): the reference's config.json as it is, and the MoE
   tensors of layers 0 and 1 rewritten byte for byte into safetensors files
   (two shards for the fused checkpoint, one with the mlx metadata for the
   split one).  `python tests/golden/make_fixtures.py ckpt` writes only these.
4. tiny_q4_sparse.npz -- the weights the QSA and gated-DeltaNet tests take
   from the same toy checkpoint, as data: layer 0's A_log, dt_bias, conv1d
   taps and output-norm gain (a linear-attention layer) and layer 3's
   indexer k_layernorm / q_layernorm gains (a QSA layer), with the config's
   shape fields (heads, head dims, ratio, budget, rope theta and sections).
   `python tests/golden/make_fixtures.py sparse` writes only this.
"""
from __future__ import annotations

import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

REF = "/root/reference/tests/fixtures"
DT = {"BF16": np.uint16, "U32": np.uint32, "I32": np.int32, "F32": np.float32, "I64": np.int64,
      "F16": np.float16, "U8": np.uint8, "I8": np.int8}


def read_safetensors(path):
    with open(path, "rb") as f:
        raw = f.read()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + n])
    base = 8 + n
    out = {}
    for k, v in hdr.items():
        if k == "__metadata__":
            continue
        a, b = v["data_offsets"]
        out[k] = np.frombuffer(raw[base + a:base + b], dtype=DT[v["dtype"]]).reshape(v["shape"]).copy()
    return out


def load_dir(d):
    t = {}
    for f in sorted(os.listdir(d)):
        if f.endswith(".safetensors"):
            t.update(read_safetensors(os.path.join(d, f)))
    return t


def f32_to_bf16(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def dequant_small(w, s, b, cols):
    """8- or 4-bit affine matrix -> bf16 [rows, cols] (qwasar.c:1444-1458)."""
    rows, words = w.shape
    bits = words * 32 // cols
    per = 32 // bits
    groups = s.shape[1]
    group = cols // groups
    j = np.arange(cols)
    q = (w[:, j // per] >> (bits * (j % per)).astype(np.uint32)) & ((1 << bits) - 1)
    v = bf16_to_f32(s)[:, j // group] * q.astype(np.float32) + bf16_to_f32(b)[:, j // group]
    return f32_to_bf16(v.astype(np.float32))


def tiny_q4():
    d = os.path.join(REF, "flashnext-tiny-q4")
    cfg = json.load(open(os.path.join(d, "config.json")))
    t = load_dir(d)
    p = "language_model.model.layers.0.mlp."
    H, E = cfg["hidden_size"], cfg["num_experts"]
    I, SI = cfg["moe_intermediate_size"], cfg["shared_expert_intermediate_size"]
    out = dict(H=H, E=E, K=cfg["num_experts_per_tok"], I=I, SI=SI, group=64, split=0,
               norm=int(cfg["norm_topk_prob"]),
               router=t[p + "gate.weight"],
               sh_gate_vec=t[p + "shared_expert_gate.weight"].reshape(H))
    for name, key, rows in (("gate_up", "experts.gate_up_proj", E * 2 * I), ("down", "experts.down_proj", E * H),
                            ("sh_gate", "shared_expert.gate_proj", SI), ("sh_up", "shared_expert.up_proj", SI),
                            ("sh_down", "shared_expert.down_proj", H)):
        out[name + "_w"] = t[p + key + ".weight"].view(np.uint32).reshape(rows, -1)
        out[name + "_s"] = t[p + key + ".scales"].reshape(rows, -1)
        out[name + "_b"] = t[p + key + ".biases"].reshape(rows, -1)
    return out


def tiny_mlx():
    d = os.path.join(REF, "flashnext-tiny-mlx")
    cfg = json.load(open(os.path.join(d, "config.json")))
    tc = cfg.get("text_config", cfg)
    t = load_dir(d)
    p = "language_model.model.layers.0.mlp."
    H, E = tc["hidden_size"], tc["num_experts"]
    I, SI = tc["moe_intermediate_size"], tc["shared_expert_intermediate_size"]
    out = dict(H=H, E=E, K=tc["num_experts_per_tok"], I=I, SI=SI, group=32, split=1,
               norm=int(tc["norm_topk_prob"]),
               router=dequant_small(t[p + "gate.weight"], t[p + "gate.scales"], t[p + "gate.biases"], H),
               sh_gate_vec=dequant_small(t[p + "shared_expert_gate.weight"], t[p + "shared_expert_gate.scales"],
                                       t[p + "shared_expert_gate.biases"], H).reshape(H))
    for name, key, rows in (("gate", "switch_mlp.gate_proj", E * I), ("up", "switch_mlp.up_proj", E * I),
                            ("down", "switch_mlp.down_proj", E * H),
                            ("sh_gate", "shared_expert.gate_proj", SI), ("sh_up", "shared_expert.up_proj", SI),
                            ("sh_down", "shared_expert.down_proj", H)):
        out[name + "_w"] = t[p + key + ".weight"].view(np.uint32).reshape(rows, -1)
        out[name + "_s"] = t[p + key + ".scales"].reshape(rows, -1)
        out[name + "_b"] = t[p + key + ".biases"].reshape(rows, -1)
    return out


def raw_entries(path):
    """(name, dtype, shape, bytes) of every tensor, and the metadata."""
    with open(path, "rb") as f:
        raw = f.read()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + n])
    meta = hdr.pop("__metadata__", None)
    base = 8 + n
    return [(k, v["dtype"], v["shape"], raw[base + v["data_offsets"][0]:base + v["data_offsets"][1]])
            for k, v in hdr.items()], meta


def write_safetensors(path, entries, meta=None):
    hdr, off, body = {}, 0, []
    if meta is not None:
        hdr["__metadata__"] = meta
    for name, dt, shape, data in sorted(entries):
        hdr[name] = {"dtype": dt, "shape": shape, "data_offsets": [off, off + len(data)]}
        off += len(data)
        body.append(data)
    h = json.dumps(hdr, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(body))


def trimmed_ckpts():
    for src, dst, shards in (("flashnext-tiny-q4", "ckpt_tiny_q4", 2), ("flashnext-tiny-mlx", "ckpt_tiny_mlx", 1)):
        d = os.path.join(REF, src)
        out = os.path.join(HERE, dst)
        os.makedirs(out, exist_ok=True)
        for f in os.listdir(out):
            os.remove(os.path.join(out, f))
        with open(os.path.join(d, "config.json"), "rb") as f:
            cfg = f.read()
        with open(os.path.join(out, "config.json"), "wb") as f:
            f.write(cfg)
        by_layer, meta = {0: [], 1: []}, None
        for fn in sorted(os.listdir(d)):
            if fn.endswith(".safetensors") and fn.startswith("model"):
                ents, m = raw_entries(os.path.join(d, fn))
                meta = meta or m
                for e in ents:
                    for layer in by_layer:
                        if e[0].startswith(f"language_model.model.layers.{layer}.mlp."):
                            by_layer[layer].append(e)
        if shards == 1:
            write_safetensors(os.path.join(out, "model.safetensors"), by_layer[0] + by_layer[1], meta)
        else:
            for layer in by_layer:
                write_safetensors(os.path.join(out, f"model-{layer + 1:05d}-of-00002.safetensors"),
                                  by_layer[layer], meta)


def tiny_sparse():
    d = os.path.join(REF, "flashnext-tiny-q4")
    t = load_dir(d)
    with open(os.path.join(d, "config.json")) as f:
        cfg = json.load(f)
    c = cfg.get("text_config", cfg)
    rp = c["rope_parameters"]
    la, sa = "language_model.model.layers.0.linear_attn.", "language_model.model.layers.3.self_attn.indexer."
    out = {
        "A_log": t[la + "A_log"], "dt_bias": t[la + "dt_bias"],
        "conv1d": t[la + "conv1d.weight"].reshape(t[la + "conv1d.weight"].shape[0], -1),
        "gdn_norm": t[la + "norm.weight"],
        "k_norm": t[sa + "k_layernorm.weight"], "q_norm": t[sa + "q_layernorm.weight"],
        "hk": np.int32(c["linear_num_key_heads"]), "hv": np.int32(c["linear_num_value_heads"]),
        "dk": np.int32(c["linear_key_head_dim"]), "dv": np.int32(c["linear_value_head_dim"]),
        "conv_k": np.int32(c["linear_conv_kernel_dim"]),
        "nq": np.int32(c["indexer_n_heads"]), "d": np.int32(c["indexer_head_dim"]),
        "ratio": np.int32(c["indexer_compress_ratio"]), "budget": np.int32(c["indexer_budget"]),
        "q_heads": np.int32(c["num_attention_heads"]), "kv_heads": np.int32(c["num_key_value_heads"]),
        "head_dim": np.int32(c["head_dim"]),
        "rotary_dim": np.int32(int(c["head_dim"] * rp["partial_rotary_factor"])),
        "rope_theta": np.float32(rp["rope_theta"]),
        "mrope_section": np.asarray(rp["mrope_section"], np.int32),
        "eps": np.float32(c["rms_norm_eps"]),
    }
    np.savez_compressed(os.path.join(HERE, "tiny_q4_sparse.npz"), **out)


def main():
    from qwasar_amd import synth
    from oracle import ref
    from tests.fixture_layers import layer_from_npz

    q4 = tiny_q4()
    np.savez_compressed(os.path.join(HERE, "tiny_q4_layer0.npz"), **q4)
    mlx = tiny_mlx()
    np.savez_compressed(os.path.join(HERE, "tiny_mlx_layer0.npz"), **mlx)

    L, x = synth.make_config(0)
    out, idx, w = ref.moe_forward(L, x)
    gold = dict(c0_x=x, c0_out=out, c0_idx=idx, c0_w=w)
    for tag, path in (("q4", "tiny_q4_layer0.npz"), ("mlx", "tiny_mlx_layer0.npz")):
        TL = layer_from_npz(os.path.join(HERE, path))
        tx = synth.make_x(77, 5, TL.H, name=f"tiny_{tag}.x")
        o, i, ww = ref.moe_forward(TL, tx)
        gold.update({f"{tag}_x": tx, f"{tag}_out": o, f"{tag}_idx": i, f"{tag}_w": ww})
    np.savez_compressed(os.path.join(HERE, "c0_golden.npz"), **gold)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    if sys.argv[1:] == ["ckpt"]:
        trimmed_ckpts()
    elif sys.argv[1:] == ["sparse"]:
        tiny_sparse()
    else:
        main()
        trimmed_ckpts()
        tiny_sparse()
