#!/usr/bin/env python3
"""Benchmark of the Flash-Next MoE layer on one MI355X.

Headline (the JSON line's `value`): BASELINE config 1 -- one MoE layer of
Flash-Next shape (H 3072, 512 experts, top-10, I 512, shared SI 512, MLX
4-bit group 64) decoding one token -- in microseconds per token, with all
expert weights resident in HBM, timed with HIP events on the backend's
stream over K back-to-back steps.  A step is one qw_op_moe_layer call on one
token (router, routing, the ten selected experts, the gated shared expert,
the combine).

Steps cycle through a pool of 64 tokens chosen (by the GPU's own routing) so
that any 12 consecutive tokens select pairwise disjoint experts: every step
reads its routed experts from HBM, not from the 256 MB Infinity Cache.

Also reported: the decode launch's own duration, HBM bandwidth on the routed
("selected-expert") bytes and on all bytes; config 2 (eight tokens a step
sharing three forced experts, judged on the batch's unique-expert bytes);
config 3 (512-token prefill with
Zipf-skewed routing) and a 2048-token prefill chunk (config 4's per-layer
step) in tokens/s and bf16-MFMA utilisation; config 4, 48 such layers
(~65 GB of weights written on the device) joined by the residual bf16 RMS
norm, through one 2048-token prefill and 256 decode steps; and the CPU
oracle's time on bounded samples of configs 0-3 (single-threaded scalar C,
the reference's own CPU path restated; see oracle/).

    python bench.py [--steps K] [--warmup W] [--no-prefill] [--no-config4] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, AMD spec
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16/fp16 MFMA, AMD spec
POOL = 64
COLD_WINDOW = 12


def q4_bytes(rows, cols, group):
    return rows * cols // 2 + (rows * cols // group) * 4


def decode_bytes(c):
    """Algorithmic bytes of one decode token, per kernel and in total."""
    H, E, K, I, SI, G = c["H"], c["E"], c["K"], c["I"], c["SI"], c["group"]
    expert_gu = 2 * q4_bytes(I, H, G)
    expert_down = q4_bytes(H, I, G)
    shared_gu = 2 * q4_bytes(SI, H, G)
    shared_down = q4_bytes(H, SI, G)
    router = 2 * E * H + 2 * H
    return {
        "routed": K * (expert_gu + expert_down),
        "all": K * (expert_gu + expert_down) + shared_gu + shared_down + router,
    }


PROFILE_JSON = os.path.join(ROOT, "profiles", "k_decode1_config1.json")


def _profile_figures():
    try:
        with open(PROFILE_JSON) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def measured_traffic(kernel):
    """HBM bytes per dispatch of `kernel` (fetch + write) from the committed
    rocprofv3 counter passes, or None when no summary covers it."""
    return _profile_figures().get("bytes_per_dispatch", {}).get(kernel)


def profiled_kernel_us(kernel):
    """`kernel`'s average duration in the committed rocprofv3 kernel trace of
    the headline decode, or None."""
    return _profile_figures().get("avg_us", {}).get(kernel)


def prefill_flops(c, rows):
    H, E, K, I, SI = c["H"], c["E"], c["K"], c["I"], c["SI"]
    return rows * (2 * K * 3 * I * H + 2 * 3 * SI * H + 2 * E * H)


def select_cold_pool(gpu, lb, cand_x, K):
    """Route candidates on the GPU; keep a cycle of POOL tokens in which any
    COLD_WINDOW consecutive ones select disjoint experts."""
    L = lb.L
    n = cand_x.shape[0]
    B = gpu.Buf
    xb, lg = B.of(cand_x), B(n * L.E * 4)
    ib, wb = B(n * K * 4), B(n * K * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_dmat_bf16(c, lg.ref(), xb.ref(), lb.router.ref(), L.H, L.E, n)
    gpu.qw_op_moe_route(c, ib.ref(), wb.ref(), lg.ref(), n, L.E, K, True)
    gpu.run(c, "route candidates")
    ids = ib.read(np.int32, (n, K))
    chosen, used = [], set(range(n))
    for _ in range(POOL):
        recent = set()
        for j in chosen[-(COLD_WINDOW - 1):]:
            recent.update(ids[j].tolist())
        if len(chosen) >= POOL - COLD_WINDOW + 1:
            for j in chosen[:COLD_WINDOW - (POOL - len(chosen))]:
                recent.update(ids[j].tolist())
        pick = next((i for i in sorted(used) if not recent.intersection(ids[i].tolist())), None)
        if pick is None:
            raise RuntimeError("could not build a cold token pool; raise the candidate count")
        chosen.append(pick)
        used.discard(pick)
    return np.ascontiguousarray(cand_x[chosen]), ids[chosen]


LEAD_ROWS = 2048          # one lead launch: the router's product over 2048 rows (~90 us)


def time_decode(gpu, lb, xpool, steps, warmup, mode):
    """Times `steps` decode steps after `warmup` untimed ones.  mode "region":
    HIP events at the region's two ends only; "steps": an event after every
    step as well (per-step durations, for the median); "kernels": events
    around every kernel launch as well (the decode kernel's own time).

    The region opens behind a lead of device work (router-shaped products,
    ~30 us of it per step to come, over a scratch row block: no expert byte
    is touched), so the host queues every step while the device is busy and
    the region holds the steps back to back.  Without it the region also
    holds whatever time the host takes to issue a step beyond the step's
    device time (on one box ~26 us a step against a 20 us kernel)."""
    L = lb.L
    B = gpu.Buf
    xb = B.of(xpool)
    ob, ib, wb = B(L.H * 4), B(L.K * 4), B(L.K * 4)
    lx, ly = B(LEAD_ROWS * L.H * 4), B(LEAD_ROWS * L.E * 4)
    row = L.H * 4
    c = gpu.qw_cmd_begin()
    for s in range(warmup):
        gpu.qw_op_moe_layer(c, ob.ref(), ib.ref(), wb.ref(), xb.ref((s % POOL) * row), lb.desc, 1)
    gpu.qw_cmd_wait(c)
    gpu.qw_prof_reset()
    gpu.qw_prof_set_enabled(True)
    gpu.qw_cmd_free(c)
    c = gpu.qw_cmd_begin()
    for _ in range(max(4, (steps * 30 + 89) // 90)):
        gpu.qw_op_dmat_bf16(c, ly.ref(), lx.ref(), lb.router.ref(), L.H, L.E, LEAD_ROWS)
    gpu.qw_cmd_mark(c, b"decode lead")           # the region opens here, on the device
    if mode == "steps":
        gpu.qw_cmd_mark(c, b"decode start")
    gpu.qw_prof_set_enabled(mode == "kernels")   # per-kernel events only when asked
    for s in range(steps):
        gpu.qw_op_moe_layer(c, ob.ref(), ib.ref(), wb.ref(), xb.ref(((warmup + s) % POOL) * row), lb.desc, 1)
        if mode == "steps":
            gpu.qw_prof_set_enabled(True)
            gpu.qw_cmd_mark(c, b"decode step")
            gpu.qw_prof_set_enabled(False)
    gpu.qw_prof_set_enabled(True)
    gpu.qw_cmd_mark(c, b"decode region")
    gpu.run(c, "decode")
    gpu.qw_prof_set_enabled(False)
    res = {"region": gpu.qw_prof_ms(b"decode region", None) if mode != "steps" else None,
           "fused": gpu.qw_prof_ms(b"moe decode", None)}
    if mode == "steps":
        buf = (ctypes.c_float * steps)()
        n = gpu.qw_prof_mark_times(b"decode step", buf, steps)
        res["per_step"] = np.array(buf[:n], np.float64)
    gpu.qw_prof_reset()
    for t in (xb, ob, ib, wb, lx, ly):
        t.free()
    return res


def hbm_ceiling(gpu, lb, reps=12):
    """The box's measured HBM read ceiling, by the read probe (every load
    independent, 16 bytes a lane, non-temporal): (a) one 2 GiB stream, past
    the 256 MB Infinity Cache; (b) ten experts' gate/up/down banks, the
    decode's routed bytes, read cold: launch r reads experts 10 s .. 10 s + 9
    for s = r mod (E / 10), so every set was last read E / 10 launches ago
    (1.35 GB of other experts in between).  Medians over `reps` launches at
    the best of a few piece sizes (a workgroup a piece)."""
    L = lb.L
    B = gpu.Buf
    out = {}
    big = B(2 << 30)
    best = None
    for blocks in (16384, 65536, 262144):      # piece bytes, one workgroup each
        ms = (ctypes.c_float * reps)()
        assert gpu.qw_probe_read((gpu.qw_ref * 1)(big.ref()), (ctypes.c_uint64 * 1)(2 << 30), 1, 1, reps,
                                 blocks, ms)
        med = float(np.median(np.array(ms[1:], np.float64)))
        if best is None or med < best[1]:
            best = (blocks, med)
    big.free()
    out["stream_2gib"] = {"gbs": round((2 << 30) / (best[1] * 1e-3) / 1e9, 1), "ms": round(best[1], 4),
                          "piece_bytes": best[0]}
    I, H, G, K = L.I, L.H, L.group, L.K
    q = lb.q
    per = []          # (buffer, byte offset, bytes) of one expert, in bank order
    for e in range(L.E):
        segs = []
        if L.split:
            for nm in ("gate", "up"):
                segs += [(q[nm].w, e * I * H // 2, I * H // 2), (q[nm].s, e * I * (H // G) * 2, I * (H // G) * 2),
                         (q[nm].b, e * I * (H // G) * 2, I * (H // G) * 2)]
        else:
            nm = "gate_up"
            segs += [(q[nm].w, e * 2 * I * H // 2, 2 * I * H // 2),
                     (q[nm].s, e * 2 * I * (H // G) * 2, 2 * I * (H // G) * 2),
                     (q[nm].b, e * 2 * I * (H // G) * 2, 2 * I * (H // G) * 2)]
        segs += [(q["down"].w, e * H * I // 2, H * I // 2), (q["down"].s, e * H * (I // G) * 2, H * (I // G) * 2),
                 (q["down"].b, e * H * (I // G) * 2, H * (I // G) * 2)]
        per.append(segs)
    nsets, nseg = L.E // K, K * len(per[0])
    refs = (gpu.qw_ref * (nsets * nseg))()
    nbytes = (ctypes.c_uint64 * (nsets * nseg))()
    for s_ in range(nsets):
        for k in range(K):
            for i, (buf, off, n) in enumerate(per[s_ * K + k]):
                refs[s_ * nseg + k * len(per[0]) + i] = buf.ref(off)
                nbytes[s_ * nseg + k * len(per[0]) + i] = n
    set_bytes = sum(n for _, _, n in per[0]) * K
    best = None
    r2 = 2 * nsets
    for blocks in (4096, 8192, 16384, 32768):  # piece bytes, one workgroup each
        ms = (ctypes.c_float * r2)()
        assert gpu.qw_probe_read(refs, nbytes, nsets, nseg, r2, blocks, ms)
        med = float(np.median(np.array(ms[nsets:], np.float64)))    # the second cycle: every set cold
        if best is None or med < best[1]:
            best = (blocks, med)
    out["ten_experts_cold"] = {"bytes": int(set_bytes), "us": round(best[1] * 1e3, 2),
                               "gbs": round(set_bytes / (best[1] * 1e-3) / 1e9, 1), "piece_bytes": best[0]}
    return out


def time_prefill(gpu, lb, x, reps):
    L = lb.L
    rows = x.shape[0]
    B = gpu.Buf
    xb, ob = B.of(x), B(rows * L.H * 4)
    ib, wb = B(rows * L.K * 4), B(rows * L.K * 4)
    c = gpu.qw_cmd_begin()
    for _ in range(2):
        gpu.qw_op_moe_layer(c, ob.ref(), ib.ref(), wb.ref(), xb.ref(), lb.desc, rows)
    gpu.run(c, "prefill warmup")
    gpu.qw_prof_reset()
    gpu.qw_prof_set_enabled(True)
    c = gpu.qw_cmd_begin()
    gpu.qw_prof_set_enabled(False)
    for _ in range(reps):
        gpu.qw_op_moe_layer(c, ob.ref(), ib.ref(), wb.ref(), xb.ref(), lb.desc, rows)
    gpu.qw_prof_set_enabled(True)
    gpu.qw_cmd_mark(c, b"prefill region")
    gpu.run(c, "prefill")
    gpu.qw_prof_set_enabled(False)
    ms = gpu.qw_prof_ms(b"prefill region", None) / reps
    gpu.qw_prof_reset()
    counts = np.bincount(ib.read(np.int32, (rows, L.K)).ravel(), minlength=L.E)
    return ms, int(counts.max()), int((counts > 0).sum())


def bench_stack(gpu, nlayers, rows, steps, warmup, seed=4444, cpu_seconds=0.0):
    """`nlayers` layers of config 1's shape (weights written
    on the device), joined by the residual bf16 RMS norm; one `rows`-token
    prefill, then `steps` decode steps, each fed a fresh N(0, 1) token."""
    from qwasar_amd import stack, synth
    cfg = dict(synth.CONFIGS[1])
    shape = {k: cfg[k] for k in ("H", "E", "K", "I", "SI", "group")}
    H = shape["H"]
    layers = [stack.DeviceLayer(seed, l, **shape) for l in range(nlayers)]
    st = stack.Stack(layers, rows)
    labels = [f"stack prefill L{l}".encode() for l in range(nlayers)]   # alive until the profile is read

    def fresh_h(c, n, name):
        gpu.qw_op_synth(c, st.h.ref(), synth.SYNTH_BF16_NORMAL, n * H, synth.sm_key(seed, name), 1.0, 0.0)

    # prefill: one untimed pass, then the timed one, a mark after each layer
    c = gpu.qw_cmd_begin()
    fresh_h(c, rows, "h0.warm")
    st.encode(c, rows)
    gpu.run(c, "stack prefill warm-up")
    c = gpu.qw_cmd_begin()
    fresh_h(c, rows, "h0")
    gpu.qw_op_residual_rms_norm_bf16(c, st.h.ref(), st.x.ref(), gpu.NULL_REF, H, rows, stack.EPS)
    gpu.qw_prof_reset()
    gpu.qw_prof_set_enabled(True)
    gpu.qw_cmd_mark(c, b"stack prefill start")
    for l in range(nlayers):
        gpu.qw_prof_set_enabled(False)
        st.encode(c, rows, first=l, count=1, start=False)
        gpu.qw_prof_set_enabled(True)
        gpu.qw_cmd_mark(c, labels[l])
    gpu.run(c, "stack prefill")
    per_layer = np.array([gpu.qw_prof_ms(labels[l], None) for l in range(nlayers)])
    gpu.qw_prof_set_enabled(False)
    gpu.qw_prof_reset()
    pf_ms = float(per_layer.sum())

    # decode
    c = gpu.qw_cmd_begin()
    for s in range(warmup):
        fresh_h(c, 1, f"dec.warm{s}")
        st.encode_fused(c, 1)
    gpu.run(c, "stack decode warm-up")
    gpu.qw_prof_reset()
    gpu.qw_prof_set_enabled(True)
    c = gpu.qw_cmd_begin()
    gpu.qw_prof_set_enabled(False)
    for s in range(steps):
        fresh_h(c, 1, f"dec{s}")
        st.encode_fused(c, 1)
    gpu.qw_prof_set_enabled(True)
    gpu.qw_cmd_mark(c, b"stack decode region")
    gpu.run(c, "stack decode")
    dec_ms = gpu.qw_prof_ms(b"stack decode region", None)
    gpu.qw_prof_set_enabled(False)
    gpu.qw_prof_reset()
    wbytes = sum(L.weight_bytes() for L in layers)
    cpu = None
    if cpu_seconds > 0:
        cpu = stack_cpu_sample(layers[0], rows, cpu_seconds, nlayers, seed)
    st.free()
    for L in layers:
        L.free()
    us_tok = dec_ms * 1000.0 / steps
    us_tl = us_tok / nlayers
    routed = decode_bytes(cfg)["routed"]
    fl = prefill_flops(cfg, rows) * nlayers
    return {"layers": nlayers, "weights_gb": round(wbytes / 1e9, 2),
            "prefill": {"rows": rows, "ms": round(pf_ms, 3), "tokens_per_s": round(rows / (pf_ms * 1e-3), 1),
                        "ms_per_layer_median": round(float(np.median(per_layer)), 3),
                        "ms_per_layer_max": round(float(per_layer.max()), 3),
                        "mfma_util": round(fl / (pf_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)},
            "decode": {"steps": steps, "us_per_token": round(us_tok, 2), "us_per_token_layer": round(us_tl, 3),
                       "routed_hbm_frac": round(routed / (us_tl * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
            "cpu": cpu,
            "includes": "per layer: the MoE block and the residual bf16 RMS norm (at decode folded into "
                        "the layer's one launch, qw_op_moe_layer_residual); decode steps include writing "
                        "the fresh token on the device and the closing residual step"}


def stack_cpu_sample(layer, rows, seconds, nlayers, seed):
    """The oracle on config 4's layer 0 (its weights read back from the
    device): decode tokens one at a time, then prefill rows 8 at a time, each
    for about `seconds`, every pass the MoE block and the residual bf16 RMS
    norm as the stack runs them; per-token-layer time scaled by the stack's
    `nlayers` layers."""
    from oracle import ref
    from qwasar_amd import synth
    L = layer.host()
    x = synth.make_x(seed + 17, 64, L.H, name="stack.cpu")

    def one(xs):
        y, _, _ = ref.moe_forward(L, xs)
        ref.rms_norm(xs + y)

    res = {}
    for name, per in (("decode", 1), ("prefill", 8)):
        n, t0 = 0, time.perf_counter()
        while (n == 0 or time.perf_counter() - t0 < seconds) and (n + 1) * per <= x.shape[0]:
            one(x[n * per:(n + 1) * per])
            n += 1
        t = (time.perf_counter() - t0) / (n * per)      # seconds a token-layer
        res[name] = {"tokens_per_s": round(1.0 / (t * nlayers), 3), "us_per_token_layer": round(t * 1e6, 1),
                     "sample": f"{n * per} tokens through layer 0 ({per} a call), scaled by {nlayers} layers"}
    res["kind"] = "port"
    res["cores"] = 1
    return res


def bench_hc(gpu, steps, H=3072, S=4, k=320, G=64, pool=96, prefill_rows=2048, seed=777):
    """The hyper-connection mixer around one block at config
    1's width: decode (one token: inject + grouped norm, mix-down, the
    injection logits, the fused mix-up) over a pool of `pool` weight sets
    (~390 MB, past the Infinity Cache), and the prefill form at
    `prefill_rows` tokens (the same with the 4-bit products as GEMMs and the
    mix as its own pass)."""
    from qwasar_amd import synth
    B = gpu.Buf
    HH = S * H

    def q4(name, rows, cols):
        w, sc, bi = B(rows * cols // 2), B(rows * cols // G * 2), B(rows * cols // G * 2)
        kk = synth.sm_key(seed, name + ".scales")
        gpu.qw_op_synth(c, w.ref(), synth.SYNTH_U32, rows * cols // 8, synth.sm_key(seed, name + ".w"), 0.0, 0.0)
        gpu.qw_op_synth(c, sc.ref(), synth.SYNTH_BF16_UNIFORM, rows * cols // G, kk, 0.001, 0.02)
        gpu.qw_op_synth(c, bi.ref(), synth.SYNTH_BF16_NEG8, rows * cols // G, kk, 0.001, 0.02)
        return w, sc, bi

    sets = []
    c = gpu.qw_cmd_begin()
    for p in range(pool):
        wn, bj = B(HH * 2), B(S * HH * 2)
        gpu.qw_op_synth(c, wn.ref(), synth.SYNTH_BF16_UNIFORM, HH, synth.sm_key(seed, f"hc{p}.norm"), 0.9, 1.1)
        gpu.qw_op_synth(c, bj.ref(), synth.SYNTH_BF16_NORMAL, S * HH, synth.sm_key(seed, f"hc{p}.inj"), 0.02, 0.0)
        sets.append((wn, q4(f"hc{p}.down", k, HH), q4(f"hc{p}.up", HH, k), bj))
    rows = prefill_rows
    h4, n4, out = B(rows * HH * 4), B(rows * HH * 4), B(rows * H * 4)
    inj, d, x, m = B(rows * S * 4), B(rows * k * 4), B(rows * H * 4), B(rows * HH * 4)
    gpu.qw_op_synth(c, h4.ref(), synth.SYNTH_F32_BF16_NORMAL, rows * HH, synth.sm_key(seed, "h4"), 1.0, 0.0)
    gpu.qw_op_synth(c, out.ref(), synth.SYNTH_F32_BF16_NORMAL, rows * H, synth.sm_key(seed, "out"), 1.0, 0.0)
    gpu.qw_op_synth(c, inj.ref(), synth.SYNTH_F32_BF16_NORMAL, rows * S, synth.sm_key(seed, "inj"), 1.0, 0.0)
    gpu.run(c, "hc mixer setup")

    h4b, injb = B(rows * HH * 4), B(rows * S * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_synth(c, injb.ref(), synth.SYNTH_F32_BF16_NORMAL, rows * S, synth.sm_key(seed, "inj"), 1.0, 0.0)
    gpu.run(c, "hc mixer setup (decode pair)")
    hpair, ipair = (h4, h4b), (inj, injb)

    def decode_step(c, p):
        # one launch: inject + norm + down + injection logits, then up + mix
        # after an in-launch hand-off; h4 and the logits alternate between two
        # buffers
        wn, (dw, ds, db), (uw, us, ub), bj = sets[p % pool]
        assert gpu.qw_op_hc_decode(c, x.ref(), hpair[(p + 1) % 2].ref(), n4.ref(), d.ref(), ipair[(p + 1) % 2].ref(),
                                   hpair[p % 2].ref(), out.ref(), ipair[p % 2].ref(), wn.ref(), dw.ref(), ds.ref(),
                                   db.ref(), bj.ref(), uw.ref(), us.ref(), ub.ref(), H, S, k, G, 1e-6, 1.0 / S)

    def decode_step_two(c, p):
        # the same step as two launches (the pre-decode op, then the mix-up op)
        wn, (dw, ds, db), (uw, us, ub), bj = sets[p % pool]
        assert gpu.qw_op_hc_pre_decode(c, hpair[(p + 1) % 2].ref(), n4.ref(), d.ref(), ipair[(p + 1) % 2].ref(),
                                       hpair[p % 2].ref(), out.ref(), ipair[p % 2].ref(), wn.ref(), dw.ref(),
                                       ds.ref(), db.ref(), bj.ref(), H, S, k, G, 1e-6)
        gpu.qw_op_hc_mix_up(c, x.ref(), d.ref(), n4.ref(), uw.ref(), us.ref(), ub.ref(), k, H, S, 1, 1.0 / S, G)

    c = gpu.qw_cmd_begin()
    for p in range(pool):
        decode_step(c, p)
    gpu.run(c, "hc decode warm-up")
    gpu.qw_prof_reset()
    gpu.qw_prof_set_enabled(True)
    c = gpu.qw_cmd_begin()
    gpu.qw_prof_set_enabled(False)
    for p in range(steps):
        decode_step(c, p)
    gpu.qw_prof_set_enabled(True)
    gpu.qw_cmd_mark(c, b"hc decode region")
    gpu.run(c, "hc decode")
    dec_ms = gpu.qw_prof_ms(b"hc decode region", None)
    gpu.qw_prof_reset()
    gpu.qw_prof_set_enabled(True)
    c = gpu.qw_cmd_begin()
    gpu.qw_prof_set_enabled(False)
    for p in range(steps):
        decode_step_two(c, p)
    gpu.qw_prof_set_enabled(True)
    gpu.qw_cmd_mark(c, b"hc decode two-launch region")
    gpu.run(c, "hc decode (two launches)")
    two_ms = gpu.qw_prof_ms(b"hc decode two-launch region", None)

    wn, (dw, ds, db), (uw, us, ub), bj = sets[0]

    def prefill(c):
        gpu.qw_op_hc_inject_norm(c, h4.ref(), out.ref(), inj.ref(), wn.ref(), n4.ref(), rows, H, S, 1e-6)
        gpu.qw_op_qmat_q4(c, d.ref(), n4.ref(), dw.ref(), ds.ref(), db.ref(), HH, k, rows, G)
        gpu.qw_op_dmat_bf16(c, inj.ref(), n4.ref(), bj.ref(), HH, S, rows)
        gpu.qw_op_silu_scale(c, d.ref(), rows * k, 1.0 / S)
        gpu.qw_op_qmat_q4(c, m.ref(), d.ref(), uw.ref(), us.ref(), ub.ref(), k, HH, rows, G)
        gpu.qw_op_hc_mix(c, x.ref(), n4.ref(), m.ref(), rows, H, S)

    c = gpu.qw_cmd_begin()
    prefill(c)
    gpu.run(c, "hc prefill warm-up")
    gpu.qw_prof_reset()
    gpu.qw_prof_set_enabled(True)
    c = gpu.qw_cmd_begin()
    gpu.qw_prof_set_enabled(False)
    reps = 5
    for _ in range(reps):
        prefill(c)
    gpu.qw_prof_set_enabled(True)
    gpu.qw_cmd_mark(c, b"hc prefill region")
    gpu.run(c, "hc prefill")
    pf_ms = gpu.qw_prof_ms(b"hc prefill region", None) / reps
    gpu.qw_prof_set_enabled(False)
    gpu.qw_prof_reset()
    for wn_, (a1, a2, a3), (b1, b2, b3), bj_ in sets:
        for t in (wn_, a1, a2, a3, b1, b2, b3, bj_):
            t.free()
    for t in (h4, n4, out, inj, d, x, m, h4b, injb):
        t.free()
    us_tok = dec_ms * 1000.0 / steps
    wbytes = 2 * (k * HH // 2 + k * HH // G * 4) + S * HH * 2 + HH * 2
    abytes = HH * 4 * 3 + H * 4 * 2 + k * 4 * 2          # h4 read and written, n4 written; out, x; d
    flops = 2.0 * rows * (2 * HH * k + HH * S)
    return {"shape": {"H": H, "S": S, "lowrank": k, "group": G},
            "decode": {"us_per_token": round(us_tok, 2), "weight_bytes": wbytes,
                       "hbm_gbs": round((wbytes + abytes) / (us_tok * 1e-6) / 1e9, 1),
                       "launches": 1, "weight_sets": pool,
                       "two_launch_us_per_token": round(two_ms * 1000.0 / steps, 2)},
            "prefill": {"rows": rows, "ms": round(pf_ms, 3),
                        "tflops": round(flops / (pf_ms * 1e-3) / 1e12, 2)}}


def bench_config2(gpu, lb, L, cfg, seed, steps, warmup, nbatch=32):
    """eight tokens a step whose router logits carry +8 on
    three experts (every token picks them), so one launch reads the union U of
    the batch's experts.  Batches are chosen by the GPU's own routing so that
    consecutive batches share no expert outside the three forced ones: each
    step reads its other experts from HBM."""
    from qwasar_amd import synth
    bias = np.zeros(L.E, np.float32)
    bias[list(synth.C2_HOT)] = synth.C2_BIAS
    r2 = synth.make_router(seed, L.E, L.H, bias)
    rb2 = gpu.Buf(wrap=r2)
    d2 = gpu.qw_moe_layer.from_buffer_copy(lb.desc)
    d2.router = rb2.ref()
    n = 2048
    cand = synth.make_x(seed + 2, n, L.H, name="bench.c2cand", const_col0=True)
    B = gpu.Buf
    xb, lg, ib, wb = B.of(cand), B(n * L.E * 4), B(n * L.K * 4), B(n * L.K * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_dmat_bf16(c, lg.ref(), xb.ref(), rb2.ref(), L.H, L.E, n)
    gpu.qw_op_moe_route(c, ib.ref(), wb.ref(), lg.ref(), n, L.E, L.K, True)
    gpu.run(c, "route config-2 candidates")
    ids = ib.read(np.int32, (n, L.K))
    for t in (xb, lg, ib, wb):
        t.free()
    hot = set(synth.C2_HOT)
    left, batches, prev = list(range(n)), [], set()
    while len(batches) < nbatch:
        cur, members = set(), []
        for i in list(left):
            e = set(ids[i].tolist()) - hot
            if not e & prev:
                members.append(i)
                cur |= e
                left.remove(i)
                if len(members) == 8:
                    break
        if len(members) < 8:
            raise RuntimeError("could not build config-2 batches; raise the candidate count")
        batches.append(members)
        prev = cur
    uniq = [len(set(ids[b].ravel().tolist())) for b in batches]
    xs = np.ascontiguousarray(cand[np.concatenate(batches)])
    xp = B.of(xs)
    ob, ib, wb = B(8 * L.H * 4), B(8 * L.K * 4), B(8 * L.K * 4)
    stride = 8 * L.H * 4

    def step(c, s):
        gpu.qw_op_moe_layer(c, ob.ref(), ib.ref(), wb.ref(), xp.ref((s % nbatch) * stride), d2, 8)

    c = gpu.qw_cmd_begin()
    for s in range(warmup):
        step(c, s)
    gpu.run(c, "config 2 warm-up")
    gpu.qw_prof_reset()
    gpu.qw_prof_set_enabled(True)
    c = gpu.qw_cmd_begin()
    gpu.qw_prof_set_enabled(False)
    for s in range(steps):
        step(c, warmup + s)
    gpu.qw_prof_set_enabled(True)
    gpu.qw_cmd_mark(c, b"config2 region")
    gpu.run(c, "config 2")
    ms = gpu.qw_prof_ms(b"config2 region", None)
    gpu.qw_prof_set_enabled(False)
    gpu.qw_prof_reset()
    for t in (xp, ob, ib, wb, rb2):
        t.free()
    us = ms * 1000.0 / steps
    u_mean = float(np.mean([uniq[(warmup + s) % nbatch] for s in range(steps)]))
    ub = u_mean * L.expert_bytes()
    nb = decode_bytes(cfg)
    other = nb["all"] - nb["routed"]
    return {"rows": 8, "forced_shared_experts": list(synth.C2_HOT), "batches": nbatch,
            "us_per_step": round(us, 3), "us_per_token": round(us / 8, 3),
            "unique_experts_mean": round(u_mean, 2), "unique_expert_bytes": int(ub),
            "unique_hbm_gbs": round(ub / (us * 1e-6) / 1e9, 1),
            "unique_hbm_frac": round(ub / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "all_hbm_frac": round((ub + other) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "ideal_us_at_peak": round(ub / HBM_PEAK_GBS / 1e3, 2)}, r2, xs


def bench_sparse(gpu, steps=40, seed=99):
    """The rest of a Flash-Next layer at the full model's shapes: QSA decode
    at 32K keys (stored-key scores over 8192 blocks, top-512 selection,
    attention of 24 query / 2 kv heads x 256 over the ~2K kept positions, gated)
    and its 2048-row prefill scoring; the gated DeltaNet's decode step (conv
    over 10240 channels, the delta rule over 48 value heads of 128x128 state)
    and its 2048-step prefill.  Layers cycle through NL copies of the caches
    and states (past the Infinity Cache) so every step reads HBM.  Times are
    device time (see timed())."""
    from qwasar_amd import synth
    B = gpu.Buf
    rng = np.random.default_rng(seed)
    f32 = lambda *sh: rng.standard_normal(sh).astype(np.float32)
    res = {}

    # ---- QSA decode at C keys
    C, ratio, nq, d, topk, qh, kvh, D = 32768, 4, 16, 128, 512, 24, 2, 256
    NL = 12
    nb = C // ratio
    cap = gpu.qw_qsa_list_cap(topk, ratio)
    c = gpu.qw_cmd_begin()
    layers = []
    for l in range(NL):
        pool, kc, vc = B(nb * d * 4), B(kvh * C * D * 2), B(kvh * C * D * 2)
        gpu.qw_op_synth(c, pool.ref(), synth.SYNTH_F32_BF16_NORMAL, nb * d, synth.sm_key(seed, f"pool{l}"), 1.0, 0.0)
        gpu.qw_op_synth(c, kc.ref(), synth.SYNTH_BF16_NORMAL, kvh * C * D, synth.sm_key(seed, f"kc{l}"), 0.5, 0.0)
        gpu.qw_op_synth(c, vc.ref(), synth.SYNTH_BF16_NORMAL, kvh * C * D, synth.sm_key(seed, f"vc{l}"), 0.5, 0.0)
        layers.append((pool, kc, vc))
    gpu.run(c, "qsa setup")
    # the caches hold bf16 patterns of N(0, 0.5): as fp16 bits they are finite
    # values of a similar spread (the kernel reads them as fp16)
    qn, q, gate = B.of(f32(1, nq, d)), B.of(f32(1, qh, D)), B.of(f32(1, qh, D))
    sc, mk, ls, out = B(nb * 4), B(C), B((1 + cap) * 4), B(qh * D * 4)

    def qsa_step(c, l):
        pool, kc, vc = layers[l % NL]
        gpu.qw_op_qsa_scores_pooled(c, sc.ref(), qn.ref(), pool.ref(), 1, nq, d, ratio, C - 1, nb)
        gpu.qw_op_qsa_select(c, mk.ref(), ls.ref(), sc.ref(), 1, ratio, C - 1, topk, C, nb)
        gpu.qw_op_attn_masked_gated(c, out.ref(), gate.ref(), q.ref(), kc.ref(), vc.ref(), ls.ref(), 1, qh, kvh, D, C,
                                    C - 1, 1.0 / 16.0, topk, ratio)

    blocker = B(1 << 30)

    def timed(label, fn, n):
        """Device ms per call of fn: the region starts after ~1 ms of other
        GPU work (writes to a 1 GiB buffer), during which the host queues every
        call, so host launch gaps stay outside the region."""
        c = gpu.qw_cmd_begin()
        for i in range(4):
            fn(c, i)
        gpu.run(c, label + " warm-up")
        gpu.qw_prof_reset()
        gpu.qw_prof_set_enabled(True)
        c = gpu.qw_cmd_begin()
        for _ in range(4):
            gpu.qw_op_synth(c, blocker.ref(), synth.SYNTH_U32, (1 << 30) // 4, 1, 0.0, 0.0)
        gpu.qw_cmd_mark(c, b"blocker")
        gpu.qw_prof_set_enabled(False)
        for i in range(n):
            fn(c, i)
        gpu.qw_prof_set_enabled(True)
        gpu.qw_cmd_mark(c, label.encode())
        gpu.run(c, label)
        ms = gpu.qw_prof_ms(label.encode(), None)
        gpu.qw_prof_set_enabled(False)
        gpu.qw_prof_reset()
        return ms / n

    ms = timed("qsa decode", qsa_step, steps)
    kept = topk * ratio + (C % ratio if C % ratio else 0)
    qbytes = (nb * d * 4 + nq * d * 4 + 2 * nb * 4 + C + (1 + cap) * 4
              + 2 * kvh * kept * D * 2 + 3 * qh * D * 4)
    res["qsa_decode"] = {"keys": C, "blocks": nb, "block_topk": topk, "q_heads": qh, "kv_heads": kvh,
                         "launches": 3, "us_per_token": round(ms * 1e3, 2), "bytes": qbytes,
                         "hbm_gbs": round(qbytes / (ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(qbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}

    # ---- QSA prefill scoring: 2048 rows at the end of the 32K context
    R = 2048
    qnR, scR = B.of(f32(R, nq, d)), B(R * nb * 4)

    def qsa_prefill(c, l):
        gpu.qw_op_qsa_scores_pooled(c, scR.ref(), qnR.ref(), layers[l % NL][0].ref(), R, nq, d, ratio, C - R, nb)

    ms = timed("qsa prefill scores", qsa_prefill, 10)
    fl = sum(2.0 * nq * d * ((C - R + r + 1) // ratio) for r in range(R))
    res["qsa_prefill_scores"] = {"rows": R, "keys": C, "ms": round(ms, 3),
                                 "tflops_fp32": round(fl / (ms * 1e-3) / 1e12, 2),
                                 "vs_fp32_peak": round(fl / (ms * 1e-3) / 1e12 / 157.3, 4)}
    for t in (qn, q, gate, sc, mk, ls, out, qnR, scR):
        t.free()
    for tt in layers:
        for t in tt:
            t.free()

    # ---- gated DeltaNet decode and prefill (48 value heads, 16 key heads, 128x128)
    hk, hv, dk, ch = 16, 48, 128, 10240
    NG = 96
    c = gpu.qw_cmd_begin()
    states = []
    for l in range(NG):
        st, cs, cs2 = B(hv * dk * dk * 4), B(3 * ch * 4), B(3 * ch * 4)
        gpu.qw_op_synth(c, st.ref(), synth.SYNTH_F32_BF16_NORMAL, hv * dk * dk, synth.sm_key(seed, f"S{l}"), 0.05, 0.0)
        gpu.qw_op_synth(c, cs.ref(), synth.SYNTH_F32_BF16_NORMAL, 3 * ch, synth.sm_key(seed, f"cs{l}"), 1.0, 0.0)
        states.append((st, cs, cs2))
    gpu.run(c, "gdn setup")
    cw = B.of(synth.to_bf16(0.3 * f32(ch, 4)))
    Al = B.of(synth.to_bf16(np.linspace(-0.5, 1.0, hv).astype(np.float32)))
    dt = B.of(synth.to_bf16(np.linspace(-0.2, 0.3, hv).astype(np.float32)))
    R = 2048
    xin, xmix = B.of(f32(R, ch)), B(R * ch * 4)
    ab, bb, yb = B.of(f32(R, hv)), B.of(f32(R, hv)), B(R * hv * dk * 4)
    prep = gpu.qw_gdn_prep(ab.ref(), bb.ref(), Al.ref(), dt.ref(), 1e-6 / dk, 1.0 / dk, 1.0 / np.sqrt(dk))

    def gdn(c, l, rows):
        st, cs, _ = states[l % NG]
        gpu.qw_op_conv1d_causal_silu(c, xmix.ref(), xin.ref(), cs.ref(), cw.ref(), ch, rows, 4, gpu.NULL_REF, 0, 0)
        # q, k, v: packed [rows, heads, 128] inputs of the recurrence
        gpu.qw_op_gated_delta_prep(c, yb.ref(), qkv[0].ref(), qkv[1].ref(), qkv[2].ref(), prep, st.ref(), hk, hv, dk,
                                   dk, rows, gpu.NULL_REF, 0, 0)

    qkv = (B.of(f32(R, hk, dk)), B.of(f32(R, hk, dk)), B.of(f32(R, hv, dk)))
    ms = timed("gdn decode", lambda c, l: gdn(c, l, 1), steps)
    gbytes = 2 * hv * dk * dk * 4 + 2 * 3 * ch * 4 + ch * 4 * 2 + ch * 4 * 2 + (2 * hk + hv) * dk * 4 + hv * dk * 4
    res["gdn_decode"] = {"hk": hk, "hv": hv, "dk": dk, "conv_channels": ch, "launches": 2,
                         "us_per_token": round(ms * 1e3, 2), "bytes": gbytes,
                         "hbm_gbs": round(gbytes / (ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(gbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    def gdn_one(c, l):
        # the one-launch step on the conv's own output channels; the layer's
        # two windows alternate
        st, cs, cs2 = states[l % NG]
        wi, wo = (cs, cs2) if (l // NG) % 2 == 0 else (cs2, cs)
        assert gpu.qw_op_gdn_decode(c, yb.ref(), xin.ref(), wi.ref(), wo.ref(), cw.ref(), prep, st.ref(), hk, hv, dk,
                                    dk)

    ms1 = timed("gdn decode one launch", gdn_one, steps)
    res["gdn_decode"]["one_launch_us_per_token"] = round(ms1 * 1e3, 2)
    ms = timed("gdn prefill", lambda c, l: gdn(c, l, R), 3)
    res["gdn_prefill"] = {"rows": R, "ms": round(ms, 3), "tokens_per_s": round(R / (ms * 1e-3), 1)}
    for t in (cw, Al, dt, xin, xmix, ab, bb, yb, blocker) + qkv:
        t.free()
    for tt in states:
        for t in tt:
            t.free()
    return res


def cpu_sample(L, x, seconds, rows_per_call):
    """Seconds per call of the oracle's moe_forward on `rows_per_call` rows of
    x at a time, over a bounded time; returns (seconds per call, calls)."""
    from oracle import ref
    n, t0 = 0, time.perf_counter()
    while (n == 0 or time.perf_counter() - t0 < seconds) and (n + 1) * rows_per_call <= x.shape[0]:
        ref.moe_forward(L, x[n * rows_per_call:(n + 1) * rows_per_call])
        n += 1
    return (time.perf_counter() - t0) / n, n


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-config2", action="store_true", help="skip config 2 (batch-8 decode)")
    ap.add_argument("--no-config4", action="store_true", help="skip the 48-layer stack (config 4)")
    ap.add_argument("--config4-only", action="store_true", help="run only the 48-layer stack and print it")
    ap.add_argument("--no-hc", action="store_true", help="skip the hyper-connection mixer")
    ap.add_argument("--no-sparse", action="store_true", help="skip QSA and the gated DeltaNet")
    ap.add_argument("--no-ceiling", action="store_true", help="skip the measured HBM read ceiling")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    from qwasar_amd import gpu, synth
    gpu.init()
    cfg = dict(synth.CONFIGS[1])
    seed = 1234
    L = synth.make_layer(seed, **{k: cfg[k] for k in ("H", "E", "K", "I", "SI", "group")})
    lb = gpu.LayerBufs(L)
    cand = synth.make_x(seed, 2048, L.H, name="bench.candidates")
    xpool, pool_ids = select_cold_pool(gpu, lb, cand, L.K)

    nb = decode_bytes(cfg)
    # the K timed steps, HIP events at the region's ends only: the value
    dec = time_decode(gpu, lb, xpool, args.steps, args.warmup, "region")
    us_mean = dec["region"] * 1000.0 / args.steps
    # the same count of steps with an event after each, for their median and
    # spread (each event adds a gap of its own to its step)
    per = time_decode(gpu, lb, xpool, args.steps, 0, "steps")["per_step"] * 1000.0
    # the same steps with events around every launch: the decode kernel's own duration
    brk = time_decode(gpu, lb, xpool, args.steps, 0, "kernels")
    k_us = brk["fused"] * 1000.0 / args.steps
    roof_gbs = nb["all"] / (k_us * 1e-6) / 1e9
    prof_us = profiled_kernel_us("k_decode1")
    ceiling = None if args.no_ceiling else hbm_ceiling(gpu, lb)

    out = {
        "metric": "moe_layer_decode_us_per_token",
        "value": round(us_mean, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_mean / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 x f16 (pow2-scaled 16-element units) -> fp32 acc",
        "data": "synthetic (seeded MLX-affine 4-bit weights, N(0,1) bf16 tokens)",
        "config": {"workload": "BASELINE config 1: Flash-Next-shaped MoE layer decode, batch 1",
                   "H": cfg["H"], "E": cfg["E"], "K": cfg["K"], "I": cfg["I"], "SI": cfg["SI"],
                   "group": cfg["group"], "tokens_per_step": 1, "token_pool": POOL,
                   "cold_window": COLD_WINDOW},
        "decode": {
            "us_per_token": round(us_mean, 3),
            "evented_steps": {"n": int(per.size), "median_us": round(float(np.median(per)), 3),
                              "p10_us": round(float(np.percentile(per, 10)), 3),
                              "p90_us": round(float(np.percentile(per, 90)), 3),
                              "note": "an event after every step; each adds its own gap"},
            "routed_bytes": nb["routed"], "all_bytes": nb["all"],
            "routed_hbm_gbs": round(nb["routed"] / (us_mean * 1e-6) / 1e9, 1),
            "routed_hbm_frac": round(nb["routed"] / (us_mean * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "all_hbm_gbs": round(nb["all"] / (us_mean * 1e-6) / 1e9, 1),
            "kernel_us": round(k_us, 3),
        },
        "roofline": {"bound": "hbm", "kernel": "k_decode1", "achieved": round(roof_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(roof_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("k_decode1"),
                     "algorithmic_bytes": nb["all"],
                     "kernel_us_live": round(k_us, 3),
                     "kernel_us_profile": prof_us,
                     "frac_from_profile": (round(nb["all"] / (prof_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                                           if prof_us else None),
                     "measured_ceiling": ceiling},
    }

    c2, c2_router, c2_x = None, None, None
    if not args.no_config2:
        c2, c2_router, c2_x = bench_config2(gpu, lb, L, cfg, seed, args.steps, args.warmup)
        out["config2"] = c2
    x3, r3 = None, None
    if not args.no_prefill:
        pf = {}
        zb = synth.zipf_bias(seed, L.E)
        r3 = synth.make_router(seed, L.E, L.H, zb)
        rb3 = gpu.Buf(wrap=r3)
        d3 = gpu.qw_moe_layer.from_buffer_copy(lb.desc)
        d3.router = rb3.ref()

        class _LB3:
            pass
        lb3 = _LB3()
        lb3.L, lb3.desc = L, d3
        for name, rows, lbx, const0 in (("config3_zipf_512", 512, lb3, True),
                                        ("chunk_2048_uniform", 2048, lb, False),
                                        ("chunk_256_uniform", 256, lb, False),
                                        ("chunk_1024_uniform", 1024, lb, False)):
            x = synth.make_x(seed + rows, rows, L.H, name=f"bench.prefill{rows}", const_col0=const0)
            if rows == 512:
                x3 = x
            ms, hot, touched = time_prefill(gpu, lbx, x, reps=5)
            fl = prefill_flops(cfg, rows)
            pf[name] = {"rows": rows, "ms": round(ms, 3), "tokens_per_s": round(rows / (ms * 1e-3), 1),
                        "useful_tflops": round(fl / (ms * 1e-3) / 1e12, 2),
                        "mfma_util": round(fl / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                        "weight_read_floor_ms": round(L.weight_bytes() / HBM_PEAK_GBS / 1e6, 3),
                        "hottest_expert_pairs": hot, "experts_touched": touched}
        rb3.free()
        # flat numbers first (the 2048-token chunk, config 4's per-layer step), then config 3
        ch, z = pf["chunk_2048_uniform"], pf["config3_zipf_512"]
        flat = {"workload": "2048-token prefill chunk of one config-1-shaped layer (config 4's per-layer step)",
                "rows": ch["rows"], "ms": ch["ms"], "tokens_per_s": ch["tokens_per_s"],
                "useful_tflops": ch["useful_tflops"], "mfma_util": ch["mfma_util"],
                "weight_read_floor_ms": ch["weight_read_floor_ms"],
                "hbm_frac_of_weight_floor": round(ch["weight_read_floor_ms"] / ch["ms"], 4),
                "config3_rows": z["rows"], "config3_ms": z["ms"], "config3_tokens_per_s": z["tokens_per_s"],
                "config3_mfma_util": z["mfma_util"], "config3_hottest_expert_pairs": z["hottest_expert_pairs"],
                "config3_experts_touched": z["experts_touched"],
                # the grouped layer at the chunk sizes the reference's own grouped-experts
                # figures are quoted at (256, 1024, 2048 rows; uniform routing)
                "chunk_sweep": {str(pf[k]["rows"]): {"ms": pf[k]["ms"], "tokens_per_s": pf[k]["tokens_per_s"],
                                                     "mfma_util": pf[k]["mfma_util"]}
                                for k in ("chunk_256_uniform", "chunk_1024_uniform", "chunk_2048_uniform")}}
        pf = flat
        out["prefill"] = pf

    if not args.no_config4:
        out["config4"] = bench_stack(gpu, 48, 2048, 256, 4, cpu_seconds=0.0 if args.no_cpu else 3.0)
    if not args.no_hc:
        out["hc_mixer"] = bench_hc(gpu, 200)
    if not args.no_sparse:
        out["sparse"] = bench_sparse(gpu)

    if not args.no_cpu:
        # the oracle (scalar C, one thread) on bounded samples of the same
        # workloads: config 1 (the headline's tokens), config 0, config 2 (the
        # first timed batches), config 3 (its first tokens) and config 4 (layer
        # 0 of the stack, scaled by its 48 layers)
        import dataclasses
        s1, n1 = cpu_sample(L, xpool, args.cpu_seconds, 1)
        by = {}
        L0, x0 = synth.make_config(0, rows=64)
        s0, n0 = cpu_sample(L0, x0, 1.0, 1)
        by["config0"] = {"us_per_token": round(s0 * 1e6, 1), "sample": f"{n0} tokens"}
        if c2 is not None:
            L2 = dataclasses.replace(L, router=c2_router)
            s2, n2 = cpu_sample(L2, c2_x, 3.0, 8)
            by["config2"] = {"us_per_step": round(s2 * 1e6, 1), "us_per_token": round(s2 * 1e6 / 8, 1),
                             "sample": f"{n2} batches of 8 tokens"}
        if x3 is not None:
            L3 = dataclasses.replace(L, router=r3)
            s3, n3 = cpu_sample(L3, x3, 3.0, 8)
            by["config3"] = {"tokens_per_s": round(8 / s3, 2), "sample": f"the first {8 * n3} of its 512 tokens"}
        if out.get("config4", {}).get("cpu"):
            by["config4"] = out["config4"]["cpu"]
        out["cpu_baseline"] = {"value": round(s1 * 1e6, 1), "unit": "us/token", "cores": 1, "kind": "port",
                               "sample": f"{n1} decode tokens of config 1 through oracle/moe_ref.c "
                                         "(scalar C, -O2, one thread), same weights and tokens",
                               "by_config": by}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
