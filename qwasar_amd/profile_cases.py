"""Single workloads for profiling under rocprofv3 (the kernel tables and
counter passes kept as summaries beside the benchmark).  Each case sets up
what bench.py sets up for it and runs only that, so a profile holds nothing
else of note:

    python3 -m qwasar_amd.profile_cases decode STEPS     config 1 decode, STEPS tokens (cold pool) after 20 warm-up
    python3 -m qwasar_amd.profile_cases prefill ROWS     one layer's prefill of ROWS uniform-routed rows, 5 passes
    python3 -m qwasar_amd.profile_cases config2 STEPS    config 2 (batch-8 decode), STEPS steps
    python3 -m qwasar_amd.profile_cases config4          the 48-layer stack (prefill 2048 rows, 256 decode steps)
    python3 -m qwasar_amd.profile_cases hc               the hyper-connection mixer
    python3 -m qwasar_amd.profile_cases sparse           QSA and the gated DeltaNet
    python3 -m qwasar_amd.profile_cases ceiling          the HBM read ceiling (stream and ten cold experts)
    python3 -m qwasar_amd.profile_cases copy BYTES       a plain device copy of BYTES: the scale for
                                                         FETCH_SIZE / WRITE_SIZE counters
"""
from __future__ import annotations

import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def _copy(nbytes: int) -> None:
    """torch's device-to-device copy of a buffer filled beforehand: a kernel
    of known traffic (nbytes read, nbytes written a pass)."""
    import torch
    a = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes}), flush=True)


def main(argv) -> None:
    if not argv:
        print(__doc__, file=sys.stderr)
        sys.exit(2)
    case, arg = argv[0], (int(argv[1]) if len(argv) > 1 else 0)
    if case == "copy":
        _copy(arg or (256 << 20))
        return
    import bench
    from qwasar_amd import gpu, synth
    gpu.init()
    cfg = dict(synth.CONFIGS[1])
    seed = 1234
    if case == "hc":
        print(json.dumps({"hc_mixer": bench.bench_hc(gpu, 200)}), flush=True)
        return
    if case == "sparse":
        print(json.dumps({"sparse": bench.bench_sparse(gpu)}), flush=True)
        return
    if case == "config4":
        print(json.dumps({"config4": bench.bench_stack(gpu, 48, 2048, 256, 4)}), flush=True)
        return
    L = synth.make_layer(seed, **{k: cfg[k] for k in ("H", "E", "K", "I", "SI", "group")})
    lb = gpu.LayerBufs(L)
    if case == "ceiling":
        print(json.dumps({"ceiling": bench.hbm_ceiling(gpu, lb)}), flush=True)
        return
    if case == "prefill":
        rows = arg or 2048
        x = synth.make_x(seed + rows, rows, L.H, name=f"bench.prefill{rows}")
        ms, _, _ = bench.time_prefill(gpu, lb, x, reps=5)
        print(json.dumps({"prefill_rows": rows, "ms": round(ms, 3)}), flush=True)
        return
    if case == "config2":
        c2, _, _ = bench.bench_config2(gpu, lb, L, cfg, seed, arg or 50, 5)
        print(json.dumps({"config2": c2}), flush=True)
        return
    if case == "decode":
        cand = synth.make_x(seed, 2048, L.H, name="bench.candidates")
        xpool, _ = bench.select_cold_pool(gpu, lb, cand, L.K)
        r = bench.time_decode(gpu, lb, xpool, arg or 200, 20, "region")   # (as bench.py: warm-up steps first)
        print(json.dumps({"decode_steps": arg or 200, "us_per_token": round(r["region"] * 1e3 / (arg or 200), 3)}),
              flush=True)
        return
    print(f"unknown case {case!r}\n{__doc__}", file=sys.stderr)
    sys.exit(2)


if __name__ == "__main__":
    main(sys.argv[1:])
