"""One-GPU benchmark of the DSALT sparse-attention hot path on MI355X.

A step is one pass of the operator over the workload's synthetic batch, with every input
resident in HBM: landmark selection, forward, and (for the training workloads) backward.
Prints one JSON line (see --help for the options).  Default workload: B=1, H=16, L=32768,
head_dim 64, bf16, w_max 512, k=128 global landmarks, forward + backward.

  python bench.py [--gpus 1] [--steps 30] [--warmup 5] [--workload NAME] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

METRIC = "DSALT attn fwd+bwd tokens/sec @L=32K bf16 (1 GPU); % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}  # dense
HERE = os.path.dirname(os.path.abspath(__file__))


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="fwdbwd_bf16_h16_l32768")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


def kernel_model(wl, T, H, D, hidden, pairs, e):
    """Algorithmic bytes and flops per launch of each kernel (no recompute, no workspace)."""
    thd = T * H * D * e
    th4 = 4 * T * H
    return {
        "sel_norms": dict(bytes=T * hidden * e + thd, flops=0),
        "attn_fwd": dict(bytes=4 * thd + th4, flops=4 * D * pairs),
        "bwd_dq": dict(bytes=6 * thd + 2 * th4, flops=4 * D * pairs),
        "bwd_dkdv": dict(bytes=6 * thd + 2 * th4, flops=4 * D * pairs),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the operator shards over "
              "(batch, head) with no communication, so run one process per GPU.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from dsalt_amd import _lib, ops
    from dsalt_amd.workloads import WORKLOADS, generate

    wl = WORKLOADS[args.workload]
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    x_cpu = generate(wl)
    x = {k: v.to(dev) for k, v in x_cpu.items()}
    T, H, D = x["q"].shape
    mode = ops.SELECT_GLOBAL if wl.select_mode == "global" else ops.SELECT_BLOCK
    scope = ops.STATS_SEQUENCE
    maxlen = wl.seqlen
    e = x["q"].element_size()

    def step():
        idx = ops.select_landmarks(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, max_seqlen=maxlen,
                                   select_mode=mode, block_size=wl.block_size, stats_scope=scope)
        out, lse = ops.attention_forward(x["q"], x["k"], x["v"], x["w"], x["cu"], idx, None, max_seqlen=maxlen,
                                         select_mode=mode, block_size=wl.block_size)
        if wl.backward:
            ops.attention_backward(x["dout"], x["q"], x["k"], x["v"], out, lse, x["w"], x["cu"], idx, None,
                                   max_seqlen=maxlen, want_dbias=False)
        return idx

    for _ in range(args.warmup):
        idx = step()
    torch.cuda.synchronize()

    # exact number of attended (query, key) pairs: window + visible landmarks
    wv = x["w"].long().clamp(min=1)
    pos = torch.arange(T, device=dev) - x["cu"].long().repeat_interleave(maxlen)[:T]
    band = torch.minimum(wv, pos + 1)
    lo = (pos - wv + 1).clamp(min=0)
    pairs = 0
    for h in range(H):
        for s in range(x["cu"].numel() - 1):
            sl = slice(s * maxlen, (s + 1) * maxlen)
            if mode == ops.SELECT_GLOBAL:
                lm = idx[h, s, 0]
                lm = lm[lm >= 0].long()
                cnt = torch.searchsorted(lm, lo[sl])
            else:
                rows = torch.arange(maxlen, device=dev)
                sets = idx[h, s].long()
                cnt = ((sets[rows // wl.block_size] >= 0) & (sets[rows // wl.block_size] < lo[sl, None])).sum(1)
            pairs += int(band[sl].sum() + cnt.sum())

    # timed region: plain steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = 1e3 * elapsed / args.steps

    # timed region with per-kernel HIP events on the launch stream
    lib.dsalt_timing_enable(1)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_step_inst = 1e3 * (time.perf_counter() - t1) / args.steps
    buf = __import__("ctypes").create_string_buffer(1 << 16)
    lib.dsalt_timing_report(buf, len(buf))
    lib.dsalt_timing_enable(0)
    kernels = {}
    for line in buf.value.decode().splitlines():
        name, n, tot = line.split()
        kernels[name] = dict(launches=int(n), avg_ms=float(tot) / int(n), ms_per_step=float(tot) / args.steps)

    model = kernel_model(wl, T, H, D, wl.hidden, pairs, e)
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"])
    roof = None
    if dom in model:
        avg_s = kernels[dom]["avg_ms"] * 1e-3
        ach = model[dom]["bytes"] / avg_s / 1e9
        traffic = None
        tpath = os.path.join(HERE, "profiles", f"traffic_{wl.name}.json")
        if os.path.exists(tpath):
            with open(tpath) as f:
                traffic = json.load(f).get(dom)
        roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                "algorithmic_bytes": model[dom]["bytes"],
                "mfma_tflops": round(model[dom]["flops"] / avg_s / 1e12, 2) if model[dom]["flops"] else None}

    dtn = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[x["q"].dtype]
    # unique algorithmic traffic of a step: q, k, v, o (+ h for the selection) and the LSE in
    # the forward; q, k, v, o, dO, dq, dk, dv and the LSE in the backward
    thd = T * H * D * e
    step_bytes = 4 * thd + T * wl.hidden * e + 4 * T * H
    if wl.backward:
        step_bytes += 8 * thd + 4 * T * H
    step_flops = (4 + (8 if wl.backward else 0)) * D * pairs
    t_roof = max(step_bytes / (HBM_PEAK_GBS * 1e9), step_flops / (MFMA_PEAK_TFLOPS[dtn] * 1e12))

    cpu = None
    if not args.no_cpu_baseline:
        from oracle.sdpa_cpu import time_baseline
        r = time_baseline(x_cpu, wl.k_lmk, scope, backward=wl.backward)
        cpu = {"value": round(r["tokens_per_s"], 2), "unit": "tokens/s", "cores": r["threads"], "kind": "port",
               "sample": (f"full-length landmark selection (C oracle, 1 thread, {r['t_select']:.2f}s) + reference "
                          f"masked-SDPA {'fwd+bwd' if wl.backward else 'fwd'} on the last {r['rows']} query rows x "
                          f"{H} heads x all {T} keys ({r['t_attention']:.2f}s, torch CPU, {r['threads']} threads, "
                          f"host cpu_count {r['cpu_count']})")}

    line = {
        "metric": METRIC,
        "value": round(T * args.steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtn,
        "data": "synthetic",
        "config": {"workload": wl.name, "batch": wl.batch, "heads": H, "seq_len": wl.seqlen, "head_dim": D,
                   "hidden": wl.hidden, "w_max": wl.w_max, "k_lmk": wl.k_lmk, "select": wl.select_mode,
                   "backward": wl.backward, "pairs": pairs},
        "roofline": roof,
        "step_roofline": {"bound": "hbm" if step_bytes / HBM_PEAK_GBS >= step_flops / (MFMA_PEAK_TFLOPS[dtn] * 1e3)
                          else "mfma", "t_roof_ms": round(t_roof * 1e3, 4),
                          "frac": round(t_roof * 1e3 / ms_step, 4), "algorithmic_bytes": step_bytes,
                          "flops": step_flops},
        "cpu_baseline": cpu,
        "kernels": {k: {kk: round(vv, 5) if isinstance(vv, float) else vv for kk, vv in v.items()}
                    for k, v in sorted(kernels.items())},
        "ms_per_step_with_kernel_events": round(ms_step_inst, 4),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
