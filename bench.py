"""One-GPU benchmark of the DSALT sparse-attention hot path on MI355X.

A step is one pass of the operator over the workload's synthetic batch, with every input
resident in HBM: landmark selection, forward, and (for the training workloads) backward.
Prints one JSON line (see --help for the options).  Default workload: B=1, H=16, L=32768,
head_dim 64, bf16, w_max 512, k=128 global landmarks, forward + backward.

  python bench.py [--gpus 1] [--steps 30] [--warmup 5] [--workload NAME] [--no-cpu-baseline]

HBM traffic per launch comes from rocprofv3 counter runs, each in a process of its own:
  rocprofv3 --pmc FETCH_SIZE -d P/fetch -o run --output-format csv -- python bench.py --steps 2 --warmup 1 --no-cpu-baseline
  rocprofv3 --pmc WRITE_SIZE -d P/write ...     (same program)
  rocprofv3 --pmc FETCH_SIZE -d P/copy_fetch -o run --output-format csv -- python bench.py --copy-calibration 1024
  rocprofv3 --pmc WRITE_SIZE -d P/copy_write ...  (same program)
  python bench.py --traffic-from P     # writes profiles/traffic_<workload>.json
The copy runs give the factor between each counter's reading and the bytes a plain copy of
known size must move; the kernels' readings are scaled by it.
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


def kernel_source_sha() -> str:
    """Hash of the HIP sources and the C header: a traffic record measured on other sources is stale."""
    import hashlib
    hs = hashlib.sha256()
    for d in (os.path.join(HERE, "dsalt_amd", "csrc"), os.path.join(HERE, "include")):
        for fn in sorted(os.listdir(d)):
            with open(os.path.join(d, fn), "rb") as f:
                hs.update(fn.encode() + b"\0" + f.read())
    return hs.hexdigest()[:16]


def cpu_model() -> str:
    """The host CPU's model name (lscpu "Model name", read from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="fwdbwd_bf16_h16_l32768")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seqlen", type=int, default=0, metavar="L",
                    help="run the operator workload with sequences of L tokens instead of its own length "
                         "(the line then carries no traffic record, which is measured at the workload's length)")
    ap.add_argument("--batch", type=int, default=0, metavar="B",
                    help="run the operator workload with B sequences instead of its own batch (no traffic record "
                         "on the line either)")
    ap.add_argument("--variant", default="auto",
                    help="tile variant bits (DSALT_VARIANT_*) of the attention kernels, or 'auto': the autotune's "
                         "winner for the workload's shape (timed before the warmup, outside the timed region)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only copy (negate) a MIB-MiB device buffer five times (HBM counter calibration) and exit")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="summarise rocprofv3 --pmc output under DIR/{fetch,write,copy_fetch,copy_write} into "
                         "profiles/traffic_<workload>.json and exit (no GPU needed)")
    ap.add_argument("--pmc-summary", metavar="DIR",
                    help="print per-kernel means of every counter found under DIR and exit (no GPU needed)")
    ap.add_argument("--kernel-stats", metavar="DIR",
                    help="print the kernel table of a rocprofv3 --kernel-trace --stats run under DIR and exit")
    return ap.parse_args()


LABELS = ("sel_norms", "sel_sums", "sel_stats", "sel_z", "sel_scores", "sel_part", "sel_merge", "sel_prune_hist",
          "sel_prune_prefix", "sel_prune_mark", "sel_prune_list", "sel_topk", "gather",
          "row_plan", "attn_fwd", "bwd_prep", "bwd_dq", "bwd_dkdv", "bwd_lmk", "bwd_lmk_sum", "train_windows", "train_dw",
          "rope", "silu_mul", "probs", "ce_rows")


def short_kernel_name(name: str) -> str:
    """Label of a library kernel (the one dsalt_timing_report uses) from a profiler kernel name."""
    import re
    # the label must start the identifier (a mangled length prefix, "::" or the start): no
    # match inside library names such as reduce_kernel or vectorized_gather_kernel
    m = re.search(r"(?<![A-Za-z_])(sel_norms|sel_sums|sel_stats|sel_z|sel_scores|sel_part|sel_merge|sel_prune_hist|"
                  r"sel_prune_prefix|sel_prune_mark|sel_prune_list|sel_topk|gather|row_plan|fwd|bwd_prep|bwd_dq|"
                  r"bwd_dkdv|bwd_lmk_sum|train_windows|train_dw|rope|silu_mul|probs|ce|"
                  r"bwd_lmk)_kernel", name)
    if not m:
        return name
    return {"fwd": "attn_fwd", "ce": "ce_rows"}.get(m.group(1), m.group(1))


def read_pmc(root: str) -> dict:
    """{kernel label: {counter: mean value per dispatch}} over every counter_collection.csv under root."""
    import csv
    acc = {}
    for dirpath, _, files in os.walk(root):
        for fn in files:
            if not fn.endswith("counter_collection.csv"):
                continue
            with open(os.path.join(dirpath, fn), newline="") as f:
                for row in csv.DictReader(f):
                    k = short_kernel_name(row["Kernel_Name"])
                    key = (row["Counter_Name"], row.get("Dispatch_Id", ""))
                    d = acc.setdefault(k, {})
                    d[key] = d.get(key, 0.0) + float(row["Counter_Value"])
    out = {}
    for k, d in acc.items():
        per = {}
        for (cname, _), v in d.items():
            per.setdefault(cname, []).append(v)
        out[k] = {c: sum(v) / len(v) for c, v in per.items()}
        out[k]["dispatches"] = max(len(v) for v in per.values())
    return out


def traffic_from(root: str, wl_name: str, copy_mib: int = 1024, variant: str = "auto") -> dict:
    """HBM bytes per launch of each kernel: FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled by
    the ratio of a plain copy's known bytes to that counter's reading for the copy."""
    known = copy_mib * 2**20

    def copy_reading(sub, counter):
        d = read_pmc(os.path.join(root, sub))
        best = max(d.values(), key=lambda c: c.get(counter, 0.0))
        return best[counter] * 1024.0

    f_fac = known / copy_reading("copy_fetch", "FETCH_SIZE")
    w_fac = known / copy_reading("copy_write", "WRITE_SIZE")
    fetch = read_pmc(os.path.join(root, "fetch"))
    write = read_pmc(os.path.join(root, "write"))
    b = f"python -u bench.py --workload {wl_name} --steps 2 --warmup 1 --no-cpu-baseline"
    if variant != "auto":  # the tiling the counted runs used
        b += f" --variant {variant}"
    res = {"_commands": [f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d <out>/fetch -o run -- {b}",
                         f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d <out>/write -o run -- {b}",
                         f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d <out>/copy_fetch -o run -- "
                         f"python -u bench.py --copy-calibration {copy_mib}",
                         f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d <out>/copy_write -o run -- "
                         f"python -u bench.py --copy-calibration {copy_mib}",
                         f"python bench.py --traffic-from <out> --workload {wl_name}"
                         + (f" --variant {variant}" if variant != "auto" else "")],
           "_calibration": {"copy_bytes": known, "fetch_factor": f_fac, "write_factor": w_fac},
           "_sources": kernel_source_sha()}
    for k in sorted(set(fetch) & set(write) & set(LABELS)):
        fb = fetch[k]["FETCH_SIZE"] * 1024.0 * f_fac
        wb = write[k]["WRITE_SIZE"] * 1024.0 * w_fac
        res[k] = {"fetch_bytes": round(fb), "write_bytes": round(wb), "bytes": round(fb + wb)}
    path = os.path.join(HERE, "profiles", f"traffic_{wl_name}.json")
    with open(path, "w") as f:
        json.dump(res, f, indent=1)
    return res


def kernel_model(wl, T, H, D, hidden, pairs, e, G=None):
    """Algorithmic bytes and flops per launch of each kernel (no recompute, no workspace);
    K and V (and dK, dV) count their own G heads when they are read unexpanded."""
    G = G or H
    thd = T * H * D * e
    tgd = T * G * D * e
    th4 = 4 * T * H
    tr = th4 if wl.train else 0  # training variant: per-head window gradients written by bwd_dq
    return {
        "sel_norms": dict(bytes=T * hidden * e + tgd, flops=0),
        "attn_fwd": dict(bytes=2 * thd + 2 * tgd + th4, flops=4 * D * pairs),
        "bwd_dq": dict(bytes=4 * thd + 2 * tgd + 2 * th4 + tr, flops=4 * D * pairs),
        "bwd_dkdv": dict(bytes=2 * thd + 4 * tgd + 2 * th4, flops=4 * D * pairs),
    }


def probs_bench(args, wl):
    """Export of one sequence's attention probabilities (window band + landmark slots) after
    a forward of the workload: a step is one dsalt_export_probs call over the whole
    sequence, every head (the forward runs once, untimed)."""
    import ctypes

    import torch

    from dsalt_amd import _lib, ops
    from dsalt_amd.workloads import generate

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    x = {k: v.to(dev) for k, v in generate(wl).items()}
    T, H, D = x["q"].shape
    L = wl.seqlen
    idx = ops.select_landmarks(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, max_seqlen=L,
                               stats_scope=ops.STATS_SEQUENCE)
    _, lse = ops.attention_forward(x["q"], x["k"], x["v"], x["w"], x["cu"], idx, None, max_seqlen=L)
    w_cap = wl.w_max

    def step():
        return ops.export_probs(x["q"], x["k"], x["w"], x["cu"], idx, lse, seq=0, rows=L, w_cap=w_cap, max_seqlen=L,
                                seq_len=L)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    lib.dsalt_timing_enable(1)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    buf = ctypes.create_string_buffer(1 << 14)
    lib.dsalt_timing_report(buf, len(buf))
    lib.dsalt_timing_enable(0)
    kernels = {}
    for line in buf.value.decode().splitlines():
        name, n, tot = line.split()
        kernels[name] = dict(launches=int(n), avg_ms=float(tot) / int(n))
    e = x["q"].element_size()
    alg = H * L * (w_cap + wl.k_lmk) * 4 + 2 * L * H * D * e + 8 * L * H  # outputs + q, k + w, lse
    avg = kernels["probs"]["avg_ms"] * 1e-3
    ach = alg / avg / 1e9
    line = {"metric": "attention-probability export rows/sec @L=32K (window band + landmark slots, all heads)",
            "value": round(L * args.steps / elapsed, 1), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(1e3 * elapsed / args.steps, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32 out / bf16 in", "data": "synthetic",
            "config": {"workload": "probs_" + wl.name, "heads": H, "seq_len": L, "head_dim": D, "w_cap": w_cap,
                       "k_lmk": wl.k_lmk, "dense_bytes_avoided": H * L * L * 4},
            "roofline": {"bound": "hbm", "kernel": "probs", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None, "algorithmic_bytes": alg},
            "cpu_baseline": None,
            "kernels": {k: {kk: round(vv, 5) if isinstance(vv, float) else vv for kk, vv in v.items()}
                        for k, v in kernels.items()}}
    print(json.dumps(line), flush=True)


def ce_bench(args):
    """LM-head loss of the Qwen2.5-3B shape: hidden states [32768, 2048] bf16, vocabulary
    151936, tied weight; a step is loss + gradients (input and weight) by the fused linear
    cross-entropy.  The reference's default path (torch logits per 2048-row chunk +
    F.cross_entropy, autograd backward) is timed beside it on the same GPU."""
    import ctypes

    import torch

    from dsalt_amd import _lib
    from dsalt_amd.kernels.cross_entropy import LigerFusedLinearCrossEntropyFunction
    from dsalt_amd.model.dsalt_lm import _chunked_cross_entropy

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    BT, H, V = 32768, 2048, 151936
    g = torch.Generator(device="cpu").manual_seed(3000)
    x = (torch.randn(BT, H, generator=g) * 0.5).to(torch.bfloat16).to(dev).requires_grad_(True)
    w = (torch.randn(V, H, generator=g) * 0.02).to(torch.bfloat16).to(dev).requires_grad_(True)
    t = torch.randint(0, V, (BT,), generator=g).to(dev)

    def fused():
        x.grad = w.grad = None
        LigerFusedLinearCrossEntropyFunction.apply(x, w, t)[0].backward()

    def chunked():
        x.grad = w.grad = None
        _chunked_cross_entropy(x, w, t, 2048).backward()

    def timed(fn, n):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n

    t_fused = timed(fused, args.steps)
    t_ref = timed(chunked, max(1, args.steps // 2))
    lib.dsalt_timing_enable(1)
    for _ in range(args.steps):
        fused()
    torch.cuda.synchronize()
    buf = ctypes.create_string_buffer(1 << 14)
    lib.dsalt_timing_report(buf, len(buf))
    lib.dsalt_timing_enable(0)
    kernels = {}
    for line in buf.value.decode().splitlines():
        name, n, tot = line.split()
        kernels[name] = dict(launches=int(n), avg_ms=float(tot) / int(n), ms_per_step=float(tot) / args.steps)
    ce = kernels["ce_rows"]
    rows_per_launch = BT / (ce["launches"] / args.steps)
    alg = rows_per_launch * V * 2 * 2 + rows_per_launch * 16  # logits read, gradient written, targets/loss
    ach = alg / (ce["avg_ms"] * 1e-3) / 1e9
    flops = 6.0 * BT * H * V
    line = {"metric": "fused linear cross-entropy tokens/sec (loss + input and weight gradients), V=151936 bf16",
            "value": round(BT / t_fused, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(t_fused * 1e3, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "ce_qwen3b_l32768", "rows": BT, "hidden": H, "vocab": V},
            "roofline": {"bound": "hbm", "kernel": "ce_rows", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None, "algorithmic_bytes": alg},
            "step_roofline": {"bound": "mfma", "flops": flops, "t_roof_ms": round(flops / 2.5e15 * 1e3, 3),
                              "frac": round(flops / 2.5e15 / t_fused, 4)},
            "torch_chunked_same_gpu": {"ms_per_step": round(t_ref * 1e3, 3), "tokens_per_s": round(BT / t_ref, 1)},
            "cpu_baseline": None,
            "kernels": {k: {kk: round(vv, 5) if isinstance(vv, float) else vv for kk, vv in v.items()}
                        for k, v in kernels.items()}}
    print(json.dumps(line), flush=True)


def model_bench(args, wl):
    """Whole-model prefill: a step is one forward of the decoder over B x L random token ids
    (embedding, every layer, final norm and the LM head over all positions, as the
    reference's forward without labels), weights random-init in bf16, no autograd."""
    import ctypes

    import torch

    from dsalt_amd import _lib
    from dsalt_amd.model import DSALTLMHeadModel

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfg = wl.config()
    torch.manual_seed(wl.seed)
    with torch.device(dev):  # parameters initialised on the GPU; the RoPE tables follow with .to
        model = DSALTLMHeadModel.from_config(cfg).to(dev, wl.dtype).eval()
    T = wl.batch * wl.seqlen
    g = torch.Generator(device="cpu").manual_seed(wl.seed)
    ids = torch.randint(0, cfg.vocab_size, (T,), generator=g).to(dev)
    cu = torch.arange(0, T + 1, wl.seqlen, dtype=torch.int32, device=dev)

    def step():
        with torch.no_grad():
            return model(ids, cu_seqlens=cu, max_seqlen=wl.seqlen)["logits"]

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = 1e3 * elapsed / args.steps

    # second timed pass: library kernels by HIP events, and the gate/up GEMM of every FFN by
    # torch events on the stream it runs on
    ffns = [layer.ffn for layer in model.layers]
    for f in ffns:
        f.gemm_events = []
    lib.dsalt_timing_enable(1)
    torch.cuda.synchronize()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    buf = ctypes.create_string_buffer(1 << 16)
    lib.dsalt_timing_report(buf, len(buf))
    lib.dsalt_timing_enable(0)
    kernels = {}
    for line in buf.value.decode().splitlines():
        name, n, tot = line.split()
        kernels[name] = dict(launches=int(n), avg_ms=float(tot) / int(n), ms_per_step=float(tot) / args.steps)
    gemm_ms = [a.elapsed_time(b) for f in ffns for a, b in f.gemm_events]
    for f in ffns:
        f.gemm_events = None
    d, dff, V = cfg.d_model, cfg.d_ff, cfg.vocab_size
    gu_flops = 2.0 * T * d * 2 * dff
    gemm_avg = sum(gemm_ms) / len(gemm_ms)
    kernels["ffn_gate_up_gemm"] = dict(launches=len(gemm_ms), avg_ms=gemm_avg, ms_per_step=sum(gemm_ms) / args.steps)
    ach = gu_flops / (gemm_avg * 1e-3) / 1e12
    roof = {"bound": "mfma", "kernel": "ffn_gate_up_gemm (hipBLASLt via torch)", "achieved": round(ach, 1),
            "peak": MFMA_PEAK_TFLOPS["bf16"], "unit": "TFLOP/s", "frac": round(ach / MFMA_PEAK_TFLOPS["bf16"], 4),
            "traffic": None, "algorithmic_flops": gu_flops}
    kvd = cfg.n_kv_heads * (d // cfg.n_heads)
    linear_params = cfg.n_layers * (2 * d * d + 2 * d * kvd + 3 * d * dff + d * kvd) + d * V
    step_flops = 2.0 * T * linear_params
    t_roof = step_flops / (MFMA_PEAK_TFLOPS["bf16"] * 1e12)
    line = {
        "metric": "DSALT decoder prefill tokens/sec @L=32K bf16 (1 GPU)",
        "value": round(T * args.steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random token ids, random-init weights)",
        "config": {"workload": wl.name, "batch": wl.batch, "seq_len": wl.seqlen, "layers": cfg.n_layers,
                   "hidden": d, "heads": cfg.n_heads, "kv_heads": cfg.n_kv_heads, "d_ff": dff, "vocab": V,
                   "w_max": cfg.n_max, "k_lmk": cfg.k_lmk, "select": cfg.select_mode, "block_size": cfg.block_size,
                   "lm_head": "all positions"},
        "roofline": roof,
        "step_roofline": {"bound": "mfma", "t_roof_ms": round(t_roof * 1e3, 3), "frac": round(t_roof * 1e3 / ms_step, 4),
                          "flops": step_flops, "note": "linear layers (incl. LM head over all positions) only"},
        "cpu_baseline": None,
        "kernels": {k: {kk: round(vv, 5) if isinstance(vv, float) else vv for kk, vv in v.items()}
                    for k, v in sorted(kernels.items())},
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.traffic_from:
        print(json.dumps(traffic_from(args.traffic_from, args.workload, args.copy_calibration or 1024, args.variant), indent=1))
        return
    if args.kernel_stats:
        import csv
        for dirpath, _, files in os.walk(args.kernel_stats):
            for fn in sorted(files):
                if fn.endswith("kernel_stats.csv"):
                    rows = list(csv.DictReader(open(os.path.join(dirpath, fn), newline="")))
                    print(f"{'kernel':<14} {'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'pct':>6}  name")
                    for r in rows:
                        print(f"{short_kernel_name(r['Name'])[:14]:<14} {r['Calls']:>6} {float(r['AverageNs']) / 1e3:9.2f} "
                              f"{float(r['MinNs']) / 1e3:9.2f} {float(r['MaxNs']) / 1e3:9.2f} "
                              f"{float(r['Percentage']):6.2f}  {r['Name'][:70]}")
        return
    if args.pmc_summary:
        for k, d in sorted(read_pmc(args.pmc_summary).items()):
            print(k, json.dumps({c: round(v, 1) for c, v in sorted(d.items())}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the operator shards over "
              "(batch, head) with no communication, so run one process per GPU.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from dsalt_amd import _lib, ops
    from dsalt_amd.workloads import MODEL_WORKLOADS, WORKLOADS, generate

    if (args.seqlen or args.batch) and (args.workload in MODEL_WORKLOADS or args.workload not in WORKLOADS):
        print(f"--seqlen and --batch apply to the operator workloads only (not {args.workload})", file=sys.stderr)
        sys.exit(2)
    if args.workload in MODEL_WORKLOADS:
        return model_bench(args, MODEL_WORKLOADS[args.workload])
    if args.workload == "ce_qwen3b_l32768":
        return ce_bench(args)
    if args.workload.startswith("probs_"):
        return probs_bench(args, WORKLOADS[args.workload[len("probs_"):]])
    wl = WORKLOADS[args.workload]
    own_shape = (wl.batch, wl.seqlen)
    if (args.seqlen and args.seqlen != wl.seqlen) or (args.batch and args.batch != wl.batch):
        import dataclasses
        wl = dataclasses.replace(wl, seqlen=args.seqlen or wl.seqlen, batch=args.batch or wl.batch)
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        n = args.copy_calibration * 2**20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            torch.neg(src, out=dst)  # an elementwise kernel: reads n bytes, writes n bytes
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "launches": 5}), flush=True)
        return
    x_cpu = generate(wl)
    x = {k: v.to(dev) for k, v in x_cpu.items()}
    T, H, D = x["q"].shape
    G = x["k"].shape[1]
    mode = ops.SELECT_GLOBAL if wl.select_mode == "global" else ops.SELECT_BLOCK
    scope = ops.STATS_SEQUENCE
    maxlen = wl.seqlen
    e = x["q"].element_size()

    if wl.train:
        tau_win, win_edge = wl.tau_win, wl.win_edge
        starts = x["cu"][:-1].long()

        def step():
            # the training forward of the layer: hard selection from floor(w~), landmark
            # log-weights log sigmoid(s / tau_lmk) at the selected positions, then the
            # training kernels forward and backward
            idx, _, _, sc = ops.select_landmarks(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk,
                                                 max_seqlen=maxlen, stats_scope=scope, want_scores=True)
            pos = idx[:, :, 0].long()
            s_sel = sc[starts[None, :, None] + pos.clamp(min=0), torch.arange(H, device=dev)[:, None, None]]
            logw = torch.log(torch.sigmoid(s_sel / wl.tau_lmk).clamp(min=1e-20))
            logw = torch.where(pos >= 0, logw, torch.full_like(logw, float("-inf"))).unsqueeze(2)
            out, lse = ops.train_forward(x["q"], x["k"], x["v"], x["w_cont"], x["cu"], idx, logw, tau_win=tau_win,
                                         win_edge=win_edge, max_seqlen=maxlen)
            ops.train_backward(x["dout"], x["q"], x["k"], x["v"], out, lse, x["w_cont"], x["cu"], idx, logw,
                               tau_win=tau_win, win_edge=win_edge, max_seqlen=maxlen)
            return idx
    else:
        variant = 0 if args.variant == "auto" else int(args.variant)
        if args.variant == "auto":
            # the reference's flow: tile sizes autotuned once per shape, then used by every call
            import contextlib

            from dsalt_amd.kernels import autotune as AT
            idx0 = ops.select_landmarks(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, max_seqlen=maxlen,
                                        select_mode=mode, block_size=wl.block_size, stats_scope=scope)
            runner = AT.operator_runner(x["q"], x["k"], x["v"], x["w"], x["cu"], idx0,
                                        x["dout"] if wl.backward else None, max_seqlen=maxlen, select_mode=mode,
                                        block_size=wl.block_size)
            with contextlib.redirect_stdout(sys.stderr):
                variant = AT.autotune_blocks(D, dev, runner, verbose=True, dtype=x["q"].dtype)["variant"]
            del idx0

        # the forward's row plan: written by the selection's norms launch and read by the forward
        # (plan_ready) and the backward
        plan = ops.new_plan(x["q"], x["k"], x["cu"], torch.empty(H, x["cu"].numel() - 1, 1, wl.k_lmk,
                                                                 dtype=torch.int32, device=dev),
                            max_seqlen=maxlen, select_mode=mode, block_size=wl.block_size)

        def step():
            idx = ops.select_landmarks(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, max_seqlen=maxlen,
                                       select_mode=mode, block_size=wl.block_size, stats_scope=scope, plan=plan)
            out, lse = ops.attention_forward(x["q"], x["k"], x["v"], x["w"], x["cu"], idx, None, max_seqlen=maxlen,
                                             select_mode=mode, block_size=wl.block_size, plan=plan,
                                             plan_ready=True, variant=variant)
            if wl.backward:
                ops.attention_backward(x["dout"], x["q"], x["k"], x["v"], out, lse, x["w"], x["cu"], idx, None,
                                       max_seqlen=maxlen, want_dbias=False, plan=plan, variant=variant)
            return idx

    idx = step()
    # warmup right before the timed region: the GPU stays busy from the autotune through the
    # warmup into the timed steps (the exact pair count runs after the timed regions)
    for _ in range(args.warmup):
        idx = step()
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

    # exact number of attended (query, key) pairs: window + visible landmarks
    # (training variant: the band of w~ is the integer window floor(w~) + 1)
    wv = (x["w"].long() + 1) if wl.train else x["w"].long().clamp(min=1)
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

    model = kernel_model(wl, T, H, D, wl.hidden, pairs, e, G)
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"])
    roof = None
    if dom in model:
        avg_s = kernels[dom]["avg_ms"] * 1e-3
        ach = model[dom]["bytes"] / avg_s / 1e9
        traffic = None
        tpath = os.path.join(HERE, "profiles", f"traffic_{wl.name}.json")
        if os.path.exists(tpath):
            with open(tpath) as f:
                rec = json.load(f)
            # only a record measured on the current kernel sources counts
            if rec.get("_sources") == kernel_source_sha() and (wl.batch, wl.seqlen) == own_shape:
                traffic = (rec.get(dom) or {}).get("bytes")
        roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                "algorithmic_bytes": model[dom]["bytes"],
                "mfma_tflops": round(model[dom]["flops"] / avg_s / 1e12, 2) if model[dom]["flops"] else None}

    dtn = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[x["q"].dtype]
    # unique algorithmic traffic of a step: q, k, v, o (+ h for the selection) and the LSE in
    # the forward; q, k, v, o, dO, dq, dk, dv and the LSE in the backward
    thd = T * H * D * e
    tgd = T * G * D * e
    step_bytes = 2 * thd + 2 * tgd + T * wl.hidden * e + 4 * T * H
    if wl.backward:
        step_bytes += 4 * thd + 4 * tgd + 4 * T * H
    step_flops = (4 + (8 if wl.backward else 0)) * D * pairs
    t_roof = max(step_bytes / (HBM_PEAK_GBS * 1e9), step_flops / (MFMA_PEAK_TFLOPS[dtn] * 1e12))

    cpu = None
    if not args.no_cpu_baseline:
        from oracle.sdpa_cpu import time_baseline
        r = time_baseline(x_cpu, wl.k_lmk, scope, backward=wl.backward,
                          train=(wl.tau_win, wl.win_edge, wl.tau_lmk) if wl.train else None)
        cpu = {"value": round(r["tokens_per_s"], 2), "unit": "tokens/s", "cores": r["threads"], "kind": "port",
               "cpu_model": cpu_model(), "torch_threads": r["threads"], "cpu_count": r["cpu_count"],
               "sample": (f"full-length landmark selection (C oracle, 1 thread, {r['t_select']:.2f}s) + reference "
                          f"{'dense training log-bias + SDPA' if wl.train else 'masked-SDPA'} "
                          f"{'fwd+bwd' if wl.backward else 'fwd'} on the last {r['rows']} query rows x "
                          f"{H} heads x all {T} keys ({r['t_attention']:.2f}s, torch CPU, {r['threads']} threads, "
                          f"host cpu_count {r['cpu_count']})")}

    line = {
        "metric": METRIC if wl.seqlen == 32768 else METRIC.replace("@L=32K", f"@L={wl.seqlen}"),
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
        "config": {"workload": wl.name, "batch": wl.batch, "heads": H, "kv_heads": G, "seq_len": wl.seqlen,
                   "head_dim": D,
                   "hidden": wl.hidden, "w_max": wl.w_max, "k_lmk": wl.k_lmk, "select": wl.select_mode,
                   "backward": wl.backward, "pairs": pairs,
                   **({"variant": "train", "tau_win": wl.tau_win, "win_edge": wl.win_edge, "tau_lmk": wl.tau_lmk}
                      if wl.train else {"tiling_variant": variant})},
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
