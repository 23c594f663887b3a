"""Tile policy of the HIP kernels, with the reference's autotune entry points.

The reference sweeps Triton tile sizes once per ``(head_dim, compute capability)``, timing
one fwd+bwd step per candidate with GPU events and caching the fastest
(``dsalt/kernels/autotune.py:55-122,176-238,276-278``); its kernels then read the cached
choice (``dsalt_triton_bwd.py:276-277``).  The gfx950 kernels are compiled in a few tilings
per (dtype, head_dim) -- 64 query rows per 256-thread block (4 waves x 16 rows, one query
row per lane), key chunks of BLOCK_N rows staged in LDS, 16x16x32 MFMA tiles -- selected at
run time by the ``variant`` bits of the C ABI (``DSALT_VARIANT_*``):

  * FWD_BN32  forward key chunks of 32 instead of 64 rows (16-bit, head_dim 64);
  * FWD_RG2   forward blocks of 128 rows, two 16-row groups per wave (16-bit; for head_dim 64
              with FWD_BN32 the kernel is held at four waves per SIMD);
  * FWD_BN64  forward key chunks of 64 instead of 32 rows (16-bit, head_dim 128, inference;
              ignored with FWD_RG2);
  * FWD_8W    forward blocks of 128 rows in eight waves, one row group each: every staged key
              chunk serves twice the rows (16-bit, head_dim 128, inference; ignores FWD_RG2 and
              FWD_BN64);
  * DQ_BN64   backward dQ key chunks of 64 instead of 32 rows (16-bit, head_dim 64);
  * LMK_SHORT landmark-backward row chunks of 512 instead of 1024 rows (more blocks).

``_candidate_configs`` lists the tilings a shape can use, ``autotune_blocks`` times each
candidate's fwd+bwd runner and caches the winner per (head_dim, dtype, device), and
``get_tuned_config`` returns it; ``dsalt_attention`` passes the cached variant to the
kernels.  Every variant computes the same operator (the GPU tests check each against the
oracle); only the speed differs.
"""
from __future__ import annotations

import torch

from .._lib import (VARIANT_DQ_BN64, VARIANT_FWD_8W, VARIANT_FWD_BN32, VARIANT_FWD_BN64, VARIANT_FWD_RG2,
                    VARIANT_LMK_SHORT)

_TUNED_CONFIG: dict = {}

# default compiled tiles: (head_dim, element bytes) -> forward key chunk, dQ key chunk,
# dK/dV query chunk
_TILES = {(64, 2): (64, 32, 32), (128, 2): (32, 32, 32), (64, 4): (32, 32, 32), (128, 4): (16, 16, 16)}


def _elem_bytes(dtype) -> int:
    return 4 if dtype in (torch.float32, None) else 2


def _device_key(head_dim: int, device, dtype=torch.bfloat16) -> tuple:
    name = torch.cuda.get_device_properties(device).gcnArchName if torch.cuda.is_available() else "cpu"
    return (int(head_dim), _elem_bytes(dtype), str(name))


def _config_of(head_dim: int, elem_bytes: int, variant: int) -> dict:
    hd = 64 if head_dim <= 64 else 128
    bn, bnq, bq = _TILES[(hd, 4 if elem_bytes == 4 else 2)]
    half = elem_bytes == 2
    tunable = hd == 64 and half
    bm = 64
    if tunable and variant & VARIANT_FWD_BN32:
        bn = 32
    w8 = half and hd == 128 and bool(variant & VARIANT_FWD_8W)
    if half and hd == 128 and variant & VARIANT_FWD_BN64 and not variant & VARIANT_FWD_RG2 and not w8:
        bn = 64
    if half and variant & VARIANT_FWD_RG2 or w8:
        bm = 128
    if tunable and variant & VARIANT_DQ_BN64:
        bnq = 64
    return {"BLOCK_M": bm, "BLOCK_N": bn, "BLOCK_N_BWD": bnq, "BLOCK_Q_BWD": bq, "num_warps": 8 if w8 else 4,
            "num_stages": 2, "LMK_ROWS": 512 if variant & VARIANT_LMK_SHORT else 1024, "variant": int(variant)}


def _heuristic_config(head_dim: int, device=None, elem_bytes: int = 2) -> dict:
    """The library's default tiling for the shape (variant 0)."""
    return _config_of(head_dim, elem_bytes, 0)


def _candidate_configs(head_dim: int, device=None, elem_bytes: int = 2) -> list[dict]:
    """Every tiling the compiled kernels offer for the shape (the heuristic first): the forward
    tilings with the default backward, then the backward tilings with the default forward."""
    if head_dim == 64 and elem_bytes == 2:
        variants = [0, VARIANT_FWD_BN32, VARIANT_FWD_RG2, VARIANT_FWD_RG2 | VARIANT_FWD_BN32,
                    VARIANT_DQ_BN64, VARIANT_LMK_SHORT, VARIANT_DQ_BN64 | VARIANT_LMK_SHORT]
    elif head_dim == 128 and elem_bytes == 2:
        variants = [0, VARIANT_FWD_RG2, VARIANT_FWD_BN64, VARIANT_FWD_8W, VARIANT_LMK_SHORT]
    else:
        variants = [0, VARIANT_LMK_SHORT]
    return [_config_of(head_dim, elem_bytes, v) for v in variants]


# variant bits of the forward kernels and of the backward kernels (independent choices)
_FWD_BITS = VARIANT_FWD_BN32 | VARIANT_FWD_RG2 | VARIANT_FWD_BN64 | VARIANT_FWD_8W
_BWD_BITS = VARIANT_DQ_BN64 | VARIANT_LMK_SHORT


def _bench_step(run_fwd_bwd, n_warmup: int = 3, n_iter: int = 20) -> float:
    """Average time (ms) of one fwd+bwd step, timed with GPU events."""
    for _ in range(n_warmup):
        run_fwd_bwd()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(n_iter):
        run_fwd_bwd()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / n_iter


# a candidate replaces an earlier one (the heuristic first) only when it is faster by more
# than this fraction: tilings that run the same kernels for a shape (e.g. the landmark-backward
# chunking in a forward-only run) time alike, and the tie goes to the default
_MARGIN = 0.005


def _timed(cands, runners, fn_of, rounds, errors):
    """Best time per candidate variant of fn_of(runner) over `rounds` rotated passes."""
    best_ms, warm = {}, False
    for r in range(max(1, rounds)):
        order = list(range(len(cands)))
        order = order[r % len(order):] + order[:r % len(order)]
        for i in order:
            cfg, runner = cands[i], runners[i]
            if runner is None or cfg["variant"] in errors:
                continue
            fn = fn_of(runner)
            if fn is None:
                continue
            try:
                if not warm:  # clocks up before the first timed candidate
                    _bench_step(fn, n_warmup=10, n_iter=1)
                    warm = True
                ms = _bench_step(fn)
            except Exception as e:  # a candidate that cannot run is skipped
                errors[cfg["variant"]] = type(e).__name__
                continue
            best_ms[cfg["variant"]] = min(ms, best_ms.get(cfg["variant"], float("inf")))
    return best_ms


def _pick(cands, best_ms):
    best = None
    for cfg in cands:  # candidate order: the heuristic first
        ms = best_ms.get(cfg["variant"])
        if ms is not None and (best is None or ms < best_ms[best["variant"]] * (1.0 - _MARGIN)):
            best = cfg
    return best


def autotune_blocks(head_dim: int, device, make_runner, verbose: bool = True, dtype=torch.bfloat16,
                    rounds: int = 2) -> dict:
    """Time ``make_runner(cfg)()`` (one fwd+bwd with the config's tiling; ``None`` when the
    config cannot run) for each candidate; cache and return the fastest config.  The GPU is
    warmed up on the first candidate before any timing, and the candidates are timed
    ``rounds`` times in rotated order, each keeping its best time.  When the runners expose
    their phases (``runner.forward`` / ``runner.backward``, as ``operator_runner``'s do), the
    forward tilings are timed on the forward alone and the backward tilings on the backward
    alone, and the winner combines both choices."""
    key = _device_key(head_dim, device, dtype)
    if key in _TUNED_CONFIG:
        return _TUNED_CONFIG[key]
    eb = _elem_bytes(dtype)
    cands = _candidate_configs(head_dim, device, eb)
    runners, errors = [], {}
    for cfg in cands:
        runner = make_runner(cfg)
        runners.append(runner)
        if runner is None:
            errors[cfg["variant"]] = "skip"
    phased = all(r is None or hasattr(r, "forward") for r in runners)
    rows = []
    if phased:
        fw = [(c, r) for c, r in zip(cands, runners) if not c["variant"] & _BWD_BITS]
        bw = [(c, r) for c, r in zip(cands, runners) if not c["variant"] & _FWD_BITS]
        f_ms = _timed([c for c, _ in fw], [r for _, r in fw], lambda r: r.forward, rounds, errors)
        b_ms = _timed([c for c, _ in bw], [r for _, r in bw], lambda r: getattr(r, "backward", None), rounds, errors)
        f_best = _pick([c for c, _ in fw], f_ms)
        b_best = _pick([c for c, _ in bw], b_ms)
        v = (f_best["variant"] if f_best else 0) | (b_best["variant"] if b_best else 0)
        best = _config_of(head_dim, eb, v)
        rows = [("forward", c, f_ms.get(c["variant"]), f_best) for c, _ in fw] + \
               [("backward", c, b_ms.get(c["variant"]), b_best) for c, _ in bw if b_ms]
    else:
        ms = _timed(cands, runners, lambda r: r, rounds, errors)
        best = _pick(cands, ms) or _heuristic_config(head_dim, device, eb)
        rows = [("fwd+bwd", c, ms.get(c["variant"]), best) for c in cands]
    _TUNED_CONFIG[key] = best
    if verbose:
        print(f"dsalt autotune head_dim={head_dim} ({key[2]}, {key[1]}-byte elements): variant {best['variant']}")
        for phase, cfg, t, win in rows:
            mark = "  <- best" if win is not None and cfg["variant"] == win["variant"] else ""
            tt = f"{t:.4f} ms" if t is not None else errors.get(cfg["variant"], "skip")
            print(f"  {phase:8s} variant {cfg['variant']:2d}  BLOCK_M {cfg['BLOCK_M']:3d} BLOCK_N {cfg['BLOCK_N']:2d} "
                  f"BLOCK_N_BWD {cfg['BLOCK_N_BWD']:2d} LMK_ROWS {cfg['LMK_ROWS']:4d}  {tt}{mark}")
    return best


def get_tuned_config(head_dim: int, device, dtype=torch.bfloat16) -> dict | None:
    """The cached config for ``(head_dim, dtype, device)``, or None before autotune_blocks."""
    return _TUNED_CONFIG.get(_device_key(head_dim, device, dtype))


def tuned_variant(head_dim: int, device, dtype) -> int:
    """Variant bits the kernels should use: the cached winner's, else the default (0)."""
    if not _TUNED_CONFIG:
        return 0
    cfg = get_tuned_config(head_dim, device, dtype)
    return int(cfg["variant"]) if cfg else 0


def operator_runner(q, k, v, w, cu_seqlens, lmk_idx, dout, *, max_seqlen=None, select_mode=None, block_size=None):
    """``make_runner`` for autotune_blocks over the operator's own fwd+bwd on the given
    tensors (indices [H, S, n_sets, k] ascending, as ops.select_landmarks returns); with
    ``dout=None`` the forward alone (inference configurations, block-causal sets).  The runner
    exposes its phases: ``runner.forward`` and ``runner.backward`` (after a forward of the
    same tiling, which it keeps)."""
    from .. import ops

    mode = ops.SELECT_GLOBAL if select_mode is None else select_mode
    bs = block_size or 512

    def make_runner(cfg):
        variant = cfg["variant"]
        state = {}

        def forward():
            plan = ops.new_plan(q, k, cu_seqlens, lmk_idx, max_seqlen=max_seqlen, select_mode=mode, block_size=bs)
            out, lse = ops.attention_forward(q, k, v, w, cu_seqlens, lmk_idx, None, max_seqlen=max_seqlen,
                                             select_mode=mode, block_size=bs, plan=plan, variant=variant)
            state.update(plan=plan, out=out, lse=lse)

        def backward():
            if "out" not in state:
                forward()
            ops.attention_backward(dout, q, k, v, state["out"], state["lse"], w, cu_seqlens, lmk_idx, None,
                                   max_seqlen=max_seqlen, want_dbias=False, plan=state["plan"], variant=variant)

        def run():
            forward()
            if dout is not None:
                backward()
        run.forward = forward
        run.backward = backward if dout is not None else None
        return run
    return make_runner
