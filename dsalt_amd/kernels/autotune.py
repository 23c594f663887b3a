"""Tile policy of the HIP kernels, with the reference's autotune entry points.

The reference sweeps Triton tile sizes once per ``(head_dim, compute capability)``
(``dsalt/kernels/autotune.py:192-278``).  The gfx950 kernels fix their tiles at compile
time per (dtype, head_dim): 64 query rows per 256-thread block (4 waves x 16 rows, one
query row per lane), key chunks of BLOCK_N rows staged in LDS, 16x16x32 MFMA tiles.
``get_tuned_config`` reports that policy; ``autotune_blocks`` keeps the reference's
contract (time each candidate's fwd+bwd runner with GPU events, cache the fastest) over the
candidates the library offers.
"""
from __future__ import annotations

import torch

_TUNED_CONFIG: dict = {}

# compiled tile table: (head_dim, element bytes) -> forward key chunk, backward query chunk
_TILES = {(64, 2): (64, 32), (128, 2): (32, 32), (64, 4): (32, 16), (128, 4): (16, 16)}


def _device_key(head_dim: int, device) -> tuple:
    name = torch.cuda.get_device_properties(device).gcnArchName if torch.cuda.is_available() else "cpu"
    return (int(head_dim), str(name))


def _heuristic_config(head_dim: int, device=None, elem_bytes: int = 2) -> dict:
    hd = 64 if head_dim <= 64 else 128
    bn, bq = _TILES[(hd, 4 if elem_bytes == 4 else 2)]
    return {"BLOCK_M": 64, "BLOCK_N": bn, "BLOCK_N_BWD": bq, "num_warps": 4, "num_stages": 2}


def _candidate_configs(head_dim: int, device=None) -> list[dict]:
    return [_heuristic_config(head_dim, device)]


def _bench_step(run_fwd_bwd, n_warmup: int = 3, n_iter: int = 10) -> float:
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


def autotune_blocks(head_dim: int, device, make_runner, verbose: bool = True) -> dict:
    """Time ``make_runner(cfg)()`` for each candidate, cache and return the fastest config."""
    key = _device_key(head_dim, device)
    if key in _TUNED_CONFIG:
        return _TUNED_CONFIG[key]
    results = []
    for cfg in _candidate_configs(head_dim, device):
        runner = make_runner(cfg)
        if runner is None:
            continue
        try:
            results.append((cfg, _bench_step(runner)))
        except Exception as e:  # a candidate that cannot run is skipped
            if verbose:
                print(f"autotune: {cfg} failed: {type(e).__name__}")
    best = min(results, key=lambda r: r[1])[0] if results else _heuristic_config(head_dim, device)
    _TUNED_CONFIG[key] = best
    if verbose and results:
        for cfg, ms in results:
            print(f"  dsalt tiles {cfg}: {ms:.4f} ms/step")
    return best


def get_tuned_config(head_dim: int, device) -> dict | None:
    return _TUNED_CONFIG.get(_device_key(head_dim, device))
