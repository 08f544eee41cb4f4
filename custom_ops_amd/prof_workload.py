"""Fixed workload for rocprofv3 runs: N launches of mha_fwd_with_mask on one
configuration, optionally preceded by a plain device copy of known size (the
calibration kernel for the FETCH_SIZE / WRITE_SIZE counters).

    python -m custom_ops_amd.prof_workload --config cfg2 --iters 20 [--copy-mib 512]

Inputs are generated and copied to the GPU before any timed launch; the GPU
clocks are settled first with untimed launches (--settle-s).
"""
from __future__ import annotations

import argparse
import time


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--settle-s", type=float, default=0.3)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run 5 copies of a buffer of this many MiB (read N, write N)")
    args = ap.parse_args()

    import torch
    from custom_ops_amd import ops
    from custom_ops_amd.workloads import CONFIGS, make_inputs

    dev = torch.device("cuda:0")
    ops.ensure_loaded()
    if args.copy_mib:
        n = args.copy_mib * 1024 * 1024 // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):   # one elementwise kernel: reads N bytes, writes N bytes
            torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()
        del src, dst
    cfg = CONFIGS[args.config]
    q, k, v, m = (t.to(dev) for t in make_inputs(cfg))
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < args.settle_s:
        for _ in range(10):
            ops.mha_fwd_with_mask(q, k, v, m)
        torch.cuda.synchronize()
    for _ in range(args.iters):
        ops.mha_fwd_with_mask(q, k, v, m)
    torch.cuda.synchronize()
    print(f"prof_workload {cfg.name}: {args.iters} launches done", flush=True)


if __name__ == "__main__":
    main()
