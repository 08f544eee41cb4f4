"""Fixed workload for rocprofv3 runs: N launches of mha_fwd_with_mask on one
configuration, optionally preceded by a plain device copy of known size (the
calibration kernel for the FETCH_SIZE / WRITE_SIZE counters).

    python -m custom_ops_amd.prof_workload --config cfg2 --iters 20 [--copy-mib 512]
        [--mask-bcast] [--cold] [--variant order=1]
    python -m custom_ops_amd.prof_workload --config cfg2 --loop-s 10

--mask-bcast launches the same call through the C ABI with the mask's row and
batch strides set to 0: every query row then reads the same (L2-resident)
mask row, so the difference in FETCH_SIZE against the normal call is the
mask stream's HBM traffic. The arithmetic is the same; only the mask values
differ (no tile of the cfg2/cfg3 masks is entirely -inf either way).

--loop-s S keeps the GPU busy for S seconds with the attention call on
--config instead and prints the achieved rate: the steady state in which
socket power and clocks are sampled.

--cold precedes every counted launch with a 512 MiB zero and read-back (the
bench's cold, clean caches), so the kernel trace shows cold launches; without
it the launches run back to back.

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
    ap.add_argument("--mask-bcast", action="store_true",
                    help="mask row/batch strides 0: one L2-resident mask row for every query row")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run 5 copies of a buffer of this many MiB (read N, write N)")
    ap.add_argument("--variant", default="",
                    help="kernel-variant fields for every call, e.g. order=1,waves=8 (custom_ops_amd.Variant)")
    ap.add_argument("--cold", action="store_true",
                    help="flush the caches (512 MiB zero + read-back) before every counted launch")
    ap.add_argument("--loop-s", type=float, default=0.0,
                    help="run back to back for this many seconds and print the achieved rate")
    args = ap.parse_args()

    import torch
    dev = torch.device("cuda:0")
    from custom_ops_amd import ops
    from custom_ops_amd.workloads import CONFIGS, make_inputs

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
    call = lambda: ops.mha_fwd_with_mask(q, k, v, m)  # noqa: E731
    var = None
    if args.variant:
        from custom_ops_amd import Variant, mha_fwd_with_mask
        var = Variant(**{kv.split("=")[0]: int(kv.split("=")[1]) for kv in args.variant.split(",")})
        call = lambda: mha_fwd_with_mask(q, k, v, m, variant=var)  # noqa: E731
    if args.mask_bcast:
        from custom_ops_amd import _lib, fa
        out = torch.empty_like(q)
        p = fa.make_params(q, k, v, m, out, 0, var)
        p.mask_row_stride = 0
        p.mask_batch_stride = 0
        ws_bytes = _lib.workspace_bytes(p)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        if ws_bytes:
            p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
        stream = torch.cuda.current_stream(dev).cuda_stream
        call = lambda: _lib.fwd(p, stream)  # noqa: E731
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < args.settle_s:
        for _ in range(10):
            call()
        torch.cuda.synchronize()
    if args.loop_s:
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.loop_s:
            for _ in range(50):
                call()
            torch.cuda.synchronize()
            n += 50
        us = (time.perf_counter() - t0) / n * 1e6
        print(f"prof_workload {cfg.name}: loop {n} calls, {us:.2f} us/call", flush=True)
        return
    flush = red = None
    if args.cold:
        flush = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.int32, device=dev)
        red = torch.empty((), dtype=torch.int32, device=dev)
    for _ in range(args.iters):
        if args.cold:
            flush.zero_()
            torch.amax(flush, dim=0, out=red)
        call()
    torch.cuda.synchronize()
    print(f"prof_workload {cfg.name}: {args.iters} launches done", flush=True)


if __name__ == "__main__":
    main()

