"""Fixed workload for rocprofv3 runs: N launches of mha_fwd_with_mask on one
configuration, optionally preceded by a plain device copy of known size (the
calibration kernel for the FETCH_SIZE / WRITE_SIZE counters).

    python -m custom_ops_amd.prof_workload --config cfg2 --iters 20 [--copy-mib 512]
        [--mask-bcast]
    python -m custom_ops_amd.prof_workload --hbm-read-mib 2048 --iters 20
    python -m custom_ops_amd.prof_workload --config cfg2 --loop-s 10
    python -m custom_ops_amd.prof_workload --mfma random --loop-s 10

--hbm-read-mib N measures the cold HBM read ceiling instead: each iteration
writes a 512 MiB flush buffer (evicting L2 and the 256 MiB last-level cache),
then the probe kernel (csrc/hbm_probe.hip) reads an N MiB buffer once.

--mask-bcast launches the same call through the C ABI with the mask's row and
batch strides set to 0: every query row then reads the same (L2-resident)
mask row, so the difference in FETCH_SIZE against the normal call is the
mask stream's HBM traffic. The arithmetic is the same; only the mask values
differ (no tile of the cfg2/cfg3 masks is entirely -inf either way).

--loop-s S keeps the GPU busy for S seconds instead (the attention call on
--config, or with --mfma random|const the MFMA probe of csrc/hbm_probe.hip)
and prints the achieved rate: the steady state in which socket power and
clocks are sampled.

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
    ap.add_argument("--hbm-read-mib", type=int, default=0,
                    help="cold HBM read ceiling: flush, then read a buffer of this many MiB")
    ap.add_argument("--loop-s", type=float, default=0.0,
                    help="run back to back for this many seconds and print the achieved rate")
    ap.add_argument("--mfma", choices=("random", "const"), default=None,
                    help="with --loop-s: the MFMA probe instead of the attention call")
    args = ap.parse_args()

    import torch
    dev = torch.device("cuda:0")
    if args.hbm_read_mib:
        hbm_read(args.hbm_read_mib, args.iters, dev)
        return
    if args.mfma:
        mfma_loop(args.mfma, args.loop_s, dev)
        return
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
    if args.mask_bcast:
        from custom_ops_amd import _lib, fa
        out = torch.empty_like(q)
        p = fa.make_params(q, k, v, m, out)
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
    for _ in range(args.iters):
        call()
    torch.cuda.synchronize()
    print(f"prof_workload {cfg.name}: {args.iters} launches done", flush=True)


def hbm_read(mib: int, iters: int, dev) -> None:
    import ctypes
    import torch
    from custom_ops_amd.build import PROBE_PATH
    lib = ctypes.CDLL(PROBE_PATH)
    lib.mi355_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    lib.mi355_probe_read.restype = ctypes.c_int
    buf = torch.ones(mib * 1024 * 1024 // 4, dtype=torch.int32, device=dev)
    flush = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(2048, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for _ in range(iters):
        flush.fill_(1)
        rc = lib.mi355_probe_read(buf.data_ptr(), buf.numel() * 4, sink.data_ptr(), stream)
        if rc:
            raise RuntimeError(f"mi355_probe_read failed ({rc})")
    torch.cuda.synchronize()
    print(f"prof_workload hbm-read {mib} MiB: {iters} passes done", flush=True)



def mfma_loop(pattern: str, secs: float, dev) -> None:
    """The MFMA probe, one 512-thread workgroup per CU, back to back for
    `secs` seconds; prints the sustained TFLOP/s."""
    import ctypes
    import torch
    from custom_ops_amd.build import PROBE_PATH
    lib = ctypes.CDLL(PROBE_PATH)
    lib.mi355_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.mi355_probe_mfma.restype = ctypes.c_int
    ctas = torch.cuda.get_device_properties(dev).multi_processor_count
    iters = 40000
    sink = torch.zeros(ctas, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    pat = 0 if pattern == "random" else 1
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < secs:
        for _ in range(5):
            rc = lib.mi355_probe_mfma(ctas, iters, pat, sink.data_ptr(), stream)
            if rc:
                raise RuntimeError(f"mi355_probe_mfma failed ({rc})")
        torch.cuda.synchronize()
        n += 5
    dt = time.perf_counter() - t0
    flops = float(n) * ctas * 8 * iters * 4 * 32768
    print(f"prof_workload mfma {pattern}: {n} launches, {flops / dt / 1e12:.0f} TFLOP/s", flush=True)


if __name__ == "__main__":
    main()

