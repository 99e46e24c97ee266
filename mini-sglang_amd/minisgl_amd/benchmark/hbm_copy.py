"""Plain device copy of a known size, the yardstick for HBM byte counters.

Profilers' FETCH_SIZE / WRITE_SIZE are read for this copy (exactly
``--mib`` MiB read and written per launch) to get the factor that turns
them into bytes for the MLA kernels.

    python -m minisgl_amd.benchmark.hbm_copy --mib 512 --iters 5
"""

from __future__ import annotations

import argparse
import time


def main() -> None:
    import torch

    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=512)
    ap.add_argument("--iters", type=int, default=5)
    args = ap.parse_args()
    n = args.mib * (1 << 20) // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(2):
        y.copy_(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.iters):
        y.copy_(x)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.iters
    print(f"copy {args.mib} MiB: {dt * 1e6:.1f} us/launch, {2 * n * 4 / dt / 1e9:.1f} GB/s (read+write)")


if __name__ == "__main__":
    main()
