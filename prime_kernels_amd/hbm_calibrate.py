"""Copy-kernel calibration for HBM traffic counters.

Runs a plain device-to-device copy of a known size several times, so that the per-dispatch
FETCH_SIZE / WRITE_SIZE counters of a profiler pass can be related to bytes actually moved:
factor = counter value of this copy / its known size.  The same factor converts the decode
kernel's counters into HBM bytes per launch.

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -- \
        python -m prime_kernels_amd.hbm_calibrate --mib 512 --repeats 8
"""

from __future__ import annotations

import argparse
import json


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=512, help="bytes copied per launch, in MiB")
    ap.add_argument("--repeats", type=int, default=8)
    args = ap.parse_args()

    import torch

    n = args.mib * (1 << 20)
    dev = torch.device("cuda:0")
    src = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 256)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.repeats):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.repeats
    if not torch.equal(dst[:4096], src[:4096]):
        raise RuntimeError("copy mismatch")
    print(json.dumps({"copy_bytes_read_per_launch": n, "copy_bytes_written_per_launch": n,
                      "repeats": args.repeats, "ms_per_copy": round(ms, 4),
                      "copy_GBps": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)


if __name__ == "__main__":
    main()
