"""Decode throughput of SmolLM2-360M (bf16, batch 1, 1024-token context) on one MI355X.
(--batch 16: BASELINE config 4, 16 sequences with ragged contexts; --weights mxfp8: config 5.)

One step = one greedy decode step of the full model (32 layers + tied LM head + argmax), i.e. one
launch of the persistent megakernel.  The KV cache holds a synthetic 1024-token context
(N(0,1) bf16), weights are seeded random-init (N(0,0.02) bf16): BASELINE config 3.  W untimed
warmup steps, then exactly K timed steps starting at position 1024 (context 1025 .. 1024+K),
bracketed by synchronisation and HIP events on the launch stream.

Prints one JSON line with the metric, the HBM roofline of the kernel (algorithmic bytes per step
from the reference's own accounting) and a CPU baseline (the oracle's eager step on host cores).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
CONTEXT = 1024
W_LAYER_360M = 19_664_640        # bf16 projections + norms of one layer
W_LAYER_360M_MXFP8 = 10_141_440  # e4m3 projections + one e8m0 byte per 32 weights + bf16 norms
E_LMHEAD_360M = 94_371_840
KV_TOKEN_360M = 40_960
HIDDEN_BYTES = 1_920


def step_bytes(S, layers: int = 32, weights: str = "bf16") -> int:
    """Algorithmic bytes of one step whose sequences attend S tokens each (S counts the new one;
    an int for one sequence or a list for a batch): the weights and the LM head once per step,
    per sequence its cached K/V, the appended K/V and the hidden state in and out."""
    w = W_LAYER_360M if weights == "bf16" else W_LAYER_360M_MXFP8
    seqs = [S] if isinstance(S, int) else list(S)
    return layers * w + E_LMHEAD_360M + sum(KV_TOKEN_360M * s + KV_TOKEN_360M + 2 * HIDDEN_BYTES for s in seqs)


def cpu_baseline(seconds: float = 15.0) -> dict:
    """The oracle's eager bf16 step (oracle/smollm2.py) on this host's cores, full 360M model,
    1024-token synthetic context; a bounded sample of steps (about `seconds` of CPU work)."""
    import torch
    from oracle import smollm2 as O

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    geom = O.SMOLLM2_360M
    w = O.make_weights(geom, 7)
    kv = O.make_paged_kv(geom, 1, CONTEXT + 64, seed=11)
    cos_sin = O.rope_cos_sin(CONTEXT + 64)
    O.decode_step(w, [5], [CONTEXT], kv, cos_sin)  # untimed warmup
    times = []
    t_end = time.perf_counter() + seconds
    k = 1
    while time.perf_counter() < t_end and k < 60:
        t0 = time.perf_counter()
        O.decode_step(w, [5 + k], [CONTEXT + k], kv, cos_sin)
        times.append(time.perf_counter() - t0)
        k += 1
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{len(times)} greedy steps of the full 360M model at context {CONTEXT + 1}..{CONTEXT + len(times)} "
                      f"(median step {med * 1e3:.1f} ms, torch {torch.__version__} CPU eager bf16, "
                      f"os.cpu_count()={os.cpu_count()})"}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--weights", choices=("bf16", "mxfp8"), default="bf16",
                    help="projection weights: bf16 (BASELINE config 3, the default) or MXFP8 (config 5)")
    ap.add_argument("--context", type=int, default=None,
                    help="cached tokens before the first timed step (default 1024; 8192 with --weights mxfp8)")
    ap.add_argument("--batch", type=int, default=1,
                    help="sequences per step; above 1 each sequence's context is drawn uniformly from "
                         "128..4096 (BASELINE config 4 at 16; bf16 weights only)")
    ap.add_argument("--seed", type=int, default=4, help="seed of the ragged contexts and token ids")
    ap.add_argument("--lossless", action="store_true",
                    help="stream the gate/up weights through the lossless codec (batch 1, bf16)")
    args = ap.parse_args()
    context = args.context if args.context is not None else (CONTEXT if args.weights == "bf16" else 8192)
    B = args.batch
    if not 1 <= B <= 16 or (B > 1 and args.weights != "bf16"):
        print("--batch takes 1..16 sequences, with bf16 weights above 1", file=sys.stderr)
        sys.exit(2)
    if args.lossless and (B != 1 or args.weights != "bf16"):
        print("--lossless runs batch 1 with bf16 weights", file=sys.stderr)
        sys.exit(2)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every box in this setup has one MI355X and the decode "
              f"path shards by data parallelism with no exchange between GPUs; --gpus {args.gpus} is not run.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import prime_kernels_amd as pk
    from prime_kernels_amd import workload as WL
    from prime_kernels_amd._decode import StepLauncher

    mod = pk.load("decode_megakernel_360m" if args.weights == "bf16" else "decode_megakernel_360m_mxfp8")
    model = mod.MODEL
    dev = torch.device("cuda:0")
    K, W = args.steps, args.warmup
    if B == 1:
        contexts, first_ids = [context], [17]
    else:
        import numpy as np
        rng = np.random.default_rng(args.seed)
        contexts = [int(x) for x in rng.integers(128, 4097, B)]
        first_ids = [int(x) for x in rng.integers(0, 49152, B)]
    embed, final_norm, layers = WL.random_weights(pk.load("decode_megakernel_360m").MODEL, 1234, dev)
    if args.weights == "mxfp8":
        layers = mod.quantize_layers(layers)
    cache = None
    gu_bytes_saved = 0
    if args.lossless:
        from prime_kernels_amd.lossless_bf16 import EncodedGUCache, COLS, ROWS

        cache = EncodedGUCache([layer[4] for layer in layers])
        st = cache.statistics()
        # encoded gate/up bytes a step streams: plane + headers + escaped chunks, per layer
        enc = sum(ROWS * COLS + ROWS * (COLS // 8) * 4 + 16 * n for n in st["escape_chunks"])
        gu_bytes_saved = len(layers) * ROWS * COLS * 2 - enc
    cap = max(contexts) + max(K, W) + 16
    kv = WL.PagedKV(model, B, cap, device=dev, seed=5, fill="randn")
    cos_sin = WL.rope_table(cap, device=dev)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    common = dict(embed=embed, layers=layers, final_norm=final_norm, kv_caches=kv.caches, block_table=kv.block_table,
                  cos_sin_cache=cos_sin, first_id=first_ids, start_pos=contexts, batch=B, encoded_gu=cache)
    warm = StepLauncher(model, steps=max(W, 1), **common)
    for k in range(W):
        warm.launch(k, stream.cuda_stream)
    timed = StepLauncher(model, steps=K, **common)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for k in range(K):
        timed.launch(k, stream.cuda_stream)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1)
    epoch, site = timed.rt.pending_failure()
    if epoch:
        raise RuntimeError(f"a timed step gave up a bounded wait (epoch {epoch}, wait site {site})")
    ids = timed.ids.cpu()
    if not bool(((ids >= 0) & (ids < 49152)).all()):
        raise RuntimeError("greedy ids out of range")

    total_bytes = sum(step_bytes([c + 1 + k for c in contexts], weights=args.weights) - gu_bytes_saved
                      for k in range(K))
    ms_per_step = ms / K
    achieved = total_bytes / (ms * 1e-3) / 1e9
    traffic = None
    tname = (f"decode360_b{B}_ragged" if B > 1 else
             f"decode360_{'' if args.weights == 'bf16' else 'mxfp8_'}{'lossless_' if args.lossless else ''}"
             f"ctx{context}")
    tfile = ROOT / "profiles" / f"{tname}_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    wname = ("bf16 lossless-GU" if args.lossless else "bf16") if args.weights == "bf16" else "MXFP8-weight"
    ctx_name = f"ctx={context}" if B == 1 else "ragged ctx 128..4096"
    workload = (f"smollm2-360m greedy decode, batch 1, {context}-token context, K steps at context "
                f"{context + 1}..{context}+K" + (", MXFP8 projection weights" if args.weights == "mxfp8" else "")
                + (", gate/up streamed through the lossless codec" if args.lossless else "")
                if B == 1 else
                f"smollm2-360m greedy decode, batch {B}, contexts drawn uniformly from 128..4096 "
                f"(seed {args.seed}, mean {sum(contexts) / B:.0f}), K steps per sequence")
    line = {
        "metric": f"decode tok/s, SmolLM2-360M {wname} bs={B} {ctx_name}; % of HBM roofline",
        "value": round(B * K / (ms * 1e-3), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.weights == "bf16" else "e4m3 weights, bf16 activations",
        "data": "synthetic (seeded random-init weights N(0,0.02) bf16" +
                (", projections quantised to MXFP8 on the GPU" if args.weights == "mxfp8" else "") +
                ", KV context N(0,1) bf16, greedy ids fed back on device)",
        "config": {"workload": workload,
                   "batch": B, "context": context if B == 1 else contexts, "layers": 32, "weights": args.weights,
                   "gate_up": "lossless codec" if args.lossless else "dense",
                   "lm_head": "tied, fused argmax", "launch": "one cooperative kernel per step, 256 workgroups"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_step": round(total_bytes / K)},
        "host_wall_ms_per_step": round(wall * 1e3 / K, 5),
    }
    if not args.no_cpu_baseline and args.weights == "bf16" and B == 1:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
