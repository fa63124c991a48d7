"""Decode throughput of SmolLM2 on one MI355X: the hot path's one step, timed.

Default: SmolLM2-360M, bf16, batch 1, 1024-token context (the headline).
--model 135m: SmolLM2-135M, 512-token context (config 2); --batch 16: 360M with 16 ragged contexts
(config 4); --weights mxfp8: 360M MXFP8 projections at an 8192-token context (config 5); --lossless:
the 360M gate/up weights streamed through the lossless codec.

One step = one greedy decode step of the full model (all layers + tied LM head + argmax), one
kernel launch.  The KV cache holds a synthetic context (N(0,1) bf16), weights are seeded
random-init (N(0,0.02) bf16).  W untimed warmup steps, then exactly K timed steps starting at the
context length (context S+1 .. S+K), bracketed by synchronisation and HIP events on the launch
stream; greedy ids are fed back on the device.

Prints one JSON line with the metric, the HBM roofline of the kernel (algorithmic bytes per step,
the accounting of SURVEY.md's roofline row; traffic from the committed rocprofv3 FETCH/WRITE
summary of the same workload) and a CPU baseline (the oracle's eager step on the host's cores).
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
VOCAB = 49152


class Bytes:
    """Algorithmic HBM bytes of one decode step of a SmolLM2 geometry."""

    def __init__(self, hidden, inter, heads, kv_heads, layers, head_dim=64):
        qkv = (heads + 2 * kv_heads) * head_dim
        mats = qkv * hidden + hidden * hidden + 2 * inter * hidden + hidden * inter
        self.layers = layers
        self.layer_bf16 = 2 * mats + 2 * 2 * hidden                  # projections + the two norms
        self.layer_mxfp8 = mats + mats // 32 + 2 * 2 * hidden        # e4m3 + one e8m0 per 32 + norms
        self.lm_head = VOCAB * hidden * 2
        self.kv_token = layers * kv_heads * 2 * head_dim * 2         # K and V of every layer, bf16
        self.hidden_bytes = hidden * 2

    def step(self, S, weights: str = "bf16") -> int:
        """Bytes of one step whose sequences attend S tokens each (S counts the new one; an int for one
        sequence or a list for a batch): weights and LM head once, per sequence its cached K/V, the
        appended K/V and the hidden state in and out."""
        w = self.layer_bf16 if weights == "bf16" else self.layer_mxfp8
        seqs = [S] if isinstance(S, int) else list(S)
        return self.layers * w + self.lm_head + sum(self.kv_token * (s + 1) + 2 * self.hidden_bytes for s in seqs)


BYTES = {"360m": Bytes(960, 2560, 15, 5, 32), "135m": Bytes(576, 1536, 9, 3, 30)}
assert BYTES["360m"].layer_bf16 == 19_664_640 and BYTES["360m"].layer_mxfp8 == 10_141_440


def step_bytes(S, layers: int = 32, weights: str = "bf16", model: str = "360m") -> int:
    """Algorithmic bytes of one step (see Bytes.step); `layers` other than the model's scales the weights."""
    b = BYTES[model]
    full = b.step(S, weights)
    return full - (b.layers - layers) * (b.layer_bf16 if weights == "bf16" else b.layer_mxfp8)


def physical_cores() -> tuple:
    """(physical cores among the CPUs this process may run on, those CPUs, os.cpu_count())."""
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        try:
            base = f"/sys/devices/system/cpu/cpu{c}/topology/"
            cores.add((int(open(base + "physical_package_id").read()), int(open(base + "core_id").read())))
        except (OSError, ValueError):
            cores.add((0, c))
    return len(cores), len(cpus), os.cpu_count()


def cpu_baseline(model: str, context: int, steps: int = 256, seconds: float = 60.0,
                 one_thread_steps: int = 16, one_thread_seconds: float = 25.0) -> dict:
    """The oracle's eager bf16 step (oracle/smollm2.py, pinned to HF eager) on this host: the median
    wall time per greedy step over `steps` steps (or as many as `seconds` allow) with one thread per
    physical core, and a 1-thread median over a shorter sample.  Untimed first step (the prefill is
    the synthetic KV context)."""
    import torch
    from oracle import smollm2 as O

    geom = O.SMOLLM2_360M if model == "360m" else O.SMOLLM2_135M
    w = O.make_weights(geom, 7)
    kv = O.make_paged_kv(geom, 1, context + steps + 64, seed=11)
    cos_sin = O.rope_cos_sin(context + steps + 64)
    n, affinity, logical = physical_cores()

    def run(threads, max_steps, budget, first_pos):
        torch.set_num_threads(threads)
        tok = O.decode_step(w, [5], [first_pos], kv, cos_sin)["ids"][0]   # untimed
        times, t_end, k = [], time.perf_counter() + budget, 1
        while k <= max_steps and time.perf_counter() < t_end:
            t0 = time.perf_counter()
            tok = O.decode_step(w, [int(tok)], [first_pos + k], kv, cos_sin)["ids"][0]
            times.append(time.perf_counter() - t0)
            k += 1
        times.sort()
        return times[len(times) // 2], len(times)

    med, done = run(n, steps, seconds, context)
    med1, done1 = run(1, one_thread_steps, one_thread_seconds, context + steps + 2)
    return {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": n, "kind": "port",
            "one_thread": {"value": round(1.0 / med1, 3), "unit": "tok/s", "steps": done1},
            "physical_cores": n, "affinity_cpus": affinity, "os_cpu_count": logical,
            "sample": f"median of {done} greedy steps of the full {model.upper()} model at context "
                      f"{context + 1}..{context + done}, {n} threads (one per physical core of this process's "
                      f"CPU set of {affinity}; os.cpu_count()={logical}); 1 thread: median of {done1} steps "
                      f"(torch {torch.__version__} CPU eager bf16)"}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--model", choices=("360m", "135m"), default="360m",
                    help="SmolLM2-360M (default; configs 3-5) or SmolLM2-135M (config 2, 512-token context)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=60.0,
                    help="time bound of the CPU baseline's multi-thread sample (256 steps at most)")
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
    if args.model == "135m" and (args.weights != "bf16" or args.lossless):
        print("--model 135m runs bf16 weights", file=sys.stderr)
        sys.exit(2)
    default_ctx = 512 if args.model == "135m" else (1024 if args.weights == "bf16" else 8192)
    context = args.context if args.context is not None else default_ctx
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

    name = {"135m": "decode_megakernel"}.get(args.model, "decode_megakernel_360m")
    mod = pk.load(name if args.weights == "bf16" else "decode_megakernel_360m_mxfp8")
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
    embed, final_norm, layers = WL.random_weights(pk.load(name).MODEL, 1234, dev)
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

    total_bytes = sum(BYTES[args.model].step([c + 1 + k for c in contexts], args.weights) - gu_bytes_saved
                      for k in range(K))
    ms_per_step = ms / K
    achieved = total_bytes / (ms * 1e-3) / 1e9
    traffic = None
    mtag = "decode135" if args.model == "135m" else "decode360"
    tname = (f"{mtag}_b{B}_ragged" if B > 1 else
             f"{mtag}_{'' if args.weights == 'bf16' else 'mxfp8_'}{'lossless_' if args.lossless else ''}ctx{context}")
    tfile = ROOT / "profiles" / f"{tname}_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    mname = "SmolLM2-135M" if args.model == "135m" else "SmolLM2-360M"
    wname = ("bf16 lossless-GU" if args.lossless else "bf16") if args.weights == "bf16" else "MXFP8-weight"
    ctx_name = f"ctx={context}" if B == 1 else "ragged ctx 128..4096"
    layers_n = len(layers)
    workload = (f"{mname.lower()} greedy decode, batch 1, {context}-token context, K steps at context "
                f"{context + 1}..{context}+K" + (", MXFP8 projection weights" if args.weights == "mxfp8" else "")
                + (", gate/up streamed through the lossless codec" if args.lossless else "")
                if B == 1 else
                f"{mname.lower()} greedy decode, batch {B}, contexts drawn uniformly from 128..4096 "
                f"(seed {args.seed}, mean {sum(contexts) / B:.0f}), K steps per sequence")
    kernel = ("split-role batch-1 kernel (contexts up to its limit; the general kernel beyond)" if B == 1 else
              "split-role batch-1 kernel, one step per sequence" if B == 2 else "batched MFMA kernel")
    line = {
        "metric": f"decode tok/s, {mname} {wname} bs={B} {ctx_name}; % of HBM roofline",
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
                   "batch": B, "context": context if B == 1 else contexts, "layers": layers_n, "weights": args.weights,
                   "gate_up": "lossless codec" if args.lossless else "dense",
                   "lm_head": "tied, fused argmax",
                   "launch": f"persistent launches of 256 workgroups (one per CU): {kernel}"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": f"profiles/{tname}_traffic.json" if traffic is not None else None,
                     "bytes_per_step": round(total_bytes / K)},
        "host_wall_ms_per_step": round(wall * 1e3 / K, 5),
    }
    if not args.no_cpu_baseline and args.weights == "bf16" and B == 1 and not args.lossless:
        line["cpu_baseline"] = cpu_baseline(args.model, context, seconds=args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
