"""Per-layer phase and exchange-wait breakdown of a batch-1 SmolLM2-360M decode step (diagnostic).

`python -m prime_kernels_amd.exchange_breakdown [--context 1024] [--out FILE.md]` runs a synthetic
32-layer step at the given context twice with timestamps on (pk_set_trace): once on the general
persistent kernel (option PK_OPT_SPLIT_ROLE = 0), and once on the split-role kernel (the default for
contexts up to its limit).  Every workgroup's first consumer wave records a 100 MHz wall-clock
timestamp at fixed points of each layer.  The report gives, per layer, the median time of each
compute phase and of each exchange, which is the wait between the last producer of a vector
finishing and the median consumer starting on it.  The exchange-wait fraction is the exchanges'
share of the layer time.  No reference counterpart: the reference kernel has no timestamps.

Trace events used (index within a layer's 40 slots):
  general kernel, every workgroup: 1 x ready, 2 QKV done; 16 attention start (q/k/v visible),
    17 local stats, 18 global stats, 19 PV done, 5 attention written (merge leaders); 7 attention
    polled, 8 O done; 10 h1 ready, 11 gate/up done; 13 act ready, 14 down done.
  split-role kernel: group F (workgroups with wg % 8 != 0) 1, 2, 10, 11, 13, 14 as above; group A
    (wg % 8 == 0) 3 attention start, 17, 18, 19 as above, 20 chunk partials published, 7 attention
    vector summed from the partials, 8 O done.
"""

from __future__ import annotations

import argparse
import json

import numpy as np
import torch

# "(rope) scores + local stats": RoPE of q is part of it on the general kernel, done by the QKV
# producers on the split-role kernel.  "partials": from P.V to the chunk partials published (the
# leader's merge included on the general kernel); "attn hop": from there to the O workgroups
# starting (which add the partials themselves on the split-role kernel).
COLUMNS = ["QKV", "qkv hop", "(rope) scores + local stats", "stats exchange", "PV", "partials",
           "attn hop", "O", "h1 hop", "gate/up", "act hop", "down", "x hop"]
EXCHANGES = {"qkv hop", "stats exchange", "partials", "attn hop", "h1 hop", "act hop", "x hop"}
WGS = 256
SLOTS = 40


def _traced_step(split_role: bool, context: int, layers: int = 32):
    """One traced step; returns (timestamps in us [WGS, layers, SLOTS], untraced step ms)."""
    import prime_kernels_amd as pk
    from prime_kernels_amd import _native, workload as WL
    from prime_kernels_amd._decode import StepLauncher

    lib = _native.library()
    old = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, 1 if split_role else 0)
    try:
        model = pk.load("decode_megakernel_360m").MODEL
        dev = torch.device("cuda:0")
        embed, final_norm, weights = WL.random_weights(model, 1234, dev, layers=layers)
        kv = WL.PagedKV(model, 1, context + 64, layers=layers, device=dev, seed=5, fill="randn")
        st = StepLauncher(model, embed=embed, layers=weights, final_norm=final_norm, kv_caches=kv.caches,
                          block_table=kv.block_table, cos_sin_cache=WL.rope_table(context + 64, device=dev),
                          first_id=17, start_pos=context, steps=8)
        stream = torch.cuda.current_stream().cuda_stream
        for k in range(4):
            st.launch(k, stream)
        torch.cuda.synchronize()
        per_wg = layers * SLOTS + 4
        buf = torch.zeros(WGS * per_wg, dtype=torch.int64, device=dev)
        st.lib.pk_set_trace(buf.data_ptr())
        try:
            st.launch(4, stream)
            torch.cuda.synchronize()
        finally:
            st.lib.pk_set_trace(None)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        st.launch(5, stream)
        e1.record()
        torch.cuda.synchronize()
        status = st.rt.pending_failure()
        if status[0] != 0:
            raise RuntimeError(f"traced step reported failure {status}")
        raw = buf.cpu().numpy().reshape(WGS, per_wg).astype(np.float64)
    finally:
        lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old)
    t0 = raw[raw > 0].min()
    us = np.where(raw > 0, (raw - t0) * 0.01, np.nan)
    return us[:, :layers * SLOTS].reshape(WGS, layers, SLOTS), e0.elapsed_time(e1)


def _rows(ev: np.ndarray, split_role: bool) -> np.ndarray:
    """Per-layer phase durations [layers - 1, len(COLUMNS)] in us."""
    md, mx = np.nanmedian, np.nanmax
    every = np.arange(WGS)
    if split_role:
        A, F = every[every % 8 == 0], every[every % 8 != 0]
        start = 3
    else:
        A = F = every
        start = 16
    out = []
    for l in range(ev.shape[1] - 1):
        e, nxt = ev[:, l, :], ev[:, l + 1, :]
        att = np.array([w for w in A if not np.isnan(e[w, start])])
        if split_role:  # every chunk publishes its partials
            lead = np.array([w for w in att if not np.isnan(e[w, 20])])
            merged = mx(e[lead, 20])
        else:
            lead = np.array([w for w in att if not np.isnan(e[w, 5])])
            merged = mx(e[lead, 5])
        ow = np.array([w for w in A if not np.isnan(e[w, 7])])
        out.append([
            md(e[F, 2]) - md(e[F, 1]), md(e[att, start]) - mx(e[F, 2]),
            md(e[att, 17]) - md(e[att, start]), md(e[att, 18]) - md(e[att, 17]),
            md(e[att, 19]) - md(e[att, 18]), merged - md(e[att, 19]),
            md(e[ow, 7]) - merged, mx(e[ow, 8]) - md(e[ow, 7]) if split_role else md(e[ow, 8]) - md(e[ow, 7]),
            md(e[F, 10]) - mx(e[ow, 8]), md(e[F, 11]) - md(e[F, 10]),
            md(e[F, 13]) - mx(e[F, 11]), md(e[F, 14]) - md(e[F, 13]), md(nxt[F, 1]) - mx(e[F, 14])])
    return np.array(out)


def breakdown(split_role: bool, context: int) -> dict:
    ev, step_ms = _traced_step(split_role, context)
    med = np.median(_rows(ev, split_role), axis=0)
    total = float(med.sum())
    wait = float(sum(v for c, v in zip(COLUMNS, med) if c in EXCHANGES))
    return {"kernel": "split_role" if split_role else "general", "context": context,
            "untraced_step_ms": round(step_ms, 4), "median_us": [round(float(v), 3) for v in med],
            "layer_us": round(total, 3), "exchange_us": round(wait, 3), "exchange_frac": round(wait / total, 4)}


def _markdown(before: dict, after: dict, command: str) -> str:
    lines = [f"# Per-layer exchange breakdown, SmolLM2-360M batch 1, context {after['context']}", "",
             f"Command: `{command}`", "",
             "Median over layers 0..30 of each phase (us), from one traced step per kernel.  An exchange is "
             "the wait from the last producer of a vector to the median consumer starting on it.", "",
             "| phase | general kernel (before) | split-role kernel (after) |", "|---|---:|---:|"]
    for i, c in enumerate(COLUMNS):
        tag = " (exchange)" if c in EXCHANGES else ""
        lines.append(f"| {c}{tag} | {before['median_us'][i]:.2f} | {after['median_us'][i]:.2f} |")
    lines += [f"| **layer total** | {before['layer_us']:.2f} | {after['layer_us']:.2f} |",
              f"| **exchange wait** | {before['exchange_us']:.2f} | {after['exchange_us']:.2f} |",
              f"| **exchange-wait fraction** | {100 * before['exchange_frac']:.0f}% | {100 * after['exchange_frac']:.0f}% |",
              f"| untraced step (ms) | {before['untraced_step_ms']:.3f} | {after['untraced_step_ms']:.3f} |", "",
              "```json", json.dumps({"before": before, "after": after}), "```", ""]
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--context", type=int, default=1024)
    ap.add_argument("--out", default=None, help="write the markdown report here")
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("exchange_breakdown needs a GPU")
    before = breakdown(False, a.context)
    after = breakdown(True, a.context)
    cmd = f"python -m prime_kernels_amd.exchange_breakdown --context {a.context}" + (f" --out {a.out}" if a.out else "")
    text = _markdown(before, after, cmd)
    print(text, flush=True)
    if a.out:
        with open(a.out, "w") as f:
            f.write(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
