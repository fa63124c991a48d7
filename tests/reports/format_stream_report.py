"""Format the per-step JSON files that tests/test_gpu_stream.py writes (with PK_STREAM_REPORT set)
into one markdown report:

    PK_STREAM_REPORT=out python -m pytest tests/test_gpu_stream.py -m gpu -s
(the batch-16 and HF streams add their sections when their JSON files are present)
    python tests/reports/format_stream_report.py out tests/reports/stream_full_depth.md
"""

import json
import sys
from pathlib import Path

ORDER = [("stream_135m_ctx512", "config 2: SmolLM2-135M, 512-token prompt"),
         ("stream_135m_ctx1200", "SmolLM2-135M, 1200-token prompt"),
         ("stream_360m_ctx1024", "config 3: SmolLM2-360M, 1024-token prompt"),
         ("stream_360m_mxfp8_ctx8192", "config 5: SmolLM2-360M MXFP8, 8192-token prompt")]


def main(src: str, dst: str) -> None:
    out = ["# Full-depth 256-step streams against the oracle", "",
           "Made by `PK_STREAM_REPORT=out python -m pytest tests/test_gpu_stream.py -m gpu -s` on an MI355X, then "
           "`python tests/reports/format_stream_report.py out tests/reports/stream_full_depth.md`.  Teacher-forced "
           "token stream (each step feeds the oracle's greedy id); the kernel, the CPU oracle and eager PyTorch on "
           "the GPU each keep their own KV cache.  Errors are max abs over the 49,152 bf16 logits.", "",
           "| stream | kernel max / mean err | eager-GPU max / mean err | kernel min cos | eager min cos | "
           "argmax agree kernel | argmax agree eager | largest oracle margin at a kernel flip | logits bound | "
           "cache: kernel / eager max err, untouched slots equal |", "|---|---|---|---|---|---|---|---|---|---|"]
    data = {}
    for name, _ in ORDER:
        p = Path(src) / f"{name}.json"
        if p.exists():
            data[name] = json.loads(p.read_text())
    for name, title in ORDER:
        if name not in data:
            continue
        s = data[name]["summary"]
        k, e, b, cl = s["kernel"], s["eager_gpu"], s["bounds"], s["cache_layers"]
        out.append(f"| {title} | {k['max_err']:.4f} / {k['mean_err']:.4f} | {e['max_err']:.4f} / {e['mean_err']:.4f} | "
                   f"{k['min_cos']:.5f} | {e['min_cos']:.5f} | {k['argmax_agree']}/{s['steps']} | "
                   f"{e['argmax_agree']}/{s['steps']} | {max(k['mismatch_margins'], default=0):.4f} | "
                   f"{b['logits_max']:.4f} | {max(c['kernel_err'] for c in cl):.4f} / "
                   f"{max(c['eager_err'] for c in cl):.4f}, {all(c['untouched_equal'] for c in cl)} |")
    for name, title in ORDER:
        if name not in data:
            continue
        rows = data[name]["steps"]
        out += ["", f"## {title}", "",
                "Per step: `step: kernel err / eager err`, with `K` where the kernel's greedy id differs from the "
                "oracle's, `E` where eager-GPU's does, and the oracle's top-2 margin after `m=` at such steps.", "",
                "```"]
        line = []
        for r in rows:
            flag = ("K" if r["kernel_id"] != r["oracle_id"] else "") + ("E" if r["eager_id"] != r["oracle_id"] else "")
            cell = f"{r['step']:3d}: {r['kernel_err']:.3f}/{r['eager_err']:.3f}"
            if flag:
                cell += f" {flag} m={r['oracle_margin']:.3f}"
            line.append(f"{cell:<34s}")
            if len(line) == 4:
                out.append("".join(line).rstrip())
                line = []
        if line:
            out.append("".join(line).rstrip())
        out += ["```", "", "Whole cache after the stream, per layer (max abs err of the appended K/V; kernel / eager):", "",
                "```", " ".join(f"{c['layer']}:{c['kernel_err']:.3f}/{c['eager_err']:.3f}"
                                for c in data[name]["summary"]["cache_layers"]), "```"]
    b16 = Path(src) / "stream_360m_b16_ragged.json"
    if b16.exists():
        s_ = json.loads(b16.read_text())["summary"]
        k, e, b = s_["kernel"], s_["eager_gpu"], s_["bounds"]
        n = s_["steps"] * s_["sequences"]
        out += ["", "## Config 4: SmolLM2-360M, 16 ragged sequences (batched kernel)", "",
                f"Contexts {s_['contexts']}, {s_['steps']} teacher-forced steps per sequence ({n} sequence-steps).", "",
                "| kernel max / mean err | eager-GPU max / mean err | kernel min cos | eager min cos | argmax agree kernel | "
                "argmax agree eager | largest oracle margin at a kernel flip | logits bound | cache: kernel / eager max err, "
                "untouched slots equal |", "|---|---|---|---|---|---|---|---|---|",
                f"| {k['max_err']:.4f} / {k['mean_err']:.4f} | {e['max_err']:.4f} / {e['mean_err']:.4f} | {k['min_cos']:.5f} | "
                f"{e['min_cos']:.5f} | {k['argmax_agree']}/{n} | {e['argmax_agree']}/{n} | "
                f"{max(k['mismatch_margins'], default=0):.4f} | {b['logits_max']:.4f} | "
                f"{s_['cache']['kernel_max_err']:.4f} / {s_['cache']['eager_max_err']:.4f}, {s_['cache']['untouched_equal']} |"]
    hf = [("hf_config2_135m", "config 2: SmolLM2-135M, HF's 512-token prompt pass and 256 greedy ids"),
          ("hf_config3_360m", "config 3: SmolLM2-360M, HF's 1024-token prompt pass and 256 greedy ids")]
    hf_data = {n: json.loads((Path(src) / f"{n}.json").read_text()) for n, _ in hf if (Path(src) / f"{n}.json").exists()}
    if hf_data:
        out += ["", "## Against HF transformers itself (tests/golden/config*_full.npz)", "",
                "Teacher-forced over HF's own greedy stream from its prompt pass (the oracle's batched prompt pass "
                "rebuilds the cache; `HF cache bits` says whether the box's CPU reproduced HF's cache bit for bit). "
                "Errors are max abs over HF's top-32 logits of each step.", "",
                "| stream | HF cache bits | kernel max / mean err | eager-GPU max / mean err | argmax agree kernel | "
                "argmax agree eager | HF margins at kernel flips | top-32 bound |", "|---|---|---|---|---|---|---|---|"]
        for n, title in hf:
            if n not in hf_data:
                continue
            s_ = hf_data[n]["summary"]
            k, e = s_["kernel"], s_["eager_gpu"]
            steps = len(hf_data[n]["steps"])
            out.append(f"| {title} | {s_['prompt_cache_is_hf_bits']} | {k['top32_max_err']:.4f} / {k['top32_mean_err']:.4f} | "
                       f"{e['top32_max_err']:.4f} / {e['top32_mean_err']:.4f} | {k['argmax_agree']}/{steps} | "
                       f"{e['argmax_agree']}/{steps} | {k['mismatch_margins']} | {s_['bounds']['top32_max']:.4f} |")
    Path(dst).write_text("\n".join(out) + "\n")


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
