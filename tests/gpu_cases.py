"""Shared helpers for the GPU parity tests: identical inputs for the HIP kernel and the CPU oracle.

Weights and paged KV caches are built on the CPU (seeded), the oracle (oracle/smollm2.py) runs on
those CPU tensors, and the kernel runs on GPU copies of the very same bits.
"""

from __future__ import annotations

import math

import torch

from oracle import smollm2 as O

BF16 = torch.bfloat16
LOGIT_ATOL = 2e-2      # north-star tolerance on bf16 logits (max abs err)
COS_MIN = 0.9999       # north-star cosine similarity on logits


def module_for(geom: O.Geometry):
    import prime_kernels_amd as pk

    return pk.load("decode_megakernel_360m" if geom.hidden == 960 else "decode_megakernel")


class Case:
    """One decode step's inputs, on CPU (oracle) and GPU (kernel)."""

    def __init__(self, geom: O.Geometry, w: O.Weights, kv: O.PagedKV, max_pos: int, dev="cuda:0"):
        self.geom, self.w, self.kv = geom, w, kv
        self.cos_sin = O.rope_cos_sin(max_pos, geom.head_dim, geom.theta)
        self.dev = torch.device(dev)
        self.wd = w.to(self.dev)
        self.kvd = [c.to(self.dev) for c in kv.caches]
        self.btd = kv.block_table.to(self.dev)
        self.csd = self.cos_sin.to(self.dev)
        self.mod = module_for(geom)
        self.kernel_layers = self.wd.layers  # what the kernel is given (bf16, or MXFP8 10-tuples)

    def sync_kv_from_oracle(self) -> None:
        for g, c in zip(self.kvd, self.kv.caches):
            g.copy_(c)

    def kernel_step(self, ids, positions, seq_lens=None, slot_mapping=None, *, logits=True, layer_outputs=False,
                    ids_dtype=torch.int64, cs_fp32=False, block_rows=None):
        """One kernel step; `block_rows` picks the block-table rows (default: row b for sequence b)."""
        B = len(ids)
        dev = self.dev
        pos = torch.tensor(positions, dtype=torch.int64, device=dev)
        sl = torch.tensor(seq_lens if seq_lens is not None else [p + 1 for p in positions], dtype=torch.int32, device=dev)
        if slot_mapping is None:
            slot_mapping = [self.kv.slot(b, int(sl[b]) - 1) for b in range(B)]
        slots = torch.tensor(slot_mapping, dtype=torch.int64, device=dev)
        lg = torch.empty((B, self.geom.vocab), dtype=BF16, device=dev) if logits else None
        lo = torch.empty((self.geom.layers, B, self.geom.hidden), dtype=BF16, device=dev) if layer_outputs else None
        cs = self.csd.float().contiguous() if cs_fp32 else self.csd
        hid, out_ids = self.mod.decode_step(
            input_ids=torch.tensor(ids, dtype=ids_dtype, device=dev), positions=pos, seq_lens=sl,
            block_table=self.btd if block_rows is None else self.btd[list(block_rows)].contiguous(),
            slot_mapping=slots, embed=self.wd.embed, layers=self.kernel_layers,
            final_norm=self.wd.final_norm, kv_caches=self.kvd, cos_sin_cache=cs, eps=1e-5,
            num_layers=self.geom.layers, return_token_ids=True, logits_out=lg, layer_outputs=lo)
        torch.cuda.synchronize()
        rt = self.mod.workspace(dev)
        ep, site = rt.pending_failure()
        assert ep == 0, f"kernel abandoned a bounded wait (wait site {site}, epoch {ep})"
        res = {"hidden": hid.clone().cpu(), "ids": out_ids.clone().cpu()}
        if logits:
            res["logits"] = lg.cpu()
        if layer_outputs:
            res["layer_outputs"] = lo.cpu()
        return res

    def oracle_step(self, ids, positions, seq_lens=None, slot_mapping=None, layer_outputs=False):
        return O.decode_step(self.w, ids, positions, self.kv, self.cos_sin, seq_lens=seq_lens,
                             slot_mapping=slot_mapping, layer_outputs=layer_outputs)

    def eager_gpu_step(self, ids, positions, layer_outputs=False):
        """The oracle's eager algorithm on GPU tensors (PyTorch's GPU BLAS and kernels): a second
        implementation of the same rounding points, differing only in accumulation order.  Its
        distance from the CPU oracle is the noise floor a correct kernel cannot beat at full
        depth, where random-init layers amplify last-bit differences.  Call before oracle_step
        of the same step (it reads the CPU caches, which oracle_step appends to)."""
        kvg = O.PagedKV([c.to(self.dev) for c in self.kv.caches], self.btd, self.kv.block_size)
        wg = O.Weights(self.geom, self.wd.embed, self.wd.final_norm, self.wd.layers)
        r = O.decode_step(wg, ids, positions, kvg, self.csd, layer_outputs=layer_outputs)
        return {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in r.items()}

    TF_ROW = 0  # embedding row that carries a teacher-forced hidden state

    def teacher_forced_layer(self, li: int, x_in: torch.Tensor, position: int, *, logits=False):
        """Layer `li` alone through the kernel (num_layers=1, that layer's weights and cache) with
        the hidden state `x_in` [H] as its input, placed in row TF_ROW of a copy of the embedding.
        Returns the layer output [H] (and the final-norm hidden state and logits if asked; the
        embedding is tied, so logit TF_ROW is x_in's own and is not comparable)."""
        if not hasattr(self, "_embed_tf"):
            self._embed_tf = self.wd.embed.clone()
        self._embed_tf[self.TF_ROW] = x_in.to(self.dev, BF16)
        dev = self.dev
        lo = torch.empty((1, 1, self.geom.hidden), dtype=BF16, device=dev)
        lg = torch.empty((1, self.geom.vocab), dtype=BF16, device=dev) if logits else None
        hid, ids = self.mod.decode_step(
            input_ids=torch.tensor([self.TF_ROW], device=dev), positions=torch.tensor([position], device=dev),
            seq_lens=torch.tensor([position + 1], dtype=torch.int32, device=dev), block_table=self.btd,
            slot_mapping=torch.tensor([self.kv.slot(0, position)], device=dev), embed=self._embed_tf,
            layers=[self.kernel_layers[li]], final_norm=self.wd.final_norm, kv_caches=[self.kvd[li]],
            cos_sin_cache=self.csd, eps=1e-5, num_layers=1, return_token_ids=True, logits_out=lg,
            layer_outputs=lo)
        torch.cuda.synchronize()
        res = {"out": lo[0, 0].cpu(), "hidden": hid[0].cpu(), "ids": ids.cpu()}
        if logits:
            res["logits"] = lg[0].cpu()
        return res


def teacher_forced_layer_batch(case: "Case", li: int, x_in: torch.Tensor, positions, *, logits=False):
    """Layer `li` alone through the kernel for B sequences at once: x_in [B, H] is placed in
    embedding rows 0..B-1 of a copy of the embedding and token b is row b.  Returns the layer
    outputs [B, H] (and the logits [B, V] if asked; logits 0..B-1 are the inputs' own rows)."""
    B = x_in.shape[0]
    dev = case.dev
    if not hasattr(case, "_embed_tfb"):
        case._embed_tfb = case.wd.embed.clone()
    case._embed_tfb[:B] = x_in.to(dev, BF16)
    lo = torch.empty((1, B, case.geom.hidden), dtype=BF16, device=dev)
    lg = torch.empty((B, case.geom.vocab), dtype=BF16, device=dev) if logits else None
    slots = [case.kv.slot(b, positions[b]) for b in range(B)]
    case.mod.decode_step(
        input_ids=torch.arange(B, device=dev), positions=torch.tensor(positions, device=dev),
        seq_lens=torch.tensor([p + 1 for p in positions], dtype=torch.int32, device=dev), block_table=case.btd,
        slot_mapping=torch.tensor(slots, device=dev), embed=case._embed_tfb, layers=[case.kernel_layers[li]],
        final_norm=case.wd.final_norm, kv_caches=[case.kvd[li]], cos_sin_cache=case.csd, eps=1e-5, num_layers=1,
        return_token_ids=True, logits_out=lg, layer_outputs=lo)
    torch.cuda.synchronize()
    res = {"out": lo[0].cpu()}
    if logits:
        res["logits"] = lg.cpu()
    return res


def mxfp8_case(geom: O.Geometry, seed: int, contexts, *, norm_jitter=0.05, fill_seed: int | None = None) -> Case:
    """A case whose kernel runs MXFP8 weights quantised on the GPU by the library, while the
    oracle (and the eager-GPU floor) run the exact bf16 dequantisation of those same codes."""
    from oracle import mxfp8 as MX
    import prime_kernels_amd as pk

    w = O.make_weights(geom, seed, norm_jitter=norm_jitter)
    mod = pk.load("decode_megakernel_360m_mxfp8")
    dev = torch.device("cuda:0")
    qlayers = mod.quantize_layers([tuple(t.to(dev) for t in layer) for layer in w.layers])
    torch.cuda.synchronize()
    deq = [MX.dequantize_layer(tuple(t.cpu().numpy() if t.dtype == torch.uint8 else t.cpu() for t in ql))
           for ql in qlayers]
    wq = O.Weights(geom, w.embed, w.final_norm, deq)
    cap = max(contexts) + 16
    kv = O.make_paged_kv(geom, len(contexts), cap, seed=fill_seed if fill_seed is not None else seed + 3)
    case = Case(geom, wq, kv, cap + 16)
    case.mod = mod
    case.kernel_layers = qlayers
    return case


def compare_logits(k: torch.Tensor, r: torch.Tensor) -> dict:
    kf, rf = k.float(), r.float()
    err = (kf - rf).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(kf.flatten(), rf.flatten(), dim=0).item()
    return {"max_abs": err, "cos": cos}


def greedy_ok(kernel_id: int, ref_logits: torch.Tensor, tol: float = LOGIT_ATOL) -> bool:
    """Greedy id matches the oracle's argmax, or the oracle itself has a near-tie (top-1 minus the
    kernel's pick within the logit tolerance), which bf16-tolerance parity cannot resolve."""
    ref = ref_logits.float()
    best = int(torch.argmax(ref))
    if kernel_id == best:
        return True
    return (ref[best] - ref[kernel_id]).item() <= tol


def random_kv_case(geom: O.Geometry, seed: int, contexts, *, max_pos: int | None = None, norm_jitter=0.05,
                   fill_seed: int | None = None, extra_blocks: int = 0, capacity: int | None = None) -> Case:
    """`capacity`: tokens the block table addresses (default: the longest context + 16)."""
    w = O.make_weights(geom, seed, norm_jitter=norm_jitter)
    cap = capacity if capacity is not None else max(contexts) + 16
    kv = O.make_paged_kv(geom, len(contexts), cap, seed=fill_seed if fill_seed is not None else seed + 3,
                         extra_blocks=extra_blocks)
    return Case(geom, w, kv, max_pos or cap + 16)


def assert_step_parity(kres: dict, rres: dict, label: str = "") -> dict:
    out = {}
    for b in range(kres["hidden"].shape[0]):
        c = compare_logits(kres["logits"][b], rres["logits"][b])
        assert c["max_abs"] <= LOGIT_ATOL, f"{label} b={b} logits max abs err {c['max_abs']}"
        assert c["cos"] >= COS_MIN, f"{label} b={b} logits cosine {c['cos']}"
        h = compare_logits(kres["hidden"][b], rres["hidden"][b])
        assert h["cos"] >= COS_MIN, f"{label} b={b} hidden cosine {h['cos']}"
        assert greedy_ok(int(kres["ids"][b]), rres["logits"][b]), \
            f"{label} b={b} greedy id {int(kres['ids'][b])} vs oracle {int(rres['ids'][b])}"
        out[b] = c
    return out


FLOOR_FACTOR = 2.0     # full depth: kernel error may be at most this multiple of the eager-vs-eager floor


def assert_within_floor(kres: dict, rres: dict, floor: dict, label: str = "") -> dict:
    """Full-depth parity of a free-running step.  The north-star bound (LOGIT_ATOL, COS_MIN) is
    unreachable there even for PyTorch eager on the GPU against PyTorch eager on the CPU: 30+
    random-init layers amplify last-bit accumulation-order differences (GPU eager vs oracle at
    SmolLM2-360M ctx 1024 measures about 0.07 max abs, cosine 0.9996).  The bar is therefore the
    larger of the north-star bound and FLOOR_FACTOR times that measured floor; the per-layer
    teacher-forced tests hold every layer to the north-star bound itself."""
    out = {}
    for b in range(kres["logits"].shape[0]):
        c = compare_logits(kres["logits"][b], rres["logits"][b])
        f = compare_logits(floor["logits"][b], rres["logits"][b])
        atol = max(LOGIT_ATOL, FLOOR_FACTOR * f["max_abs"])
        cos_min = min(COS_MIN, 1.0 - FLOOR_FACTOR * (1.0 - f["cos"]))
        assert c["max_abs"] <= atol, f"{label} b={b} logits max abs err {c['max_abs']} > {atol} (floor {f})"
        assert c["cos"] >= cos_min, f"{label} b={b} logits cosine {c['cos']} < {cos_min} (floor {f})"
        assert greedy_ok(int(kres["ids"][b]), rres["logits"][b], tol=atol), \
            f"{label} b={b} greedy id {int(kres['ids'][b])} vs oracle {int(rres['ids'][b])}"
        out[b] = {"kernel": c, "eager_gpu_floor": f}
    return out if len(out) > 1 else out[0]


SEED_SET_HARD_ATOL = 2 * LOGIT_ATOL   # no case of a seed set may exceed this
SEED_SET_MEAN_FACTOR = 1.5            # mean error at most this multiple of eager-GPU's (or LOGIT_ATOL / 2)


def assert_seed_set_parity(cases: list, label: str = "") -> dict:
    """Parity of a shallow model over a set of seeds, each case a (kernel, eager_gpu, oracle) triple
    of single-sequence step results.  At two random-init layers the north-star bound sits at the
    noise level of accumulation order: one bf16 rounding that flips early in layer 0 spreads
    one-ulp differences through the step and moves the logits by 0.015-0.025, and over 60 seeded
    2-layer 360M steps (bf16 and MXFP8, contexts 1025..2049) PyTorch eager on the GPU exceeds
    LOGIT_ATOL against the CPU oracle on 3 and the kernel on 2; which seeds do changes whenever
    either side's summation order changes.  So every case must meet COS_MIN, pick the oracle's
    greedy id (or a near-tie) and stay within SEED_SET_HARD_ATOL, and the mean logits error over
    the set may be at most SEED_SET_MEAN_FACTOR times eager-GPU's mean on the same seeds (or
    LOGIT_ATOL / 2, whichever is larger)."""
    errs, floors = [], []
    for i, (k, e, r) in enumerate(cases):
        c = compare_logits(k["logits"][0], r["logits"][0])
        f = compare_logits(e["logits"][0], r["logits"][0])
        assert c["cos"] >= COS_MIN, f"{label} case {i}: logits cosine {c['cos']}"
        assert c["max_abs"] <= SEED_SET_HARD_ATOL, f"{label} case {i}: logits max abs err {c['max_abs']}"
        assert greedy_ok(int(k["ids"][0]), r["logits"][0]), \
            f"{label} case {i}: greedy id {int(k['ids'][0])} vs oracle {int(r['ids'][0])}"
        errs.append(c["max_abs"])
        floors.append(f["max_abs"])
    mean, floor = sum(errs) / len(errs), sum(floors) / len(floors)
    bar = max(LOGIT_ATOL / 2, SEED_SET_MEAN_FACTOR * floor)
    assert mean <= bar, f"{label}: mean logits max abs err {mean} > {bar} (eager GPU mean {floor})"
    return {"cases": len(cases), "mean": mean, "eager_mean": floor, "worst": max(errs),
            "over_atol": sum(x > LOGIT_ATOL for x in errs), "eager_over_atol": sum(x > LOGIT_ATOL for x in floors)}


def identical_fraction(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.to(BF16).view(torch.int16) == b.to(BF16).view(torch.int16)).float().mean().item())


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> int:
    return O.max_ulp(a, b)


def finite(t: torch.Tensor) -> bool:
    return bool(torch.isfinite(t.float()).all())


__all__ = ["Case", "compare_logits", "greedy_ok", "random_kv_case", "assert_step_parity", "assert_within_floor",
           "identical_fraction", "LOGIT_ATOL", "COS_MIN", "FLOOR_FACTOR", "math"]
