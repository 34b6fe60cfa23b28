"""Per-launch timelines from the kernels' own timestamps (no profiler).

The code object build/xpu_kernels_stamps.hsaco is the product code object
compiled with -DXPU_STAMPS: every GEMV, GEMM and fused Qwen3 decode kernel
has lane 0 of each wave record, as the wave leaves, its entry time on the
constant 100 MHz clock, its elapsed constant-clock and shader-clock ticks,
the kernel id, the block and the XCD. This module reads those records and
groups them into launches, so graph-mode decode (where rocprofv3's kernel
trace is not available here) gets per-kernel durations, the gaps between
dependent launches, and the shader clock of each XCD.

Phase marks: the GEMM body, the short-context attention and the long-context
P.V kernel also mark up to four points of their own (XPU_PHASE in the
sources), recorded for the first 1024 (block, wave) slots as shader-clock
ticks since the wave's entry. PHASES names them; `phases` in the output gives,
per kernel, the median ticks of each segment between consecutive marks (and
from the last mark to the wave's exit) over the waves that passed the marks.

    python -m xpu_playground_amd.timeline gemm --size 4096 --type bf16
    python -m xpu_playground_amd.timeline decode --prompt 128 --new 12

Launch grouping: launches on one stream do not overlap, so the records
sorted by entry time split into launches wherever the kernel id changes or
a wave enters after every earlier wave of the current launch has left.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
from collections import defaultdict

import numpy as np

from . import BF16, BUILD_DIR, FP16, Runtime, check

STAMPS_MODULE = os.path.join(BUILD_DIR, "xpu_kernels_stamps.hsaco")
TICK_NS = 10.0  # s_memrealtime: 100 MHz
RECORD = np.dtype([("start_lo", "<u4"), ("real_ticks", "<u4"), ("clock_ticks", "<u4"), ("tag", "<u4")])
KERNELS = {1: "gemv", 2: "gemm", 10: "qkv", 11: "attention", 12: "attn_scores", 13: "attn_pv", 14: "residual",
           15: "gate_up", 16: "logits", 17: "finish"}
PHASE_COUNT = 4
# segment names, one per mark and one for the rest of the wave after the last
PHASES = {
    "gemm": ["prologue (slice 0 staged, first fragments read)", "K loop (to the last MFMA issued)",
             "DMA drain and barrier", "epilogue (C through LDS to HBM)"],
    "attention": ["operand loads, QK-norm, RoPE", "scores and their maximum",
                  "exponentials and lane sums", "denominator, P.V chains, combine, store"],
    "attn_pv": ["softmax maximum (score and V loads issued)", "exponentials and denominator",
                "probabilities", "V tiles and their chains", "combine and store"],
}


class Stamps:
    """The stamp rings of a runtime created on the stamps code object."""

    def __init__(self, rt: Runtime):
        self.rt = rt
        self.seq_ptr, self.seq_bytes = self._global(b"xpu_stamp_seq")
        self.ring_ptr, self.ring_bytes = self._global(b"xpu_stamp_ring")
        self.phase_ptr, self.phase_bytes = self._global(b"xpu_stamp_phase")
        self.slots = self.seq_bytes // 4
        self.ring = self.ring_bytes // RECORD.itemsize // self.slots
        self.phase_slots = self.phase_bytes // 4 // PHASE_COUNT // self.ring

    def _global(self, name):
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        check(self.rt.lib.xpu_rt_module_global(self.rt.handle, name, ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value

    def reset(self) -> None:
        self.rt.synchronize()
        self.rt.memset(self.seq_ptr, 0, self.seq_bytes)
        self.rt.synchronize()

    def read(self) -> np.ndarray:
        """All records written since reset(), sorted by entry time."""
        self.rt.synchronize()
        seq = self.rt.download(self.seq_ptr, self.slots, np.uint32)
        if int(seq.max(initial=0)) > self.ring:
            raise RuntimeError(f"a stamp slot wrapped ({int(seq.max())} > {self.ring} records): time fewer launches")
        raw = self.rt.download(self.ring_ptr, self.ring_bytes, np.uint8).view(RECORD).reshape(self.slots, self.ring)
        keep = np.arange(self.ring)[None, :] < seq[:, None]
        recs = raw[keep]
        slot, pos = np.nonzero(keep)
        marks = self.rt.download(self.phase_ptr, self.phase_bytes // 4, np.uint32).reshape(
            self.phase_slots, self.ring, PHASE_COUNT)
        phases = np.zeros((slot.size, PHASE_COUNT), np.uint32)
        lo_slot = slot < self.phase_slots
        phases[lo_slot] = marks[slot[lo_slot], pos[lo_slot]]
        # entry times from the low 32 bits (43 s period) relative to the
        # earliest, across at most one wrap
        lo = recs["start_lo"].astype(np.int64)
        if lo.size and lo.max() - lo.min() > (1 << 31):
            lo = np.where(lo < (1 << 31), lo + (1 << 32), lo)
        out = np.zeros(lo.size, dtype=[("real_start", "<i8"), ("real_ticks", "<u4"), ("clock_ticks", "<u4"),
                                       ("kernel", "<u4"), ("xcc", "<u4"), ("block", "<u4"),
                                       ("phases", "<u4", (PHASE_COUNT,))])
        out["phases"] = phases
        out["real_start"] = lo - (lo.min() if lo.size else 0)
        out["real_ticks"], out["clock_ticks"] = recs["real_ticks"], recs["clock_ticks"]
        out["kernel"] = recs["tag"] >> 24
        out["xcc"] = (recs["tag"] >> 20) & 15
        out["block"] = recs["tag"] & 0xFFFF
        return out[np.argsort(out["real_start"], kind="stable")]


def launches(recs: np.ndarray) -> list[dict]:
    out: list[dict] = []
    cur = None
    for r in recs:
        start, end = int(r["real_start"]), int(r["real_start"]) + int(r["real_ticks"])
        if cur is None or r["kernel"] != cur["kernel"] or start >= cur["end"]:
            cur = {"kernel": int(r["kernel"]), "start": start, "end": end, "waves": 0, "clock": defaultdict(list),
                   "residency": [], "block_end": {}, "marks": []}
            out.append(cur)
        cur["end"] = max(cur["end"], end)
        b = int(r["block"])
        cur["block_end"][b] = max(cur["block_end"].get(b, 0), end)
        cur["waves"] += 1
        if r["real_ticks"]:
            cur["clock"][int(r["xcc"])].append(r["clock_ticks"] / (r["real_ticks"] * TICK_NS))
        cur["residency"].append(int(r["clock_ticks"]))
        if r["phases"].any():
            cur["marks"].append([int(x) for x in r["phases"]] + [int(r["clock_ticks"])])
    for i, ln in enumerate(out):
        ln["name"] = KERNELS.get(ln["kernel"], str(ln["kernel"]))
        if ln["name"] == "residual":  # o_proj follows the attention, down_proj the gate/up kernel
            ln["name"] = "down" if i and out[i - 1]["name"] == "gate_up" else "o_proj"
        ln["us"] = (ln["end"] - ln["start"]) * TICK_NS / 1e3
        ln["gap_us"] = (ln["start"] - out[i - 1]["end"]) * TICK_NS / 1e3 if i else 0.0
        ln["ghz_by_xcc"] = {x: float(np.median(v)) for x, v in sorted(ln["clock"].items())}
        ln["max_wave_cycles"] = max(ln["residency"])
        ln["median_wave_cycles"] = float(np.median(ln["residency"]))
    return out


def phase_segments(marks: list[list[int]]) -> list[float] | None:
    """Median shader-clock ticks of each segment, over the waves that passed
    every mark the kernel's waves pass (marks of 0 are marks not passed):
    entry to the first mark, mark to mark, the last mark to the exit."""
    if not marks:
        return None
    m = np.asarray(marks, np.int64)
    used = [i for i in range(PHASE_COUNT) if m[:, i].any()]
    m = m[np.all(m[:, used] > 0, axis=1)][:, used + [PHASE_COUNT]]
    if not m.size:
        return None
    seg = np.diff(np.concatenate([np.zeros((m.shape[0], 1), np.int64), m], axis=1), axis=1)
    return [round(float(v), 0) for v in np.median(seg, axis=0)]


def phase_table(name: str, marks: list[list[int]]) -> dict | None:
    seg = phase_segments(marks)
    if seg is None:
        return None
    labels = PHASES.get(name, [f"segment {i}" for i in range(len(seg))])
    return {"waves": len(marks), "median_cycles": dict(zip(labels, seg))}


def summarize(lns: list[dict]) -> dict:
    by = defaultdict(list)
    for ln in lns:
        by[ln["name"]].append(ln)
    table = {}
    for name, group in by.items():
        clocks = [c for ln in group for c in ln["ghz_by_xcc"].values()]
        table[name] = {
            "launches": len(group),
            "mean_us": round(float(np.mean([g["us"] for g in group])), 3),
            "mean_gap_before_us": round(float(np.mean([g["gap_us"] for g in group])), 3),
            "total_us": round(float(np.sum([g["us"] + g["gap_us"] for g in group])), 1),
            "median_wave_cycles": round(float(np.median([g["median_wave_cycles"] for g in group])), 0),
            "max_wave_cycles": int(max(g["max_wave_cycles"] for g in group)),
            "shader_ghz_min_med_max": [round(min(clocks), 3), round(float(np.median(clocks)), 3),
                                       round(max(clocks), 3)] if clocks else None,
        }
        phases = phase_table(name, [mk for g in group for mk in g["marks"]])
        if phases:
            table[name]["phases"] = phases
    return table


def run_gemm(args) -> dict:
    rt = Runtime(module_path=args.module)
    st = Stamps(rt)
    dt = FP16 if args.type == "fp16" else BF16
    m, n, k = (args.size,) * 3 if args.size else (args.m, args.n, args.k)
    a, b, c = rt.alloc(m * k * 2), rt.alloc(k * n * 2), rt.alloc(m * n * 2)
    rt.fill_uniform(dt, a, m * k, 5)
    rt.fill_uniform(dt, b, k * n, 6)
    rt.synchronize()
    st.reset()
    for _ in range(args.steps):
        rt.gemm(dt, a, b, c, m, n, k)
    lns = [ln for ln in launches(st.read()) if ln["name"] == "gemm"]
    flop = 2.0 * m * n * k
    per = [{"us": round(ln["us"], 2), "tflops": round(flop / (ln["us"] * 1e-6) / 1e12, 1),
            "ghz_by_xcc": {x: round(v, 3) for x, v in ln["ghz_by_xcc"].items()},
            "median_wave_cycles": ln["median_wave_cycles"], "max_wave_cycles": ln["max_wave_cycles"],
            "gap_us": round(ln["gap_us"], 2), "phases": phase_table("gemm", ln["marks"])} for ln in lns]
    rt.close()
    return {"workload": f"gemm {args.type} {m}x{n}x{k}", "launches": per}


def run_decode(args) -> dict:
    from . import qwen3

    rt = Runtime(module_path=args.module)
    st = Stamps(rt)
    cfg = qwen3.preset(args.preset)
    max_seq = args.prompt + args.new
    eng = qwen3.Engine(cfg, max_seq=max_seq, seed=0, gain_std=0.0, runtime=rt)
    eng.set_mode(qwen3.GRAPH if args.mode == "graph" else qwen3.EAGER)
    prompt = qwen3.prompt_tokens(args.prompt, 1, cfg.vocab)
    eng.generate(prompt, args.new, stop_on_eos=False)  # builds the graphs
    st.reset()
    out, pm, dm = eng.generate(prompt, args.new, stop_on_eos=False)
    lns = launches(st.read())
    # the decode steps: the launches after the last prompt step's finish
    finishes = [i for i, ln in enumerate(lns) if ln["name"] == "finish"]
    first = finishes[-(len(out) - 1) - 1] + 1 if len(finishes) >= len(out) else 0
    steps = lns[first:]
    token_us = (steps[-1]["end"] - steps[0]["start"]) * TICK_NS / 1e3 / max(1, len(out) - 1)
    # the attention kernel: its query-head blocks against the blocks that
    # prefetch the layer's remaining weights
    att = [ln for ln in steps if ln["name"] == "attention"]
    heads_us = [(max(v for b, v in ln["block_end"].items() if b < cfg.heads) - ln["start"]) * TICK_NS / 1e3
                for ln in att]
    rest_us = [(max((v for b, v in ln["block_end"].items() if b >= cfg.heads), default=ln["start"]) - ln["start"])
               * TICK_NS / 1e3 for ln in att]
    eng.close()
    rt.close()
    return {"workload": f"{args.preset} decode, {args.prompt} prompt ids, {args.new} new tokens, {args.mode} mode",
            "decode_ms_events": round(dm, 3), "tok_s_events": round((len(out) - 1) / dm * 1e3, 1),
            "token_us_stamps": round(token_us, 2), "kernels_per_token": len(steps) / max(1, len(out) - 1),
            "attention_head_blocks_mean_us": round(float(np.mean(heads_us)), 3) if heads_us else None,
            "attention_prefetch_blocks_mean_us": round(float(np.mean(rest_us)), 3) if rest_us else None,
            "per_kernel": summarize(steps)}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="what", required=True)
    g = sub.add_parser("gemm")
    g.add_argument("--size", type=int, default=4096)
    g.add_argument("--m", type=int, default=0)
    g.add_argument("--n", type=int, default=0)
    g.add_argument("--k", type=int, default=0)
    g.add_argument("--type", choices=["bf16", "fp16"], default="bf16")
    g.add_argument("--steps", type=int, default=25)
    d = sub.add_parser("decode")
    d.add_argument("--preset", default="qwen3-0.6b")
    d.add_argument("--prompt", type=int, default=128)
    d.add_argument("--new", type=int, default=12)
    d.add_argument("--mode", choices=["graph", "eager"], default="graph")
    for p in (g, d):
        p.add_argument("--module", default=STAMPS_MODULE, help="a code object built with -DXPU_STAMPS")
    args = ap.parse_args(argv)
    if not os.path.exists(args.module):
        print(f"{args.module} is missing: build it (make -C xpu_playground_amd/csrc)", file=sys.stderr)
        return 1
    if args.what == "gemm" and (args.m or args.n or args.k):
        args.size = 0
    res = run_gemm(args) if args.what == "gemm" else run_decode(args)
    print(json.dumps(res, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
