"""Decode fusion probe: whole-layer kernel sequences of the Qwen3-0.6B shape
(28 layers, random weights, one decode position) captured in one HIP graph
and timed by HIP events, with per-kernel durations and launch gaps from the
kernels' own timestamps (the code object build/fusion_probe.hsaco, made by
the Makefile beside this file: the product kernels plus the probe kernels
of fusion_probe.hip, built with -DXPU_STAMPS).

Sequences per layer:
  base       QKV GEMV, attention (256 blocks: 16 heads + weight prefetch),
             o_proj + residual, RMSNorm + [gate; up] + SiLU, down + residual:
             the shipped decode's kernels and grids
  base_nopf  the same with the attention on 16 blocks (no weight prefetch)
  ctrl       the probe's unfolded attention (control for the fold kernels)
  fold16     o_proj folded into the attention, 16 blocks per head (256
             blocks, no prefetch), partials summed by the [gate; up] kernel
  fold16_g256  fold16 with the [gate; up] kernel on 256 blocks instead of 768
  fold8pf    8 blocks per head (128) + 128 prefetch blocks
  fold4pf    4 blocks per head (64) + 192 prefetch blocks
  qkv32      the QKV GEMV on 32 blocks, one head's 128 rows per block: the
             grid a QK-norm / RoPE epilogue in the QKV kernel needs

    python3 tests/fusion_probe/fusion_probe.py --position 160
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from xpu_playground_amd import BF16, Args, Runtime, check  # noqa: E402
from xpu_playground_amd import timeline as tl  # noqa: E402

MODULE = os.path.join(HERE, "build", "fusion_probe.hsaco")
H, I, HEADS, KV, HD, LAYERS, MAX_SEQ, VOCAB = 1024, 3072, 16, 8, 128, 28, 256, 151936
QD, QKV = HEADS * HD, (HEADS + 2 * KV) * HD
EPS, SCALE = 1e-6, float(np.float32(1 / np.sqrt(128.0)))
VARIANTS = ["base", "base_nopf", "ctrl", "fold16", "fold16_g256", "fold8pf", "fold4pf", "qkv32"]


class Model:
    """Random bf16 weights of `layers` layers (each layer's qkv, o, [gate;
    up] and down contiguous, as in the engine's arena), K/V caches filled
    to MAX_SEQ, two residual buffers, the decode position in `state`."""

    def __init__(self, rt: Runtime, position: int, layers: int = LAYERS):
        if not 0 <= position < MAX_SEQ:
            raise ValueError(f"position {position} outside the probe's short-context range [0, {MAX_SEQ})")
        self.rt = rt
        self.layers = []
        self.owned = []
        seed = 1
        n_w = QKV * H + H * QD + 2 * I * H + H * I
        for _ in range(layers):
            base = self._alloc(n_w * 2)
            w = {"qkv": base, "o": base + QKV * H * 2}
            w["gu"] = w["o"] + H * QD * 2
            w["down"] = w["gu"] + 2 * I * H * 2
            w["end"] = w["down"] + H * I * 2
            rt.fill_uniform(BF16, base, n_w, seed)
            seed += 1
            for name, n in (("in_norm", H), ("post_norm", H), ("q_norm", HD), ("k_norm", HD),
                            ("kc", KV * MAX_SEQ * HD), ("vc", KV * MAX_SEQ * HD)):
                w[name] = self._alloc(n * 2)
                rt.fill_uniform(BF16, w[name], n, seed)
                seed += 1
            self.layers.append(w)
        self.x = [self._alloc(H * 2), self._alloc(H * 2)]
        rt.fill_uniform(BF16, self.x[0], H, 99)
        rt.fill_uniform(BF16, self.x[1], H, 98)
        self.qkv = self._alloc(QKV * 2)
        self.attn = self._alloc(QD * 2)
        self.h = self._alloc(I * 2)
        self.parts = self._alloc(HEADS * H * 4)
        self.rope = self._alloc(2 * HD * 2)  # cos row, sin row
        rt.fill_uniform(BF16, self.rope, 2 * HD, 7)
        self.state = rt.upload(np.array([position, 0, 0, 0], np.uint32))
        self.owned.append(self.state)
        rt.synchronize()

    def _alloc(self, nbytes):
        p = self.rt.alloc(nbytes)
        self.owned.append(p)
        return p

    def close(self):
        for p in self.owned:
            self.rt.free(p)
        self.owned = []

    def _attn_args(self, w, prefetch):
        return (Args().ptr(self.qkv).ptr(w["q_norm"]).ptr(w["k_norm"]).ptr(self.rope).ptr(self.rope + HD * 2)
                .ptr(w["kc"]).ptr(w["vc"]).ptr(self.attn).ptr(self.state).u32(HEADS).u32(KV).u32(MAX_SEQ)
                .f32(EPS).f32(SCALE).ptr(w["o"]).u64(w["end"] - w["o"] if prefetch else 0))

    def layer(self, variant, w, x_in, x_out):
        """(kernel, grid, args) of one layer, and the buffer that holds the
        residual stream after it."""
        seq = [("xpu_q3_norm_gemv_r2_v2", 32 if variant == "qkv32" else 512,
                Args().ptr(w["qkv"]).ptr(x_in).ptr(w["in_norm"]).ptr(self.qkv).u32(QKV).u32(H).f32(EPS).ptr(0)
                .ptr(self.state).u32(VOCAB))]
        if variant.startswith("fold"):
            s = int(variant[4:].split("_")[0].rstrip("pf"))
            prefetch = variant.endswith("pf")
            seq.append((f"probe_attn_fold{s}", 256 if prefetch else HEADS * s,
                        self._attn_args(w, prefetch).ptr(w["o"]).ptr(self.parts).u32(H)))
            seq.append(("probe_swiglu_partials", 256 if variant.endswith("_g256") else 768,
                        Args().ptr(w["gu"]).ptr(x_in).ptr(self.parts).u32(HEADS).ptr(x_out).ptr(w["post_norm"])
                        .ptr(self.h).u32(I).u32(H).f32(EPS)))
            seq.append(("xpu_q3_gemv_residual_r1_v6", 256,
                        Args().ptr(w["down"]).ptr(self.h).ptr(x_out).u32(H).u32(I)))
            return seq, x_out
        if variant == "ctrl":
            seq.append(("probe_attn_ctrl", 256, self._attn_args(w, True).ptr(w["o"]).ptr(self.parts).u32(H)))
        else:
            nopf = variant == "base_nopf"
            seq.append(("xpu_q3_attention", HEADS if nopf else 256, self._attn_args(w, not nopf).u32(1)))
        seq.append(("xpu_q3_gemv_residual_r1_v4", 256,
                    Args().ptr(w["o"]).ptr(self.attn).ptr(x_in).u32(H).u32(QD)))
        seq.append(("xpu_q3_norm_gemv_swiglu_r2_v2", 768,
                    Args().ptr(w["gu"]).ptr(x_in).ptr(w["post_norm"]).ptr(self.h).u32(I).u32(H).f32(EPS)))
        seq.append(("xpu_q3_gemv_residual_r1_v6", 256, Args().ptr(w["down"]).ptr(self.h).ptr(x_in).u32(H).u32(I)))
        return seq, x_in

    def enqueue(self, variant, keep):
        xa, xb = self.x
        for w in self.layers:
            seq, xo = self.layer(variant, w, xa, xb)
            for name, grid, args in seq:
                keep.append(args)
                self.rt.launch_grid(name, grid, 256, 0, args)
            if xo != xa:
                xa, xb = xb, xa


def time_variant(m: Model, st: tl.Stamps, variant: str, reps: int) -> dict:
    rt = m.rt
    keep: list = []
    check(rt.lib.xpu_rt_capture_begin(rt.handle))
    m.enqueue(variant, keep)
    graph = ctypes.c_void_p()
    check(rt.lib.xpu_rt_capture_end(rt.handle, ctypes.byref(graph)))
    try:
        for _ in range(10):
            check(rt.lib.xpu_rt_graph_launch(rt.handle, graph))
        rt.synchronize()
        e0, e1 = rt.event(), rt.event()
        e0.record()
        for _ in range(reps):
            check(rt.lib.xpu_rt_graph_launch(rt.handle, graph))
        e1.record()
        rt.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / reps
        # timestamps over a few replays (each stamp slot holds 2048 records)
        st.reset()
        replays = 8
        for _ in range(replays):
            check(rt.lib.xpu_rt_graph_launch(rt.handle, graph))
        per = tl.summarize(tl.launches(st.read()))
    finally:
        check(rt.lib.xpu_rt_graph_destroy(graph))
    return {"us_per_token_layers": round(us, 2),
            "per_kernel": {k: {"launches_per_token": v["launches"] / replays, "mean_us": v["mean_us"],
                               "mean_gap_before_us": v["mean_gap_before_us"],
                               "us_per_token": round(v["total_us"] / replays, 1)} for k, v in per.items()}}


def check_layer(rt: Runtime, position: int, fold: int = 16) -> dict:
    """One layer through `base` and through the fold: the residual stream
    after o_proj (x + o, bf16) and the [gate; up] + SiLU output of each."""
    m = Model(rt, position, layers=1)
    try:
        w = m.layers[0]
        x0 = rt.download(m.x[0], H, np.uint16)
        out = {}
        for variant in ("base", f"fold{fold}"):
            rt.copy_to(m.x[0], x0)
            seq, xo = m.layer(variant, w, m.x[0], m.x[1])
            for name, grid, args in seq[:-1]:  # up to the [gate; up] kernel
                rt.launch_grid(name, grid, 256, 0, args)
            rt.synchronize()
            out[variant] = (rt.download(xo, H, np.uint16), rt.download(m.h, I, np.uint16))
        return out
    finally:
        m.close()


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="decode fusion probe (Qwen3-0.6B shape)")
    ap.add_argument("--position", type=int, default=160)
    ap.add_argument("--variants", default=",".join(VARIANTS))
    ap.add_argument("--reps", type=int, default=60)
    ap.add_argument("--out", default="")
    args = ap.parse_args(argv)
    if not os.path.exists(MODULE):
        print(f"{MODULE} is missing: make -C {HERE}", file=sys.stderr)
        return 1
    rt = Runtime(module_path=MODULE)
    st = tl.Stamps(rt)
    m = Model(rt, args.position)
    res = {"position": args.position, "variants": {}}
    for v in args.variants.split(","):
        if v not in VARIANTS:
            raise SystemExit(f"unknown variant {v}")
        print(f"== {v} (position {args.position})", flush=True)
        r = time_variant(m, st, v, args.reps)
        res["variants"][v] = r
        print(f"   {r['us_per_token_layers']:.2f} us for {LAYERS} layers", flush=True)
    m.close()
    rt.close()
    text = json.dumps(res, indent=1)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text)
    else:
        print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
