#!/usr/bin/env python3
"""Where the CPU oracle's Qwen3 decode departs from transformers, op by op
(run in the build container, never on the GPU box).

For a case of make_qwen3_golden.py, transformers' Qwen3ForCausalLM (eager,
bf16, the model qwen3/reference.py:15-24 builds) runs the one-position step
path (the engine's order, qwen3/main.cpp:343-352) over the prompt and the
greedy steps, with every op's bf16 input and output recorded. Each op is
then recomputed by the oracle's own primitive from transformers' input
(op-local: no error carried in from earlier ops), and the two outputs are
compared code by code:

  in_norm, post_norm, final_norm   RMSNorm            orc_rmsnorm
  q_norm, k_norm                   per-head RMSNorm   orc_rmsnorm
  rope_q, rope_k                   RoPE rotation      the oracle's formula, with
                                   transformers' cos/sin rows and with the
                                   oracle's tables (rope_*_tables)
  q, k, v, o, gate, up, down,      GEMV               orc_gemv_canonical
  lm_head
  attention                        one query head     orc_attention_head
  add_attn, add_mlp                residual add       orc_add
  silu_mul                         bf16(silu(g)) * u  orc_silu_mul

For every op: elements compared, elements that differ, the largest code
distance (bf16 codes of one sign are ordered, so the distance is the number
of representable steps between the two values), and for the sums (GEMVs,
norms' outputs) how many outputs of each side equal the FP64 result rounded
to bf16 (both sides accumulate in FP32; if each misses the FP64 rounding
about equally often, the difference is summation order, not a rounding
point). The cumulative view composes the oracle's primitives into its decode
(bit-identical to orc_qwen3_decode, checked on the logits) and reports the
first position, layer and op where its stream leaves transformers'.

Usage: python tests/golden/qwen3_op_diff.py [case ...]   (default small-varied)
Writes tests/golden/qwen3_opdiff_<case>.json.
"""
from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)
import oracle_lib as orc  # noqa: E402
from make_qwen3_golden import build_hf, case  # noqa: E402


def codes(t) -> np.ndarray:
    import torch

    return t.detach().contiguous().view(torch.int16).numpy().astype(np.uint16).reshape(-1)


def code_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Number of bf16 steps between two codes (sign-magnitude mapped to an
    ordered integer line; +0 and -0 are one point)."""
    def line(c):
        c = c.astype(np.int64)
        return np.where(c & 0x8000, -(c & 0x7FFF), c)
    return np.abs(line(a) - line(b))


class Stat:
    def __init__(self):
        self.n = self.diff = self.maxd = 0
        self.hist = {}
        self.exact_hf = self.exact_orc = self.exact_n = 0
        self.max_rel = 0.0  # max |hf - oracle| over the op output's max |value|, per call

    def add(self, hf: np.ndarray, orc_out: np.ndarray, exact=None):
        d = code_distance(hf, orc_out)
        self.n += d.size
        self.diff += int(np.count_nonzero(d))
        self.maxd = max(self.maxd, int(d.max()) if d.size else 0)
        a, b = orc.bf16_to_f32(hf).astype(np.float64), orc.bf16_to_f32(orc_out).astype(np.float64)
        scale = float(np.max(np.abs(a))) if a.size else 0.0
        if scale > 0 and np.all(np.isfinite(a)) and np.all(np.isfinite(b)):
            self.max_rel = max(self.max_rel, float(np.max(np.abs(a - b))) / scale)
        for v, c in zip(*np.unique(d, return_counts=True)):
            self.hist[int(v)] = self.hist.get(int(v), 0) + int(c)
        if exact is not None:
            self.exact_n += exact.size
            self.exact_hf += int(np.count_nonzero(hf == exact))
            self.exact_orc += int(np.count_nonzero(orc_out == exact))

    def json(self):
        # a code distance is large where cancellation leaves an output near
        # zero; the largest difference relative to the output vector's
        # largest magnitude shows its size on the vector's own scale (one
        # bf16 ulp of the largest value is 2^-8 to 2^-7 of it)
        out = {"elements": self.n, "differ": self.diff, "max_code_distance": self.maxd,
               "max_diff_over_vector_max": self.max_rel,
               "distance_histogram": {str(k): v for k, v in sorted(self.hist.items())}}
        if self.exact_n:
            out["equal_fp64_rounded"] = {"transformers": self.exact_hf, "oracle": self.exact_orc,
                                         "of": self.exact_n}
        return out


def f64_to_bf16(y: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even of FP64 values to bf16 codes in one rounding:
    through FP32, except where the FP32 value is itself a bf16 halfway point,
    which the FP64 value's side of it decides."""
    x32 = y.astype(np.float32)
    bits = x32.view(np.uint32).astype(np.uint64)
    rne = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    tie = (bits & 0xFFFF) == 0x8000
    above = np.abs(y) > np.abs(x32.astype(np.float64))
    below = np.abs(y) < np.abs(x32.astype(np.float64))
    out = np.where(tie & above, (bits >> 16) + 1, np.where(tie & below, bits >> 16, rne))
    return out.astype(np.uint16)


def gemv_exact(w: np.ndarray, x: np.ndarray, rows: int, k: int) -> np.ndarray:
    return f64_to_bf16(orc.gemv_f64(w, x, rows, k, k, 0))


def analyse(name: str) -> dict:
    import torch
    import transformers.models.qwen3.modeling_qwen3 as mq

    preset, seed, gain_std, pseed, n_prompt, n_new, n_logits, options = case(name)
    tied = "untied" not in options
    t0 = time.time()
    model = build_hf(preset, seed, gain_std, tied)
    cfg = orc.config(preset, tied=int(tied))
    H, D, heads, kvh, I, V = cfg.hidden, cfg.head_dim, cfg.heads, cfg.kv_heads, cfg.intermediate, cfg.vocab
    L = cfg.layers
    prompt = orc.tokens(n_prompt, pseed, V)
    # the prompt and the steps whose logits the golden fixture records
    max_seq = n_prompt + min(n_new, n_logits)
    o_cos, o_sin = orc.rope_tables(max_seq, D, cfg.rope_theta)
    W = {}
    for layer in range(L):
        for kind in (orc.W_Q, orc.W_K, orc.W_V, orc.W_O, orc.W_QNORM, orc.W_KNORM, orc.W_GATE, orc.W_UP,
                     orc.W_DOWN, orc.W_INNORM, orc.W_POSTNORM):
            W[kind, layer] = orc.fill_tensor(cfg, seed, gain_std, kind, layer)
    W[orc.W_EMBED, 0] = orc.fill_tensor(cfg, seed, gain_std, orc.W_EMBED, 0)
    W[orc.W_FINALNORM, 0] = orc.fill_tensor(cfg, seed, gain_std, orc.W_FINALNORM, 0)
    lm_head = W[orc.W_EMBED, 0] if tied else orc.fill_tensor(cfg, seed, gain_std, orc.W_LMHEAD, 0)

    # ---- record every op of transformers' step path
    rec = {}
    cur = {"pos": 0}

    def put(key, value):
        rec[(cur["pos"],) + key] = value

    hooks = []
    for li, layer in enumerate(model.model.layers):
        def mod_hook(tag, li=li):
            def h(_m, inp, out):
                put((li, tag, "in"), codes(inp[0]))
                put((li, tag, "out"), codes(out))
            return h
        at = layer.self_attn
        for tag, m in (("in_norm", layer.input_layernorm), ("q", at.q_proj), ("k", at.k_proj), ("v", at.v_proj),
                       ("q_norm", at.q_norm), ("k_norm", at.k_norm), ("o", at.o_proj),
                       ("post_norm", layer.post_attention_layernorm), ("gate", layer.mlp.gate_proj),
                       ("up", layer.mlp.up_proj), ("down", layer.mlp.down_proj)):
            hooks.append(m.register_forward_hook(mod_hook(tag)))
        hooks.append(layer.register_forward_hook(
            lambda _m, inp, out, li=li: put((li, "layer", "out"), codes(out[0] if isinstance(out, tuple) else out))))
    def final_norm_hook(_m, inp, out):  # a forward hook must return None to leave the output alone
        put((L, "final_norm", "in"), codes(inp[0]))
        put((L, "final_norm", "out"), codes(out))

    hooks.append(model.model.norm.register_forward_hook(final_norm_hook))
    hooks.append(model.lm_head.register_forward_hook(lambda _m, inp, out: put((L, "lm_head", "out"), codes(out))))

    orig_attn = mq.eager_attention_forward
    orig_rope = mq.apply_rotary_pos_emb

    def attn(module, query, key, value, attention_mask, scaling, dropout=0.0, **kw):
        out, w = orig_attn(module, query, key, value, attention_mask, scaling, dropout, **kw)
        li = module.layer_idx
        put((li, "attention", "q"), codes(query))        # [1, heads, 1, D], after RoPE
        # the cache is [1, kvh, S, D]; only this position's row is new (the
        # rows before it were recorded at their own positions)
        put((li, "attention", "k"), codes(key[:, :, -1]))
        put((li, "attention", "v"), codes(value[:, :, -1]))
        put((li, "attention", "out"), codes(out))        # [1, 1, heads, D]
        return out, w

    def rope(q, k, cos, sin, unsqueeze_dim=1):
        qo, ko = orig_rope(q, k, cos, sin, unsqueeze_dim)
        rec[(cur["pos"], "rope_cos")] = codes(cos)
        rec[(cur["pos"], "rope_sin")] = codes(sin)
        return qo, ko

    mq.eager_attention_forward = attn
    mq.apply_rotary_pos_emb = rope
    # the attention class binds the rotary function at class creation when
    # kernels are enabled; patch the bound name too where it exists
    for layer in model.model.layers:
        if hasattr(layer.self_attn, "rotary_fn"):
            layer.self_attn.rotary_fn = rope
    stream = []
    try:
        with torch.no_grad():
            past = None
            tok = int(prompt[0])
            for p in range(max_seq - 1):
                cur["pos"] = p
                out = model(input_ids=torch.tensor([[tok]]), past_key_values=past, use_cache=True)
                past = out.past_key_values
                nxt = int(torch.argmax(out.logits[0, -1].float()))
                if p + 1 < n_prompt:
                    tok = int(prompt[p + 1])
                else:
                    stream.append(nxt)
                    tok = nxt
                rec[(p, "token_in")] = int(prompt[p]) if p < n_prompt else stream[p - n_prompt]
    finally:
        mq.eager_attention_forward = orig_attn
        mq.apply_rotary_pos_emb = orig_rope
        for h in hooks:
            h.remove()
    print(f"[{name}] transformers steps recorded {time.time() - t0:.1f}s", flush=True)
    positions = max_seq - 1

    # ---- op-local comparison
    S = {k: Stat() for k in ("in_norm", "q", "k", "v", "q_norm", "k_norm", "rope_q", "rope_k", "rope_q_tables",
                             "rope_k_tables", "rope_table_cos", "rope_table_sin", "attention", "o", "add_attn",
                             "post_norm", "gate", "up", "silu_mul", "down", "add_mlp", "final_norm", "lm_head")}

    def rope_rot(v, cos_row, sin_row):
        # the oracle's rotation without its norm: orc_qk_norm_rope with a
        # unit-gain norm is not separable, so restate the rotation of
        # oracle.c (out = bf16(bf16(v*cos) + bf16(rot(v)*sin))) on codes
        f = orc.bf16_to_f32(v)
        half = v.size // 2
        rot = np.concatenate([-f[half:], f[:half]])
        a = orc.bf16_to_f32(orc.encode(f * orc.bf16_to_f32(cos_row), 0))
        b = orc.bf16_to_f32(orc.encode(rot * orc.bf16_to_f32(sin_row), 0))
        return orc.encode(a + b, 0)

    hk = np.zeros((L, kvh, max_seq, D), np.uint16)  # transformers' caches, rebuilt row by row
    hv = np.zeros((L, kvh, max_seq, D), np.uint16)
    for p in range(positions):
        S["rope_table_cos"].add(rec[(p, "rope_cos")], o_cos[p * D:(p + 1) * D])
        S["rope_table_sin"].add(rec[(p, "rope_sin")], o_sin[p * D:(p + 1) * D])
        hcos, hsin = rec[(p, "rope_cos")], rec[(p, "rope_sin")]
        for li in range(L):
            g = lambda tag, io="out": rec[(p, li, tag, io)]  # noqa: E731
            S["in_norm"].add(g("in_norm"), orc.rmsnorm(g("in_norm", "in"), W[orc.W_INNORM, li]))
            xn = g("in_norm")
            for tag, kind, rows in (("q", orc.W_Q, heads * D), ("k", orc.W_K, kvh * D), ("v", orc.W_V, kvh * D)):
                S[tag].add(g(tag), orc.gemv_canonical(W[kind, li], xn, rows, H, H, 0),
                           gemv_exact(W[kind, li], xn, rows, H))
            for tag, kind, n in (("q_norm", orc.W_QNORM, heads), ("k_norm", orc.W_KNORM, kvh)):
                src = g(tag, "in").reshape(n, D)
                S[tag].add(g(tag), np.concatenate([orc.rmsnorm(src[i], W[kind, li]) for i in range(n)]))
            qn = g("q_norm").reshape(heads, D)
            kn = g("k_norm").reshape(kvh, D)
            q_roped = rec[(p, li, "attention", "q")].reshape(heads, D)
            hk[li, :, p] = rec[(p, li, "attention", "k")].reshape(kvh, D)
            hv[li, :, p] = rec[(p, li, "attention", "v")].reshape(kvh, D)
            kcache, vcache = hk[li, :, :p + 1], hv[li, :, :p + 1]
            S["rope_q"].add(q_roped.reshape(-1), np.concatenate([rope_rot(qn[i], hcos, hsin) for i in range(heads)]))
            S["rope_k"].add(kcache[:, p].reshape(-1), np.concatenate([rope_rot(kn[i], hcos, hsin) for i in range(kvh)]))
            oc, os_ = o_cos[p * D:(p + 1) * D], o_sin[p * D:(p + 1) * D]
            S["rope_q_tables"].add(q_roped.reshape(-1), np.concatenate([rope_rot(qn[i], oc, os_) for i in range(heads)]))
            S["rope_k_tables"].add(kcache[:, p].reshape(-1), np.concatenate([rope_rot(kn[i], oc, os_) for i in range(kvh)]))
            att = rec[(p, li, "attention", "out")].reshape(heads, D)
            mine = []
            for h in range(heads):
                gk = h // (heads // kvh)
                mine.append(orc.attention_head(q_roped[h], np.ascontiguousarray(kcache[gk]).reshape(-1),
                                               np.ascontiguousarray(vcache[gk]).reshape(-1), D, p + 1, D))
            S["attention"].add(att.reshape(-1), np.concatenate(mine))
            S["o"].add(g("o"), orc.gemv_canonical(W[orc.W_O, li], g("o", "in"), H, heads * D, heads * D, 0),
                       gemv_exact(W[orc.W_O, li], g("o", "in"), H, heads * D))
            S["add_attn"].add(g("post_norm", "in"), orc.add(g("in_norm", "in"), g("o")))
            S["post_norm"].add(g("post_norm"), orc.rmsnorm(g("post_norm", "in"), W[orc.W_POSTNORM, li]))
            pn = g("post_norm")
            for tag, kind in (("gate", orc.W_GATE), ("up", orc.W_UP)):
                S[tag].add(g(tag), orc.gemv_canonical(W[kind, li], pn, I, H, H, 0), gemv_exact(W[kind, li], pn, I, H))
            S["silu_mul"].add(g("down", "in"), orc.silu_mul(g("gate"), g("up")))
            S["down"].add(g("down"), orc.gemv_canonical(W[orc.W_DOWN, li], g("down", "in"), H, I, I, 0),
                          gemv_exact(W[orc.W_DOWN, li], g("down", "in"), H, I))
            S["add_mlp"].add(g("layer"), orc.add(g("post_norm", "in"), g("down")))
        S["final_norm"].add(rec[(p, L, "final_norm", "out")],
                            orc.rmsnorm(rec[(p, L, "final_norm", "in")], W[orc.W_FINALNORM, 0]))
        fn = rec[(p, L, "final_norm", "out")]
        S["lm_head"].add(rec[(p, L, "lm_head", "out")], orc.gemv_canonical(lm_head, fn, V, H, H, 0),
                         gemv_exact(lm_head, fn, V, H))
    print(f"[{name}] op-local comparison done {time.time() - t0:.1f}s", flush=True)

    # ---- cumulative: the oracle's own decode, composed from its primitives
    kc = np.zeros((L, kvh, max_seq, D), np.uint16)
    vc = np.zeros((L, kvh, max_seq, D), np.uint16)
    first = None
    per_layer = []  # [position][layer] max code distance of the residual stream after the layer
    logits_equal_model = True
    m = orc.Model(cfg, seed=seed, gain_std=gain_std, max_seq=max_seq)
    for p in range(positions):
        tok = rec[(p, "token_in")]
        x = W[orc.W_EMBED, 0][tok * H:(tok + 1) * H].copy()
        cos_row, sin_row = o_cos[p * D:(p + 1) * D], o_sin[p * D:(p + 1) * D]
        row = []

        def check(op, li, mine, theirs):
            nonlocal first
            d = int(code_distance(mine, theirs).max())
            if d and first is None:
                first = {"position": p, "layer": li, "op": op, "max_code_distance": d,
                         "differing": int(np.count_nonzero(mine != theirs)), "of": int(mine.size)}
            return d

        for li in range(L):
            g = lambda tag, io="out": rec[(p, li, tag, io)]  # noqa: E731
            xn = orc.rmsnorm(x, W[orc.W_INNORM, li])
            check("in_norm", li, xn, g("in_norm"))
            q = orc.gemv_canonical(W[orc.W_Q, li], xn, heads * D, H, H, 0)
            k = orc.gemv_canonical(W[orc.W_K, li], xn, kvh * D, H, H, 0)
            v = orc.gemv_canonical(W[orc.W_V, li], xn, kvh * D, H, H, 0)
            check("q", li, q, g("q"))
            check("k", li, k, g("k"))
            check("v", li, v, g("v"))
            for gi in range(kvh):
                kc[li, gi, p] = orc.qk_norm_rope(k[gi * D:(gi + 1) * D], W[orc.W_KNORM, li], cos_row, sin_row)
                vc[li, gi, p] = v[gi * D:(gi + 1) * D]
            check("k_rope_cache", li, kc[li, :, p].reshape(-1), rec[(p, li, "attention", "k")])
            att = []
            qr_all = []
            for h in range(heads):
                gk = h // (heads // kvh)
                qr = orc.qk_norm_rope(q[h * D:(h + 1) * D], W[orc.W_QNORM, li], cos_row, sin_row)
                qr_all.append(qr)
                att.append(orc.attention_head(qr, kc[li, gk, :p + 1].reshape(-1), vc[li, gk, :p + 1].reshape(-1), D,
                                              p + 1, D))
            check("q_rope", li, np.concatenate(qr_all), rec[(p, li, "attention", "q")])
            att = np.concatenate(att)
            check("attention", li, att, rec[(p, li, "attention", "out")])
            o = orc.gemv_canonical(W[orc.W_O, li], att, H, heads * D, heads * D, 0)
            check("o", li, o, g("o"))
            x = orc.add(x, o)
            check("add_attn", li, x, g("post_norm", "in"))
            pn = orc.rmsnorm(x, W[orc.W_POSTNORM, li])
            check("post_norm", li, pn, g("post_norm"))
            gt = orc.gemv_canonical(W[orc.W_GATE, li], pn, I, H, H, 0)
            up = orc.gemv_canonical(W[orc.W_UP, li], pn, I, H, H, 0)
            check("gate", li, gt, g("gate"))
            check("up", li, up, g("up"))
            sm = orc.silu_mul(gt, up)
            check("silu_mul", li, sm, g("down", "in"))
            dn = orc.gemv_canonical(W[orc.W_DOWN, li], sm, H, I, I, 0)
            check("down", li, dn, g("down"))
            x = orc.add(x, dn)
            row.append(check("add_mlp", li, x, g("layer")))
        fn = orc.rmsnorm(x, W[orc.W_FINALNORM, 0])
        check("final_norm", L, fn, rec[(p, L, "final_norm", "out")])
        lg = orc.gemv_canonical(lm_head, fn, V, H, H, 0)
        lg_diff = check("lm_head", L, lg, rec[(p, L, "lm_head", "out")])
        _, ref_logits = m.decode(tok, p, want_logits=True)
        logits_equal_model &= bool(np.array_equal(ref_logits, lg))
        hf_l = orc.bf16_to_f32(rec[(p, L, "lm_head", "out")]).astype(np.float64)
        my_l = orc.bf16_to_f32(lg).astype(np.float64)
        per_layer.append({"position": p, "residual_max_code_distance_by_layer": row,
                          "logits_max_code_distance": lg_diff,
                          "logits_max_abs": float(np.max(np.abs(hf_l - my_l)))})
    m.close()
    print(f"[{name}] cumulative comparison done {time.time() - t0:.1f}s", flush=True)
    return {
        "case": name,
        "preset": preset,
        "positions": positions,
        "prompt_length": n_prompt,
        "composed_oracle_equals_orc_qwen3_decode": logits_equal_model,
        "op_local": {k: v.json() for k, v in S.items()},
        "cumulative_first_departure": first,
        "cumulative_by_position": per_layer,
    }


def main() -> None:
    names = sys.argv[1:] or ["small-varied"]
    for name in names:
        res = analyse(name)
        path = os.path.join(HERE, f"qwen3_opdiff_{name}.json")
        with open(path, "w") as f:
            json.dump(res, f, indent=1)
        print(f"wrote {path}", flush=True)
        for op, st in res["op_local"].items():
            ex = st.get("equal_fp64_rounded")
            exs = f"  fp64-rounded: hf {ex['transformers']} orc {ex['oracle']} of {ex['of']}" if ex else ""
            print(f"  {op:16s} differ {st['differ']:8d}/{st['elements']:9d} max {st['max_code_distance']:5d} "
                  f"rel {st['max_diff_over_vector_max']:.2e}{exs}")
        print("  first departure:", res["cumulative_first_departure"])


if __name__ == "__main__":
    main()
