#!/usr/bin/env python3
"""Writes the Qwen3 golden fixtures of tests/golden/ (run in the build
container, never on the GPU box).

The reference's oracle is qwen3/reference.py: transformers'
Qwen3ForCausalLM in eager bf16, greedy generate (reference.py:15-24,39-44;
pinned transformers==4.51.0, qwen3/requirements.txt:2). This script builds
that model class from the installed transformers (5.15.0 here; the Qwen3
eager rounding points - RMSNorm, RoPE, eager attention, SiLU MLP - are the
same in both versions) for a shape of the Qwen3 family, loads the synthetic
weights of the CPU oracle's generator (N(0, 0.02^2) matrices, norm gains
1 + N(0, gain_std^2)), and records:
  * hf_generate: model.generate(prompt, greedy, no EOS stop) - the batched
    prompt path reference.py takes;
  * hf_steps: the same prompt fed one position at a time with the KV cache
    (the engine's order, qwen3/main.cpp:343-352), its greedy tokens and, per
    step, the top-16 logits (index, value);
  * oracle: the CPU oracle's tokens and top-16 logits for the same steps.

Usage: python tests/golden/make_qwen3_golden.py [tiny|qwen3-0.6b ...]
"""
from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as orc  # noqa: E402

CASES = {
    # name: (preset, weight seed, gain_std, prompt seed, prompt length, new tokens, logit steps)
    "tiny": ("tiny", 5, 0.1, 1, 16, 32, 32),
    "qwen3-0.6b": ("qwen3-0.6b", 0, 0.0, 1, 128, 128, 32),
}


def build_hf(preset: str, seed: int, gain_std: float):
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM

    p = orc.PRESETS[preset]
    cfg = Qwen3Config(vocab_size=p["vocab"], hidden_size=p["hidden"], intermediate_size=p["intermediate"],
                      num_hidden_layers=p["layers"], num_attention_heads=p["heads"],
                      num_key_value_heads=p["kv_heads"], head_dim=128, max_position_embeddings=40960,
                      rms_norm_eps=1e-6, rope_theta=1e6, tie_word_embeddings=True, hidden_act="silu",
                      attention_bias=False)
    cfg._attn_implementation = "eager"
    # the way from_pretrained(..., torch_dtype=torch.bfloat16) builds it
    # (qwen3/reference.py:15-24): parameters in bf16, while the RoPE inv_freq
    # buffer, computed explicitly in FP32, stays FP32 (a blanket .to(bf16)
    # would round it to bf16 and shift every cos/sin table entry)
    model = Qwen3ForCausalLM._from_config(cfg, dtype=torch.bfloat16).eval()
    assert model.model.rotary_emb.inv_freq.dtype == torch.float32
    oc = orc.config(preset)
    hd, h, inter = 128, p["hidden"], p["intermediate"]

    def t(kind, layer, shape):
        a = orc.fill_tensor(oc, seed, gain_std, kind, layer)
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).reshape(shape)

    with torch.no_grad():
        for l, layer in enumerate(model.model.layers):
            at = layer.self_attn
            at.q_proj.weight.copy_(t(orc.W_Q, l, (p["heads"] * hd, h)))
            at.k_proj.weight.copy_(t(orc.W_K, l, (p["kv_heads"] * hd, h)))
            at.v_proj.weight.copy_(t(orc.W_V, l, (p["kv_heads"] * hd, h)))
            at.o_proj.weight.copy_(t(orc.W_O, l, (h, p["heads"] * hd)))
            at.q_norm.weight.copy_(t(orc.W_QNORM, l, (hd,)))
            at.k_norm.weight.copy_(t(orc.W_KNORM, l, (hd,)))
            layer.mlp.gate_proj.weight.copy_(t(orc.W_GATE, l, (inter, h)))
            layer.mlp.up_proj.weight.copy_(t(orc.W_UP, l, (inter, h)))
            layer.mlp.down_proj.weight.copy_(t(orc.W_DOWN, l, (h, inter)))
            layer.input_layernorm.weight.copy_(t(orc.W_INNORM, l, (h,)))
            layer.post_attention_layernorm.weight.copy_(t(orc.W_POSTNORM, l, (h,)))
        model.model.embed_tokens.weight.copy_(t(orc.W_EMBED, 0, (p["vocab"], h)))
        model.model.norm.weight.copy_(t(orc.W_FINALNORM, 0, (h,)))
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    return model


def topk(values: np.ndarray, k: int = 16):
    idx = np.argsort(-values, kind="stable")[:k]
    return [[int(i), float(values[i])] for i in idx]


def make(name: str) -> dict:
    import torch
    import transformers

    preset, seed, gain_std, pseed, n_prompt, n_new, n_logits = CASES[name]
    t0 = time.time()
    model = build_hf(preset, seed, gain_std)
    vocab = orc.PRESETS[preset]["vocab"]
    prompt = orc.tokens(n_prompt, pseed, vocab)
    with torch.no_grad():
        gen = model.generate(torch.from_numpy(prompt.astype(np.int64))[None], max_new_tokens=n_new,
                             do_sample=False, use_cache=True, eos_token_id=None, pad_token_id=0)
        hf_generate = gen[0, n_prompt:].tolist()
        print(f"[{name}] generate done {time.time() - t0:.1f}s", flush=True)
        out = None
        past = None
        for p in range(n_prompt):
            out = model(input_ids=torch.tensor([[int(prompt[p])]]), past_key_values=past, use_cache=True)
            past = out.past_key_values
        steps, logits = [], []
        for i in range(n_new):
            row = out.logits[0, -1].float().numpy()
            nxt = int(np.argmax(row))
            steps.append(nxt)
            if i < n_logits:
                logits.append(topk(row))
            if i + 1 == n_new:
                break
            out = model(input_ids=torch.tensor([[nxt]]), past_key_values=past, use_cache=True)
            past = out.past_key_values
        print(f"[{name}] steps done {time.time() - t0:.1f}s", flush=True)
    m = orc.Model(orc.config(preset), seed=seed, gain_std=gain_std, max_seq=n_prompt + n_new)
    o_tokens, o_logits = m.generate(prompt, n_new, logit_steps=n_logits)
    m.close()
    o_top = [topk(orc.decode(o_logits[i], 0)) for i in range(n_logits)]
    print(f"[{name}] oracle done {time.time() - t0:.1f}s", flush=True)
    return {
        "case": name,
        "preset": preset,
        "weight_seed": seed,
        "gain_std": gain_std,
        "prompt_seed": pseed,
        "prompt": prompt.tolist(),
        "new_tokens": n_new,
        "transformers_version": transformers.__version__,
        "torch_version": torch.__version__,
        "hf_generate": hf_generate,
        "hf_steps": steps,
        "hf_steps_top16": logits,
        "oracle_tokens": o_tokens.tolist(),
        "oracle_top16": o_top,
    }


def main() -> None:
    names = sys.argv[1:] or list(CASES)
    for name in names:
        fixture = make(name)
        path = os.path.join(HERE, f"qwen3_{name}.json")
        with open(path, "w") as f:
            json.dump(fixture, f, separators=(",", ":"))
        same = sum(a == b for a, b in zip(fixture["hf_steps"], fixture["oracle_tokens"]))
        print(f"wrote {path}: oracle == hf_steps for {same}/{len(fixture['hf_steps'])} tokens; "
              f"hf_generate == hf_steps for "
              f"{sum(a == b for a, b in zip(fixture['hf_generate'], fixture['hf_steps']))}", flush=True)


if __name__ == "__main__":
    main()
