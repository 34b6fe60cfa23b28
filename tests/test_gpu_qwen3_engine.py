"""Qwen3 decode engine on gfx950 vs the CPU oracle: tokens, logits and hidden
states bit for bit in all three modes (graph, eager, the reference's kernel
sequence), the BASELINE 0.6B workload against the golden fixtures, the
checkpoint path and the NaN sentinel."""
import json
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as orc
import qwen3_fixtures as qf
from checkpoint_util import write_checkpoint
import xpu_playground_amd as xpu
from xpu_playground_amd import qwen3

pytestmark = pytest.mark.gpu

MODES = [qwen3.GRAPH, qwen3.EAGER, qwen3.REFERENCE]


@pytest.mark.parametrize("mode", MODES)
def test_decode_steps_match_oracle_bitwise(rt, mode):
    cfg = orc.config("tiny")
    m = orc.Model(cfg, seed=5, gain_std=0.1, max_seq=48)
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=48, seed=5, gain_std=0.1, runtime=rt)
    eng.set_mode(mode)
    prompt = orc.tokens(20, 9, cfg.vocab)
    token = int(prompt[0])
    for pos in range(40):
        print(f"mode={mode} pos={pos}", flush=True)
        ref_tok, ref_logits = m.decode(token, pos, want_logits=True)
        tok = eng.decode(token, pos)
        assert np.array_equal(eng.logits(), ref_logits), pos
        assert np.array_equal(eng.hidden(), m.hidden()), pos
        assert tok == ref_tok
        token = int(prompt[pos + 1]) if pos + 1 < len(prompt) else tok
    eng.close()


def test_generate_small_config_all_modes_agree(rt):
    cfg = orc.config("small")
    prompt = orc.tokens(24, 4, cfg.vocab)
    m = orc.Model(cfg, seed=3, gain_std=0.05, max_seq=96)
    ref, _ = m.generate(prompt, 48)
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=96, seed=3, gain_std=0.05, runtime=rt)
    for mode in MODES:
        eng.set_mode(mode)
        out, pm, dm = eng.generate(prompt, 48, stop_on_eos=False)
        assert out.tolist() == ref.tolist(), mode
    eng.close()


@pytest.mark.parametrize("split_from", [0, 257])
def test_attention_past_one_softmax_chunk(rt, split_from):
    # positions beyond 4096 take the chunked (recomputing) attention path, in
    # one block per head (split_from 0) or split over compute units
    cfg = orc.config("tiny", layers=1, vocab=512)
    n_prompt = 4100
    prompt = orc.tokens(n_prompt, 6, cfg.vocab)
    m = orc.Model(cfg, seed=8, gain_std=0.1, max_seq=n_prompt + 4)
    ref, logits = m.generate(prompt, 4, logit_steps=4)
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=n_prompt + 4, seed=8, gain_std=0.1, runtime=rt)
    eng.set_attention_split(split_from)
    out, _, _ = eng.generate(prompt, 4, stop_on_eos=False)
    assert out.tolist() == ref.tolist()
    assert np.array_equal(eng.logits(), logits[3])
    eng.close()


@pytest.mark.parametrize("heads", [16, 32])
@pytest.mark.parametrize("mode", [qwen3.GRAPH, qwen3.EAGER])
@pytest.mark.parametrize("split_from", [0, 1, 257])
def test_split_attention_every_position_matches_oracle(rt, mode, split_from, heads):
    # 16 or 32 query heads over 8 kv heads (the 0.6B and 8B groupings): every
    # position 0..299 through decode, with the attention split over compute
    # units never, at every step, or from the 257th position on (both
    # captured graphs in one run)
    cfg = orc.config("small", layers=1, vocab=1024, heads=heads)
    max_seq = 304
    m = orc.Model(cfg, seed=6, gain_std=0.1, max_seq=max_seq)
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=max_seq, seed=6, gain_std=0.1, runtime=rt)
    eng.set_mode(mode)
    eng.set_attention_split(split_from)
    prompt = orc.tokens(160, 12, cfg.vocab)
    token = int(prompt[0])
    print(f"mode={mode} split_from={split_from} heads={heads}", flush=True)
    for pos in range(300):
        ref_tok, ref_logits = m.decode(token, pos, want_logits=True)
        tok = eng.decode(token, pos)
        assert np.array_equal(eng.logits(), ref_logits), pos
        assert tok == ref_tok, pos
        token = int(prompt[pos + 1]) if pos + 1 < len(prompt) else tok
    eng.close()


def test_split_attention_setter(rt):
    cfg = orc.config("tiny")
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=16, seed=1, gain_std=0.1, runtime=rt)
    for v in (0, 1, 257, 1 << 20):
        eng.set_attention_split(v)
    eng.close()


def engine_logit_rows(eng, fx):
    """Feed the fixture's prompt and then the engine's own tokens one
    position at a time (eager mode); the bf16 logits rows of the first
    logit_steps generated tokens."""
    prompt = fx["prompt"]
    rows = []
    token = int(prompt[0])
    for p in range(len(prompt) + fx["logit_steps"] - 1):
        tok = eng.decode(token, p)
        if p >= len(prompt) - 1:
            rows.append(eng.logits().copy())
        token = int(prompt[p + 1]) if p + 1 < len(prompt) else tok
    return rows


def test_baseline_workload_qwen3_0_6b(rt):
    # 128 seeded prompt ids, 128 greedy steps
    fx = qf.load("qwen3-0.6b")
    cfg = qwen3.preset("qwen3-0.6b")
    eng = qwen3.Engine(cfg, max_seq=256, seed=fx["weight_seed"], gain_std=fx["gain_std"], runtime=rt)
    prompt = np.array(fx["prompt"], np.uint32)
    assert np.array_equal(prompt, qwen3.prompt_tokens(128, fx["prompt_seed"], cfg.vocab))
    out, pm, dm = eng.generate(prompt, fx["new_tokens"], stop_on_eos=False)
    print(f"0.6B: prompt {pm:.2f} ms, decode {dm:.2f} ms ({(len(out) - 1) / dm * 1e3:.1f} tok/s)")
    # bit-exact canonical arithmetic: all 128 tokens equal the oracle's; the
    # decode bar against transformers: the first 32 identical to both of its
    # paths (all 128 equal its step-by-step decode)
    assert out.tolist() == fx["oracle_tokens"] == fx["hf_steps"]
    assert out[:32].tolist() == fx["hf_generate"][:32]
    # logits of the first 32 generated tokens: the very rows whose
    # full-vocabulary distance to transformers the fixture records (and
    # tests/test_oracle_qwen3.py holds to the bar)
    eng.set_mode(qwen3.EAGER)
    rows = engine_logit_rows(eng, fx)
    assert [qf.row_hash(r) for r in rows] == fx["oracle_logits_sha256"]
    worst = max(max(st["oracle_vs_generate"], st["oracle_vs_steps"]) for st in fx["logit_stats"])
    print(f"max |logit - transformers| over 32 steps x {cfg.vocab} ids: {worst}")
    eng.close()


@pytest.mark.parametrize("name", ["tiny", "tiny-varied", "small-varied", "small-varied-b"])
def test_transformers_fixtures_varied_streams(rt, name):
    # greedy streams with up to 32 distinct tokens in 32 steps: the engine's
    # tokens equal transformers' (both paths) and its logits rows are the
    # oracle's measured rows, bit for bit, in graph and eager modes
    fx = qf.load(name)
    cfg = orc.config(fx["preset"])
    n_prompt = len(fx["prompt"])
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=n_prompt + fx["new_tokens"], seed=fx["weight_seed"],
                       gain_std=fx["gain_std"], runtime=rt)
    out, _, _ = eng.generate(np.array(fx["prompt"], np.uint32), fx["new_tokens"], stop_on_eos=False)
    assert out.tolist() == fx["oracle_tokens"] == fx["hf_generate"] == fx["hf_steps"]
    for mode in (qwen3.GRAPH, qwen3.EAGER):
        eng.set_mode(mode)
        assert [qf.row_hash(r) for r in engine_logit_rows(eng, fx)] == fx["oracle_logits_sha256"], mode
    eng.close()


@pytest.mark.parametrize("name", qf.FORCED)
def test_transformers_fixtures_teacher_forced(rt, name):
    # the teacher-forced fixtures: the reference engine's untied lm_head
    # (small-untied) and the BASELINE 0.6B shape with a stream that changes
    # (28 distinct tokens in 32 steps). Fed the prompt and then
    # transformers' step-path tokens, the engine's logits rows are the
    # oracle's measured rows bit for bit, in graph and eager modes, so the
    # fixture's distances to transformers and its token checks
    # (tests/test_oracle_qwen3.py) hold for the GPU path
    fx = qf.load(name)
    cfg = orc.config(fx["preset"], tied=fx["tied"])
    inputs = qf.forced_inputs(fx)
    n_prompt = len(fx["prompt"])
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=len(inputs) + 1, seed=fx["weight_seed"],
                       gain_std=fx["gain_std"], runtime=rt)
    for mode in (qwen3.GRAPH, qwen3.EAGER):
        eng.set_mode(mode)
        rows, toks = [], []
        for p, tok in enumerate(inputs):
            t = eng.decode(int(tok), p)
            if p >= n_prompt - 1:
                rows.append(eng.logits().copy())
                toks.append(t)
        print(f"{name} mode {mode}: {sum(a == b for a, b in zip(toks, fx['hf_steps']))} of 32 tokens equal "
              f"transformers' step path", flush=True)
        assert toks == fx["oracle_tokens"][:len(toks)]
        assert [qf.row_hash(r) for r in rows] == fx["oracle_logits_sha256"], mode
    eng.close()


@pytest.mark.parametrize("tied,sharded", [(1, False), (0, True)])
def test_checkpoint_loading(rt, tmp_path, tied, sharded):
    cfg = orc.config("tiny", tied=tied)
    write_checkpoint(str(tmp_path), cfg, seed=11, gain_std=0.1, sharded=sharded)
    eng = qwen3.Engine(runtime=rt, model_dir=str(tmp_path), max_seq=32)
    assert eng.cfg.tied == tied and eng.cfg.hidden == cfg.hidden
    m = orc.Model(cfg, seed=11, gain_std=0.1, max_seq=32)
    prompt = orc.tokens(10, 2, cfg.vocab)
    ref, _ = m.generate(prompt, 8)
    out, _, _ = eng.generate(prompt, 8, stop_on_eos=False)
    assert out.tolist() == ref.tolist()
    eng.close()


def test_non_finite_logits_raise(rt, tmp_path):
    # main.cpp:223-224: a NaN anywhere in the logits is an error
    cfg = orc.config("tiny")
    write_checkpoint(str(tmp_path), cfg, seed=1, gain_std=0.0, nan_embed=True)
    eng = qwen3.Engine(runtime=rt, model_dir=str(tmp_path), max_seq=16)
    for mode in MODES:
        eng.set_mode(mode)
        with pytest.raises(xpu.XpuError, match="NaN"):
            eng.decode(3, 0)
    eng.close()


def test_command_line_matches_oracle(tmp_path):
    cfg = orc.config("tiny")
    prompt = orc.tokens(12, 5, cfg.vocab)
    ids = tmp_path / "ids.txt"
    ids.write_text(" ".join(map(str, prompt.tolist())) + "\n")
    m = orc.Model(cfg, seed=0, gain_std=0.0, max_seq=64)
    ref, _ = m.generate(prompt, 10, stop_on_eos=True)
    exe = os.path.join(xpu.BUILD_DIR, "qwen3_hip")
    out = subprocess.run([exe, "--synthetic", "tiny", "--input-ids", str(ids), "--max-new-tokens", "10",
                          "--max-seq-len", "64"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert json.loads(out.stdout)["generated_ids"] == ref.tolist()
    bad = subprocess.run([exe, "--synthetic", "tiny", "--input-ids", str(ids), "--max-new-tokens", "60",
                          "--max-seq-len", "64"], capture_output=True, text=True, timeout=120)
    assert bad.returncode == 1 and "exceeds --max-seq-len" in bad.stderr


@pytest.mark.parametrize("preset,n_prompt,max_seq", [("small", 40, 96), ("small", 2, 16), ("small", 1, 16),
                                                      ("small", 300, 320), ("small", 256, 272), ("small", 257, 272)])
def test_batched_prefill_bit_identical(rt, preset, n_prompt, max_seq):
    # every prompt position in one batch per layer (chunks of 256 positions;
    # 257 leaves the last position alone in its chunk), the last position
    # finished by the decode step's kernels: same tokens, logits and hidden
    # state as feeding the prompt through decode one position at a time, and
    # as the oracle, for the first generated token and after 16 more
    cfg = orc.config(preset)
    new = min(16, max_seq - n_prompt)
    prompt = orc.tokens(n_prompt, 12, cfg.vocab)
    m = orc.Model(cfg, seed=4, gain_std=0.1, max_seq=max_seq)
    ref, ref_logits = m.generate(prompt, new, logit_steps=new)
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=max_seq, seed=4, gain_std=0.1, runtime=rt)
    results = {}
    for batched in (True, False):
        eng.set_prefill(batched)
        for mode in (qwen3.GRAPH, qwen3.EAGER):
            print(f"{preset} n_prompt={n_prompt} batched={batched} mode={mode}", flush=True)
            eng.set_mode(mode)
            out, pm, dm = eng.generate(prompt, new, stop_on_eos=False)
            results[(batched, mode)] = (out.tolist(), eng.logits().copy(), eng.hidden().copy(), pm)
    for key, (toks, logits, hidden, pm) in results.items():
        assert toks == ref.tolist(), key
        assert np.array_equal(logits, ref_logits[new - 1]), key
        assert np.array_equal(hidden, m.hidden()), key
    print({k: round(v[3], 3) for k, v in results.items()})
    # the first generated token alone: the prompt's own last step
    eng.set_prefill(True)
    eng.set_mode(qwen3.GRAPH)
    out, _, _ = eng.generate(prompt, 1, stop_on_eos=False)
    assert out.tolist() == ref.tolist()[:1]
    assert np.array_equal(eng.logits(), ref_logits[0])
    eng.close()


def test_batched_prefill_needs_kernels_for_the_shape(rt):
    # hidden 256 is not a multiple of 512: no batched kernels, stepwise prompt
    cfg = orc.config("tiny")
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=32, seed=1, gain_std=0.1, runtime=rt)
    with pytest.raises(xpu.XpuError, match="batched prefill"):
        eng.set_prefill(True)
    prompt = orc.tokens(10, 3, cfg.vocab)
    m = orc.Model(cfg, seed=1, gain_std=0.1, max_seq=32)
    ref, _ = m.generate(prompt, 6)
    out, _, _ = eng.generate(prompt, 6, stop_on_eos=False)
    assert out.tolist() == ref.tolist()
    eng.close()


def test_prefill_cli_flag():
    exe = os.path.join(xpu.BUILD_DIR, "qwen3_hip")
    bad = subprocess.run([exe, "--synthetic", "tiny", "--input-ids", "-", "--max-new-tokens", "1", "--prefill", "x"],
                         input="1 2 3\n", capture_output=True, text=True, timeout=120)
    assert bad.returncode == 1 and "--prefill must be" in bad.stderr


def run_steps_all_modes(rt, cfg, seed, steps, max_seq, label):
    """decode `steps` positions (the first half from a seeded prompt) in
    every mode; logits, hidden state and tokens bit for bit against the oracle"""
    m = orc.Model(cfg, seed=seed, gain_std=0.1, max_seq=max_seq)
    prompt = orc.tokens(steps // 2, seed + 1, cfg.vocab)
    ref = []
    token = int(prompt[0])
    for pos in range(steps):
        tok, logits = m.decode(token, pos, want_logits=True)
        ref.append((tok, logits, m.hidden().copy()))
        token = int(prompt[pos + 1]) if pos + 1 < len(prompt) else tok
    m.close()
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=max_seq, seed=seed, gain_std=0.1, runtime=rt)
    for mode in MODES:
        eng.set_mode(mode)
        token = int(prompt[0])
        for pos in range(steps):
            print(f"{label} mode={mode} pos={pos}", flush=True)
            tok = eng.decode(token, pos)
            assert np.array_equal(eng.logits(), ref[pos][1]), (mode, pos)
            assert np.array_equal(eng.hidden(), ref[pos][2]), (mode, pos)
            assert tok == ref[pos][0], (mode, pos)
            token = int(prompt[pos + 1]) if pos + 1 < len(prompt) else tok
    eng.close()


def test_reference_engine_shape_qwen3_8b(rt):
    # the reference's own shape (qwen3/model.hpp:11-22): hidden 4096,
    # intermediate 12288, 32 query / 8 kv heads, untied lm_head; two layers
    # and a 4096-id vocabulary keep the oracle fast. down_proj (K = 12288)
    # runs the LDS-staged residual GEMV, the other projections the
    # register-vector kernels with 8 chunks per lane.
    cfg = orc.config("qwen3-8b", layers=2, vocab=4096)
    assert cfg.tied == 0
    run_steps_all_modes(rt, cfg, seed=21, steps=8, max_seq=16, label="8b")


def test_wide_shape_takes_the_lds_staged_kernels(rt):
    # hidden 5120 (> 4096 = 8 chunks of 512 per lane) with 40 query heads
    # over 8 kv heads (a group of 5): RMSNorm + QKV, gate/up + SiLU, the
    # o_proj / down residual GEMVs and the final norm + lm_head all take
    # their LDS-staged kernels
    cfg = orc.config("small", hidden=5120, intermediate=6656, heads=40, kv_heads=8, layers=1, vocab=2048, tied=0)
    run_steps_all_modes(rt, cfg, seed=23, steps=6, max_seq=8, label="wide")


def test_mode_switch_mid_sequence_is_rejected(rt):
    # reference mode keeps the KV caches position-major, graph and eager
    # chunk-major: continuing a sequence across that switch is an error;
    # graph <-> eager may alternate; position 0 starts afresh
    cfg = orc.config("tiny")
    m = orc.Model(cfg, seed=5, gain_std=0.1, max_seq=16)
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=16, seed=5, gain_std=0.1, runtime=rt)
    seq = [3, 17, 400, 9]
    ref = [m.decode(t, p) for p, t in enumerate(seq)]
    for first, second in [(qwen3.GRAPH, qwen3.REFERENCE), (qwen3.REFERENCE, qwen3.EAGER)]:
        eng.set_mode(first)
        eng.decode(seq[0], 0)
        eng.decode(seq[1], 1)
        eng.set_mode(second)
        with pytest.raises(xpu.XpuError, match="other mode's layout"):
            eng.decode(seq[2], 2)
        assert [eng.decode(t, p) for p, t in enumerate(seq)] == ref
    eng.set_mode(qwen3.GRAPH)
    out = [eng.decode(seq[0], 0)]
    eng.set_mode(qwen3.EAGER)
    out.append(eng.decode(seq[1], 1))
    eng.set_mode(qwen3.GRAPH)
    out += [eng.decode(seq[2], 2), eng.decode(seq[3], 3)]
    assert out == ref
    eng.close()


# "small" also has the batched GEMV form; "tiny" (hidden 256) and the
# reference's own Qwen3-8B shape (qwen3/model.hpp:11-22; two layers, 4096
# ids; intermediate 12288, 4 query heads per kv head) only the GEMM form
# (tiny with one layer, 4110 ids: two chunks of the GEMM form; the decode
# step of the last prompt position attends over caches written by both, the
# second chunk's from position 4096 on. With one layer the prompt's own
# attention output is not used, the last layer stops at its caches; the MFMA
# attention with p0 > 0 is covered by test_gpu_prefill_attention.py)
GEMM_PROMPT_CASES = [("small", {}, 40, 96), ("small", {}, 300, 320), ("small", {}, 2, 16), ("tiny", {}, 30, 48),
                     ("qwen3-8b", {"layers": 2, "vocab": 4096}, 24, 40), ("tiny", {"layers": 1}, 4110, 4160),
                     ("tiny", {"layers": 1}, 4097, 4112)]


@pytest.mark.parametrize("preset,over,n_prompt,max_seq", GEMM_PROMPT_CASES)
def test_gemm_prefill_within_rounding(rt, preset, over, n_prompt, max_seq):
    # the projections of the prompt positions on the MFMA GEMM: each
    # projection output is within the GEMM's bar of the canonical one, so
    # the caches differ from the oracle's by bf16 rounding and the logits and
    # hidden state of the first new token by a small multiple of it; a
    # dropped residual, a swapped gate/up half or a transposed weight moves
    # them by O(1)
    cfg = orc.config(preset, **over)
    prompt = orc.tokens(n_prompt, 12, cfg.vocab)
    m = orc.Model(cfg, seed=4, gain_std=0.1, max_seq=max_seq)
    ref, ref_logits = m.generate(prompt, 1, logit_steps=1)
    want = orc.decode(ref_logits[0], xpu.BF16).astype(np.float64)
    want_h = orc.decode(m.hidden(), xpu.BF16).astype(np.float64)
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=max_seq, seed=4, gain_std=0.1, runtime=rt)
    eng.set_prefill("gemm")
    for mode in (qwen3.GRAPH, qwen3.EAGER):
        print(f"gemm prefill {preset} n_prompt={n_prompt} mode={mode}", flush=True)
        eng.set_mode(mode)
        out, _, _ = eng.generate(prompt, 1, stop_on_eos=False)
        got = orc.decode(eng.logits(), xpu.BF16).astype(np.float64)
        got_h = orc.decode(eng.hidden(), xpu.BF16).astype(np.float64)
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        rel_h = np.linalg.norm(got_h - want_h) / np.linalg.norm(want_h)
        dmax = float(np.abs(got - want).max())
        print(f"logits rel-L2 {rel:.3e} max|d| {dmax:.3e} (max|logit| {np.abs(want).max():.3e}), "
              f"hidden rel-L2 {rel_h:.3e}", flush=True)
        # measured: logits and hidden rel-L2 4e-3 - 1.2e-2, max |d| up to
        # 5.9e-2 at these shapes: the GEMM form misses the decode's 2e-2
        # max-abs bar (it is opt-in and labelled so); these bounds hold it
        # where it is
        assert rel <= 1.5e-2 and rel_h <= 1.5e-2, (rel, rel_h)
        assert dmax <= 6.5e-2, dmax
        top2 = np.sort(want)[-2:]
        if top2[1] - top2[0] > 2 * dmax:
            assert out.tolist() == ref.tolist()
    # the exact forms on the same engine: batched where the shape has it,
    # else stepwise
    eng.set_prefill("batched" if preset == "small" else "stepwise")
    eng.generate(prompt, 1, stop_on_eos=False)
    assert np.array_equal(eng.logits(), ref_logits[0])
    eng.close()


def test_gemm_prefill_full_0_6b_shape(rt):
    # the BASELINE workload's prompt (configs[4]: 0.6B shape, 28 layers,
    # 128 seeded ids) in the GEMM form against the bit-exact batched form,
    # whose first generated token's logits row is the oracle's (the hash the
    # qwen3-0.6b fixture records)
    fx = qf.load("qwen3-0.6b")
    cfg = qwen3.preset("qwen3-0.6b")
    prompt = np.array(fx["prompt"], np.uint32)
    eng = qwen3.Engine(cfg, max_seq=256, seed=fx["weight_seed"], gain_std=fx["gain_std"], runtime=rt)
    eng.set_mode(qwen3.EAGER)
    out_b, _, _ = eng.generate(prompt, 1, stop_on_eos=False)
    exact = eng.logits().copy()
    assert qf.row_hash(exact) == fx["oracle_logits_sha256"][0]
    eng.set_prefill("gemm")
    out_g, _, _ = eng.generate(prompt, 1, stop_on_eos=False)
    got = orc.decode(eng.logits(), xpu.BF16).astype(np.float64)
    want = orc.decode(exact, xpu.BF16).astype(np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    dmax = float(np.abs(got - want).max())
    print(f"0.6B GEMM-form prompt: logits rel-L2 {rel:.3e}, max|d| {dmax:.3e}", flush=True)
    # measured 1.36e-2 - 1.56e-2 and 0.041 - 0.049 (DESIGN's figures): above
    # the decode's 2e-2 max-abs bar, held here as a regression bound
    assert rel <= 2e-2 and dmax <= 6e-2, (rel, dmax)
    top2 = np.sort(want)[-2:]
    if top2[1] - top2[0] > 2 * dmax:
        assert out_g.tolist() == out_b.tolist()
    eng.close()


def test_gemm_prefill_mode_checks(rt):
    # 8 query heads per kv head: no MFMA attention kernel (1, 2 or 4), and
    # hidden 256 has no batched GEMV form either
    cfg = orc.config("tiny", heads=8, kv_heads=1)
    eng = qwen3.Engine(qwen3.config_from(cfg), max_seq=32, seed=1, gain_std=0.1, runtime=rt)
    with pytest.raises(xpu.XpuError, match="gemm prefill"):
        eng.set_prefill("gemm")
    with pytest.raises(xpu.XpuError, match="batched prefill"):
        eng.set_prefill("batched")
    with pytest.raises(xpu.XpuError, match="prefill mode"):
        xpu.check(eng.lib.xpu_qwen3_set_prefill(eng.handle, 3))
    eng.close()
