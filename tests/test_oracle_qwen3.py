"""CPU oracle of the Qwen3 decode, pinned by closed forms, the reference's
own CPU primitive test (qwen3/tests/test_cpu_reference.cpp, built in
oracle/_ref), transformers' rotary embedding, and the golden fixtures of
tests/golden/ (transformers Qwen3ForCausalLM, the library
qwen3/reference.py calls)."""
import json
import math
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as orc
import qwen3_fixtures as qf



def b(v):
    return orc.encode(np.asarray(v, np.float32), 0)


def f(codes):
    return orc.decode(np.asarray(codes, np.uint16), 0)


def test_reference_cpu_primitive_test_passes():
    exe = os.path.join(orc.REF_DIR, "test_cpu_reference")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref not built (reference sources absent)")
    out = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and "PASS" in out.stdout


def test_exp_within_one_ulp():
    xs = np.concatenate([np.linspace(-103.9, 88.7, 200001), np.linspace(-1, 1, 20001)]).astype(np.float32)
    got = np.array([orc.lib().orc_exp(float(x)) for x in xs[::7]], np.float32)
    ref = np.exp(xs[::7].astype(np.float64))
    normal = ref > 1.2e-38
    ulp = np.spacing(ref[normal].astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got[normal] - ref[normal]) / ulp) <= 1.0
    assert orc.lib().orc_exp(0.0) == 1.0
    assert orc.lib().orc_exp(-200.0) == 0.0 and math.isinf(orc.lib().orc_exp(100.0))


def test_rmsnorm_constant_input_returns_gains():
    # x*rsqrt(mean(x^2)+eps) rounds to +-1 for a constant input, so the
    # output is the gain vector itself (pins the per-index gain multiply)
    w = orc.encode((1 + 0.1 * np.random.default_rng(0).standard_normal(1024)).astype(np.float32), 0)
    assert np.array_equal(orc.rmsnorm(b(np.full(1024, 0.75)), w), w)
    assert np.array_equal(f(orc.rmsnorm(b(np.full(128, -3.0)), w[:128])), -f(w[:128]))


def test_rmsnorm_matches_float64_within_rounding():
    rng = np.random.default_rng(1)
    for width in (128, 1000, 1024, 4096):
        x = b(rng.standard_normal(width))
        w = b(1 + 0.1 * rng.standard_normal(width))
        fx = f(x).astype(np.float64)
        exact = f(w) * (fx / np.sqrt(np.mean(fx * fx) + 1e-6))
        got = f(orc.rmsnorm(x, w)).astype(np.float64)
        assert np.all(np.abs(got - exact) <= 2.0**-7 * np.abs(exact) + 1e-30)


def test_rope_tables_match_transformers_rotary_embedding():
    import torch
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    cfg = Qwen3Config(hidden_size=1024, num_attention_heads=16, head_dim=128, rope_theta=1e6,
                      max_position_embeddings=40960)
    rope = Qwen3RotaryEmbedding(cfg)
    pos = torch.tensor([[0, 1, 2, 100, 1000, 4095, 12345, 40959]])
    cos, sin = rope(torch.zeros(1, dtype=torch.bfloat16), pos)
    ct, st = orc.rope_tables(40960)
    ct, st = ct.reshape(40960, 128), st.reshape(40960, 128)
    for i, p in enumerate(pos[0].tolist()):
        hc = cos[0, i].view(torch.int16).numpy().view(np.uint16)
        hs = sin[0, i].view(torch.int16).numpy().view(np.uint16)
        # same bf16 codes except where torch's FP32 pow/cos sit 1 ulp off the
        # correctly rounded value right at a bf16 rounding boundary
        assert np.sum(hc != ct[p]) <= 2 and np.sum(hs != st[p]) <= 2
        assert np.all(np.abs(f(hc) - f(ct[p])) <= 2.0**-8) and np.all(np.abs(f(hs) - f(st[p])) <= 2.0**-8)


def test_rope_at_position_zero_is_identity():
    # qwen3/tests/test_cpu_reference.cpp:96-103
    q = b((np.arange(128) - 64) / 64.0)
    w = b(np.ones(128))
    ct, st = orc.rope_tables(1)
    assert np.array_equal(orc.qk_norm_rope(q, w, ct, st), orc.rmsnorm(q, w))


def test_rope_rotation_matches_float64():
    rng = np.random.default_rng(2)
    ct, st = orc.rope_tables(300)
    v = b(rng.standard_normal(128))
    w = b(np.ones(128))
    n = f(orc.rmsnorm(v, w)).astype(np.float64)
    for p in (1, 17, 299):
        c, s = f(ct[p * 128:(p + 1) * 128]).astype(np.float64), f(st[p * 128:(p + 1) * 128]).astype(np.float64)
        rot = np.concatenate([-n[64:], n[:64]])
        exact = n * c + rot * s
        got = f(orc.qk_norm_rope(v, w, ct[p * 128:(p + 1) * 128], st[p * 128:(p + 1) * 128])).astype(np.float64)
        assert np.all(np.abs(got - exact) <= 3 * 2.0**-8 * (np.abs(n * c) + np.abs(rot * s)) + 1e-6)


def test_attention_closed_forms():
    # one cached position: softmax weight 1, output = v exactly
    # (test_cpu_reference.cpp:136-141)
    q = b(np.full(128, 0.25))
    v = b(np.random.default_rng(3).standard_normal(128))
    assert np.array_equal(orc.attention_head(q, q, v, 128, 1), v)
    # two equal keys: weights 1/2 each, output = bf16((v0 + v1) / 2)
    k2 = np.concatenate([q, q])
    v2 = b(np.random.default_rng(4).standard_normal(256))
    expect = b((f(v2[:128]) + f(v2[128:])) * 0.5)
    assert np.array_equal(orc.attention_head(q, k2, v2, 128, 2), expect)


def test_attention_matches_float64_softmax():
    rng = np.random.default_rng(5)
    n = 300
    q = b(rng.standard_normal(128))
    k = b(rng.standard_normal(n * 128))
    v = b(rng.standard_normal(n * 128))
    s = (f(k).reshape(n, 128).astype(np.float64) @ f(q).astype(np.float64)) / math.sqrt(128)
    p = np.exp(s - s.max())
    p /= p.sum()
    exact = p @ f(v).reshape(n, 128).astype(np.float64)
    got = f(orc.attention_head(q, k, v, 128, n)).astype(np.float64)
    assert np.max(np.abs(got - exact)) < 0.02 * max(1.0, np.abs(exact).max())


def test_add_silu_mul_closed_forms():
    a = b([1.0, -2.0, 0.5, 3.0])
    c = b([2.0, 0.25, -0.5, 4.0])
    assert np.array_equal(orc.add(a, c), b([3.0, -1.75, 0.0, 7.0]))
    g = b([0.0, 20.0, -20.0, 1.0])
    u = b([1.0, 1.0, 1.0, 0.0])
    out = f(orc.silu_mul(g, u))
    assert out[0] == 0.0 and out[1] == 20.0 and abs(out[2]) < 1e-6 and out[3] == 0.0
    rng = np.random.default_rng(6)
    g = b(4 * rng.standard_normal(3072))
    u = b(rng.standard_normal(3072))
    fg = f(g).astype(np.float64)
    exact = fg / (1 + np.exp(-fg)) * f(u)
    assert np.all(np.abs(f(orc.silu_mul(g, u)) - exact) <= 2 * 2.0**-8 * np.abs(exact) + 1e-6)


def test_argmax_ties_and_non_finite():
    # qwen3/tests/test_cpu_reference.cpp:158-161, test_gpu_dispatch.cpp:195-209
    logits = b(np.full(151936, -1.0))
    logits[17] = logits[42] = b([3.0])[0]
    assert orc.argmax(logits) == 17
    logits[5] = b([np.nan])[0]
    assert orc.argmax(logits) == 0xFFFFFFFF
    logits[5] = b([-np.inf])[0]
    assert orc.argmax(logits) == 0xFFFFFFFF
    assert orc.argmax(b(np.zeros(10))) == 0


def test_engine_step_by_step_equals_generate():
    cfg = orc.config("tiny")
    prompt = orc.tokens(9, 3, cfg.vocab)
    m1 = orc.Model(cfg, seed=2, gain_std=0.1, max_seq=32)
    gen, _ = m1.generate(prompt, 12)
    m2 = orc.Model(cfg, seed=2, gain_std=0.1, max_seq=32)
    nxt = 0
    for p, t in enumerate(prompt):
        nxt = m2.decode(int(t), p)
    steps = []
    for i in range(12):
        steps.append(nxt)
        nxt = m2.decode(nxt, len(prompt) + i)
    assert steps == gen.tolist()
    assert np.all(np.isfinite(f(m2.hidden())))


@pytest.mark.parametrize("name", qf.NAMES)
def test_oracle_meets_the_decode_bar_against_transformers(name):
    fx = qf.load(name)
    n = min(32, fx["new_tokens"])
    stats = fx["logit_stats"]
    assert len(stats) == fx["logit_steps"] == 32
    if name in qf.FORCED:
        # teacher-forced: transformers' token wherever its top-2 margin is
        # above twice the step's distance (qwen3_fixtures.py)
        assert fx["teacher_forced"]
        dec = [step for step, st in enumerate(stats) if qf.decisive(st)]
        same = [step for step, st in enumerate(stats) if st["argmax"][0] == fx["hf_steps"][step]]
        assert set(dec) <= set(same), (name, sorted(set(dec) - set(same)))
        print(f"{name}: {len(dec)} decisive steps of 32, all with transformers' token; {len(same)} of 32 overall")
        assert (len(dec), len(same)) == qf.DECISIVE[name]
    else:
        # tokens: the oracle's greedy stream equals transformers' generate
        # (the reference.py path) and step-by-step streams for the first 32
        # steps (the 0.6B fixture: all 128 equal the step path; transformers'
        # own two paths part at step 102 there)
        assert fx["oracle_tokens"][:n] == fx["hf_generate"][:n] == fx["hf_steps"][:n]
        if name == "qwen3-0.6b":
            assert fx["oracle_tokens"] == fx["hf_steps"]
    if name in qf.VARIED:
        assert len(set(fx["hf_steps"][:n])) >= 16  # a stream that changes
    # logits over the full vocabulary, per step
    d = [qf.step_distance(st) for st in stats]
    within = sum(x <= qf.BAR for x in d)
    print(f"{name}: {within} of 32 steps within {qf.BAR}, largest distance {max(d)}")
    if name in qf.OPEN_GAP:
        want_within, bound = qf.OPEN_GAP[name]
        assert within == want_within and max(d) <= bound, (name, within, max(d))
    else:
        assert within == 32, (name, d)
    for step, st in enumerate(stats):
        # the recorded maxima bound the recorded top-16 entries
        for top, key in (("hf_steps_top16", "oracle_vs_steps"), ("hf_generate_top16", "oracle_vs_generate")):
            if st[key] is None:
                continue
            ovals = dict(map(tuple, fx["oracle_top16"][step]))
            for i, v in fx[top][step]:
                if i in ovals:
                    assert abs(ovals[i] - v) <= st[key] + 1e-9


# ops that round once from FP32 operands: exact given the same inputs
ELEMENTWISE = ["add_attn", "add_mlp", "silu_mul", "rope_q", "rope_k", "rope_q_tables", "rope_k_tables",
               "rope_table_cos", "rope_table_sin"]
NORMS = ["in_norm", "post_norm", "final_norm", "q_norm", "k_norm"]
SUMS = ["q", "k", "v", "o", "gate", "up", "down", "lm_head"]


@pytest.mark.parametrize("name", qf.NAMES)
def test_departure_from_transformers_is_summation_order(name):
    # tests/golden/qwen3_opdiff_<name>.json (qwen3_op_diff.py): each op of
    # the oracle recomputed from transformers' own inputs along the step path
    ev = qf.load_opdiff(name)
    ops = ev["op_local"]
    assert ev["composed_oracle_equals_orc_qwen3_decode"]
    assert ev["positions"] == len(qf.load(name)["prompt"]) + 31
    for op in ELEMENTWISE:
        assert ops[op]["differ"] == 0, (name, op, ops[op])
    for op in NORMS:
        # the sum of squares is a sum: rarely, one code of bf16(x * rsqrt),
        # which a gain of up to ~4 (1 + N(0, 1)) carries to at most two
        assert ops[op]["max_code_distance"] <= 2 and ops[op]["differ"] <= 2e-5 * ops[op]["elements"], (name, op)
    for op in SUMS:
        # both sides accumulate in FP32 in different orders: few outputs
        # differ, and the oracle equals the FP64 result rounded to bf16 at
        # least about as often as transformers does
        st = ops[op]
        assert st["differ"] <= 2e-3 * st["elements"], (name, op, st["differ"])
        ex = st["equal_fp64_rounded"]
        miss_o, miss_t = ex["of"] - ex["oracle"], ex["of"] - ex["transformers"]
        assert miss_o <= 1.5 * miss_t + 2, (name, op, ex)
    assert ops["attention"]["differ"] <= 1e-4 * ops["attention"]["elements"]
    # the first place the oracle's own stream leaves transformers' is a sum
    first = ev["cumulative_first_departure"]
    assert first is not None and first["op"] in SUMS + ["attention"], first


@pytest.mark.parametrize("name", ["tiny", "tiny-varied", "small-varied", "small-varied-b", "small-untied"])
def test_oracle_reproduces_the_measured_logit_rows(name):
    # the live oracle computes the rows whose statistics the fixture holds,
    # bit for bit (SHA-256 of each bf16 row); teacher-forced fixtures are fed
    # transformers' step-path tokens
    fx = qf.load(name)
    cfg = orc.config(fx["preset"], tied=fx.get("tied", 1))
    m = orc.Model(cfg, seed=fx["weight_seed"], gain_std=fx["gain_std"], max_seq=len(fx["prompt"]) + fx["new_tokens"])
    if fx.get("teacher_forced"):
        n_prompt, logits, tokens = len(fx["prompt"]), [], []
        for p, tok in enumerate(qf.forced_inputs(fx)):
            t, row = m.decode(int(tok), p, want_logits=True)
            if p >= n_prompt - 1:
                logits.append(row)
                tokens.append(t)
        m.close()
        assert tokens == fx["oracle_tokens"][:len(tokens)]
    else:
        tokens, logits = m.generate(np.array(fx["prompt"], np.uint32), fx["new_tokens"], logit_steps=fx["logit_steps"])
        m.close()
        assert tokens.tolist() == fx["oracle_tokens"]
    assert [qf.row_hash(r) for r in logits] == fx["oracle_logits_sha256"]
    for step in range(fx["logit_steps"]):
        row = f(logits[step])
        for i, v in fx["oracle_top16"][step]:
            assert row[i] == np.float32(v)


def test_config_reader_accepts_qwen3_and_rejects_others(tmp_path):
    # qwen3/tests/test_cpu_reference.cpp:178-209, generalised to the family
    from xpu_playground_amd import XpuError, qwen3

    valid = {"hidden_size": 1024, "intermediate_size": 3072, "head_dim": 128, "num_attention_heads": 16,
             "num_key_value_heads": 8, "num_hidden_layers": 28, "vocab_size": 151936,
             "max_position_embeddings": 40960, "eos_token_id": 151645, "rms_norm_eps": 1e-6,
             "rope_theta": 1000000, "tie_word_embeddings": True, "hidden_act": "silu", "model_type": "qwen3",
             "torch_dtype": "bfloat16"}
    (tmp_path / "config.json").write_text(json.dumps(valid))
    cfg = qwen3.read_config(str(tmp_path))
    assert (cfg.hidden, cfg.layers, cfg.heads, cfg.kv_heads, cfg.tied) == (1024, 28, 16, 8, 1)
    assert abs(cfg.rms_eps - 1e-6) < 1e-12 and cfg.rope_theta == 1e6
    for key, bad in [("hidden_size", 4095), ("model_type", "llama"), ("torch_dtype", "float32"),
                     ("head_dim", 64), ("num_key_value_heads", 3), ("hidden_act", "gelu")]:
        (tmp_path / "config.json").write_text(json.dumps({**valid, key: bad}))
        with pytest.raises(XpuError):
            qwen3.read_config(str(tmp_path))
    (tmp_path / "config.json").write_text(json.dumps({k: v for k, v in valid.items() if k != "vocab_size"}))
    with pytest.raises(XpuError):
        qwen3.read_config(str(tmp_path))
    (tmp_path / "config.json").write_text("{\"hidden_size\": 1024,")
    with pytest.raises(XpuError):
        qwen3.read_config(str(tmp_path))


def test_product_host_generators_match_oracle():
    from xpu_playground_amd import qwen3

    cfg = orc.config("tiny")
    pc = qwen3.config_from(cfg)
    for kind in range(13):
        for layer in (0, 1):
            a = orc.fill_tensor(cfg, 7, 0.1, kind, layer)
            assert np.array_equal(a, qwen3.fill_tensor(pc, 7, 0.1, kind, layer, a.size)), (kind, layer)
    c8 = orc.config("qwen3-8b", layers=1, vocab=3000)
    a = orc.fill_tensor(c8, 3, 0.0, orc.W_LMHEAD, 0)
    assert np.array_equal(a, qwen3.fill_tensor(qwen3.config_from(c8), 3, 0.0, orc.W_LMHEAD, 0, a.size))
    c1, s1 = orc.rope_tables(512)
    c2, s2 = qwen3.rope_tables(512)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)
    assert np.array_equal(orc.tokens(1000, 1, 151936), qwen3.prompt_tokens(1000, 1, 151936))


def test_weight_generator_statistics():
    cfg = orc.config("small")
    w = f(orc.fill_tensor(cfg, 0, 0.0, orc.W_GATE, 0))
    assert abs(w.mean()) < 2e-4 and abs(w.std() - 0.02) < 2e-4
    assert np.all(f(orc.fill_tensor(cfg, 0, 0.0, orc.W_INNORM, 0)) == 1.0)
