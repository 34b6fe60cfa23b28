"""The reference's eight Qwen3 kernel entries on gfx950 through the runtime's
work-item launch (qwen3/tests/test_gpu_dispatch.cpp restated), compared bit
for bit with the CPU oracle and with the reference's closed forms."""
import numpy as np
import pytest

import oracle_lib as orc
import xpu_playground_amd as xpu
from xpu_playground_amd import Args

pytestmark = pytest.mark.gpu


def b(v):
    return orc.encode(np.asarray(v, np.float32), 0)


def f(codes):
    return orc.decode(np.asarray(codes, np.uint16), 0)


def close(actual, expected, atol=0.03, rtol=0.02):
    # test_gpu_dispatch.cpp:17-25
    assert np.all(np.isfinite(actual))
    assert np.all(np.abs(actual - expected) <= atol + rtol * np.abs(expected))


def test_embedding(rt):
    hidden, vocab, token = 1024, 40, 17
    table = b(((np.arange(vocab * hidden) % 29) - 14) / 16.0)
    dt, dout = rt.upload(table), rt.alloc(hidden * 2)
    rt.launch("QwenEmbedding", hidden, Args().ptr(dt).ptr(dout).u32(token).u32(hidden))
    assert np.array_equal(rt.download(dout, hidden, np.uint16), table[token * hidden:(token + 1) * hidden])


@pytest.mark.parametrize("width", [128, 1024, 4096, 3000])
def test_rmsnorm(rt, width):
    x = b(((np.arange(width) % 31) - 15) / 32.0)
    w = orc.encode((1.0 + 0.1 * np.sin(np.arange(width))).astype(np.float32), 0)
    dx, dw, do = rt.upload(x), rt.upload(w), rt.alloc(width * 2)
    rt.launch("QwenRmsNorm", 1, Args().ptr(dx).ptr(dw).ptr(do).u32(width).f32(1e-6))
    out = rt.download(do, width, np.uint16)
    assert np.array_equal(out, orc.rmsnorm(x, w))
    fx = f(x)
    close(f(out), fx * f(w) / np.sqrt(np.mean(fx * fx) + 1e-6))


def test_gemv_32x32(rt):
    rows = cols = 32
    vec = b(((np.arange(cols) % 7) - 3) / 8.0)
    mat = b(((np.arange(rows * cols) % 11) - 5) / 16.0)
    dm, dv, do = rt.upload(mat), rt.upload(vec), rt.alloc(rows * 2)
    rt.launch("QwenGemv", rows, Args().ptr(dm).ptr(dv).ptr(do).u32(rows).u32(cols))
    out = rt.download(do, rows, np.uint16)
    assert np.array_equal(out, orc.gemv_canonical(mat, vec, rows, cols, cols, 0))
    close(f(out), f(mat).reshape(rows, cols) @ f(vec))


def qkv_case(heads, kv_heads, seed):
    rng = np.random.default_rng(seed)
    q = b(rng.standard_normal(heads * 128))
    k = b(rng.standard_normal(kv_heads * 128))
    v = b(rng.standard_normal(kv_heads * 128))
    return q, k, v


def launch_qkv(rt, dq, dk, dv, dqn, dkn, dcos, dsin, dkc, dvc, pos, maximum, heads, kv):
    rt.launch("QwenQkvRopeCache", heads,
              Args().ptr(dq).ptr(dk).ptr(dv).ptr(dqn).ptr(dkn).ptr(dcos).ptr(dsin).ptr(dkc).ptr(dvc)
              .u32(pos).u32(maximum).u32(heads).u32(kv))


def test_qkv_rope_cache_and_attention_position_zero(rt):
    # test_gpu_dispatch.cpp:102-142: cos = 1, sin = 0, position 0; the value
    # cache receives v, attention over one position returns v of head / group
    heads, kv = 32, 8
    q = b(((np.arange(heads * 128) % 17) - 8) / 16.0)
    k = b(((np.arange(kv * 128) % 13) - 6) / 16.0)
    v = b(((np.arange(kv * 128) % 19) - 9) / 16.0)
    norm = b(np.ones(128))
    cos, sin = b(np.ones(128)), b(np.zeros(128))
    dq, dk, dv, dn, dc, ds = map(rt.upload, (q, k, v, norm, cos, sin))
    dkc, dvc = rt.alloc(kv * 128 * 2), rt.alloc(kv * 128 * 2)
    launch_qkv(rt, dq, dk, dv, dn, dn, dc, ds, dkc, dvc, 0, 1, heads, kv)
    assert np.array_equal(rt.download(dvc, kv * 128, np.uint16), v)
    dout = rt.alloc(heads * 128 * 2)
    rt.launch("QwenAttention", heads, Args().ptr(dq).ptr(dkc).ptr(dvc).ptr(dout).u32(0).u32(heads).u32(kv))
    att = f(rt.download(dout, heads * 128, np.uint16)).reshape(heads, 128)
    for h in range(heads):
        close(att[h], f(v).reshape(kv, 128)[h // (heads // kv)])


def test_qkv_rope_cache_final_slot(rt):
    # test_gpu_dispatch.cpp:144-167: position 40959 of a 40960-entry cache
    heads, kv, maximum = 16, 8, 40960
    q, k, v = qkv_case(heads, kv, 3)
    cos_t, sin_t = orc.rope_tables(maximum)
    norm = b(np.ones(128))
    dq, dk, dv, dn = map(rt.upload, (q, k, v, norm))
    dc, ds = rt.upload(cos_t), rt.upload(sin_t)
    cache = maximum * kv * 128
    dkc, dvc = rt.alloc(cache * 2), rt.alloc(cache * 2)
    launch_qkv(rt, dq, dk, dv, dn, dn, dc, ds, dkc, dvc, maximum - 1, maximum, heads, kv)
    last = (maximum - 1) * kv * 128
    assert np.array_equal(rt.download(dvc + last * 2, kv * 128, np.uint16), v)
    kc = rt.download(dkc + last * 2, kv * 128, np.uint16).reshape(kv, 128)
    row = slice((maximum - 1) * 128, maximum * 128)
    for g in range(kv):
        assert np.array_equal(kc[g], orc.qk_norm_rope(k[g * 128:(g + 1) * 128], norm, cos_t[row], sin_t[row]))
    # out of range position: nothing written (kernels.hpp:74-75)
    rt.memset(dvc, 0, 16)
    launch_qkv(rt, dq, dk, dv, dn, dn, dc, ds, dkc, dvc, maximum, maximum, heads, kv)
    assert np.all(rt.download(dvc, 8, np.uint16) == 0)
    rt.free(dkc)
    rt.free(dvc)


@pytest.mark.parametrize("pos", [0, 5, 255, 4200])
def test_qkv_rope_cache_and_attention_random(rt, pos):
    heads, kv, maximum = 16, 8, 4608
    group = heads // kv
    rng = np.random.default_rng(pos)
    q, k, v = qkv_case(heads, kv, pos + 1)
    qn = orc.encode((1 + 0.1 * rng.standard_normal(128)).astype(np.float32), 0)
    kn = orc.encode((1 + 0.1 * rng.standard_normal(128)).astype(np.float32), 0)
    cos_t, sin_t = orc.rope_tables(maximum)
    kc = b(rng.standard_normal(maximum * kv * 128))
    vc = b(rng.standard_normal(maximum * kv * 128))
    dq, dk, dv, dqn, dkn, dc, ds, dkc, dvc = map(rt.upload, (q, k, v, qn, kn, cos_t, sin_t, kc, vc))
    launch_qkv(rt, dq, dk, dv, dqn, dkn, dc, ds, dkc, dvc, pos, maximum, heads, kv)
    row = slice(pos * 128, (pos + 1) * 128)
    q_exp = np.concatenate([orc.qk_norm_rope(q[h * 128:(h + 1) * 128], qn, cos_t[row], sin_t[row]) for h in range(heads)])
    k_normed = np.concatenate([orc.rmsnorm(k[g * 128:(g + 1) * 128], kn) for g in range(kv)])
    assert np.array_equal(rt.download(dq, heads * 128, np.uint16), q_exp)
    assert np.array_equal(rt.download(dk, kv * 128, np.uint16), k_normed)
    kc_gpu = rt.download(dkc, maximum * kv * 128, np.uint16)
    for g in range(kv):
        slot = (pos * kv + g) * 128
        kc[slot:slot + 128] = orc.qk_norm_rope(k[g * 128:(g + 1) * 128], kn, cos_t[row], sin_t[row])
        vc[slot:slot + 128] = v[g * 128:(g + 1) * 128]
    assert np.array_equal(kc_gpu, kc)
    dout = rt.alloc(heads * 128 * 2)
    rt.launch("QwenAttention", heads, Args().ptr(dq).ptr(dkc).ptr(dvc).ptr(dout).u32(pos).u32(heads).u32(kv))
    att = rt.download(dout, heads * 128, np.uint16)
    for h in range(heads):
        g = h // group
        exp = orc.attention_head(q_exp[h * 128:(h + 1) * 128], kc[g * 128:], vc[g * 128:], kv * 128, pos + 1)
        assert np.array_equal(att[h * 128:(h + 1) * 128], exp), h
    for p in (dq, dk, dv, dqn, dkn, dc, ds, dkc, dvc, dout):
        rt.free(p)


def test_add_and_silu_multiply(rt):
    # test_gpu_dispatch.cpp:170-194
    width = 3072
    left = b(((np.arange(width) % 11) - 5) / 8.0)
    right = b(((np.arange(width) % 7) - 3) / 8.0)
    dl, dr = rt.upload(left), rt.upload(right)
    rt.launch("QwenAdd", width // 32, Args().ptr(dl).ptr(dr).u32(width))
    out = rt.download(dl, width, np.uint16)
    assert np.array_equal(out, orc.add(left, right))
    close(f(out), f(left) + f(right))
    rng = np.random.default_rng(5)
    gate = b(rng.standard_normal(width) * 4)
    rt.copy_to(dl, gate)
    rt.launch("QwenSiluMultiply", width // 32, Args().ptr(dl).ptr(dr).u32(width))
    out = rt.download(dl, width, np.uint16)
    assert np.array_equal(out, orc.silu_mul(gate, right))
    g = f(gate)
    close(f(out), g / (1 + np.exp(-g)) * f(right))


def test_argmax_tie_nan_and_random(rt):
    # test_gpu_dispatch.cpp:195-209
    width = 151936
    logits = b(np.full(width, -1.0))
    logits[17] = logits[42] = b([3.0])[0]
    dl, dt = rt.upload(logits), rt.alloc(4)

    def run():
        rt.launch("QwenArgmax", 1, Args().ptr(dl).ptr(dt).u32(width))
        return int(rt.download(dt, 1, np.uint32)[0])

    assert run() == 17
    logits[3] = b([np.nan])[0]
    rt.copy_to(dl, logits)
    assert run() == 0xFFFFFFFF
    logits[3] = b([np.inf])[0]
    rt.copy_to(dl, logits)
    assert run() == 0xFFFFFFFF
    rand = b(np.random.default_rng(1).standard_normal(width))
    rt.copy_to(dl, rand)
    assert run() == orc.argmax(rand)


def test_cpp_runtime_wrapper_contract_program():
    # include/xpu_runtime.hpp (the LevelZeroRuntime-shaped wrapper) from C++:
    # queries, reserve check, alignment, copies, fragment lookup errors and a
    # three-launch chain with a closed-form answer
    import os
    import subprocess

    exe = os.path.join(xpu.BUILD_DIR, "runtime_contract_check")
    out = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert "runtime contract: PASS" in out.stdout
