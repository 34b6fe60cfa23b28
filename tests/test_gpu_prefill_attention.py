"""The prompt chunk's attention on MFMA (xpu_q3_pf_attention_mfma_g<G>,
the engine's GEMM prompt mode) against the oracle's attention
(orc_attention_head, qwen3/kernels.hpp:157-192) for every query row and
head, with the per-token kernel of the batched prompt mode
(xpu_q3_pf_attention) as the bit-exact control on the same caches.

The MFMA kernel rounds the scores where the oracle does (bf16(q . k), then
bf16(s * scale)) but runs the softmax online in one sweep, as the
reference's own kernel does (qwen3/kernels.hpp:174-190): p = bf16(exp(s -
m)) with the running max m, the output rescaled as m grows and divided by
the FP32 sum at the end, where the oracle rounds p = bf16(exp(s - M) / sum)
with the final max. Its FP32 sums run in the MFMA's order and its exp is
the hardware's exp2. So about half of the output codes equal the oracle's
and the rest sit a bf16 step away. The bars: rel-L2 <= 1e-2 over the chunk;
every element within 2 bf16 ulps of the row's largest |out| plus 1/64 of
it; and against the attention computed in FP64 from the same bf16 q, k and
v with no rounding inside, the kernel's rel-L2 error at most 1.25 times
the oracle's plus 1e-4 (the two roundings of p are equally accurate; a
wrong scale, mask or rescale is not). Cache positions past the chunk hold
NaN codes, which a read of a key beyond the block's last query would
spread into the output."""
import numpy as np
import pytest

import oracle_lib as orc
import xpu_playground_amd as xpu
from xpu_playground_amd import Args

pytestmark = pytest.mark.gpu

NAN = 0x7FC0


def run_case(rt, p0, T, heads, kv, max_seq, q_gain, seed):
    g = heads // kv
    q = orc.uniform(T * heads * 128, seed, xpu.BF16)
    if q_gain != 1.0:
        q = orc.encode(orc.decode(q, xpu.BF16) * q_gain, xpu.BF16)
    n = p0 + T
    kpos = np.full((kv, max_seq, 128), NAN, np.uint16)
    vpos = np.full((kv, max_seq, 128), NAN, np.uint16)
    kpos[:, :n] = orc.uniform(kv * n * 128, seed + 1, xpu.BF16).reshape(kv, n, 128)
    vpos[:, :n] = orc.uniform(kv * n * 128, seed + 2, xpu.BF16).reshape(kv, n, 128)
    # chunk-major [kv][16][max_seq][8]
    kcm = np.ascontiguousarray(kpos.reshape(kv, max_seq, 16, 8).transpose(0, 2, 1, 3))
    vcm = np.ascontiguousarray(vpos.reshape(kv, max_seq, 16, 8).transpose(0, 2, 1, 3))
    scale = float(np.float32(1.0 / np.sqrt(128.0)))
    dq, dk, dv = rt.upload(q), rt.upload(kcm), rt.upload(vcm)
    outs = {}
    try:
        for name in (f"xpu_q3_pf_attention_mfma_g{g}", "xpu_q3_pf_attention"):
            da = rt.alloc(T * heads * 128 * 2)
            try:
                rt.memset(da, 0xFF, T * heads * 128 * 2)
                if name.startswith("xpu_q3_pf_attention_mfma"):
                    qt = 64 if g == 1 else 32  # queries per block
                    blocks = (T + qt - 1) // qt * kv
                    args = Args().ptr(dq).ptr(dk).ptr(dv).ptr(da).u32(p0).u32(T).u32(heads).u32(kv).u32(max_seq)
                    print(f"{name} p0={p0} T={T} heads={heads} kv={kv} blocks={blocks}", flush=True)
                    rt.launch_grid(name, blocks, 256, 0, args.f32(scale))
                else:
                    args = Args().ptr(dq).ptr(dk).ptr(dv).ptr(da).u32(p0).u32(heads).u32(kv).u32(max_seq)
                    print(f"{name} p0={p0} T={T}", flush=True)
                    rt.launch_grid(name, heads, 256, 0, args.f32(scale), grid_y=T)
                rt.synchronize()
                outs[name] = rt.download(da, T * heads * 128, np.uint16).reshape(T, heads, 128)
            finally:
                rt.free(da)
    finally:
        for p in (dq, dk, dv):
            rt.free(p)
    # every output of the whole chunk written (the buffer started as 0xFFFF,
    # a NaN code) and finite
    for o in outs.values():
        assert np.all(np.isfinite(orc.decode(o.reshape(-1), xpu.BF16)))
    # query rows checked on the CPU: all of them up to 300, else a spread of
    # rows (every 61st, the middle, the last three: the first and last key
    # tiles, the two key halves and their merge)
    rows = list(range(T)) if T <= 300 else sorted(set(range(0, T, 61)) | {T // 2, T - 3, T - 2, T - 1})
    qr = q.reshape(T, heads, 128)
    ref = np.empty((len(rows), heads, 128), np.uint16)
    exact = np.empty((len(rows), heads, 128))
    qd = orc.decode(qr.reshape(-1), xpu.BF16).astype(np.float64).reshape(T, heads, 128)
    kd = orc.decode(kpos[:, :n].reshape(-1), xpu.BF16).astype(np.float64).reshape(kv, n, 128)
    vd = orc.decode(vpos[:, :n].reshape(-1), xpu.BF16).astype(np.float64).reshape(kv, n, 128)
    for i, t in enumerate(rows):
        for h in range(heads):
            ref[i, h] = orc.attention_head(qr[t, h], kpos[h // g], vpos[h // g], 128, p0 + t + 1)
            sc = kd[h // g, : p0 + t + 1] @ qd[t, h] / np.sqrt(128.0)
            w = np.exp(sc - sc.max())
            exact[i, h] = (w / w.sum()) @ vd[h // g, : p0 + t + 1]
    return (outs[f"xpu_q3_pf_attention_mfma_g{g}"][rows], outs["xpu_q3_pf_attention"][rows], ref, exact)


CASES = [(0, 300, 16, 8, 1.0), (0, 300, 16, 8, 8.0), (37, 129, 16, 8, 4.0), (0, 1, 16, 8, 1.0), (5, 2, 16, 8, 1.0),
         (200, 64, 32, 8, 4.0), (0, 100, 8, 8, 4.0), (513, 200, 16, 8, 2.0), (64, 191, 16, 4, 4.0),
         # chunks of the engine's size (up to 4096 positions: 64 key tiles
         # per half, long rescale sweeps, the two-half merge) and a chunk
         # after a full one
         (0, 2048, 16, 8, 4.0), (0, 4096, 16, 8, 2.0), (4096, 64, 16, 8, 4.0)]


@pytest.mark.parametrize("p0,T,heads,kv,q_gain", CASES)
def test_mfma_prefill_attention(rt, p0, T, heads, kv, q_gain):
    got, control, ref, exact = run_case(rt, p0, T, heads, kv, p0 + T + 40, q_gain, 900 + p0 + T)
    assert np.array_equal(control, ref), "per-token kernel differs from the oracle"
    g = orc.decode(got.reshape(-1), xpu.BF16).astype(np.float64).reshape(got.shape)
    r = orc.decode(ref.reshape(-1), xpu.BF16).astype(np.float64).reshape(ref.shape)
    assert np.all(np.isfinite(g))
    rel = np.linalg.norm(g - r) / np.linalg.norm(r)
    rowmax = np.abs(r).max(axis=2, keepdims=True)
    ulp = np.exp2(np.floor(np.log2(np.maximum(rowmax, 1e-30))) - 7)
    err = np.abs(g - r)
    same = float(np.mean(got == ref))
    print(f"rel-L2 {rel:.3e}, max err / row max {float((err / rowmax).max()):.3e}, identical codes {same:.4f}",
          flush=True)
    assert rel <= 1e-2, rel
    bad = err > 2 * ulp + rowmax / 64
    assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:5])
    e_kernel = np.linalg.norm(g - exact) / np.linalg.norm(exact)
    e_oracle = np.linalg.norm(r - exact) / np.linalg.norm(exact)
    print(f"against FP64: kernel rel-L2 {e_kernel:.3e}, oracle {e_oracle:.3e}", flush=True)
    assert e_kernel <= 1.25 * e_oracle + 1e-4, (e_kernel, e_oracle)
