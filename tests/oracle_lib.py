"""ctypes bindings to the CPU oracle (oracle/liboracle.so) for the tests.

The oracle is the checker: tests compare the HIP path with it; nothing in the
product imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_double, c_float, c_int, c_uint16, c_uint32, c_uint64, c_void_p

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(REPO, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")
REF_DIR = os.path.join(ORACLE_DIR, "_ref")

EOS_TOKENS = (151645, 151643)

W_Q, W_K, W_V, W_O, W_QNORM, W_KNORM, W_GATE, W_UP, W_DOWN, W_INNORM, W_POSTNORM, W_EMBED, W_FINALNORM, W_LMHEAD = range(14)


class OrcConfig(ctypes.Structure):
    _fields_ = [
        ("hidden", c_uint32),
        ("intermediate", c_uint32),
        ("layers", c_uint32),
        ("heads", c_uint32),
        ("kv_heads", c_uint32),
        ("head_dim", c_uint32),
        ("vocab", c_uint32),
        ("rms_eps", c_float),
        ("rope_theta", c_double),
        ("tied", c_uint32),
    ]


PRESETS = {
    # Qwen3-0.6B architecture
    "qwen3-0.6b": dict(hidden=1024, intermediate=3072, layers=28, heads=16, kv_heads=8, head_dim=128, vocab=151936),
    # reference engine shape (qwen3/model.hpp:11-22)
    "qwen3-8b": dict(hidden=4096, intermediate=12288, layers=36, heads=32, kv_heads=8, head_dim=128, vocab=151936,
                     tied=0),
    # small shapes for fast tests
    "tiny": dict(hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=1000),
    "small": dict(hidden=1024, intermediate=3072, layers=2, heads=16, kv_heads=8, head_dim=128, vocab=4096),
}


def config(name: str = "qwen3-0.6b", **over) -> OrcConfig:
    d = dict(tied=1)
    d.update(PRESETS[name])
    d.update(over)
    return OrcConfig(rms_eps=1e-6, rope_theta=1e6, **d)


def build() -> None:
    subprocess.run(["make", "-s", "-C", ORACLE_DIR, "all"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = ctypes.CDLL(ORACLE_SO)
        u16p = POINTER(c_uint16)
        sigs = {
            "orc_f32_to_bf16": (c_uint16, [c_float]),
            "orc_bf16_to_f32": (c_float, [c_uint16]),
            "orc_f32_to_fp16": (c_uint16, [c_float]),
            "orc_fp16_to_f32": (c_float, [c_uint16]),
            "orc_encode_n": (None, [c_void_p, c_void_p, c_uint64, c_int]),
            "orc_decode_n": (None, [c_void_p, c_void_p, c_uint64, c_int]),
            "orc_hash": (c_uint64, [c_uint64, c_uint64]),
            "orc_fill_uniform": (None, [c_void_p, c_uint64, c_uint64, c_int]),
            "orc_fill_normal_bf16": (None, [c_void_p, c_uint64, c_uint64, c_float]),
            "orc_fill_gain_bf16": (None, [c_void_p, c_uint64, c_uint64, c_float]),
            "orc_fill_tokens": (None, [c_void_p, c_uint64, c_uint64, c_uint32]),
            "orc_fill_reference_gemv": (None, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_int]),
            "orc_gemv_rows_seq": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint64, c_int]),
            "orc_gemv_f64": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint64, c_int]),
            "orc_gemv_canonical": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint64, c_int]),
            "orc_canonical_dot": (c_float, [c_void_p, c_void_p, c_uint32, c_int]),
            "orc_canonical_sum": (c_float, [c_void_p, c_uint32]),
            "orc_time_gemv_seq": (c_double, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_int, c_int]),
            "orc_gemm_f64": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_int, c_void_p, c_uint32]),
            "orc_gemm_f32_rows": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_int, c_void_p, c_uint32]),
            "orc_time_gemm_f32": (c_double, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_int, c_uint32, c_int]),
            "orc_gemm_f32_blocked": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_int]),
            "orc_time_gemm_blocked": (c_double, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_int, c_int]),
            "orc_exp": (c_float, [c_float]),
            "orc_rmsnorm": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_float]),
            "orc_rope_tables": (None, [c_void_p, c_void_p, c_uint32, c_uint32, c_double]),
            "orc_qk_norm_rope": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_float]),
            "orc_attention_head": (None, [c_void_p, c_void_p, c_void_p, c_uint64, c_uint32, c_uint32, c_void_p]),
            "orc_add": (None, [c_void_p, c_void_p, c_uint32]),
            "orc_silu_mul": (None, [c_void_p, c_void_p, c_uint32]),
            "orc_argmax": (c_uint32, [c_void_p, c_uint32]),
            "orc_qwen3_tensor_elems": (c_uint64, [POINTER(OrcConfig), c_int]),
            "orc_qwen3_fill_tensor": (None, [POINTER(OrcConfig), c_uint64, c_float, c_int, c_uint32, c_void_p]),
            "orc_qwen3_create": (c_void_p, [POINTER(OrcConfig), c_uint64, c_float, c_uint32]),
            "orc_qwen3_destroy": (None, [c_void_p]),
            "orc_qwen3_weight": (u16p, [c_void_p, c_int, c_uint32]),
            "orc_qwen3_decode": (c_uint32, [c_void_p, c_uint32, c_uint32, c_void_p]),
            "orc_qwen3_hidden": (u16p, [c_void_p]),
            "orc_qwen3_generate": (
                c_uint32,
                [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_void_p, c_void_p, c_uint32],
            ),
            "orc_set_threads": (None, [c_int]),
            "orc_get_threads": (c_int, []),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(a: np.ndarray) -> c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(c_void_p)


# ---------------------------------------------------------------- codecs
def bf16_to_f32(codes: np.ndarray) -> np.ndarray:
    return (codes.astype(np.uint32) << 16).view(np.float32)


def decode(codes: np.ndarray, dtype: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint16)
    out = np.empty(codes.shape, np.float32)
    lib().orc_decode_n(ptr(codes), ptr(out), codes.size, dtype)
    return out


def encode(values: np.ndarray, dtype: int) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(values.shape, np.uint16)
    lib().orc_encode_n(ptr(values), ptr(out), values.size, dtype)
    return out


def bf16_ulp(value: float) -> float:
    """Spacing of bf16 codes at |value| (the gap to the next code up)."""
    code = int(encode(np.float32([abs(value)]), 0)[0])
    pair = decode(np.array([code, code + 1], np.uint16), 0)
    return float(pair[1] - pair[0])


# ---------------------------------------------------------------- synth
def uniform(n: int, seed: int, dtype: int) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().orc_fill_uniform(ptr(out), n, seed, dtype)
    return out


def tokens(n: int, seed: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().orc_fill_tokens(ptr(out), n, seed, vocab)
    return out


def reference_gemv_inputs(m: int, k: int, ld: int, dtype: int):
    a = np.empty(m * ld, np.uint16)
    x = np.empty(k, np.uint16)
    lib().orc_fill_reference_gemv(ptr(a), ptr(x), m, k, ld, dtype)
    return a, x


# ---------------------------------------------------------------- GEMV / GEMM
def gemv_canonical(a: np.ndarray, x: np.ndarray, m: int, k: int, lda: int, dtype: int) -> np.ndarray:
    y = np.empty(m, np.uint16)
    lib().orc_gemv_canonical(ptr(a), ptr(x), ptr(y), m, k, lda, dtype)
    return y


def gemv_f64(a: np.ndarray, x: np.ndarray, m: int, k: int, lda: int, dtype: int) -> np.ndarray:
    y = np.empty(m, np.float64)
    lib().orc_gemv_f64(ptr(a), ptr(x), ptr(y), m, k, lda, dtype)
    return y


def gemv_rows_seq(a: np.ndarray, x: np.ndarray, rows: int, k: int, lda: int, dtype: int) -> np.ndarray:
    y = np.empty(rows, np.float32)
    lib().orc_gemv_rows_seq(ptr(a), ptr(x), ptr(y), rows, k, lda, dtype)
    return y


def gemm_f64(a, b, m, n, k, dtype, rows=None) -> np.ndarray:
    if rows is None:
        c = np.empty((m, n), np.float64)
        lib().orc_gemm_f64(ptr(a), ptr(b), ptr(c), m, n, k, dtype, None, m)
    else:
        rows = np.ascontiguousarray(rows, dtype=np.uint32)
        c = np.empty((len(rows), n), np.float64)
        lib().orc_gemm_f64(ptr(a), ptr(b), ptr(c), m, n, k, dtype, ptr(rows), len(rows))
    return c


def gemm_f32_rows(a, b, m, n, k, dtype, rows) -> np.ndarray:
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    c = np.empty((len(rows), n), np.float32)
    lib().orc_gemm_f32_rows(ptr(a), ptr(b), ptr(c), m, n, k, dtype, ptr(rows), len(rows))
    return c


# ---------------------------------------------------------------- Qwen3
def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(w, np.uint16)
    out = np.empty_like(x)
    lib().orc_rmsnorm(ptr(x), ptr(w), ptr(out), x.size, eps)
    return out


def rope_tables(max_seq: int, head_dim: int = 128, theta: float = 1e6):
    c = np.empty(max_seq * head_dim, np.uint16)
    s = np.empty(max_seq * head_dim, np.uint16)
    lib().orc_rope_tables(ptr(c), ptr(s), max_seq, head_dim, theta)
    return c, s


def qk_norm_rope(v: np.ndarray, w: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray, eps: float = 1e-6):
    v = np.array(v, np.uint16)
    lib().orc_qk_norm_rope(ptr(v), ptr(np.ascontiguousarray(w, np.uint16)), ptr(np.ascontiguousarray(cos_row)),
                           ptr(np.ascontiguousarray(sin_row)), v.size, eps)
    return v


def attention_head(q, kcache, vcache, stride, n, head_dim=128):
    out = np.empty(head_dim, np.uint16)
    lib().orc_attention_head(ptr(np.ascontiguousarray(q, np.uint16)), ptr(np.ascontiguousarray(kcache, np.uint16)),
                             ptr(np.ascontiguousarray(vcache, np.uint16)), stride, n, head_dim, ptr(out))
    return out


def add(left, right):
    left = np.array(left, np.uint16)
    lib().orc_add(ptr(left), ptr(np.ascontiguousarray(right, np.uint16)), left.size)
    return left


def silu_mul(gate, up):
    gate = np.array(gate, np.uint16)
    lib().orc_silu_mul(ptr(gate), ptr(np.ascontiguousarray(up, np.uint16)), gate.size)
    return gate


def argmax(logits) -> int:
    logits = np.ascontiguousarray(logits, np.uint16)
    return int(lib().orc_argmax(ptr(logits), logits.size))


def fill_tensor(cfg: OrcConfig, seed: int, gain_std: float, kind: int, layer: int) -> np.ndarray:
    n = lib().orc_qwen3_tensor_elems(ctypes.byref(cfg), kind)
    out = np.empty(n, np.uint16)
    lib().orc_qwen3_fill_tensor(ctypes.byref(cfg), seed, gain_std, kind, layer, ptr(out))
    return out


class Model:
    """CPU oracle decode (qwen3/main.cpp:159-226 restated)."""

    def __init__(self, cfg: OrcConfig, seed: int = 0, gain_std: float = 0.0, max_seq: int = 256):
        self.cfg = cfg
        self.handle = lib().orc_qwen3_create(ctypes.byref(cfg), seed, gain_std, max_seq)

    def close(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.orc_qwen3_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def weight(self, kind: int, layer: int = 0) -> np.ndarray:
        n = lib().orc_qwen3_tensor_elems(ctypes.byref(self.cfg), kind)
        p = lib().orc_qwen3_weight(self.handle, kind, layer)
        return np.ctypeslib.as_array(p, shape=(n,)).copy()

    def decode(self, token: int, position: int, want_logits: bool = False):
        logits = np.empty(self.cfg.vocab, np.uint16) if want_logits else None
        t = lib().orc_qwen3_decode(self.handle, token, position, ptr(logits) if want_logits else None)
        return (int(t), logits) if want_logits else int(t)

    def hidden(self) -> np.ndarray:
        p = lib().orc_qwen3_hidden(self.handle)
        return np.ctypeslib.as_array(p, shape=(self.cfg.hidden,)).copy()

    def generate(self, prompt, max_new: int, stop_on_eos: bool = False, logit_steps: int = 0):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max_new, np.uint32)
        logits = np.zeros((max(logit_steps, 1), self.cfg.vocab), np.uint16)
        n = lib().orc_qwen3_generate(self.handle, ptr(prompt), len(prompt), max_new, int(stop_on_eos), ptr(out),
                                     ptr(logits), logit_steps)
        return out[:n], (logits[:logit_steps] if logit_steps else None)


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)
