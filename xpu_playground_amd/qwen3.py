"""Qwen3 decode engine bindings (include/xpu_qwen3.h).

Engine mirrors the reference's Engine (qwen3/main.cpp:118-329): decode(token,
position) -> next token, plus the prompt + greedy generate loop
(main.cpp:342-352). Everything runs on the gfx950 kernels; there is no CPU
path.
"""
from __future__ import annotations

import ctypes
from ctypes import c_double, c_uint32, c_void_p

import numpy as np

from . import Qwen3Config, Runtime, check, library

GRAPH, EAGER, REFERENCE = 0, 1, 2
EOS_TOKENS = (151645, 151643)  # qwen3/model.hpp:19-20


def available() -> bool:
    return hasattr(library(), "xpu_qwen3_create")


def preset(name: str) -> Qwen3Config:
    cfg = Qwen3Config()
    check(library().xpu_qwen3_preset(name.encode(), ctypes.byref(cfg)))
    return cfg


def config_from(other) -> Qwen3Config:
    """Copy any structure with the same field names (e.g. the oracle's)."""
    cfg = Qwen3Config()
    for name, _ in Qwen3Config._fields_:
        setattr(cfg, name, getattr(other, name))
    return cfg


def read_config(model_dir: str) -> Qwen3Config:
    cfg = Qwen3Config()
    check(library().xpu_qwen3_read_config(model_dir.encode(), ctypes.byref(cfg)))
    return cfg


def validate_checkpoint(model_dir: str) -> Qwen3Config:
    """Host-only validation of a checkpoint directory (no GPU needed)."""
    cfg = Qwen3Config()
    check(library().xpu_qwen3_validate_checkpoint(model_dir.encode(), ctypes.byref(cfg)))
    return cfg


def prompt_tokens(n: int, seed: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    check(library().xpu_synth_tokens(out.ctypes.data_as(c_void_p), n, seed, vocab))
    return out


def fill_tensor(cfg: Qwen3Config, seed: int, gain_std: float, kind: int, layer: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint16)
    check(library().xpu_qwen3_fill_tensor(ctypes.byref(cfg), seed, gain_std, kind, layer,
                                          out.ctypes.data_as(c_void_p), count))
    return out


def rope_tables(max_seq: int, head_dim: int = 128, theta: float = 1e6):
    c = np.empty(max_seq * head_dim, np.uint16)
    s = np.empty(max_seq * head_dim, np.uint16)
    check(library().xpu_qwen3_rope_tables(c.ctypes.data_as(c_void_p), s.ctypes.data_as(c_void_p), max_seq,
                                          head_dim, theta))
    return c, s


class Engine:
    def __init__(self, cfg: Qwen3Config | None = None, max_seq: int = 256, seed: int = 0, gain_std: float = 0.0,
                 runtime: Runtime | None = None, model_dir: str | None = None):
        self.lib = library()
        self.runtime = runtime
        if runtime is not None:
            runtime.add_dependent(self)  # closed before the runtime it allocates from
        handle = c_void_p()
        rt = runtime.handle if runtime else None
        if model_dir is not None:
            check(self.lib.xpu_qwen3_create_from_checkpoint(rt, model_dir.encode(), max_seq, ctypes.byref(handle)))
            self.cfg = Qwen3Config()
            self.handle = handle
            check(self.lib.xpu_qwen3_get_config(handle, ctypes.byref(self.cfg)))
        else:
            check(self.lib.xpu_qwen3_create(rt, ctypes.byref(cfg), max_seq, seed, gain_std, ctypes.byref(handle)))
            self.handle = handle
            self.cfg = cfg
        self.max_seq = max_seq

    def close(self):
        if getattr(self, "handle", None):
            self.lib.xpu_qwen3_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_mode(self, mode: int) -> None:
        check(self.lib.xpu_qwen3_set_mode(self.handle, mode))

    PREFILL_MODES = {"stepwise": 0, "batched": 1, "gemm": 2}

    def set_prefill(self, mode) -> None:
        """Prompt processing in generate: "batched" (default; True),
        "stepwise" (False) or "gemm" (the projections on the MFMA GEMM)."""
        if isinstance(mode, bool):
            mode = "batched" if mode else "stepwise"
        check(self.lib.xpu_qwen3_set_prefill(self.handle, self.PREFILL_MODES[mode]))

    def set_attention_split(self, min_context: int) -> None:
        """Split the attention over compute units for contexts of at least
        min_context positions (0: never); results are bit-identical."""
        check(self.lib.xpu_qwen3_set_attention_split(self.handle, c_uint32(min_context)))

    def decode(self, token: int, position: int) -> int:
        nxt = c_uint32()
        check(self.lib.xpu_qwen3_decode(self.handle, token, position, ctypes.byref(nxt)))
        return nxt.value

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab, np.uint16)
        check(self.lib.xpu_qwen3_logits(self.handle, out.ctypes.data_as(c_void_p), out.size))
        return out

    def hidden(self) -> np.ndarray:
        out = np.empty(self.cfg.hidden, np.uint16)
        check(self.lib.xpu_qwen3_hidden(self.handle, out.ctypes.data_as(c_void_p), out.size))
        return out

    def generate(self, prompt, max_new: int, stop_on_eos: bool = True):
        """Returns (token ids, prompt ms, decode ms)."""
        prompt = np.ascontiguousarray(prompt, np.uint32)
        arr = (c_uint32 * len(prompt))(*prompt.tolist())
        out = (c_uint32 * max(max_new, 1))()
        n = c_uint32()
        pm, dm = c_double(), c_double()
        check(self.lib.xpu_qwen3_generate(self.handle, arr, len(prompt), max_new, int(stop_on_eos), out,
                                          ctypes.byref(n), ctypes.byref(pm), ctypes.byref(dm)))
        return np.array(out[:n.value], np.uint32), pm.value, dm.value
