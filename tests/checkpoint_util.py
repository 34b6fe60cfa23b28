"""Checkpoint directories for the loader tests: a Hugging Face style Qwen3
checkpoint (config.json, model.safetensors or shards plus an index) holding
the oracle's synthetic weights, and hand-built safetensors files for the
malformed cases."""
import json
import os
import struct

import numpy as np

import oracle_lib as orc


def write_checkpoint(directory, cfg, seed, gain_std, sharded=False, nan_embed=False):
    import torch
    from safetensors.torch import save_file

    names = ["self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
             "self_attn.o_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
             "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight", "input_layernorm.weight",
             "post_attention_layernorm.weight"]
    h, hd = cfg.hidden, cfg.head_dim
    shapes = [(cfg.heads * hd, h), (cfg.kv_heads * hd, h), (cfg.kv_heads * hd, h), (h, cfg.heads * hd), (hd,),
              (hd,), (cfg.intermediate, h), (cfg.intermediate, h), (h, cfg.intermediate), (h,), (h,)]

    def tensor(kind, layer, shape):
        a = orc.fill_tensor(cfg, seed, gain_std, kind, layer)
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).reshape(shape)

    tensors = {}
    for layer in range(cfg.layers):
        for kind, (n, shape) in enumerate(zip(names, shapes)):
            tensors[f"model.layers.{layer}.{n}"] = tensor(kind, layer, shape)
    emb = tensor(orc.W_EMBED, 0, (cfg.vocab, h))
    if nan_embed:
        emb = emb.clone()
        emb[:, 7] = float("nan")
    tensors["model.embed_tokens.weight"] = emb
    tensors["model.norm.weight"] = tensor(orc.W_FINALNORM, 0, (h,))
    if not cfg.tied:
        tensors["lm_head.weight"] = tensor(orc.W_LMHEAD, 0, (cfg.vocab, h))
    config = {"hidden_size": h, "intermediate_size": cfg.intermediate, "head_dim": hd,
              "num_attention_heads": cfg.heads, "num_key_value_heads": cfg.kv_heads,
              "num_hidden_layers": cfg.layers, "vocab_size": cfg.vocab, "max_position_embeddings": 40960,
              "eos_token_id": 151645, "rms_norm_eps": 1e-6, "rope_theta": 1000000.0,
              "tie_word_embeddings": bool(cfg.tied), "hidden_act": "silu", "model_type": "qwen3",
              "torch_dtype": "bfloat16", "rope_scaling": None}
    with open(os.path.join(directory, "config.json"), "w") as fh:
        json.dump(config, fh)
    if not sharded:
        save_file(tensors, os.path.join(directory, "model.safetensors"))
        return
    keys = sorted(tensors)
    half = len(keys) // 2
    shards = {"model-00001-of-00002.safetensors": keys[:half], "model-00002-of-00002.safetensors": keys[half:]}
    weight_map = {}
    for shard, ks in shards.items():
        save_file({k: tensors[k] for k in ks}, os.path.join(directory, shard))
        weight_map.update({k: shard for k in ks})
    total = sum(t.numel() * 2 for t in tensors.values())
    with open(os.path.join(directory, "model.safetensors.index.json"), "w") as fh:
        json.dump({"metadata": {"total_size": total}, "weight_map": weight_map}, fh)


def write_raw_safetensors(path, entries, payload_bytes, header_extra=None):
    """A safetensors file whose header lists `entries` ({name: (dtype, shape,
    [begin, end])}, written as given, valid or not) over `payload_bytes`
    zero bytes."""
    header = {name: {"dtype": dt, "shape": shape, "data_offsets": offs} for name, (dt, shape, offs) in entries.items()}
    if header_extra:
        header.update(header_extra)
    text = json.dumps(header).encode()
    with open(path, "wb") as fh:
        fh.write(struct.pack("<Q", len(text)))
        fh.write(text)
        fh.write(b"\0" * payload_bytes)


def read_header(path):
    with open(path, "rb") as fh:
        n = struct.unpack("<Q", fh.read(8))[0]
        return json.loads(fh.read(n)), 8 + n, os.path.getsize(path)
