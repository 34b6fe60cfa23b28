"""The checkpoint loader's validation rules on the host (no GPU): the config
reader, the safetensors tensor directory (qwen3/model.cpp:288-368,448-495)
and the JSON reader underneath them."""
import json
import os

import pytest

import oracle_lib as orc
from checkpoint_util import read_header, write_checkpoint, write_raw_safetensors
from xpu_playground_amd import XpuError, qwen3


def tiny(**over):
    return orc.config("tiny", layers=1, vocab=64, **over)


@pytest.mark.parametrize("tied,sharded", [(1, False), (0, True), (1, True)])
def test_valid_checkpoints_pass(tmp_path, tied, sharded):
    cfg = tiny(tied=tied)
    write_checkpoint(str(tmp_path), cfg, seed=1, gain_std=0.1, sharded=sharded)
    got = qwen3.validate_checkpoint(str(tmp_path))
    assert (got.hidden, got.layers, got.vocab, got.tied) == (cfg.hidden, 1, 64, tied)


def rejects(tmp_path, match):
    with pytest.raises(XpuError, match=match):
        qwen3.validate_checkpoint(str(tmp_path))


def sharded(tmp_path):
    write_checkpoint(str(tmp_path), tiny(tied=0), seed=1, gain_std=0.0, sharded=True)
    index = json.load(open(tmp_path / "model.safetensors.index.json"))
    return index


def save_index(tmp_path, index):
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))


def test_index_total_size_must_match(tmp_path):
    index = sharded(tmp_path)
    index["metadata"]["total_size"] += 2
    save_index(tmp_path, index)
    rejects(tmp_path, "total_size does not match")
    index["metadata"]["total_size"] = -1
    save_index(tmp_path, index)
    rejects(tmp_path, "total_size must be an unsigned integer")


def test_index_and_shard_headers_must_agree(tmp_path):
    index = sharded(tmp_path)
    wm = index["weight_map"]
    a, b = sorted(set(wm.values()))
    moved = next(k for k, v in wm.items() if v == a)
    wm[moved] = b  # the index now maps a tensor to the shard that lacks it
    save_index(tmp_path, index)
    rejects(tmp_path, "does not map to it|absent from shard")


def test_index_names_a_missing_tensor(tmp_path):
    index = sharded(tmp_path)
    index["weight_map"]["model.layers.0.extra.weight"] = sorted(set(index["weight_map"].values()))[0]
    save_index(tmp_path, index)
    rejects(tmp_path, "absent from shard")


def test_bad_shard_names(tmp_path):
    index = sharded(tmp_path)
    key = next(iter(index["weight_map"]))
    for bad in ("../model.safetensors", "", 3):
        index["weight_map"][key] = bad
        save_index(tmp_path, index)
        rejects(tmp_path, "invalid shard name")


def rewrite_single(tmp_path, edit):
    """Rewrite model.safetensors with edit(header) applied, payload kept."""
    path = tmp_path / "model.safetensors"
    header, start, size = read_header(path)
    edit(header)
    entries = {k: (v["dtype"], v["shape"], v["data_offsets"]) for k, v in header.items() if k != "__metadata__"}
    write_raw_safetensors(path, entries, size - start)


@pytest.fixture
def single(tmp_path):
    write_checkpoint(str(tmp_path), tiny(), seed=1, gain_std=0.0)
    return tmp_path


def test_offsets_past_the_payload_or_overflowing(single):
    name = "model.norm.weight"

    def past_end(h):
        b, e = h[name]["data_offsets"]
        h[name]["data_offsets"] = [2 ** 64 - 1024, 2 ** 64 - 1024 + (e - b)]  # 8 + header + end wraps past 2^64

    rewrite_single(single, past_end)
    rejects(single, "beyond shard")

    def too_big(h):
        h[name]["data_offsets"] = [0, 2 ** 64]  # not a 64-bit integer

    rewrite_single(single, too_big)
    rejects(single, "invalid data offsets")


def test_overlapping_payloads(single):
    def overlap(h):
        names = sorted(h, key=lambda k: h[k]["data_offsets"][0])
        a, b = names[0], names[1]
        size = h[b]["data_offsets"][1] - h[b]["data_offsets"][0]
        start = h[a]["data_offsets"][1] - 2
        h[b]["data_offsets"] = [start, start + size]

    rewrite_single(single, overlap)
    rejects(single, "overlapping safetensors payloads")


def test_dtype_shape_and_size_rules(single):
    rewrite_single(single, lambda h: h["model.norm.weight"].update(dtype="F32"))
    rejects(single, "not BF16")


def test_byte_size_must_match_shape(tmp_path):
    write_checkpoint(str(tmp_path), tiny(), seed=1, gain_std=0.0)
    rewrite_single(tmp_path, lambda h: h["model.norm.weight"].update(shape=[tiny().hidden - 1]))
    rejects(tmp_path, "byte size does not match")


def test_wrong_shape_missing_and_unexpected_tensors(tmp_path):
    cfg = tiny()
    write_checkpoint(str(tmp_path), cfg, seed=1, gain_std=0.0)
    path = tmp_path / "model.safetensors"
    header, start, size = read_header(path)
    entries = {k: (v["dtype"], v["shape"], v["data_offsets"]) for k, v in header.items() if k != "__metadata__"}
    # a config with another intermediate size: every MLP tensor has the wrong shape
    conf = json.load(open(tmp_path / "config.json"))
    (tmp_path / "config.json").write_text(json.dumps({**conf, "intermediate_size": 2 * cfg.intermediate}))
    rejects(tmp_path, "wrong shape")
    (tmp_path / "config.json").write_text(json.dumps(conf))
    missing = dict(entries)
    del missing["model.layers.0.mlp.up_proj.weight"]
    write_raw_safetensors(path, missing, size - start)
    rejects(tmp_path, "missing tensor: model.layers.0.mlp.up_proj.weight")
    extra = dict(entries)
    extra["model.layers.1.mlp.up_proj.weight"] = ("BF16", [2], [size - start, size - start + 4])
    write_raw_safetensors(path, extra, size - start + 4)
    rejects(tmp_path, "unexpected tensor in checkpoint: model.layers.1.mlp.up_proj.weight")
    extra["model.layers.1.mlp.up_proj.weight"] = entries["model.layers.0.mlp.up_proj.weight"]
    write_raw_safetensors(path, extra, size - start)
    rejects(tmp_path, "overlapping")


def test_header_length_and_truncation(tmp_path):
    write_checkpoint(str(tmp_path), tiny(), seed=1, gain_std=0.0)
    path = tmp_path / "model.safetensors"
    data = path.read_bytes()
    path.write_bytes((len(data)).to_bytes(8, "little") + data[8:])  # header longer than the file
    rejects(tmp_path, "header length")
    path.write_bytes(data[:5])
    rejects(tmp_path, "truncated")


@pytest.mark.parametrize("text,match", [
    ('{"a": 1,}', "malformed JSON at offset 8"),
    ('{"a" 1}', "':' after a member name"),
    ('[1, 2', "',' or ']'"),
    ('{"a": 01}', "malformed JSON"),
    ('{"a": "\\x"}', "valid escape"),
    ('{"a": tru}', "a value"),
    ('{} {}', "end of document"),
    ('{"a": "tab\there"}', "raw control character"),
    # qwen3/model.cpp:204-205: a repeated member name fails, also after
    # unescaping and inside nested objects
    ('{"a": 1, "a": 2}', 'duplicate object key "a"'),
    ('{"a": 1, "\\u0061": 2}', 'duplicate object key "a"'),
    ('{"x": [{"b": 1, "c": 2, "b": 3}]}', 'duplicate object key "b"'),
])
def test_json_reader_rejects_malformed_documents(tmp_path, text, match):
    (tmp_path / "config.json").write_text(text)
    with pytest.raises(XpuError, match=match):
        qwen3.read_config(str(tmp_path))


def test_json_reader_escapes_nesting_and_exact_integers(tmp_path):
    valid = {"hidden_size": 1024, "intermediate_size": 3072, "head_dim": 128, "num_attention_heads": 16,
             "num_key_value_heads": 8, "num_hidden_layers": 28, "vocab_size": 151936, "rms_norm_eps": 1e-6,
             "tie_word_embeddings": False, "hidden_act": "silu", "torch_dtype": "bfloat16",
             "rope_parameters": {"rope_type": "default", "rope_theta": 5e5}, "name": "café \U0001d11e \"q\"",
             "list": [[], {}, [1, [2, {"x": None}]]]}
    text = json.dumps(valid, ensure_ascii=True).replace('"silu"', '"\\u0073ilu"')
    (tmp_path / "config.json").write_text(text.replace('"hidden_act"', '"model_type": "qwen3", "hidden_act"'))
    cfg = qwen3.read_config(str(tmp_path))
    assert cfg.rope_theta == 5e5 and cfg.tied == 0 and cfg.vocab == 151936
    # the same names in different objects are not duplicates; a second
    # hidden_size in the top-level object is
    (tmp_path / "config.json").write_text(text.replace('"hidden_act"', '"model_type": "qwen3", "hidden_act"')
                                          .replace('"list": [', '"list": [{"hidden_size": 1}, '))
    assert qwen3.read_config(str(tmp_path)).hidden == 1024
    (tmp_path / "config.json").write_text(text.replace('"hidden_act"', '"model_type": "qwen3", "hidden_act"')
                                          .replace('"list": [', '"hidden_size": 2048, "list": ['))
    with pytest.raises(XpuError, match='duplicate object key "hidden_size"'):
        qwen3.read_config(str(tmp_path))
    for bad in ("1024.0", "1e3", "-1", "18446744073709551616", "4294967296"):
        (tmp_path / "config.json").write_text(
            json.dumps({**valid, "model_type": "qwen3"}).replace('"hidden_size": 1024', f'"hidden_size": {bad}'))
        with pytest.raises(XpuError, match="hidden_size"):
            qwen3.read_config(str(tmp_path))


def test_safetensors_header_with_a_repeated_tensor_name(tmp_path):
    # a header naming one tensor twice is malformed JSON for the reader
    # (qwen3/model.cpp:204-205), not a second definition that wins
    write_checkpoint(str(tmp_path), tiny(), seed=1, gain_std=0.0)
    path = tmp_path / "model.safetensors"
    header, start, size = read_header(path)
    name = "model.norm.weight"
    text = json.dumps(header)
    entry = json.dumps({name: header[name]})[1:-1]
    text = text[:-1] + ", " + entry + "}"
    data = path.read_bytes()[start:]
    with open(path, "wb") as fh:
        fh.write(len(text).to_bytes(8, "little"))
        fh.write(text.encode())
        fh.write(data)
    rejects(tmp_path, f'duplicate object key "{name}"')
