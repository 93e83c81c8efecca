"""The .yuf container: Python writer/reader and the C++ loader behind the ABI.

Checks follow vulkan/src/checkpoint.rs:90-149 (magic, version, JSON header,
exact payload size) and export_checkpoint.py:32-146 (layout, tensor order).
"""

import json
import os
import struct

import numpy as np
import pytest

from yufmusicgen_amd._lib import YufError
from yufmusicgen_amd.checkpoint import read_yuf, write_yuf
from yufmusicgen_amd.config import PRESETS
from yufmusicgen_amd.engine import Checkpoint
from yufmusicgen_amd.synth import synth_weights, tensor_specs


@pytest.fixture(scope="module")
def tiny_yuf(tmp_path_factory):
    cfg = PRESETS["state_test"]
    path = tmp_path_factory.mktemp("ck") / "tiny.yuf"
    weights = synth_weights(cfg, seed=3)
    write_yuf(path, cfg, weights)
    return path, cfg, weights


def test_python_roundtrip_and_export_order(tiny_yuf):
    path, cfg, weights = tiny_yuf
    header, tensors = read_yuf(path)
    assert header["format"] == "yufmusicgen-checkpoint" and header["version"] == 1
    assert [t["name"] for t in header["tensors"]] == [n for n, _ in tensor_specs(cfg)]
    # Offsets are contiguous float indices (export_checkpoint.py:90-100).
    offsets = [t["offset"] for t in header["tensors"]]
    counts = [t["count"] for t in header["tensors"]]
    assert offsets == list(np.cumsum([0] + counts[:-1]))
    # mix_r..mix_g contiguous and in registration order (model.rs:962).
    names = [t["name"] for t in header["tensors"]]
    i = names.index("blocks.0.time_mix.mix_r")
    assert names[i:i + 6] == [f"blocks.0.time_mix.mix_{c}" for c in "rwkvag"]
    for name, value in weights.items():
        np.testing.assert_array_equal(tensors[name], value)


def test_cpp_loader_matches(tiny_yuf):
    path, cfg, weights = tiny_yuf
    ck = Checkpoint.load(path)
    c = ck.config
    assert (c["vocab_size"], c["d_model"], c["n_layers"], c["n_heads"], c["head_size"], c["rosa_size"]) == (
        cfg.vocab_size, cfg.d_model, cfg.n_layers, cfg.n_heads, cfg.head_size, cfg.rosa_size)
    assert c["low_rank"] == weights["blocks.0.time_mix.w1"].shape[1]
    assert c["midi_offset"] == 260 and c["tie_embeddings"] == 1
    for name in ("token_embedding.weight", "blocks.1.time_mix.w2", "blocks.0.rosa.householder", "final_norm.bias"):
        np.testing.assert_array_equal(ck.tensor(name), weights[name])
    with pytest.raises(YufError) as err:
        ck.tensor("no.such.tensor")
    assert err.value.status == -6


def test_low_rank_comes_from_w1_shape(tmp_path):
    """d_model 1024: Python rounding gives 64, the Rust formula 96 (checkpoint.rs:27-30)."""
    cfg = PRESETS["wide"]
    small = type(cfg)(vocab_size=1024, d_model=1024, n_layers=1, n_heads=16, head_size=64, rosa_size=8)
    assert small.low_rank == 64
    path = tmp_path / "wide.yuf"
    write_yuf(path, small, synth_weights(small, seed=0))
    assert Checkpoint.load(path).config["low_rank"] == 64


def _corrupt(path, tmp_path, mutate):
    data = bytearray(path.read_bytes())
    out = tmp_path / "bad.yuf"
    out.write_bytes(bytes(mutate(data)))
    return out


@pytest.mark.parametrize("case", ["magic", "version", "truncated", "extra", "json", "format", "shape", "no_tie",
                                  "no_dropout", "no_midi", "midi_fields", "small_vocab", "no_header_version"])
def test_cpp_loader_rejects_malformed_files(tiny_yuf, tmp_path, case):
    """The rejections of vulkan/src/checkpoint.rs:90-149: magic, version, size,
    JSON, format; serde's required fields (tie_embeddings, dropout, the midi
    header, the header's version, :14-24, :58-80); and ModelConfig::validate's
    vocab_size >= d_model (:44-46)."""
    path = tiny_yuf[0]
    header_len = struct.unpack("<Q", path.read_bytes()[8:16])[0]

    def rewrite_header(data, fn):
        header = json.loads(bytes(data[16:16 + header_len]))
        fn(header)
        blob = json.dumps(header).encode()
        return data[:8] + struct.pack("<Q", len(blob)) + blob + data[16 + header_len:]

    mutate = {
        "magic": lambda d: b"NOPE" + d[4:],
        "version": lambda d: d[:4] + struct.pack("<I", 3) + d[8:],
        "truncated": lambda d: d[:-4],
        "extra": lambda d: d + b"\0\0\0\0",
        "json": lambda d: d[:16] + b"{" * 3 + d[19:],
        "format": lambda d: rewrite_header(d, lambda h: h.update(format="other")),
        "shape": lambda d: rewrite_header(d, lambda h: h["tensors"][0].update(shape=[1, 2])),
        "no_tie": lambda d: rewrite_header(d, lambda h: h["model_config"].pop("tie_embeddings")),
        "no_dropout": lambda d: rewrite_header(d, lambda h: h["model_config"].pop("dropout")),
        "no_midi": lambda d: rewrite_header(d, lambda h: h.pop("midi")),
        "midi_fields": lambda d: rewrite_header(d, lambda h: h["midi"].pop("tokenization")),
        "small_vocab": lambda d: rewrite_header(d, lambda h: h["model_config"].update(
            vocab_size=h["model_config"]["d_model"] - 1)),
        "no_header_version": lambda d: rewrite_header(d, lambda h: h.pop("version")),
    }[case]
    bad = _corrupt(path, tmp_path, mutate)
    with pytest.raises(YufError) as err:
        Checkpoint.load(bad)
    assert err.value.status == -3, str(err.value)


def test_missing_file_is_io_error(tmp_path):
    with pytest.raises(YufError) as err:
        Checkpoint.load(tmp_path / "absent.yuf")
    assert err.value.status == -2


def test_golden_fixture_loads(golden_dir):
    ck = Checkpoint.load(os.path.join(golden_dir, "model_state_test.yuf"))
    assert ck.config["d_model"] == 32 and ck.config["n_layers"] == 2


# ----------------------------------------------------------------- version 2
def _bf16_round(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    return r.view(np.float32)


@pytest.fixture(scope="module")
def bf16_yuf(tmp_path_factory):
    cfg = PRESETS["state_test"]
    path = tmp_path_factory.mktemp("ck2") / "bf16.yuf"
    weights = synth_weights(cfg, seed=4)
    write_yuf(path, cfg, weights, linear_bf16=True)
    return path, cfg, weights


def test_v2_bf16_roundtrip_python_and_cpp(bf16_yuf):
    """nn.Linear weights stored as bf16 (round to nearest even, checked against
    the bit-level rule), everything else f32 and unchanged, in both readers."""
    path, cfg, weights = bf16_yuf
    header, tensors = read_yuf(path)
    assert header["version"] == 2 and struct.unpack("<I", path.read_bytes()[4:8])[0] == 2
    kinds = {t["name"]: t["dtype"] for t in header["tensors"]}
    assert kinds["blocks.0.time_mix.receptance.weight"] == "bf16" and kinds["blocks.0.ffn_in.weight"] == "bf16"
    assert kinds["token_embedding.weight"] == "f32" and kinds["blocks.0.time_mix.k_k"] == "f32"
    for t in header["tensors"]:
        assert t["offset"] % (2 if t["dtype"] == "bf16" else 4) == 0
    ck = Checkpoint.load(path)
    for name, value in weights.items():
        expect = _bf16_round(value) if kinds[name] == "bf16" else np.asarray(value, dtype=np.float32)
        np.testing.assert_array_equal(tensors[name], expect)
        np.testing.assert_array_equal(ck.tensor(name), expect)
    # bf16 tensors take half the bytes.
    f32_bytes = sum(np.asarray(v).size for v in weights.values()) * 4
    bf16_count = sum(np.asarray(weights[n]).size for n, k in kinds.items() if k == "bf16")
    assert header["payload_bytes"] <= f32_bytes - 2 * bf16_count + 2 * len(weights)


def test_v2_all_f32_stays_version_1(tmp_path):
    cfg = PRESETS["state_test"]
    path = tmp_path / "f.yuf"
    write_yuf(path, cfg, synth_weights(cfg, seed=4), dtypes={})
    assert read_yuf(path)[0]["version"] == 1


@pytest.mark.parametrize("case", ["dtype", "misaligned", "payload", "outside", "no_payload_field"])
def test_v2_loader_rejects_malformed_files(bf16_yuf, tmp_path, case):
    path = bf16_yuf[0]
    header_len = struct.unpack("<Q", path.read_bytes()[8:16])[0]

    def rewrite_header(data, fn):
        header = json.loads(bytes(data[16:16 + header_len]))
        fn(header)
        blob = json.dumps(header).encode()
        return data[:8] + struct.pack("<Q", len(blob)) + blob + data[16 + header_len:]

    def first_bf16(h):
        return next(t for t in h["tensors"] if t["dtype"] == "bf16")

    mutate = {
        "dtype": lambda d: rewrite_header(d, lambda h: first_bf16(h).update(dtype="f16")),
        "misaligned": lambda d: rewrite_header(d, lambda h: first_bf16(h).update(offset=first_bf16(h)["offset"] + 1)),
        "payload": lambda d: d[:-2],
        "outside": lambda d: rewrite_header(d, lambda h: h["tensors"][-1].update(offset=h["payload_bytes"])),
        "no_payload_field": lambda d: rewrite_header(d, lambda h: h.pop("payload_bytes")),
    }[case]
    bad = _corrupt(path, tmp_path, mutate)
    with pytest.raises(YufError) as err:
        Checkpoint.load(bad)
    assert err.value.status == -3, str(err.value)
    with pytest.raises((ValueError, KeyError)):
        read_yuf(bad)


def test_header_json_exposes_midi_header_without_a_second_load(tiny_yuf):
    """``yuf_ckpt_header_json``: the verbatim JSON the Rust loop reads as
    ``checkpoint.header`` (midi_offset, midi_vocab_size, vocab, tokenizer_json;
    vulkan/src/generation.rs:102-117), byte-identical to the file's header."""
    path, cfg, _ = tiny_yuf
    ck = Checkpoint.load(path)
    raw = open(path, "rb").read()
    (header_len,) = struct.unpack("<Q", raw[8:16])
    assert ck.header_json.encode("utf-8") == raw[16:16 + header_len]
    assert ck.version == 1
    h = ck.header
    assert h["midi"]["midi_offset"] == 260
    assert h["midi"]["midi_vocab_size"] + 260 == cfg.vocab_size == h["model_config"]["vocab_size"]
    assert len(h["midi"]["vocab"]) == h["midi"]["midi_vocab_size"]
    assert "tokenizer_json" in h["midi"]


def test_header_json_of_version_2_file(tmp_path):
    cfg = PRESETS["state_test"]
    path = tmp_path / "v2.yuf"
    write_yuf(path, cfg, synth_weights(cfg, seed=4), linear_bf16=True)
    ck = Checkpoint.load(path)
    assert ck.version == 2 and ck.header["version"] == 2 and ck.header["payload_bytes"] > 0
