"""The ``.yuf`` checkpoint container: writer and reader (Python side).

Format (``vulkan/scripts/export_checkpoint.py:32-146``, read by
``vulkan/src/checkpoint.rs:90-149``):

    b"YUFM" | u32 LE version (1) | u64 LE header_len | UTF-8 JSON header | f32 LE blob

The JSON header carries ``format`` = "yufmusicgen-checkpoint", ``version``,
``model_config``, ``midi`` {tokenization, midi_offset = 260, midi_vocab_size,
vocab[], tokenizer_json}, ``source``, ``lm_head_alias`` and ``tensors``
[{name, shape, offset (in floats), count}].  The file size must equal
``data_start + 4 * sum(count)``.  The tied LM head is not stored.

Version 2 (this build's extension for bf16 weights; written only when some
tensor is bf16, so all-f32 files stay version 1): each tensor entry also has
``dtype`` ("f32" or "bf16", little-endian) and its ``offset`` counts bytes from
the start of the payload, a multiple of the element size; the header has
``payload_bytes`` and the file size must equal ``data_start + payload_bytes``.
Readers return float32 (a bf16 value widens exactly).

The engine (``libyufhip.so``) has its own C++ loader with the same checks;
this module writes the synthetic checkpoints the tests and the benchmark use.
"""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

from .config import ModelConfig

MAGIC = b"YUFM"
VERSION = 1
VERSION_TYPED = 2
FORMAT = "yufmusicgen-checkpoint"
MIDI_OFFSET = 260
DTYPE_SIZE = {"f32": 4, "bf16": 2}
# nn.Linear weights by name suffix (the tensors a bf16 checkpoint stores as bf16).
LINEAR_SUFFIXES = (
    "receptance.weight", "key.weight", "value.weight", "output.weight", "time_mix.w1", "time_mix.w2",
    "time_mix.a1", "time_mix.a2", "time_mix.g1", "time_mix.g2", "input.weight", "write_gate.weight",
    "read_gate.weight", "ffn_in.weight", "ffn_gate.weight", "ffn_out.weight",
)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even; NaN stays NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def write_yuf(path, cfg: ModelConfig, tensors: dict, source: dict | None = None, dtypes: dict | None = None,
              linear_bf16: bool = False) -> None:
    """Write ``tensors`` (name -> float32 array, in the given order) to ``path``.

    ``dtypes`` maps tensor names to "f32" / "bf16"; ``linear_bf16`` stores every
    nn.Linear weight as bf16.  Any bf16 tensor makes the file version 2."""
    path = Path(path)
    kinds = {}
    for name in tensors:
        kind = (dtypes or {}).get(name, "bf16" if linear_bf16 and name.endswith(LINEAR_SUFFIXES) else "f32")
        if kind not in DTYPE_SIZE:
            raise ValueError(f"unknown tensor dtype {kind!r} for {name}")
        kinds[name] = kind
    typed = any(k != "f32" for k in kinds.values())
    entries, payloads, offset = [], [], 0
    for name, value in tensors.items():
        arr = np.ascontiguousarray(value, dtype=np.float32)
        if typed:
            raw = bf16_bits(arr).astype("<u2").tobytes() if kinds[name] == "bf16" else arr.astype("<f4").tobytes()
            offset = -(-offset // DTYPE_SIZE[kinds[name]]) * DTYPE_SIZE[kinds[name]]
            entries.append({"name": name, "shape": list(arr.shape), "dtype": kinds[name], "offset": offset,
                            "count": int(arr.size)})
            payloads.append((offset, raw))
            offset += len(raw)
        else:
            entries.append({"name": name, "shape": list(arr.shape), "offset": offset, "count": int(arr.size)})
            payloads.append((4 * offset, arr.astype("<f4").tobytes()))
            offset += int(arr.size)
    version = VERSION_TYPED if typed else VERSION
    midi_vocab = max(0, cfg.vocab_size - MIDI_OFFSET)
    header = {
        "format": FORMAT,
        "version": version,
        "model_config": {
            "vocab_size": cfg.vocab_size,
            "d_model": cfg.d_model,
            "n_layers": cfg.n_layers,
            "n_heads": cfg.n_heads,
            "head_size": cfg.head_size,
            "rosa_size": cfg.rosa_size,
            "dropout": cfg.dropout,
            "tie_embeddings": cfg.tie_embeddings,
        },
        "midi": {
            "tokenization": "REMI",
            "midi_offset": MIDI_OFFSET,
            "midi_vocab_size": midi_vocab,
            "vocab": [f"Synthetic_{i}" for i in range(midi_vocab)],
            "tokenizer_json": None,
        },
        "source": source or {"checkpoint": "synthetic", "step": -1, "phase": ""},
        "lm_head_alias": "token_embedding.weight" if cfg.tie_embeddings else None,
        "tensors": entries,
    }
    if typed:
        header["payload_bytes"] = offset
    blob = json.dumps(header, ensure_ascii=False).encode("utf-8")
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "wb") as handle:
        handle.write(MAGIC)
        handle.write(struct.pack("<I", version))
        handle.write(struct.pack("<Q", len(blob)))
        handle.write(blob)
        written = 0
        for start, raw in payloads:
            handle.write(b"\0" * (start - written))
            handle.write(raw)
            written = start + len(raw)


def read_yuf(path):
    """Return ``(header dict, {name: float32 array})`` with the checks of checkpoint.rs:90-149."""
    path = Path(path)
    with open(path, "rb") as handle:
        if handle.read(4) != MAGIC:
            raise ValueError(f"{path} is not a .yuf checkpoint (bad magic)")
        (version,) = struct.unpack("<I", handle.read(4))
        if version not in (VERSION, VERSION_TYPED):
            raise ValueError(f"unsupported .yuf version {version}")
        (header_len,) = struct.unpack("<Q", handle.read(8))
        header = json.loads(handle.read(header_len).decode("utf-8"))
        if header.get("format") != FORMAT:
            raise ValueError(f"unexpected .yuf payload format {header.get('format')!r}")
        data_start = handle.tell()
    size = path.stat().st_size
    tensors = {}
    if version == VERSION:
        total = sum(int(t["count"]) for t in header["tensors"])
        if size != data_start + 4 * total:
            raise ValueError(f"checkpoint size mismatch: file has {size} bytes, header expects {data_start + 4 * total}")
        data = np.memmap(path, dtype="<f4", mode="r", offset=data_start, shape=(total,))
        for t in header["tensors"]:
            tensors[t["name"]] = np.array(data[t["offset"]:t["offset"] + t["count"]]).reshape(t["shape"])
        return header, tensors
    payload = int(header.get("payload_bytes", -1))
    if payload < 0 or size != data_start + payload:
        raise ValueError(f"checkpoint size mismatch: file has {size} bytes, header expects {data_start + payload}")
    raw = np.memmap(path, dtype=np.uint8, mode="r", offset=data_start, shape=(payload,)) if payload else np.zeros(0, np.uint8)
    for t in header["tensors"]:
        kind, off, count = t.get("dtype"), int(t["offset"]), int(t["count"])
        if kind not in DTYPE_SIZE:
            raise ValueError(f"tensor {t['name']}: unknown dtype {kind!r}")
        width = DTYPE_SIZE[kind]
        if off < 0 or off % width or off + width * count > payload:
            raise ValueError(f"tensor {t['name']} lies outside the payload or is misaligned")
        chunk = np.array(raw[off:off + width * count])
        values = chunk.view("<f4").astype(np.float32) if kind == "f32" else bf16_to_f32(chunk.view("<u2"))
        tensors[t["name"]] = values.reshape(t["shape"])
    return header, tensors


def config_from_header(header: dict) -> ModelConfig:
    mc = header["model_config"]
    return ModelConfig(**{k: mc[k] for k in ModelConfig.__dataclass_fields__ if k in mc})
