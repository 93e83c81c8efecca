"""The ``.yuf`` checkpoint container: writer and reader (Python side).

Format (``vulkan/scripts/export_checkpoint.py:32-146``, read by
``vulkan/src/checkpoint.rs:90-149``):

    b"YUFM" | u32 LE version (1) | u64 LE header_len | UTF-8 JSON header | f32 LE blob

The JSON header carries ``format`` = "yufmusicgen-checkpoint", ``version``,
``model_config``, ``midi`` {tokenization, midi_offset = 260, midi_vocab_size,
vocab[], tokenizer_json}, ``source``, ``lm_head_alias`` and ``tensors``
[{name, shape, offset (in floats), count}].  The file size must equal
``data_start + 4 * sum(count)``.  The tied LM head is not stored.

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
FORMAT = "yufmusicgen-checkpoint"
MIDI_OFFSET = 260


def write_yuf(path, cfg: ModelConfig, tensors: dict, source: dict | None = None) -> None:
    """Write ``tensors`` (name -> float32 array, in the given order) to ``path``."""
    path = Path(path)
    entries, offset = [], 0
    for name, value in tensors.items():
        arr = np.ascontiguousarray(value, dtype=np.float32)
        entries.append({"name": name, "shape": list(arr.shape), "offset": offset, "count": int(arr.size)})
        offset += int(arr.size)
    midi_vocab = max(0, cfg.vocab_size - MIDI_OFFSET)
    header = {
        "format": FORMAT,
        "version": VERSION,
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
    blob = json.dumps(header, ensure_ascii=False).encode("utf-8")
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "wb") as handle:
        handle.write(MAGIC)
        handle.write(struct.pack("<I", VERSION))
        handle.write(struct.pack("<Q", len(blob)))
        handle.write(blob)
        for name, value in tensors.items():
            handle.write(np.ascontiguousarray(value, dtype="<f4").tobytes())


def read_yuf(path):
    """Return ``(header dict, {name: float32 array})`` with the checks of checkpoint.rs:90-149."""
    path = Path(path)
    with open(path, "rb") as handle:
        if handle.read(4) != MAGIC:
            raise ValueError(f"{path} is not a .yuf checkpoint (bad magic)")
        (version,) = struct.unpack("<I", handle.read(4))
        if version != VERSION:
            raise ValueError(f"unsupported .yuf version {version}")
        (header_len,) = struct.unpack("<Q", handle.read(8))
        header = json.loads(handle.read(header_len).decode("utf-8"))
        if header.get("format") != FORMAT:
            raise ValueError(f"unexpected .yuf payload format {header.get('format')!r}")
        data_start = handle.tell()
    total = sum(int(t["count"]) for t in header["tensors"])
    size = path.stat().st_size
    if size != data_start + 4 * total:
        raise ValueError(f"checkpoint size mismatch: file has {size} bytes, header expects {data_start + 4 * total}")
    data = np.memmap(path, dtype="<f4", mode="r", offset=data_start, shape=(total,))
    tensors = {}
    for t in header["tensors"]:
        tensors[t["name"]] = np.array(data[t["offset"]:t["offset"] + t["count"]]).reshape(t["shape"])
    return header, tensors


def config_from_header(header: dict) -> ModelConfig:
    mc = header["model_config"]
    return ModelConfig(**{k: mc[k] for k in ModelConfig.__dataclass_fields__ if k in mc})
