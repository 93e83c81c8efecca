"""Python host mirror of the engine API (the C ABI of ``include/yuf_engine.h``).

Keeps the reference engine's surface -- ``Checkpoint.load`` /
``Model(ckpt)`` / ``model.step(token)`` / ``model.reset_state()`` and the
sampler's ``Mt19937`` / ``sample_token`` / ``argmax`` (vulkan/src/checkpoint.rs,
vulkan/src/compute/model.rs:24-65, vulkan/src/sampler.rs) -- and adds the
batched multi-stream calls (prefill, step, state save/load) the HIP engine
provides.  Host arrays are numpy; the ``*_device`` calls take torch GPU
tensors (torch is only the device-memory plumbing).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from ._lib import ModelConfigC, RngC, c_float_p, check, lib

LOGITS_NONE, LOGITS_LAST, LOGITS_ALL = 0, 1, 2
_MODES = {"none": LOGITS_NONE, "last": LOGITS_LAST, "all": LOGITS_ALL}


def _config_dict(c: ModelConfigC) -> dict:
    return {name: getattr(c, name) for name, _ in ModelConfigC._fields_}


class Checkpoint:
    """A loaded ``.yuf`` file (``Checkpoint::load``, checkpoint.rs:90-149)."""

    def __init__(self, handle):
        self._h = handle

    @classmethod
    def load(cls, path) -> "Checkpoint":
        handle = ctypes.c_void_p()
        check(lib().yuf_ckpt_load(str(Path(path)).encode(), ctypes.byref(handle)))
        return cls(handle)

    @property
    def config(self) -> dict:
        c = ModelConfigC()
        check(lib().yuf_ckpt_config(self._h, ctypes.byref(c)))
        return _config_dict(c)

    @property
    def header_json(self) -> str:
        """The file's JSON header verbatim (``checkpoint.header``, checkpoint.rs:60-81)."""
        text = ctypes.c_char_p()
        size = ctypes.c_size_t()
        version = ctypes.c_uint32()
        check(lib().yuf_ckpt_header_json(self._h, ctypes.byref(text), ctypes.byref(size), ctypes.byref(version)))
        return ctypes.string_at(text, size.value).decode("utf-8")

    @property
    def header(self) -> dict:
        import json

        return json.loads(self.header_json)

    @property
    def version(self) -> int:
        text = ctypes.c_char_p()
        version = ctypes.c_uint32()
        check(lib().yuf_ckpt_header_json(self._h, ctypes.byref(text), None, ctypes.byref(version)))
        return int(version.value)

    def tensor(self, name: str) -> np.ndarray:
        """``Checkpoint::tensor`` + ``tensor_dims`` (checkpoint.rs:151-168); a copy."""
        data = c_float_p()
        count = ctypes.c_int64()
        ndim = ctypes.c_int32()
        dims = (ctypes.c_int64 * 8)()
        check(lib().yuf_ckpt_tensor(self._h, name.encode(), ctypes.byref(data), ctypes.byref(count),
                                    ctypes.byref(ndim), dims))
        flat = np.ctypeslib.as_array(data, shape=(count.value,)).copy()
        return flat.reshape([dims[i] for i in range(ndim.value)])

    def close(self) -> None:
        if self._h:
            lib().yuf_ckpt_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Engine:
    """Device-resident weights and ``max_streams`` recurrent-state slots."""

    WEIGHT_TYPES = {"f32": 0, "bf16": 1}

    def __init__(self, ckpt: Checkpoint, max_streams: int = 1, max_tokens: int = 4096, weight_dtype: str = "f32"):
        """``weight_dtype`` "bf16": bf16 projection weights with fp32 accumulation
        (``yuf_engine_create_ex``); "f32" (default): everything fp32."""
        if weight_dtype not in self.WEIGHT_TYPES:
            raise ValueError(f"weight_dtype must be one of {sorted(self.WEIGHT_TYPES)}, got {weight_dtype!r}")
        handle = ctypes.c_void_p()
        check(lib().yuf_engine_create_ex(ckpt._h, int(max_streams), int(max_tokens),
                                         self.WEIGHT_TYPES[weight_dtype], ctypes.byref(handle)))
        self._h = handle
        self.weight_dtype = weight_dtype
        c = ModelConfigC()
        check(lib().yuf_engine_config(self._h, ctypes.byref(c)))
        self.config = _config_dict(c)
        self.vocab = self.config["vocab_size"]
        self.max_streams = int(max_streams)

    # ---------------------------------------------------------------- host API
    @staticmethod
    def _slots(n, slots):
        arr = np.arange(n, dtype=np.int32) if slots is None else np.ascontiguousarray(slots, dtype=np.int32)
        if arr.shape != (n,):
            raise ValueError("slots must have one entry per stream")
        return arr

    def prefill(self, tokens, slots=None, logits: str = "last"):
        """Run ``tokens`` [n, T] through the model from each slot's current state.

        Returns logits ``[n, V]`` ("last"), ``[n, T, V]`` ("all") or None ("none")."""
        tok = np.ascontiguousarray(tokens, dtype=np.int32)
        if tok.ndim != 2:
            raise ValueError("tokens must have shape [n, T]")
        n, steps = tok.shape
        mode = _MODES[logits]
        sl = self._slots(n, slots)
        out = None
        if mode == LOGITS_LAST:
            out = np.empty((n, self.vocab), np.float32)
        elif mode == LOGITS_ALL:
            out = np.empty((n, steps, self.vocab), np.float32)
        check(lib().yuf_prefill(self._h, n, sl.ctypes.data, steps, tok.ctypes.data,
                                None if out is None else out.ctypes.data, mode))
        return out

    def step(self, tokens, slots=None) -> np.ndarray:
        """One token per stream -> logits [n, V] (``Model::step``, model.rs:54-60)."""
        tok = np.ascontiguousarray(np.atleast_1d(tokens), dtype=np.int32)
        n = tok.shape[0]
        out = np.empty((n, self.vocab), np.float32)
        check(lib().yuf_step(self._h, n, self._slots(n, slots).ctypes.data, tok.ctypes.data, out.ctypes.data))
        return out

    def reset_state(self, slot: int = -1) -> None:
        check(lib().yuf_state_reset(self._h, int(slot)))

    @property
    def state_size(self) -> int:
        return int(lib().yuf_state_size(self._h))

    def save_state(self, slot: int) -> np.ndarray:
        blob = np.empty(self.state_size // 4, np.float32)
        check(lib().yuf_state_save(self._h, int(slot), blob.ctypes.data))
        return blob

    def load_state(self, slot: int, blob) -> None:
        arr = np.ascontiguousarray(blob, dtype=np.float32)
        if arr.size * 4 != self.state_size:
            raise ValueError(f"state blob must hold {self.state_size // 4} floats")
        check(lib().yuf_state_load(self._h, int(slot), arr.ctypes.data))

    # -------------------------------------------------------------- device API
    @property
    def stream(self) -> int:
        return int(lib().yuf_engine_stream(self._h) or 0)

    def prefill_device(self, tokens_dev, logits_dev, slots, logits: str = "last") -> None:
        """Asynchronous on the engine's stream; tokens [n, T] int32, logits float32 GPU tensors."""
        n, steps = tokens_dev.shape
        sl = self._slots(n, slots)
        check(lib().yuf_prefill_device(self._h, n, sl.ctypes.data, steps, tokens_dev.data_ptr(),
                                       None if logits_dev is None else logits_dev.data_ptr(), _MODES[logits]))

    def step_device(self, tokens_dev, logits_dev, slots) -> None:
        n = tokens_dev.shape[0]
        check(lib().yuf_step_device(self._h, n, self._slots(n, slots).ctypes.data, tokens_dev.data_ptr(),
                                    logits_dev.data_ptr()))

    def take_error(self) -> None:
        """Raise if a device entry point read an out-of-range token id since the
        last check (``yuf_engine_take_error``; synchronises the engine stream)."""
        check(lib().yuf_engine_take_error(self._h))

    def time_wkv_step(self, iters: int = 50):
        """Mean duration (us) and stream count of the last decode step's
        first-layer WKV-7 step kernel, relaunched alone ``iters`` times with its
        own inputs (``yuf_engine_time_wkv_step``; the engine state is unchanged)."""
        us, n = ctypes.c_float(), ctypes.c_int()
        check(lib().yuf_engine_time_wkv_step(self._h, iters, ctypes.byref(us), ctypes.byref(n)))
        return float(us.value), int(n.value)

    def close(self) -> None:
        if self._h:
            lib().yuf_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """Single-stream drop-in for the reference ``Model`` (model.rs:24-65)."""

    def __init__(self, ckpt: Checkpoint):
        self.engine = Engine(ckpt, max_streams=1, max_tokens=4096)
        self.config = self.engine.config

    def step(self, token: int) -> np.ndarray:
        return self.engine.step([int(token)])[0]

    def reset_state(self) -> None:
        self.engine.reset_state(0)


# ------------------------------------------------------------------- sampling
class Mt19937:
    """torch's CPU generator (``torch.manual_seed``), sampler.rs:22-82."""

    def __init__(self, seed: int):
        self._rng = RngC()
        lib().yuf_rng_seed(ctypes.byref(self._rng), int(seed) & 0xFFFFFFFFFFFFFFFF)

    def copy(self) -> "Mt19937":
        """An independent generator in the same state."""
        other = Mt19937.__new__(Mt19937)
        other._rng = RngC()
        ctypes.memmove(ctypes.byref(other._rng), ctypes.byref(self._rng), ctypes.sizeof(RngC))
        return other

    def next_u32(self) -> int:
        return int(lib().yuf_rng_next_u32(ctypes.byref(self._rng)))

    def next_uniform(self) -> float:
        return float(lib().yuf_rng_next_uniform(ctypes.byref(self._rng)))

    def exp_draws(self, vocab: int, k: int):
        """The Exp(1) draws one host sample over ``vocab`` logits consumes:
        (the first ``k`` as float32, the first later position whose uniform is
        0 or -1) -- the device sampler's exact-mode input."""
        q = np.empty(k, np.float32)
        fz = ctypes.c_int32()
        check(lib().yuf_rng_exp_draws(ctypes.byref(self._rng), int(vocab), int(k), q.ctypes.data if k else None,
                                      ctypes.byref(fz)))
        return q, int(fz.value)


def sample_token(logits, temperature: float, top_p: float, rng: Mt19937, top_k: int = 0) -> int:
    """Token-for-token torch's CPU ``sample_token`` (cli/generate.py:45-56) under the same seed."""
    arr = np.ascontiguousarray(logits, dtype=np.float32)
    out = lib().yuf_sample(arr.ctypes.data, arr.size, float(temperature), float(top_p), int(top_k),
                           ctypes.byref(rng._rng))
    if out < 0:
        check(out)
    return int(out)


def argmax(logits) -> int:
    arr = np.ascontiguousarray(logits, dtype=np.float32)
    out = lib().yuf_argmax(arr.ctypes.data, arr.size)
    if out < 0:
        check(out)
    return int(out)


def generation_mask(logits, index: int, blocked_raw_ids=(), midi_offset: int = 260, eos_id: int = 2,
                    min_before_eos: int = 16) -> np.ndarray:
    """The generation loop's mask (vulkan/src/generation.rs:195-203): MIDI ids
    only, minus blocked Program ids, plus EOS from step ``min_before_eos``."""
    arr = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty_like(arr)
    blocked = np.ascontiguousarray(blocked_raw_ids, dtype=np.int32)
    check(lib().yuf_generation_mask(arr.ctypes.data, arr.size, index, midi_offset, eos_id, min_before_eos,
                                    blocked.ctypes.data if blocked.size else None, blocked.size,
                                    out.ctypes.data))
    return out


def sample_device(logits_dev, tokens_dev, temperature: float, top_k: int, seed: int, counter: int, stream=None):
    """Top-k sampling of every row of ``logits_dev`` [n, V] on the GPU."""
    n, vocab = logits_dev.shape
    import torch

    st = torch.cuda.current_stream().cuda_stream if stream is None else stream
    check(lib().yuf_sample_device(n, vocab, logits_dev.data_ptr(), float(temperature), int(top_k), int(seed),
                                  int(counter), tokens_dev.data_ptr(), st))


def sample_device_masked(logits_dev, tokens_dev, temperature: float, top_p: float, top_k: int, *,
                         mask: dict | None = None, index=0, exp_draws=None, first_zero=None, seed: int = 0,
                         counter: int = 0, stream=None) -> None:
    """Generation mask + sampler of every row of ``logits_dev`` [n, V] on the GPU
    (``yuf_sample_device_masked``).  ``mask``: dict(midi_offset=260, eos_id=2,
    min_before_eos=16, blocked=(...)) or None; ``index``: an int for every
    stream or an int32 GPU tensor [n]; ``exp_draws`` [n, top_k] float32 and
    ``first_zero`` [n] int32 GPU tensors (from ``Mt19937.exp_draws``) select
    the exact mode, else the counter-based draws of ``seed`` / ``counter``.
    ``top_k`` 0 (or >= V) samples over the whole vocabulary (V <= 24576), the
    reference's top-p sampling; its exact mode takes all V draws,
    ``exp_draws`` [n, V] from ``Mt19937.exp_draws(V, V)``."""
    import torch

    n, vocab = logits_dev.shape
    st = torch.cuda.current_stream().cuda_stream if stream is None else stream
    mo, eos, mbe, blocked = -1, 2, 16, np.zeros(0, np.int32)
    if mask is not None:
        mo = int(mask.get("midi_offset", 260))
        eos = int(mask.get("eos_id", 2))
        mbe = int(mask.get("min_before_eos", 16))
        blocked = np.ascontiguousarray(mask.get("blocked", ()), dtype=np.int32)
    idx_host, idx_dev = (int(index), None) if isinstance(index, (int, np.integer)) else (0, index)
    check(lib().yuf_sample_device_masked(
        n, vocab, logits_dev.data_ptr(), float(temperature), float(top_p), int(top_k), mo, eos, mbe, idx_host,
        None if idx_dev is None else idx_dev.data_ptr(), blocked.ctypes.data if blocked.size else None, blocked.size,
        None if exp_draws is None else exp_draws.data_ptr(), None if first_zero is None else first_zero.data_ptr(),
        int(seed), int(counter), tokens_dev.data_ptr(), st))
