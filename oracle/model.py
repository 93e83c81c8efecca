"""Full YufMusicGen forward / step -- CPU restatement (test infrastructure only).

Follows ``yufmusicgen/model.py`` op for op with ``use_cuda_kernel=False`` and
``use_rosa_scan=False`` (the reference recurrences; the torch-scan ROSA path
``model.py:224-258`` multiplies by the raw read gate and is not reproduced):

* TimeMix inputs   ``model.py:97-131``      token shift x + (x - x_prev) * mu
* WKV-7 scan       ``model.py:145-165``      (``oracle.wkv7``)
* TimeMix output   ``model.py:195-197``      W_o(LN_out(y) * g); next previous = normed x[:, -1]
* ROSA             ``model.py:290-342``      (``oracle.rosa``)
* Block            ``model.py:365-378``      pre-LN residual TimeMix -> ROSA -> FFN
* Model            ``model.py:406-431``      embedding, blocks, final LN, tied LM head

Weights are a dict keyed by the reference's ``state_dict`` names (the names
the ``.yuf`` container carries, ``vulkan/src/compute/model.rs:916-951``).

``bf16_linear=True`` restates the bf16-weight configuration (C5's weight type):
every nn.Linear weight and the LM head (not the embedding gather) is rounded to
bf16 -- torch's float32 -> bfloat16 cast, round to nearest even -- and the model
then computes in ``dtype`` as the fp32 reference does (projection inputs are
not rounded; norms, gates and both recurrences are unchanged).  This is the
reference PyTorch module loaded with bf16-valued weights.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
from torch.nn import functional as F

from .rosa import rosa_scan
from .wkv7 import wkv7_scan, wkv7_scan_chunked

LN_EPS = 1e-5  # nn.LayerNorm default, model.py:89,346-356


@dataclass
class LayerState:
    previous: torch.Tensor  # [B, d]      normed input of the last token (model.py:197)
    memory: torch.Tensor  # [B, H, N, N] WKV state, (i=value row, j=key column)
    rosa: torch.Tensor  # [B, D]


# nn.Linear weights (by name suffix), including the low-rank pairs.
_LINEAR_SUFFIXES = (
    "receptance.weight", "key.weight", "value.weight", "output.weight", "time_mix.w1", "time_mix.w2",
    "time_mix.a1", "time_mix.a2", "time_mix.g1", "time_mix.g2", "input.weight", "write_gate.weight",
    "read_gate.weight", "ffn_in.weight", "ffn_gate.weight", "ffn_out.weight",
)


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float32).to(torch.bfloat16).to(x.dtype)


def split16(x: torch.Tensor) -> torch.Tensor:
    """An activation as the bf16-weight kernels multiply it: hi = bf16(x),
    lo = bf16(x - hi), hi + lo (|x - (hi + lo)| <= 2^-16 |x|)."""
    hi = _bf16(x)
    return hi + _bf16(x - hi)


class OracleModel:
    def __init__(self, config: dict, weights: dict, dtype=torch.float64, bf16_linear: bool = False,
                 chunked_scan: bool = False, split_activations: bool = False):
        self.cfg = dict(config)
        self.dtype = dtype
        self.bf16_linear = bool(bf16_linear)
        # chunked_scan: the WKV-7 scan in its 16-token chunk form
        # (wkv7_scan_chunked, the same recurrence regrouped; pinned against the
        # sequential loop in tests/test_oracle_wkv7.py) -- for long sequences,
        # where the per-token loop dominates the oracle's time.
        self.chunked_scan = bool(chunked_scan)
        # split_activations: every projection multiplies split16(x) instead of
        # x -- the engine's bf16-weight products, which split each fp32
        # activation into two bf16 parts (a model of that engine, not of the
        # reference, whose fp32 program multiplies x itself).
        self.split_activations = bool(split_activations)
        self.d = int(self.cfg["d_model"])
        self.n_layers = int(self.cfg["n_layers"])
        self.heads = int(self.cfg["n_heads"])
        self.head_size = int(self.cfg["head_size"])
        self.rosa_size = int(self.cfg["rosa_size"])
        self.vocab = int(self.cfg["vocab_size"])
        self.w = {name: torch.as_tensor(np.asarray(value), dtype=dtype) for name, value in weights.items()}
        if "lm_head.weight" not in self.w:
            # Tied head (model.py:390-391; export_checkpoint.py:70-74).
            self.w["lm_head.weight"] = self.w["token_embedding.weight"]
        if self.bf16_linear:
            for name in list(self.w):
                if name == "lm_head.weight" or name.endswith(_LINEAR_SUFFIXES):
                    self.w[name] = _bf16(self.w[name])

    # ------------------------------------------------------------------ state
    def initial_state(self, batch: int) -> list:
        return [
            LayerState(
                torch.zeros(batch, self.d, dtype=self.dtype),
                torch.zeros(batch, self.heads, self.head_size, self.head_size, dtype=self.dtype),
                torch.zeros(batch, self.rosa_size, dtype=self.dtype),
            )
            for _ in range(self.n_layers)
        ]

    # ---------------------------------------------------------------- helpers
    def _p(self, layer: int, suffix: str) -> torch.Tensor:
        return self.w[f"blocks.{layer}.{suffix}"]

    def _ln(self, x, layer_prefix: str):
        return F.layer_norm(x, (self.d,), self.w[layer_prefix + ".weight"], self.w[layer_prefix + ".bias"], LN_EPS)

    def _mm(self, x: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
        """x @ m for a projection (m already in its product orientation)."""
        if self.split_activations:
            x = split16(x)
        return x @ m

    # ---------------------------------------------------------------- TimeMix
    def timemix_inputs(self, layer: int, x: torch.Tensor, previous: torch.Tensor):
        """model.py:97-131: returns (r, w_raw, k_adjusted, v, -kk, kk*a, g)."""
        p = lambda s: self._p(layer, "time_mix." + s)  # noqa: E731
        shifted = torch.cat((previous[:, None], x[:, :-1]), dim=1)
        delta = x - shifted
        xr = x + delta * p("mix_r")
        xw = x + delta * p("mix_w")
        xk = x + delta * p("mix_k")
        xv = x + delta * p("mix_v")
        xa = x + delta * p("mix_a")
        xg = x + delta * p("mix_g")
        mm = self._mm
        r = mm(xr, p("receptance.weight").T)
        w = p("w0") + mm(torch.tanh(mm(xw, p("w1"))), p("w2"))
        k = mm(xk, p("key.weight").T)
        v = mm(xv, p("value.weight").T)
        a = torch.sigmoid(p("a0") + mm(mm(xa, p("a1")), p("a2")))
        g = torch.sigmoid(mm(mm(xg, p("g1")), p("g2")))
        batch, steps, _ = k.shape
        shape = (batch, steps, self.heads, self.head_size)
        kk = F.normalize((k * p("k_k")).view(shape), dim=-1, p=2.0, eps=1e-12)
        a_heads = a.view(shape)
        k_adj = (k * (1.0 + (a - 1.0) * p("k_a"))).view(shape)
        return r.view(shape), w.view(shape), k_adj, v.view(shape), -kk, kk * a_heads, g

    def timemix(self, layer: int, x: torch.Tensor, state: LayerState):
        r, w, k, v, a, b, g = self.timemix_inputs(layer, x, state.previous)
        scan = wkv7_scan_chunked if self.chunked_scan and x.shape[1] > 1 else wkv7_scan
        y, memory = scan(r, w, k, v, a, b, state.memory)
        y = y.reshape(x.shape)
        p = lambda s: self._p(layer, "time_mix." + s)  # noqa: E731
        z = F.layer_norm(y, (self.d,), p("out_norm.weight"), p("out_norm.bias"), LN_EPS)
        out = self._mm(z * g, p("output.weight").T)
        return out, x[:, -1].clone(), memory

    # ------------------------------------------------------------------- ROSA
    def rosa(self, layer: int, x: torch.Tensor, memory: torch.Tensor):
        p = lambda s: self._p(layer, "rosa." + s)  # noqa: E731
        cand = self._mm(x, p("input.weight").T) + p("input.bias")
        write = self._mm(x, p("write_gate.weight").T) + p("write_gate.bias")
        read_gate = self._mm(x, p("read_gate.weight").T) + p("read_gate.bias")
        decay = torch.sigmoid(p("decay"))
        direction = F.normalize(p("householder"), dim=0)
        read, memory = rosa_scan(cand, write, read_gate, decay, direction, memory, gated=True)
        return self._mm(read, p("output.weight").T), memory

    # ------------------------------------------------------------------ block
    def block(self, layer: int, x: torch.Tensor, state: LayerState):
        pre = f"blocks.{layer}."
        tm_out, previous, memory = self.timemix(layer, self._ln(x, pre + "norm_time"), state)
        x = x + tm_out
        rosa_out, rosa_mem = self.rosa(layer, self._ln(x, pre + "norm_rosa"), state.rosa)
        x = x + rosa_out
        f = self._ln(x, pre + "norm_ffn")
        hidden = F.silu(self._mm(f, self._p(layer, "ffn_in.weight").T)) * self._mm(f, self._p(layer, "ffn_gate.weight").T)
        x = x + self._mm(hidden, self._p(layer, "ffn_out.weight").T)
        return x, LayerState(previous, memory, rosa_mem)

    # ------------------------------------------------------------------ model
    def forward(self, ids, state=None, logits: str = "all"):
        """model.py:406-422.  ``logits`` = "all" | "last" | "none"."""
        ids = torch.as_tensor(np.asarray(ids), dtype=torch.long)
        if ids.ndim != 2:
            raise ValueError("input_ids must have shape [batch, time]")
        if state is None:
            state = self.initial_state(ids.shape[0])
        hidden = self.w["token_embedding.weight"][ids]
        new_state = []
        for layer in range(self.n_layers):
            hidden, st = self.block(layer, hidden, state[layer])
            new_state.append(st)
        if logits == "none":
            return None, new_state
        if logits == "last":
            hidden = hidden[:, -1:]
        normed = F.layer_norm(hidden, (self.d,), self.w["final_norm.weight"], self.w["final_norm.bias"], LN_EPS)
        out = self._mm(normed, self.w["lm_head.weight"].T)
        return (out[:, -1] if logits == "last" else out), new_state

    def step(self, ids, state=None):
        """model.py:424-431: one token per stream, returns logits[:, -1]."""
        ids = torch.as_tensor(np.asarray(ids), dtype=torch.long)
        if ids.ndim == 1:
            ids = ids[:, None]
        out, state = self.forward(ids, state)
        return out[:, -1], state


def state_to_blob(state: list) -> np.ndarray:
    """Per-stream flat blob ``[prev d | wkv H*N*N (i,j) | rosa D]`` per layer, float32.

    The order is ``BlockState``'s (model.py:29-38); returns ``[B, n_layers * (d + H*N*N + D)]``.
    """
    parts = []
    for st in state:
        batch = st.previous.shape[0]
        parts += [st.previous.reshape(batch, -1), st.memory.reshape(batch, -1), st.rosa.reshape(batch, -1)]
    return torch.cat(parts, dim=1).to(torch.float32).numpy()


def blob_to_state(blob: np.ndarray, cfg: dict, dtype=torch.float64) -> list:
    d, h, n, dr = (int(cfg[k]) for k in ("d_model", "n_heads", "head_size", "rosa_size"))
    blob = torch.as_tensor(np.asarray(blob), dtype=dtype)
    batch = blob.shape[0]
    out, off = [], 0
    for _ in range(int(cfg["n_layers"])):
        prev = blob[:, off:off + d]
        off += d
        mem = blob[:, off:off + h * n * n].reshape(batch, h, n, n)
        off += h * n * n
        ro = blob[:, off:off + dr]
        off += dr
        out.append(LayerState(prev.clone(), mem.clone(), ro.clone()))
    return out
