"""Write golden vectors from the reference's own PyTorch code (run once, in the build container).

The reference (``/root/reference``, YufeiV/YufMusicGen) is imported read-only,
on the CPU, with ``use_cuda_kernel=False`` and ``use_rosa_scan=False`` (the
reference recurrences; ``model.py:175-193``, ``:303-337``).  Only the inputs
and outputs are stored here -- as ``.npz`` data and ``.yuf`` weights written
by this build's own writer; no reference source travels with the fixtures.

What the vectors pin that no closed form does:

* ``wkv7_ref.npz``   -- ``RWKV7TimeMix._torch_recurrence`` (model.py:145-165)
  from a non-zero initial state;
* ``rosa_ref.npz``   -- ``ROSAMemory._reference_recurrence`` (model.py:260-288)
  from a non-zero memory;
* ``model_state_test.{yuf,npz}`` -- the whole ``YufMusicGen.forward`` for the
  configuration of ``tests/test_model_state.py`` (token shift sign, mix
  order, LayerNorm placement, gate, tied head), full sequence and continued
  from a carried state, with the final per-layer states;
* ``model_tiny.npz`` -- C1's tiny model (weights regenerated from the seed by
  ``yufmusicgen_amd.synth``; a checksum guards the generator), prompt logits
  and the 256-step greedy continuation of C1.

Usage (from the repository root, never on the GPU box):
    python tests/golden/make_golden.py [wkv rosa state_test tiny]   (default: all)
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, "/root/reference")

from yufmusicgen.config import ModelConfig as RefConfig  # noqa: E402  (reference, read-only)
from yufmusicgen.model import ROSAMemory, RWKV7TimeMix, YufMusicGen  # noqa: E402

from yufmusicgen_amd.checkpoint import write_yuf  # noqa: E402
from yufmusicgen_amd.config import PRESETS  # noqa: E402
from yufmusicgen_amd.synth import synth_weights  # noqa: E402


def ref_model(preset: str, weights: dict) -> YufMusicGen:
    cfg = PRESETS[preset]
    ref_cfg = RefConfig(
        vocab_size=cfg.vocab_size, d_model=cfg.d_model, n_layers=cfg.n_layers, n_heads=cfg.n_heads,
        head_size=cfg.head_size, rosa_size=cfg.rosa_size, use_cuda_kernel=False, use_rosa_scan=False,
    )
    model = YufMusicGen(ref_cfg).eval()
    state = {name: torch.from_numpy(np.array(value)) for name, value in weights.items()}
    state["lm_head.weight"] = state["token_embedding.weight"]
    model.load_state_dict(state, strict=True)
    return model


def flatten_state(state) -> dict:
    out = {}
    for layer, block in enumerate(state):
        out[f"state.{layer}.previous"] = block.timemix.previous.numpy()
        out[f"state.{layer}.memory"] = block.timemix.memory.numpy()
        out[f"state.{layer}.rosa"] = block.rosa.numpy()
    return out


def wkv_golden() -> None:
    g = torch.Generator().manual_seed(11)
    batch, steps, heads, size = 2, 7, 2, 8
    shape = (batch, steps, heads, size)
    r, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    w_raw = torch.randn(shape, generator=g) * 2.0
    kappa = torch.nn.functional.normalize(torch.randn(shape, generator=g), dim=-1)
    a = -kappa
    b = kappa * torch.sigmoid(torch.randn(shape, generator=g))
    s0 = torch.randn(batch, heads, size, size, generator=g) * 0.5
    y, s = RWKV7TimeMix._torch_recurrence(r, w_raw, k, v, a, b, s0.clone())
    np.savez(HERE / "wkv7_ref.npz", r=r.numpy(), w_raw=w_raw.numpy(), k=k.numpy(), v=v.numpy(),
             a=a.numpy(), b=b.numpy(), s0=s0.numpy(), y=y.numpy(), s=s.numpy())


def rosa_golden() -> None:
    g = torch.Generator().manual_seed(12)
    batch, steps, dim = 2, 7, 12
    cand, write, read_raw = (torch.randn(batch, steps, dim, generator=g) for _ in range(3))
    decay = torch.sigmoid(torch.randn(dim, generator=g) + 2.0)
    direction = torch.nn.functional.normalize(torch.randn(dim, generator=g), dim=0)
    m0 = torch.randn(batch, dim, generator=g)
    read, m = ROSAMemory._reference_recurrence(cand, write, read_raw, decay, direction, m0.clone())
    np.savez(HERE / "rosa_ref.npz", cand=cand.numpy(), write=write.numpy(), read_raw=read_raw.numpy(),
             decay=decay.numpy(), direction=direction.numpy(), m0=m0.numpy(), read=read.numpy(), m=m.numpy())


def model_state_test_golden() -> None:
    cfg = PRESETS["state_test"]
    weights = synth_weights(cfg, seed=7, std=0.2)
    write_yuf(HERE / "model_state_test.yuf", cfg, weights, source={"checkpoint": "golden", "step": 7, "phase": ""})
    model = ref_model("state_test", weights)
    tokens = torch.from_numpy(np.random.default_rng(7).integers(0, cfg.vocab_size, size=(2, 9)))
    with torch.no_grad():
        full_logits, full_state = model(tokens)
        head_logits, head_state = model(tokens[:, :5])
        tail_logits, tail_state = model(tokens[:, 5:], head_state)
    out = {"tokens": tokens.numpy().astype(np.int32), "logits": full_logits.numpy(),
           "head_logits": head_logits.numpy(), "tail_logits": tail_logits.numpy()}
    out.update({f"full.{k}": v for k, v in flatten_state(full_state).items()})
    out.update({f"tail.{k}": v for k, v in flatten_state(tail_state).items()})
    np.savez(HERE / "model_state_test.npz", **out)


def model_tiny_golden() -> None:
    cfg = PRESETS["tiny"]
    weights = synth_weights(cfg, seed=1, std=0.02)
    checksum = np.array([float(np.sum(v.astype(np.float64))) for v in weights.values()])
    model = ref_model("tiny", weights)
    prompt = torch.from_numpy(np.random.default_rng(1).integers(0, cfg.vocab_size, size=(1, 32)))
    with torch.no_grad():
        logits, state = model(prompt)
        last = logits[:, -1]
        greedy, greedy_logits = [], []
        for _ in range(256):
            token = torch.argmax(last, dim=-1)
            greedy.append(int(token))
            last, state = model.step(token, state)
            greedy_logits.append(last.numpy()[0])
    np.savez(HERE / "model_tiny.npz", prompt=prompt.numpy().astype(np.int32), prompt_logits=logits.numpy(),
             greedy=np.array(greedy, np.int32), greedy_logits=np.stack(greedy_logits), weight_checksum=checksum,
             seed=np.array(1), std=np.array(0.02))


if __name__ == "__main__":
    torch.manual_seed(0)
    makers = {"wkv": wkv_golden, "rosa": rosa_golden, "state_test": model_state_test_golden,
              "tiny": model_tiny_golden}
    for name in sys.argv[1:] or list(makers):
        makers[name]()
    for path in sorted(HERE.glob("*.np[zy]")) + sorted(HERE.glob("*.yuf")):
        print(f"{path.name}: {path.stat().st_size} bytes")
