"""CPU oracle for the YufMusicGen recurrent hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU (float64 by default, float32
for the timed CPU baseline), the reference algorithm of YufeiV/YufMusicGen for
the recurrent language-model forward pass:

* ``wkv7``    -- the WKV-7 TimeMix scan        (reference ``yufmusicgen/model.py:145-165``)
* ``rosa``    -- the ROSA Householder scan     (reference ``yufmusicgen/model.py:260-288``)
* ``model``   -- the full model forward / step (reference ``yufmusicgen/model.py:97-445``)
* ``sampler`` -- temperature / top-p sampling  (reference ``yufmusicgen/cli/generate.py:45-56``)

It is the checker, never the product: only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it.  Nothing in
``yufmusicgen_amd`` imports or calls it, and the product path fails loudly
when its HIP library is missing instead of falling back to this code.

How each function is pinned (beyond retyping the reference):

* ``wkv7.wkv7_scan``: the O(T^2) closed form for a = b = 0, the exact T = 1
  and T = 2 cases written as outer products, the delta-rule write property
  (with unit decay, a = -kappa, b = k = kappa the updated state maps kappa to
  v exactly), linearity in v, padding invariance of the reference's T-padding
  (``cuda_ops.py:160-186``), the chunked (16-token) form, and golden vectors
  written by the reference's own ``_torch_recurrence`` (``tests/golden``).
* ``rosa.rosa_scan``: H(H(x)) = x, norm preservation, a dense float64
  matrix-power unrolling of the linear time-invariant recurrence, and golden
  vectors from the reference's ``_reference_recurrence``.
* ``model.OracleModel``: the reference's own invariant (full-sequence forward
  equals the step loop, ``tests/test_model_state.py:9-28``) and golden logits
  and states from the reference model (``tests/golden``).
* ``sampler``: torch's own ``torch.multinomial`` under ``torch.manual_seed``.
"""

from . import wkv7, rosa, model, sampler  # noqa: F401
