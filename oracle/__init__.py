"""CPU oracle for the GPT forward hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with PyTorch tensors, the arithmetic of the
reference's GPT-2 forward (falcons-eyes/cutileGPT, ``cutile_gpt/models/gpt.py``
and ``cutile_gpt/kernels/*.py``).  It is the checker that the HIP kernels of
``cutilegpt_amd`` are compared with.  Only ``tests/``, ``__graft_entry__.smoke``
and the ``cpu_baseline`` leg of ``bench.py`` may import it; the product path
(``cutilegpt_amd``) never does and has no CPU fallback.

How each function is pinned (checked against something other than itself):

* ``gelu_tanh``        closed form at fixed points, odd/even identity
                       gelu(x) - gelu(-x) = x, limits, and
                       ``torch.nn.functional.gelu(approximate='tanh')``.
* ``layer_norm``       ``torch.nn.functional.layer_norm`` in float64, constant
                       rows, shift/scale invariance.
* ``linear``           brute-force triple loop on tiny shapes, one-hot weights.
* ``causal_attention`` brute-force per-query loop, row 0 == V[0], equal keys
                       give the prefix mean of V, score-shift invariance,
                       ``torch.nn.functional.scaled_dot_product_attention``.
* ``online_attention`` equal to ``causal_attention`` in float64 (the online
                       form is exact algebra), with or without lazy rescaling;
                       with P rounded to bf16 it equals the two-pass rounding
                       where the first key block holds every row's maximum.
* ``embedding``        exact gather vs indexing.
* ``gpt_forward``      ``transformers.GPT2LMHeadModel`` (an installed library
                       implementation of the same architecture) with identical
                       weights, and the committed golden fixtures.
* ``generate``         ``transformers`` greedy ``generate(do_sample=False)``.
* ``forward_cached`` / ``generate_cached``  equal to ``gpt_forward`` / the
                       full-recompute ``generate`` on small models (tokens and
                       per-step logits).

Nothing here is "parity unpinned" except the reference's own approximate GPU
numerics (TF32 MMA, ``exp2(flush_to_zero)``, approximate division), which no
fixture or test of the reference records; the oracle computes true fp32/fp64.
"""

from .gpt_ref import (  # noqa: F401
    Flow,
    FLOWS,
    gelu_tanh,
    layer_norm,
    linear,
    causal_attention,
    online_attention,
    embedding,
    gpt_forward,
    forward_cached,
    generate,
    generate_cached,
    init_weights,
    round_to,
)
