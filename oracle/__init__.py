"""CPU oracle for the sparse-prefill hot path — TEST INFRASTRUCTURE ONLY.

This package is a numpy (fp32) restatement of the reference's v2 selection
path and of its block-sparse attention semantics.  It is the checker that the
HIP kernels are compared against, nothing more:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
  ``bench.py`` may import it;
* the product path (the package beside this directory) never imports it and
  fails loudly when its HIP library is missing — there is no CPU fallback.

Modules
-------
``selector``   K-block summaries, per-row block scores, tile max-pool,
               visibility + sink/self forcing, top-k, sigma margin, router
               (row/cell grain, quantile/abs) and sentinel emission —
               ``src/sparse_attention.py:588-748`` of the reference.
``selector_v1`` the v1 per-row selector ``_block_select_mask`` (keep mask;
               topk / quest / router / belief / rollout) —
               ``src/sparse_attention.py:208-382``.
``score_dump`` order statistics and score-noise estimate of the reference's
               score-dump diagnostic (``src/dump_block_scores.py:104-207``).
``attention``  block-sparse attention over ``kv_idx`` (kernel semantics of
               ``src/triton_block_attn.py:184-264``), the masked dense
               formulation of ``reference_attn`` (``:301-312``) and
               ``_compute_kv_idx`` (``:125-146``).

How each function is pinned (beyond restating the reference) is listed in the
module docstrings; the tests under ``tests/test_oracle_*.py`` hold the checks.
"""

from . import selector, selector_v1, attention, score_dump  # noqa: F401
