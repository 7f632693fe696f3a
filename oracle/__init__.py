"""CPU oracle for the Bifrost converted-layer core — TEST INFRASTRUCTURE ONLY.

This package restates, in plain fp32/fp64 PyTorch on the CPU, the algorithms of the reference's hot path
(ValeroisAI/Heimdall):

  * ``gdn``    — chunked gated delta rule (UT/WY form), its GQA form, the single-token step and a brute-force
                 token recurrence (``Heimdall/heimdall/kernels.py:81-138``, ``Heimdall/heimdall/motor.py:70-102``).
  * ``window`` — sliding-window + sink attention with per-row log-sum-exp (``Heimdall/heimdall/hibrit.py:341-361``).
  * ``layer``  — the converted layer's student path: memory inputs, write-on-exit, gamma mix, ring/sink/state cache
                 (``Heimdall/heimdall/hibrit.py:193-240,327-424``), plus a per-token brute-force restatement.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it, and only as the
checker (or the timed CPU baseline). The product package ``heimdall_amd`` never imports it and has no CPU path.

Every function is pinned by a check in ``tests/test_oracle_*.py`` that does not restate its formula: brute-force
recurrence in fp64, chunk-size and padding invariance, closed forms (pure decay, exact overwrite), an independent
third-party restatement (``transformers`` Qwen3.5 torch fallback), textbook masked softmax, cache/full invariance,
and golden vectors written by the reference itself (``tests/golden/``).
"""
