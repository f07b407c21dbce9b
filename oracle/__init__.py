"""CPU oracle of the paged-KV attention path. TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's own definitions of what the path computes. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it, and only as the checker (or as
the timed CPU baseline): the product package never imports it and has no CPU fallback.

- ``oracle.attention``: softmax attention (the reference test suite's ``_attend``), the block-table page gather,
  the KV slot scatter, and decode / varlen / dense attention built from them.
- ``oracle.context``: the per-token loops that define the prefill and decode context tensors.

Every function cites the reference file:line it follows; ``tests/test_oracle.py`` pins each against closed forms,
brute force on tiny inputs, an independent library routine (torch SDPA in float64) and the reference tests'
known-answer cases.
"""
