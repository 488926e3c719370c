"""CPU oracle for the prefill->decode KV handoff and decode attention.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import anything under ``oracle/``, and
only as the oracle results are compared with (or, for the baseline, as the
timed CPU restatement of the reference). The product package ``rngd_pd_amd``
never imports it.

Modules:
  native     ctypes wrapper over liboracle.so (pdk_oracle.c): pack, scatter,
             gather, cache append, decode attention (double accumulation),
             greedy argmax, bf16 truncate/widen.
  wire       numpy/pickle restatement of the reference's bf16 wire codec
             (ser/deser) and /dev/shm file protocol, plus the reference's KV
             generator and the whole CPU shm handoff used as the baseline.
  attention  numpy restatement of cpu_layer's attention on the reference's
             dense layout, and dense<->paged layout conversion by indexing.

Pinning: every function here is checked in tests/test_oracle.py against an
independent formulation (numpy transposes and fancy indexing, torch float64
attention, closed forms) and against the reference's own test vectors
(tests/test_airm.py seeds and shapes). See each function's docstring for the
reference lines it follows.
"""
