"""Benchmark harness of the HIP grouped-GEMM path: cases, providers, measurement, CSV, validation.

* ``harness.cases``     - what to measure: MoE EP/TP per-rank cases, single-GEMM shape sweeps and
                          the (G, M, N, K) heatmap, as immutable ``Case`` records;
* ``harness.providers`` - how to run one case: the HIP grouped / single / expert-sorted launches
                          and the torch baselines, behind one ``Provider`` interface;
* ``harness.measure``   - the staged pipeline per (case, providers): admission, rotating-ring
                          allocation, tuning, correctness gate, graph timing;
* ``harness.rows``      - the CSV row of a measurement (the result wire format of utils.io);
* ``harness.cli``       - ``python -m harness``: the experiment driver and its flags;
* ``harness.validate``  - ``python -m harness.validate``: the result contract checker;
* ``harness.compare``   - ``python -m harness.compare``: HIP grouped GEMM against library
                          baselines on identical operands.
"""
