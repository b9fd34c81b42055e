"""CPU oracle for the Gemma 4 rollout prefill + KV-cache decode path.

TEST INFRASTRUCTURE ONLY. Nothing under ``oracle/`` is part of the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it, and only as the
checker (or, for the CPU baseline, as the thing timed on the host), never as a code path of the
GPU library.
"""
