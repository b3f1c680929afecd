"""CPU oracle for the MaskAhead KV read/keep path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference (brain-lab-research/MaskAhead,
``src/maskahead``) computes on the hot path, so the HIP kernels of ``maskahead_amd``
can be checked against it on identical seeded inputs.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
it, and only as the checker or as the timed CPU baseline.  The product package never
imports anything from here; a missing HIP library is an error there, never a silent
fallback to this code.

Modules
  codec.c / codec.py   int4 nibble pack/unpack, f16/bf16 conversion, KIVI dequant,
                       top-k with index-ascending tie-break, keep-set selection,
                       compaction -- plain C, loaded through ctypes (bit-exact work).
  attention.py         torch restatement of the floating-point semantics: quantizer
                       rule, split-K attention with prefix statistics, prefix mass /
                       value score, value_score in bf16, selector importance.
  selection.py         numpy/torch wrappers over the C selection routines and the
                       boundary-tolerance helpers the parity tests use.

Each function names the reference file:line it follows.  How every function is
pinned (golden vectors written from the reference in this container, closed forms,
brute force, invariants) is listed in tests/test_oracle_*.py; a function without
such a check says "parity unpinned" in its docstring.
"""
