"""CPU oracle for the decode-time state path (TEST INFRASTRUCTURE ONLY).

This package restates, in plain PyTorch on the CPU, the arithmetic of the reference engine's decode state
path (sott0n/tt-qwen-resident) so the HIP kernels can be checked against it on identical seeded inputs.
Only the tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it, and
only as the checker: the product path (the HIP library behind ``qwen36_state``) never calls into it.

Every function cites the reference file:line it restates. The reference itself cannot be imported (its
modules import ``ttnn`` at load time and the tt-metal submodule is empty), so nothing here runs it.

Pinning (what independently fixes each function; the tests under ``tests/test_oracle_*.py`` hold them):

  conv1d_update      brute-force per-channel loop, impulse response, shift invariant, carry exactness
  l2norm             unit norm up to eps, scale invariance
  gdn_gates          scalar ``math`` restatement of softplus (threshold 20) and sigmoid
  gdn_step           fp64 brute-force loops on d=4, decay=1/beta=0 identity, S=0 rank-1 write,
                     decay=1/beta=1 "write v at key k", column separability
  gdn_verify         T=1 equals gdn_step exactly; snapshots equal sequential steps exactly
  rollback           equals the snapshot bit-exactly
  paged_append/fill  pure-Python index loops; bit-exact
  gqa_decode         fp64 softmax; one position gives the V row; split-K merge equals one pass;
                     softmax shift invariance; causal mask against per-token truncation
  gdn_chunk_prefill  the sequential recurrence (gdn_step applied T times); the chunked WY/UT form is a
                     second, independent restatement checked against it in fp64
  weight_stream      (module ``oracle.weight_stream``) golden OCP MX encodings and block quantizations,
                     the nearest-representable property, a hand-indexed layout case, the MLP half's closed
                     forms (D = 0 identity, linearity in D, rmsnorm scale invariance) and scalar loops

Functions whose exact rounding only the reference's third-party ops could pin (tt-metal's
``chunk_gated_delta_rule`` tile staging) are matched within tolerance, not bit-for-bit: parity for that
rounding is unpinned by design (the arithmetic lives in the absent tt-metal submodule).
"""
from .state_path import *  # noqa: F401,F403
