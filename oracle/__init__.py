"""CPU oracle for the int8 KV-cache decode path — TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithms in numpy so that tests,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` can
check (and time) the HIP path against them. Nothing in ``nova_amd`` imports it:
the product path runs the hand-written HIP kernels or raises.

Modules and what each one pins (every function cites the reference line it
restates):

- ``oracle.kvquant``  int8 token-axis / channel-axis asymmetric quantize and
  dequantize (``src/nova/kvquant.py:118-176``), the per-token symmetric
  extension (``scheme="tok"``), and the int8 byte accounting
  (``src/nova/kvquant.py:232-289``). Pinned by the golden vectors written from
  the reference itself (``tests/golden/make_golden.py``) and by closed-form
  invariants (constant tensors, code range, half-step error bound).
- ``oracle.attn``     dequantize-then-softmax attention for one decode step
  (``tests/test_kvattn.py:62-70``), the fp16 tail attention with its
  log-sum-exp (``src/nova/kvattn.py:447-482``) and the log-sum-exp merge
  (``src/nova/kvattn.py:852-862``). Pinned against torch's math SDPA, an
  fp64 brute force, and special cases (one token, constant V, empty mask).
- ``oracle.stream``   the streaming-cache state machine: ring write, whole-ring
  requantize, device scalars, ring mask, bulk prefill quantize
  (``src/nova/kvattn.py:668-862``). Pinned by reference-generated state
  vectors and by invariants (ring-mask count, finish_prefill == quantizer).
- ``oracle.decode``   capacity buckets and the additive mask row
  (``src/nova/decode.py:39-48,200-205``). Pinned by the reference's own table
  (``tests/test_decode_mask_bucket.py:29-37``).

The per-token symmetric scheme ("tok") has no counterpart in the reference;
its oracle follows kvquant's rounding conventions (fp32 arithmetic,
round-half-even, 1e-8 floor, fp16-stored scale) and is pinned by closed-form
checks only.
"""
