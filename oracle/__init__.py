"""CPU oracle for the FlashAttention-2 forward path.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as a
checker or as the timed CPU baseline, never as the product path.

Two restatements of the reference (Dell710000/ascend-rsfa,
ascend_rsfa/flash_attention_forward.py):

* ``attention.reference_attention`` - the closed form the reference is judged
  against, ``softmax(q k^T * sm_scale + causal mask) v`` in fp32 (the golden
  ``npu_fusion_attention`` semantics of benchmarks/run_correctness_test.py:68-92,
  BNSD layout, causal keeps key n <= query m).
* ``attention.blockwise_attention`` - the reference's own tiled algorithm with
  its rounding points, in plain C (``fa2_blockwise.c``).

How each is pinned (no reference tensors exist to compare with: the reference
ships none, and its golden op needs an Ascend NPU) is listed in the docstring
of ``attention.py`` and tested in tests/test_oracle.py.
"""
