"""CPU oracle for the HIP realizer -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

This package restates, in NumPy, the reference's CPU realizer for the hot
path: ``_realize.realize`` (packages/browsergrad-jit/src/python/_realize.py:
1854-1923) with its AMP cast pass (``_amp.insert_cast_pass``, _amp.py:
183-261) and the op handlers the five BASELINE configs touch.  Each function
cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import anything from here, and only as the checker (or as the timed
CPU comparator in bench.py).  The product path (``browsergrad_amd``) never
imports it and fails loudly when the HIP library is missing.

How each part is pinned (see tests/test_oracle_golden.py):
  * GEMM: reference known answers [58,64,139,154], 70, [19,22,43,50],
    identity / 2*I, float64 brute force on tiny shapes, and the AMP
    invariant ones(1x4096) @ ones(4096x1) in f16 -> exactly 4096.0.
  * fused elementwise: closed forms exp(a+b)/a and log(exp(x)*y), and the
    ops-list encoding of the reference tests.
  * softmax / attention: uniform rows, rows sum to 1, the reference's
    softmax rows, the CS336 attention fixtures (non-causal, causal, hard
    causal boundary) and a float64 brute-force attention.
  * LayerNorm / GELU: closed forms and the reference's GELU known values.
  * casts: f32->f16 against NumPy astype (the reference's own arithmetic),
    f32->bf16 by exhaustive comparison of every bf16 bit pattern's round
    trip and of RNE ties against an integer restatement.
  * AMP graph: CAST placement and output dtypes of MATMUL / ADD / softmax
    ops against the policy table of _amp.py:56-69.
"""
