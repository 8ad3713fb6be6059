"""CPU oracle for the paged KV-cache decode path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, what the reference engine computes on the KV
path it drives through ``llm.generate`` (wavelet/inference/engine.py:887,
:1045, :1274). It is the checker the HIP kernels are compared against and the
CPU baseline that bench.py times beside them. Only ``tests/``,
``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg may import it; the
product (``wavelet_amd``) never does, and has no CPU fallback.

Modules
-------
``oracle.fp8``    e4m3fn encode/decode and the power-of-two absmax scale
                  (wavelet/trainer/models/deepseek_v4/attention.py:41-50).
``oracle.paged``  slot-mapped append (bf16 / fp8 with per-(block, head)
                  scales), block-table gather, GQA and MLA paged decode
                  attention (attention.py:81-96; wavelet/kernels/patch.py:173-196).

How each function is pinned (tests/test_oracle.py)
-------------------------------------------------
* ``fp8.e4m3_encode`` / ``e4m3_decode``: all 65,536 bf16 bit patterns and 2^20
  random fp32 bit patterns against torch's ``float8_e4m3fn`` cast (a library
  routine); decode against the 256-entry torch table.
* ``fp8.pow2_scale``: every positive finite bf16 amax against torch's
  ``exp2(ceil(log2(max(a,1e-10)/448)))`` (the reference expression, evaluated
  by torch's libm), plus the invariant ``a/448 <= s < 2*a/448``.
* ``paged.append_bf16`` / ``gather``: round trip (gather(append(x)) == x,
  bit-exact) on seeded workloads, untouched slots unchanged, ``slot=-1``
  skipped, brute-force per-element loop on tiny inputs.
* ``paged.append_fp8``: a scalar pure-Python re-implementation (math.frexp,
  per-element loop) on small runs including scale growth and subnormal
  re-encoding; invariants (dequantised |x - x_hat| <= half an e4m3 ulp of
  x/s times s before any growth; scales are powers of two and monotone).
* ``paged.decode_gqa`` / ``decode_mla``: torch
  ``scaled_dot_product_attention`` in float64 on the gathered K/V (library
  routine); known answers: L=1 gives v0, identical keys give mean(V), and the
  ignore-slot case of tests/test_deepseek_attention.py:100-118
  (output ``sigmoid(0.625)*[2,-1]`` with NaN in never-read slots); MLA against
  an explicit non-absorbed expansion with random W_UK / W_UV on tiny sizes.
"""
