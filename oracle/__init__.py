"""CPU oracle for the W4A8 per-group linear -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's CPU W4A8 path
(GongCheng1919/vllm-ascend910: fakequant_lab/quant.py, fakequant_lab/fake_linear.py,
fakequant_lab/run_selftest.py, npu_ops/python/w4a8_ops.py, npu_ops/kernel/mg_kgeom.h),
each function citing the reference lines it follows.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker: the product (the package ``vllm-ascend910_amd``)
never imports, links or calls anything here.

How each function is pinned (tests/test_oracle.py):
  * bf16 rounding        -- torch's .to(bfloat16) and the reference's own
                            FP32ToBF16 (oracle/_ref, int4_cube_lab/host/bf16.h:17-27)
  * per-token quantiser  -- exact rational arithmetic (fractions.Fraction) on
                            random and constructed inputs: half-way ties,
                            all-zero rows, +-128 clamping
  * int4 pack / geometry -- the reference's own C++ packers and geometry
                            (oracle/_ref: gemm_ref.cpp PackInt4Grouped,
                            mg_kgeom.h) and exhaustive nibble round trips
  * group partials       -- brute-force int64 dot products
  * fp32 GEMM / bf16 out -- the reference's ReferenceMidGroupGemm and
                            ReferencePerchannelGemm (oracle/_ref) and a float64
                            restatement of run_selftest.py's _exact_reference;
                            tests/golden/reference_vectors.npz holds outputs of
                            the reference's C++ (packing, plane split, ksums,
                            geometry, the three GEMM orders) written by
                            tests/golden/make_golden.py, checked on CPU and GPU
  * torch addcmul_ FMA   -- fma32 (one rounding of acc + partial*s) equals
    contraction             torch CPU's addcmul_ on every element of random and
                            broadcast cases, and exact rational rounding
                            (tests/test_oracle.py)
"""
