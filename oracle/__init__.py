"""CPU oracle for scratch_llm's quantized-linear path — TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithms (andreidhoang/scratch_llm,
``src/scratch_llm/quant/{int4_group,int8,awq,nvfp4_mxfp4}.py`` and
``src/scratch_llm/k3/checkpoint.py:92-144``) on the CPU so the HIP kernels can be checked against
it. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker or the timed CPU baseline; the product package
``scratch_llm_amd`` never imports it and has no CPU path.

Modules:
  quant_ref   numpy restatement, fp32 arithmetic identical to the reference's (IEEE division,
              round-half-to-even), plus float64 linears for tolerance checks.
  torch_path  the reference's own CPU linear path (torch dequantize, then ``F.linear``), restated
              with torch on the CPU; timed as the CPU baseline.
  nvfp4_ceil_ref  numpy restatement of the second NVFP4 convention (the b_r6 GEMM rung's operands:
              ceil-rounded UE4M3 block scales, E2M1 ties to even), float64 as the reference.
  decode_ref, fp8_ref  the decode step and the FP8 quantizers (see their docstrings).

Pinning status of every function is listed in quant_ref's module docstring.
"""
