"""CPU oracle for the ExQ INT4 MoE expert-dispatch path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``exq_amd``) imports this
package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
(or, for ``cpu_baseline``, as the timed CPU restatement of the reference's
PyTorch CPU path) -- never as the thing measured for the GPU or shipped.

Every function restates the reference algorithm in numpy (float32 IEEE
arithmetic, round-half-to-even, stable sorts) and cites the reference file and
line range it follows.  The reference lives in alityb/exq:

* ``quant``     -- INT4 RTN packing, INT8 per-channel quantisation, fake-quant
                   (exq/kernels/moe_int4_kernel.py, exq/eval/quant_shim.py,
                   scripts/bench_int4.py).
* ``routing``   -- canonical token->expert sort, expert boundaries, block
                   padding, slot compaction (exq/kernels/moe_grouped_gemm.py,
                   exq/kernels/cuda_src/exq_dispatch.cu, the sgl_kernel call
                   site in exq/runtime/sglang_backend.py).
* ``moe``       -- gather, SiLU-and-mul, grouped GEMM, weighted combine and the
                   full fp32 dequantise-then-matmul MoE layer
                   (exq/kernels/moe_grouped_gemm.py:267-290 and the pipeline
                   order of exq/runtime/sglang_backend.py:65-158).
* ``artifact``  -- quant-plan reader rules (exq/kernels/exq_artifact.py).
* ``cpu_baseline`` -- the reference's PyTorch CPU path, restated in torch for
                   the timed CPU baseline.

Pinning status of each function is recorded in its docstring ("pinned by: ...")
and checked in ``tests/test_oracle_*.py``.
"""
