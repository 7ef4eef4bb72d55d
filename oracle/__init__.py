"""TEST INFRASTRUCTURE -- the CPU oracle for the WarpIR MI355X backend.

Nothing in ``warpir_amd`` imports, links or runs anything here.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker / the reported CPU baseline.

* ``torch_ref``       -- the reference's numerical oracles: ``torch.mm`` on
  fp32-upcast bf16 (``tests/test_modal_gpu.py:115``) and naive fp32
  ``softmax(q k^T * scale) v`` (``tests/test_modal_attention.py:92-98``),
  plus the log-sum-exp closed form and the seeded input recipe.
* ``ir_interp``       -- a block-granular CPU interpreter of the tile IR
  with the reference lowering's storage semantics (iter_arg aliasing,
  in-place MMA accumulation, drain counter; ``warpir/lowering/lowering.py``).
* ``sched_bruteforce`` -- exhaustive enumeration of the modulo-scheduling
  model (``warpir/passes/modulo_scheduler.py:51-101``) in C, and of the
  warp-assignment model (``warpir/passes/warp_assigner.py:31-119``) in
  Python for small instances.

Pinning (what checks each function beyond a restatement):
* ``torch_ref.gemm_ref`` / ``attention_ref`` -- closed forms: identity B
  returns A; one-hot V columns return P; constant K gives uniform
  softmax (mean of V); LSE of constant scores is ``log(n) + s``.
* ``ir_interp`` -- config 1 (GEMM 1024^3 through passes) equals
  ``torch.matmul``; attention IR equals naive attention; SSA and
  pipelined forms agree bit for bit.
* ``sched_bruteforce`` -- the reference GEMM model's unique optimum
  (ii=6, makespan 40, stage_of {0, 0, 2}) derived by hand in the
  survey, and the printer golden text generated from the reference.
"""
