"""Write the printer golden fixtures from the reference's own printer.

Run in the build container only (``/root/reference`` does not exist on
the GPU box); the outputs are committed as small text fixtures:

    python tests/golden/make_printer_golden.py

What is pinned, and why this needs the reference itself: the text form of
the IR (``warpir/printing/printer.py:38-191``) is a set of format strings
whose byte-exact output no closed form or invariant fixes.  The script
imports the reference's pure-Python ``warpir.ir`` / ``warpir.printing``
and its two IR builders (``tests/gemm_baseline_v2.py:31-88``,
``tests/attention_baseline.py:46-186``) and prints:

* ``gemm_ssa.txt``       -- the GEMM builder's SSA kernel
* ``attention_ssa.txt``  -- the attention builder's SSA kernel
* ``gemm_pipelined.txt`` -- the buffer-form kernel that the reference's
  ``kernel_pass`` builds for the GEMM (``modulo_scheduler.py:239-358``)
  for its optimal schedule ii=6, stage_of={loads: 0, mma: 2}.  The
  reference pass itself needs OR-Tools (absent here), so this script
  assembles the same op sequence from the reference's IR classes,
  following ``modulo_scheduler.py:244-356`` step by step, and prints it
  with the reference printer.

The reference is imported in a fresh interpreter whose ``sys.path``
starts with ``/root/reference`` so that this repository's ``warpir``
alias package cannot shadow it.
"""
from __future__ import annotations

import os
import subprocess
import sys

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))

_CHILD = r'''
import sys
sys.path.insert(0, REF)
sys.path.insert(0, REF + "/tests")
from warpir.printing import format_kernel
from warpir.ir import (AllocSharedOp, BufSlotExpr, ForOp, Kernel, MMABufOp, SharedBufferType,
                       TMALoadBufOp, TMALoadOp, TMAStoreOp, MMAOp, Value, WaitBufOp, YieldOp, ZeroOp)
from gemm_baseline_v2 import build_gemm_kernel
from attention_baseline import build_attention_kernel

gemm = build_gemm_kernel()
att = build_attention_kernel()
open(OUT + "/gemm_ssa.txt", "w").write(format_kernel(gemm) + "\n")
open(OUT + "/attention_ssa.txt", "w").write(format_kernel(att) + "\n")

# Buffer form of the GEMM for ii=6, stage_of = {load_a: 0, load_b: 0, mma: 2}, 3 stages,
# assembled the way modulo_scheduler.py:244-356 does.
zero, loop, store = gemm.body
loads = [o for o in loop.body if isinstance(o, TMALoadOp)]
mma = next(o for o in loop.body if isinstance(o, MMAOp))
yld = next(o for o in loop.body if isinstance(o, YieldOp))
stages, mma_stage = 3, 2
bufs = {ld.result: Value(ld.source.name.lower() + "_bufs", SharedBufferType(ld.result.type, stages))
        for ld in loads}
body = [zero] + [AllocSharedOp(result=bufs[ld.result]) for ld in loads]
for step in range(stages - 1):
    for ld in loads:
        sub = ld.substitute({loop.induction_var: step})
        body.append(TMALoadBufOp(buf=bufs[ld.result], slot=step, source=ld.source, coords=sub.coords))
cslot = BufSlotExpr(value=loop.induction_var, offset=-mma_stage, modulus=stages)
lslot = BufSlotExpr(value=loop.induction_var, offset=0, modulus=stages)
inner = [WaitBufOp(bufs=tuple(bufs[ld.result] for ld in loads), slot=cslot)]
for ld in loads:
    inner.append(TMALoadBufOp(buf=bufs[ld.result], slot=lslot, source=ld.source, coords=ld.coords))
inner.append(MMABufOp(result=mma.result, a_buf=bufs[mma.a], a_slot=cslot, b_buf=bufs[mma.b],
                      b_slot=cslot, accum=mma.accum))
inner.append(yld)
body.append(ForOp(induction_var=loop.induction_var, start=stages - 1, stop=loop.stop, step=loop.step,
                  tile_size=loop.tile_size, iter_args=loop.iter_args, body=tuple(inner),
                  results=loop.results))
for ep in range(stages - 1):
    dslot = BufSlotExpr(value=None, offset=ep, modulus=stages)
    body.append(WaitBufOp(bufs=tuple(bufs[ld.result] for ld in loads), slot=dslot))
    body.append(MMABufOp(result=Value(mma.result.name + "_ep" + str(ep), mma.result.type),
                         a_buf=bufs[mma.a], a_slot=dslot, b_buf=bufs[mma.b], b_slot=dslot,
                         accum=loop.results[0]))
# modulo_scheduler.py:174-178 copies non-loop ops in program order, so the store follows
# the drain steps.
body.append(store)
piped = Kernel(name=gemm.name, inputs=gemm.inputs, outputs=gemm.outputs, body=tuple(body))
open(OUT + "/gemm_pipelined.txt", "w").write(format_kernel(piped) + "\n")
print("wrote", OUT)
'''


def main() -> int:
    if not os.path.isdir(REF):
        print("reference tree not present; fixtures are used as committed")
        return 0
    code = f"REF = {REF!r}\nOUT = {HERE!r}\n" + _CHILD
    env = dict(os.environ, PYTHONPATH="")
    return subprocess.call([sys.executable, "-S", "-c", code], cwd="/tmp", env=env)


if __name__ == "__main__":
    raise SystemExit(main())
