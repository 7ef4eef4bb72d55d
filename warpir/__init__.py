"""Import alias: ``warpir.<module>`` resolves to ``warpir_amd.<module>``.

Lets IR builder scripts written against the reference package
(``from warpir.ir import ...``, ``from warpir.passes.modulo_scheduler
import kernel_pass``, ``from warpir.printing import print_kernel``) run
unchanged on this backend.  The lowering target differs by design:
``warpir.lowering`` exports ``CDNA4Lowerer`` in place of the reference's
ThunderKittens lowerer.
"""
import importlib
import sys

_ALIASED = (
    "ir", "ir.ops", "ir.types",
    "printing", "printing.printer",
    "passes", "passes.modulo_scheduler", "passes.warp_assigner",
    "passes.register_counter", "passes.memory_annotator",
    "lowering", "runtime",
)

for _name in _ALIASED:
    _mod = importlib.import_module("warpir_amd." + _name)
    sys.modules[__name__ + "." + _name] = _mod
    if "." not in _name:
        globals()[_name] = _mod
