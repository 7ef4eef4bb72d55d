"""MI355X (gfx950 / CDNA4) backend for the WarpIR tile IR.

Sub-packages:

* ``ir``        -- the tile IR (types, SSA ops, buffer ops, loops)
* ``printing``  -- text form of the IR
* ``passes``    -- modulo scheduling and wavefront assignment
* ``lowering``  -- IR -> gfx950 HIP source (``CDNA4Lowerer``)
* ``runtime``   -- hipcc code-object cache + ctypes binding of the C-ABI
                   launcher library (``libwarpir_rt.so``)
* ``workloads`` -- IR builders for the GEMM and FlashAttention workloads
"""
__version__ = "0.1.0"
