"""Host runtime: code-object cache + ctypes binding of ``libwarpir_rt.so``.

The reference host harness JIT-builds each generated kernel with a pybind
launch wrapper (``tests/test_modal_gpu.py:80-99``) and launches it with
``gemm<<<grid, 128>>>(global_vars{...})`` (``:24-50``).  Here the flow is:

1. ``CDNA4Lowerer.lower(kernel)`` -> HIP source;
2. ``compile_source`` -> ``hipcc --genco --offload-arch=gfx950`` code object,
   cached in ``warpir_amd/_kcache/<sha256>.hsaco`` (built ahead of time by
   ``__graft_entry__.build()`` so GPU runs never compile);
3. ``KernelHandle`` loads it through the C ABI of ``include/warpir_rt.h``
   (``wir_module_load`` / ``wir_module_get_function``), packs the kernel's
   globals struct (inputs then outputs, ``lowering.py:291-298``) from
   PyTorch tensors' pointers, shapes and strides, and calls ``wir_launch``
   on the current PyTorch stream.  The runtime never allocates user memory.

Errors: any non-zero HIP status raises ``HipError`` with
``wir_error_string``; a failed compile raises ``CompileError`` with the
hipcc log.  There is no fallback path: without the native library or a
GPU the launch raises.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import shutil
import subprocess
import threading
from typing import Dict, Optional, Sequence, Tuple

from warpir_amd.ir.ops import Kernel, Value
from warpir_amd.ir.types import GPUType, GlobalType, ScalarType
from warpir_amd.lowering.cdna4 import HIPCC_FLAGS_MARKER

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libwarpir_rt.so")
CACHE_DIR = os.environ.get("WARPIR_KCACHE", os.path.join(PKG_DIR, "_kcache"))
ARCH = "gfx950"
# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in generated code.
HIPCC_FLAGS = ("-O3", "-std=c++17", "--genco", f"--offload-arch={ARCH}",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")

_EXPORTS = (
    "wir_abi_version", "wir_set_device", "wir_device_info", "wir_module_load", "wir_module_unload",
    "wir_module_get_function", "wir_launch", "wir_function_attrs", "wir_stream_sync",
    "wir_device_sync", "wir_event_create", "wir_event_destroy", "wir_event_record",
    "wir_event_elapsed_ms", "wir_error_string",
)


class HipError(RuntimeError):
    """A HIP call behind the C ABI returned an error."""


class CompileError(RuntimeError):
    """hipcc rejected a generated kernel."""


# ---------------------------------------------------------------------------
# native library
# ---------------------------------------------------------------------------
_lib_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def library() -> ctypes.CDLL:
    """The loaded ``libwarpir_rt.so`` with argument types declared."""
    global _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        vp, sz, ci, cu = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint
        sig = {
            "wir_abi_version": ([], ci),
            "wir_set_device": ([ci], ci),
            "wir_device_info": ([ci, ctypes.POINTER(ci), ctypes.POINTER(ci), ctypes.POINTER(ci),
                                 ctypes.c_char_p, sz], ci),
            "wir_module_load": ([vp, sz, ctypes.POINTER(vp)], ci),
            "wir_module_unload": ([vp], ci),
            "wir_module_get_function": ([vp, ctypes.c_char_p, ctypes.POINTER(vp)], ci),
            "wir_launch": ([vp, cu, cu, cu, cu, cu, cu, cu, vp, vp, sz], ci),
            "wir_function_attrs": ([vp, ctypes.POINTER(ci), ctypes.POINTER(ci), ctypes.POINTER(ci)], ci),
            "wir_stream_sync": ([vp], ci),
            "wir_device_sync": ([], ci),
            "wir_event_create": ([ctypes.POINTER(vp)], ci),
            "wir_event_destroy": ([vp], ci),
            "wir_event_record": ([vp, vp], ci),
            "wir_event_elapsed_ms": ([vp, vp, ctypes.POINTER(ctypes.c_float)], ci),
            "wir_error_string": ([ci], ctypes.c_char_p),
            "wir_gemm_splitk": ([vp, vp, vp, vp, vp, vp, sz, ci, ci, ci, ci, vp], ci),
            "wir_gemm_splitk_noalloc": ([vp, vp, vp, vp, vp, ci, ci, ci, ci, vp], ci),
            "wir_gemm_splitk_fused": ([vp, vp, vp, vp, vp, sz, vp, sz, ci, ci, ci, ci, vp], ci),
        }
        for name, (args, res) in sig.items():
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = args, res
        _lib = lib
        return lib


def check(code: int, what: str = "HIP call") -> None:
    if code != 0:
        msg = library().wir_error_string(code)
        raise HipError(f"{what} failed: {msg.decode() if msg else code} (code {code})")


def device_info(device: int = 0) -> Dict[str, object]:
    lib = library()
    cus, clk, lds = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    arch = ctypes.create_string_buffer(64)
    check(lib.wir_device_info(device, ctypes.byref(cus), ctypes.byref(clk), ctypes.byref(lds), arch, 64),
          "wir_device_info")
    return {"num_cus": cus.value, "clock_khz": clk.value, "lds_per_block": lds.value,
            "arch": arch.value.decode()}


# ---------------------------------------------------------------------------
# compilation cache
# ---------------------------------------------------------------------------
def source_key(source: str) -> str:
    h = hashlib.sha256()
    h.update(" ".join(HIPCC_FLAGS).encode())
    h.update(b"\0")
    h.update(source.encode())
    return h.hexdigest()[:32]


def hsaco_path(source: str) -> str:
    return os.path.join(CACHE_DIR, source_key(source) + ".hsaco")


# Extra hipcc flags a generated source may ask for on its first line (after
# the lowering's HIPCC_FLAGS_MARKER); only these are accepted.
_ALLOWED_SOURCE_FLAGS = {("-mllvm", "-amdgpu-mfma-vgpr-form=1")}


def source_flags(source: str) -> Tuple[str, ...]:
    """The hipcc flags named on *source*'s first line, if it carries the marker."""
    first = source.split("\n", 1)[0]
    if not first.startswith(HIPCC_FLAGS_MARKER):
        return ()
    words = first[len(HIPCC_FLAGS_MARKER):].split()
    if len(words) % 2 or any(tuple(words[i:i + 2]) not in _ALLOWED_SOURCE_FLAGS for i in range(0, len(words), 2)):
        raise CompileError(f"unsupported hipcc flags in the source marker: {' '.join(words)}")
    return tuple(words)


def compile_source(source: str, force: bool = False) -> str:
    """Compile *source* for gfx950 into the cache; returns the ``.hsaco`` path."""
    out = hsaco_path(source)
    if os.path.exists(out) and not force:
        return out
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        raise CompileError(f"{out} is not cached and hipcc is not available")
    os.makedirs(CACHE_DIR, exist_ok=True)
    base = out[: -len(".hsaco")]
    src_path = base + ".hip"
    with open(src_path, "w") as f:
        f.write(source)
    tmp = f"{base}.{os.getpid()}.tmp"
    cmd = [hipcc, *HIPCC_FLAGS, *source_flags(source), "-Rpass-analysis=kernel-resource-usage", src_path,
           "-o", tmp]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    with open(base + ".log", "w") as f:
        f.write(" ".join(cmd) + "\n" + proc.stdout)
    if proc.returncode != 0:
        raise CompileError(f"hipcc failed for {src_path}:\n{proc.stdout[-4000:]}")
    os.replace(tmp, out)
    return out


def resource_usage(source: str) -> Dict[str, int]:
    """VGPR/AGPR/SGPR/spill/LDS/occupancy figures from the cached compile log."""
    log = hsaco_path(source)[: -len(".hsaco")] + ".log"
    usage: Dict[str, int] = {}
    if not os.path.exists(log):
        return usage
    keys = {"VGPRs:": "vgpr", "AGPRs:": "agpr", "SGPRs:": "sgpr", "ScratchSize [bytes/lane]:": "scratch",
            "Occupancy [waves/SIMD]:": "occupancy", "VGPRs Spill:": "vgpr_spill",
            "LDS Size [bytes/block]:": "lds"}
    with open(log) as f:
        for line in f:
            for k, name in keys.items():
                if k in line:
                    try:
                        usage[name] = int(line.rsplit(k, 1)[1].strip().split()[0])
                    except (ValueError, IndexError):
                        pass
    return usage



def compiled_register_count(target=None):
    """A register estimator for ``CostModel.register_estimate``: the registers
    per lane hipcc gives the kernel's gfx950 lowering (VGPRs + AGPRs + spilled
    VGPRs), from the compile remarks.  Compiles through the code-object cache,
    so each distinct kernel is compiled once.  ``target`` is the
    ``CDNA4Target`` the kernel will be lowered with."""
    from warpir_amd.lowering import CDNA4Lowerer

    def estimate(kernel: Kernel) -> int:
        src = CDNA4Lowerer(target).lower(kernel)
        compile_source(src)
        u = resource_usage(src)
        return u.get("vgpr", 0) + u.get("agpr", 0) + u.get("vgpr_spill", 0)

    return estimate

# ---------------------------------------------------------------------------
# kernel arguments
# ---------------------------------------------------------------------------
class GL(ctypes.Structure):
    """Host mirror of ``wir::gl<T>`` (pointer, 4 dims, 3 strides in elements)."""

    _fields_ = [("data", ctypes.c_void_p), ("b", ctypes.c_int), ("d", ctypes.c_int),
                ("r", ctypes.c_int), ("c", ctypes.c_int), ("sb", ctypes.c_longlong),
                ("sd", ctypes.c_longlong), ("sr", ctypes.c_longlong)]


def kernarg_struct(kernel: Kernel):
    """ctypes structure laid out as the emitted ``<name>_globals`` struct."""
    fields = []
    for v in list(kernel.inputs) + list(kernel.outputs):
        fields.append((v.name, GL if isinstance(v.type, GlobalType) else ctypes.c_int))
    return type(f"{kernel.name}_globals", (ctypes.Structure,), {"_fields_": fields})


def _global_view(v: Value, t) -> Tuple[Tuple[int, int, int, int], Tuple[int, int, int]]:
    """4-D (b, d, r, c) shape and (sb, sd, sr) element strides of tensor *t* for global *v*."""
    shape, strides = list(t.shape), list(t.stride())
    gt: GlobalType = v.type
    if gt.cols == 1 and (not shape or shape[-1] != 1):
        shape.append(1)
        strides.append(1)
    if len(shape) > 4:
        raise ValueError(f"{v.name}: tensors of rank {len(shape)} are not supported")
    while len(shape) < 4:
        shape.insert(0, 1)
        strides.insert(0, 0)
    if shape[3] > 1 and strides[3] != 1:
        raise ValueError(f"{v.name}: the last dimension must be contiguous (stride 1)")
    for want, got, what in zip((gt.batch, gt.depth, gt.rows, gt.cols), shape, "bdrc"):
        if want != -1 and want != got:
            raise ValueError(f"{v.name}: dimension {what} is {got}, the IR type fixes {want}")
    return tuple(shape), (strides[0], strides[1], strides[2])


# ---------------------------------------------------------------------------
# loaded kernels
# ---------------------------------------------------------------------------
class KernelHandle:
    """A lowered, compiled WarpIR kernel, launched through the C ABI."""

    def __init__(self, kernel: Kernel, lowerer=None, source: Optional[str] = None):
        from warpir_amd.lowering import CDNA4Lowerer

        self.kernel = kernel
        self.lowerer = lowerer or CDNA4Lowerer()
        self.source = source if source is not None else self.lowerer.lower(kernel)
        if self.lowerer.kernel is not kernel:
            self.lowerer.lower(kernel)
        self.path = compile_source(self.source)
        self.args_type = kernarg_struct(kernel)
        self._module = None
        self._function = None
        self._load_lock = threading.Lock()
        # packed kernel arguments and launch configuration per argument signature
        # (tensor pointers, shapes, strides, dtypes and int values), so repeated
        # launches with the same buffers skip validation and packing
        self._pack_cache: Dict[tuple, tuple] = {}
        self._loaded_stores = [v.name for v in kernel.outputs]
        self._loaded_globals = self._loaded_sources()

    def _loaded_sources(self):
        from warpir_amd.ir.ops import TMALoadBufOp, TMALoadOp
        from warpir_amd.lowering.cdna4 import _walk
        return {op.source.name for op in _walk(self.kernel.body) if isinstance(op, (TMALoadOp, TMALoadBufOp))}

    def resources(self) -> Dict[str, int]:
        return resource_usage(self.source)

    def load(self) -> None:
        if self._function is not None:
            return
        with self._load_lock:   # one module per handle, also when threads race here
            if self._function is not None:
                return
            lib = library()
            with open(self.path, "rb") as f:
                image = f.read()
            self._image = ctypes.create_string_buffer(image, len(image))
            mod = ctypes.c_void_p()
            check(lib.wir_module_load(self._image, len(image), ctypes.byref(mod)), "wir_module_load")
            fn = ctypes.c_void_p()
            check(lib.wir_module_get_function(mod, self.kernel.name.encode(), ctypes.byref(fn)),
                  f"wir_module_get_function({self.kernel.name})")
            self._module, self._function = mod, fn

    def pack(self, args: Dict[str, object]):
        """Validate tensors / ints and build the kernel-argument struct and grid."""
        import torch

        packed = self.args_type()
        shapes = {}
        device = None
        for v in list(self.kernel.inputs) + list(self.kernel.outputs):
            if v.name not in args:
                raise ValueError(f"missing kernel argument {v.name!r}")
            x = args[v.name]
            if isinstance(v.type, GlobalType):
                if not isinstance(x, torch.Tensor):
                    raise TypeError(f"{v.name} must be a torch.Tensor")
                want = torch.bfloat16 if v.type.data_type == GPUType.bf16 else torch.float32
                if x.dtype != want:
                    raise TypeError(f"{v.name}: dtype {x.dtype}, expected {want}")
                if not x.is_cuda:
                    raise ValueError(f"{v.name} must be a GPU tensor")
                if device is None:
                    device = x.device
                elif x.device != device:
                    raise ValueError("all tensors must be on one device")
                shape, strides = _global_view(v, x)
                esz = x.element_size()
                vector = v.type.data_type == GPUType.fp32 and v.type.sub_tile_type.cols == 1
                if vector:   # fp32 L x 1 vectors move 4 bytes per lane
                    if x.data_ptr() % 4:
                        raise ValueError(f"{v.name}: must be 4-byte aligned")
                elif (v.name in self._loaded_globals or shape[3] > 1) and x.numel():
                    # (an empty tensor is never read or written: every tile of it
                    # lies outside it, and loads of such tiles read the zero page)
                    if x.data_ptr() % 16 or (strides[2] * esz) % 16 or (shape[3] * esz) % 16:
                        raise ValueError(f"{v.name}: rows must be 16-byte aligned and a multiple of 16 bytes "
                                         "(the tile-load granule)")
                for dim in shape:
                    if dim >= 2 ** 31:
                        raise ValueError(f"{v.name}: dimension {dim} does not fit in int32")
                setattr(packed, v.name, GL(x.data_ptr(), *shape, *strides))
                shapes[v.name] = shape
            elif isinstance(v.type, ScalarType):
                if not isinstance(x, int):
                    raise TypeError(f"{v.name} must be an int")
                if not -(2 ** 31) <= x < 2 ** 31:
                    raise ValueError(f"{v.name}={x} does not fit in int32")
                setattr(packed, v.name, x)
        cfg = self.lowerer.launch_config(self.kernel, {k: s for k, s in shapes.items()})
        # every output empty (e.g. attention over S = 0): the launch would write nothing
        empty = all(args[v.name].numel() == 0 for v in self.kernel.outputs
                    if isinstance(v.type, GlobalType)) and any(isinstance(v.type, GlobalType)
                                                               for v in self.kernel.outputs)
        return packed, cfg, device, empty

    def _signature(self, args: Dict[str, object]):
        """Hashable summary of the arguments that fixes the packed struct, or None."""
        import torch

        sig = []
        for v in list(self.kernel.inputs) + list(self.kernel.outputs):
            x = args.get(v.name)
            if isinstance(x, torch.Tensor):
                sig.append((x.data_ptr(), tuple(x.shape), tuple(x.stride()), x.dtype, x.device))
            elif isinstance(x, int):
                sig.append(x)
            else:
                return None
        return tuple(sig) if len(args) == len(sig) else None

    def __call__(self, stream=None, **args) -> None:
        import torch

        key = self._signature(args)
        hit = self._pack_cache.get(key) if key is not None else None
        if hit is None:
            hit = self.pack(args)
            if key is not None:
                if len(self._pack_cache) >= 64:
                    self._pack_cache.clear()
                self._pack_cache[key] = hit
        packed, cfg, device, empty = hit
        gx, gy, gz = cfg.grid
        if empty or not (gx and gy and gz):
            return   # an empty problem: no output element to write, or no workgroup
        self.load()
        if stream is None:
            stream = torch.cuda.current_stream(device).cuda_stream
        elif hasattr(stream, "cuda_stream"):
            stream = stream.cuda_stream
        bx, by, bz = cfg.block
        check(library().wir_launch(self._function, gx, gy, gz, bx, by, bz, cfg.dyn_lds,
                                   ctypes.c_void_p(stream), ctypes.byref(packed), ctypes.sizeof(packed)),
              f"wir_launch({self.kernel.name})")

    def __del__(self):
        if self._module is not None and _lib is not None:
            try:
                _lib.wir_module_unload(self._module)
            except Exception:  # interpreter shutdown
                pass


def compile_kernel(kernel: Kernel, lowerer=None) -> KernelHandle:
    """Lower, compile (or fetch from the cache) and wrap *kernel* for launching."""
    return KernelHandle(kernel, lowerer)


_raw_lock = threading.Lock()


class RawKernel:
    """A hand-written kernel from a prebuilt code object in the package
    (``__graft_entry__.build()`` compiles them), launched through the C ABI
    with a ctypes argument structure on the current stream."""

    def __init__(self, filename: str, symbol: str):
        self.path = os.path.join(PKG_DIR, filename)
        self.symbol = symbol
        self._module = None
        self._function = None

    def _load(self) -> None:
        if self._function is not None:
            return
        with _raw_lock:
            if self._function is None:
                self._load_locked()

    def _load_locked(self) -> None:
        if not os.path.exists(self.path):
            raise CompileError(f"{self.path} is not built (run __graft_entry__.build())")
        lib = library()
        with open(self.path, "rb") as f:
            self._image = f.read()
        mod, fn = ctypes.c_void_p(), ctypes.c_void_p()
        check(lib.wir_module_load(self._image, len(self._image), ctypes.byref(mod)), f"wir_module_load({self.path})")
        check(lib.wir_module_get_function(mod, self.symbol.encode(), ctypes.byref(fn)),
              f"wir_module_get_function({self.symbol})")
        self._module, self._function = mod, fn

    def launch(self, grid: Tuple[int, int, int], block: Tuple[int, int, int], args: ctypes.Structure,
               stream=None) -> None:
        import torch

        if not all(grid):
            return   # no workgroups: nothing to launch
        self._load()
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        check(library().wir_launch(self._function, *grid, *block, 0, ctypes.c_void_p(stream), ctypes.byref(args),
                                   ctypes.sizeof(args)), f"wir_launch({self.symbol})")

    def __del__(self):
        if _lib is not None and self._module:
            try:
                _lib.wir_module_unload(self._module)
            except Exception:
                pass


class Event:
    """A HIP timing event recorded on a stream through the C ABI."""

    def __init__(self):
        self._ev = ctypes.c_void_p()
        check(library().wir_event_create(ctypes.byref(self._ev)), "wir_event_create")

    def record(self, stream) -> None:
        check(library().wir_event_record(self._ev, ctypes.c_void_p(stream)), "wir_event_record")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(library().wir_event_elapsed_ms(self._ev, end._ev, ctypes.byref(ms)), "wir_event_elapsed_ms")
        return ms.value

    def __del__(self):
        if _lib is not None and self._ev:
            try:
                _lib.wir_event_destroy(self._ev)
            except Exception:
                pass


__all__ = ["HipError", "CompileError", "KernelHandle", "RawKernel", "compile_kernel", "compile_source",
           "library", "device_info", "Event", "kernarg_struct", "GL", "hsaco_path", "resource_usage"]
