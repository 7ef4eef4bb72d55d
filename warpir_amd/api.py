"""Host entry points for the two workloads, over the generated kernels.

These play the role of the reference harness's launch wrappers
(``launch_gemm(A, B, C)``, ``tests/test_modal_gpu.py:24-50``;
``launch_attention(Q, K, V, O)``, ``tests/test_modal_attention.py:25-39``):
validate shapes, allocate nothing but the outputs the caller did not
pass, and launch the WarpIR-generated HIP kernel through the C ABI on the
current stream.  They raise on a CPU tensor or a missing GPU; there is no
fallback implementation.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

from warpir_amd import kernels

GEMM_VARIANT = "gemm_256_k64"
SKINNY_GEMM_VARIANT = "gemm_128x32_k64"   # M <= 128: 128x32 tiles, 256 workgroups at N = 8192
MID_GEMM_VARIANT = "gemm_128_k64"         # fewer 256x256 tiles than CUs: 128x128 tiles


def gemm_variant(m: int, n: int, k: Optional[int] = None) -> str:
    """Kernel variant for an M x N (x K) GEMM on the 256 CUs of one MI355X.

    Measured at N = K = 8192 with four B operands cycled (512 MiB, so B
    streams from HBM), microseconds per product: M=64 split-K x4 42.4 vs
    128x32 67.1; M=128 split-K x4 38.8 vs 128x32 60.4; M=256 128x64 68.5
    vs split-K x2 69.6."""
    if m <= 128 and k is not None and splitk_count(m, n, k) >= 4:
        return SPLITK_GEMM_VARIANT
    if m <= 128:
        return SKINNY_GEMM_VARIANT
    if m <= 256:
        return "gemm_128x64_k64"
    if math.ceil(m / 256) * math.ceil(n / 256) < 256:
        return MID_GEMM_VARIANT
    return GEMM_VARIANT


# 128x128 tiles, 64-deep K steps; kernel_pass sizes the rings per operand:
# B (streamed from HBM) seven slots loaded six steps ahead, A (the row panel
# every program re-reads from L2) three slots, filling 160 KiB of LDS
# (measured at M=128, N=K=8192: 36.6 us against 37.8 for 128-deep steps with
# three B slots, and 41.5 for 32-deep steps with fourteen).  The slices are
# summed by the separate reduction kernel (two launches in one C call), also
# the form of wir_gemm_splitk_noalloc.
SPLITK_TWO_LAUNCH_VARIANT = "gemm_128_splitk_k64_b7"
SPLITK_GEMM_VARIANT = SPLITK_TWO_LAUNCH_VARIANT
# The same GEMM summing the slices itself (one launch: the last slice to store
# an output tile adds the partials).  Correct, but slower on MI355X: its
# device-scope release and acquire write back and invalidate an XCD's whole
# L2 per workgroup (58 against 38 microseconds at M=128, N=K=8192).
SPLITK_FUSED_VARIANT = "gemm_128_splitk_fused"
_reduce_kernel = None
# Zeroed per-tile arrival counters of the fused split-K kernels, one buffer
# per (device, stream): the kernel leaves them zero, so launches ordered on
# one stream share a buffer and launches on different streams never do.
_arrivals: dict = {}
_arrivals_lock = __import__("threading").Lock()


def _arrival_counters(device, stream: int, count: int):
    import torch

    key = (device.index, stream)
    with _arrivals_lock:
        buf = _arrivals.get(key)
        if buf is None or buf.numel() < count:
            buf = torch.zeros(max(count, 256), dtype=torch.int32, device=device)
            _arrivals[key] = buf
        return buf


_fused_variants: dict = {}


def _fused(variant: str) -> bool:
    """Whether the split-K variant sums its slices itself (a reduce_slices op)."""
    from warpir_amd.ir import ReduceSlicesOp
    if variant not in _fused_variants:
        _fused_variants[variant] = any(isinstance(op, ReduceSlicesOp) for op in kernels.handle(variant).kernel.body)
    return _fused_variants[variant]


def splitk_count(m: int, n: int, k: int, num_cus: int = 256) -> int:
    """Number of K slices for the split-K kernel: enough 128x128 tiles x
    slices to cover the CUs, with every slice a whole number of 64-deep
    K steps.  1 means no split (also for an empty product)."""
    if m <= 0 or n <= 0 or k <= 0:
        return 1
    tiles = math.ceil(m / 128) * math.ceil(n / 128)
    best = 1
    for s in range(2, 17):
        if tiles * s > num_cus:
            break
        if k % (64 * s) == 0:
            best = s
    return best


_splitk_checked: set = set()


def _splitk_functions(variant: str):
    """(GEMM, reduction) kernel functions of a split-K variant, loaded.  The
    first use of a variant checks that its launch geometry is the one the C
    ABI's split-K entry points build (128x128 tiles, 256 threads, slices on
    blockIdx.z)."""
    from warpir_amd.runtime import RawKernel

    global _reduce_kernel
    h = kernels.handle(variant)
    if variant not in _splitk_checked:
        cfg = h.lowerer.launch_config(h.kernel, {"A": (1, 2, 256, 512), "B": (1, 2, 512, 384),
                                                 "C_global": (1, 2, 256, 384)})
        if cfg.grid != (3, 2, 2) or tuple(cfg.block) != (256, 1, 1):
            raise ValueError(f"{variant}: launch geometry {cfg} is not the split-K entry points' "
                             "(128x128 tiles, 256 threads)")
        _splitk_checked.add(variant)
    h.load()
    if _fused(variant):
        return h._function, None
    if _reduce_kernel is None:
        _reduce_kernel = RawKernel("splitk_reduce.hsaco", "wir_splitk_reduce")
    _reduce_kernel._load()
    return h._function, _reduce_kernel._function


def gemm_split_k(a, b, out=None, splits: Optional[int] = None, workspace=None, variant: Optional[str] = None):
    """``out = a @ b`` as ``splits`` K slices run side by side (``blockIdx.z``)
    plus an fp32 reduction: the form for short M and long K, where the
    output alone has too few tiles to fill the chip.  The default variant
    sums the slices with the separate reduction kernel; the fused variant
    (``SPLITK_FUSED_VARIANT``) sums them inside the GEMM kernel (one launch,
    per-tile arrival counters kept per device and stream).  ``workspace`` is an
    fp32 tensor of at least ``splits * M * N`` elements (allocated if
    omitted); ``variant`` names a split-K kernel variant (default
    ``SPLITK_GEMM_VARIANT``)."""
    import ctypes

    import torch

    from warpir_amd.runtime import check, library

    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"gemm: shapes {tuple(a.shape)} @ {tuple(b.shape)} do not chain")
    m, k = a.shape
    n = b.shape[1]
    if k == 0:
        raise ValueError("gemm_split_k: K must be positive (api.gemm takes K = 0)")
    splits = splits or splitk_count(m, n, k)
    if k % (64 * splits) or n % 8 or not a.is_contiguous() or not b.is_contiguous():
        raise ValueError(f"gemm_split_k: K={k} must split into {splits} multiples of 64, N % 8 == 0, "
                         "contiguous operands")
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise TypeError("gemm_split_k: a and b must be bf16")
    if out is None:
        out = torch.empty(m, n, dtype=torch.bfloat16, device=a.device)
    # the reduction writes M * N bf16 values flat from out's first element
    if tuple(out.shape) != (m, n) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError(f"gemm_split_k: out must be a contiguous bf16 [{m}, {n}] tensor, got "
                         f"{out.dtype} {tuple(out.shape)} with strides {tuple(out.stride())}")
    if out.device != a.device:
        raise ValueError("gemm_split_k: out must be on the operands' device")
    if workspace is None:
        workspace = torch.empty(splits * m * n, dtype=torch.float32, device=a.device)
    if workspace.numel() < splits * m * n or workspace.dtype != torch.float32:
        raise ValueError("gemm_split_k: workspace must be fp32 with splits * M * N elements")
    if workspace.device != a.device or not workspace.is_contiguous():
        raise ValueError("gemm_split_k: workspace must be a contiguous tensor on the operands' device")
    if not a.is_cuda or b.device != a.device:
        raise ValueError("gemm_split_k: a, b, out and workspace must be on one GPU")
    if any(t.data_ptr() % 16 for t in (a, b, out, workspace)):
        raise ValueError("gemm_split_k: a, b, out and workspace must be 16-byte aligned")
    if m == 0 or n == 0:
        return out
    gemm_fn, reduce_fn = _splitk_functions(variant or SPLITK_GEMM_VARIANT)
    stream = torch.cuda.current_stream(a.device).cuda_stream
    if reduce_fn is None:   # the slices are summed inside the GEMM kernel
        tiles = math.ceil(m / 128) * math.ceil(n / 128)
        arr = _arrival_counters(a.device, stream, tiles)
        check(library().wir_gemm_splitk_fused(gemm_fn, a.data_ptr(), b.data_ptr(), out.data_ptr(),
                                              workspace.data_ptr(), workspace.numel(), arr.data_ptr(),
                                              arr.numel(), m, n, k, splits, ctypes.c_void_p(stream)),
              "wir_gemm_splitk_fused")
        return out
    check(library().wir_gemm_splitk(gemm_fn, reduce_fn, a.data_ptr(), b.data_ptr(), out.data_ptr(),
                                    workspace.data_ptr(), workspace.numel(), m, n, k, splits,
                                    ctypes.c_void_p(stream)), "wir_gemm_splitk")
    return out


NOALLOC_SCRATCH_FLOATS = 8 * 1024 * 1024   # WIR_NOALLOC_SCRATCH_FLOATS of include/warpir_rt.h


def gemm_split_k_noalloc(a, b, out, splits: Optional[int] = None, stream=None):
    """``out = a @ b`` by the split-K GEMM and the separate reduction kernel
    (``SPLITK_TWO_LAUNCH_VARIANT``; the same sums, bit for bit, as
    ``gemm_split_k``), with the fp32 partials in the native library's own
    device scratch: no device
    memory is allocated (``wir_gemm_splitk_noalloc``).  ``out`` is required.
    Raises ``HipError`` when ``splits * M * N`` exceeds the scratch
    (``NOALLOC_SCRATCH_FLOATS``).  Calls that overlap on one device share the
    scratch and race; order them on one stream."""
    import ctypes

    import torch

    from warpir_amd.runtime import check, library

    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"gemm: shapes {tuple(a.shape)} @ {tuple(b.shape)} do not chain")
    m, k = a.shape
    n = b.shape[1]
    if k == 0:
        raise ValueError("gemm_split_k_noalloc: K must be positive (api.gemm takes K = 0)")
    splits = splits or splitk_count(m, n, k)
    for name, t, shape in (("a", a, (m, k)), ("b", b, (k, n)), ("out", out, (m, n))):
        if (not isinstance(t, torch.Tensor) or tuple(t.shape) != shape or t.dtype != torch.bfloat16
                or not t.is_contiguous()):
            raise ValueError(f"gemm_split_k_noalloc: {name} must be a contiguous bf16 {list(shape)} tensor")
    if not a.is_cuda or b.device != a.device or out.device != a.device:
        raise ValueError("gemm_split_k_noalloc: a, b and out must be on one GPU")
    if m == 0 or n == 0:
        return out
    gemm_fn, reduce_fn = _splitk_functions(SPLITK_TWO_LAUNCH_VARIANT)
    if stream is None:
        stream = torch.cuda.current_stream(a.device).cuda_stream
    elif hasattr(stream, "cuda_stream"):
        stream = stream.cuda_stream
    with torch.cuda.device(a.device):
        check(library().wir_gemm_splitk_noalloc(gemm_fn, reduce_fn, a.data_ptr(),
                                                b.data_ptr(), out.data_ptr(), m, n, k, splits,
                                                ctypes.c_void_p(stream)),
              "wir_gemm_splitk_noalloc")
    return out


def _splitk_operands_ok(a, b, out) -> bool:
    """Whether ``gemm_split_k`` accepts these tensors: bf16, contiguous and
    16-byte aligned (it addresses them as dense row-major arrays)."""
    import torch

    return all(t.dtype == torch.bfloat16 and t.is_contiguous() and t.data_ptr() % 16 == 0
               for t in (a, b, out))


def gemm(a, b, out=None, variant: Optional[str] = None, workspace=None):
    """``out[M, N] = a[M, K] @ b[K, N]`` in bf16 with fp32 accumulation.

    The variant follows ``gemm_variant``: 256x256 tiles by default, smaller
    tiles for outputs with fewer tiles than CUs, split-K for M <= 128 and
    long K (``workspace`` as in ``gemm_split_k``).  An empty output (M or
    N = 0) launches nothing; K = 0 gives zeros (the kernel's loop runs no
    step and its tile loads read the zero page).
    """
    import torch

    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"gemm: shapes {tuple(a.shape)} @ {tuple(b.shape)} do not chain")
    m, k = a.shape
    n = b.shape[1]
    if k % 8 or n % 8:
        raise ValueError("gemm: K and N must be multiples of 8 (16-byte rows)")
    if out is None:
        out = torch.empty(m, n, dtype=torch.bfloat16, device=a.device)
    if variant is None:
        variant = gemm_variant(m, n, k)
        if variant == SPLITK_GEMM_VARIANT and not _splitk_operands_ok(a, b, out):
            # the split-K entry points take dense operands only; the tiled
            # kernel reads row-strided views through the globals' row stride
            variant = SKINNY_GEMM_VARIANT
    if variant == SPLITK_GEMM_VARIANT:
        return gemm_split_k(a, b, out=out, workspace=workspace)
    kernels.handle(variant)(A=a, B=b, N=k, C_global=out)
    return out


def attention_forward(q, k, v, causal: bool = False, out=None, lse=None,
                      variant: Optional[str] = None) -> Tuple[object, object]:
    """FlashAttention forward over ``[B, H, S, D]`` bf16; returns ``(O, LSE)``.

    ``LSE[b, h, s] = logsumexp_j(q_s . k_j / sqrt(D))`` in fp32 (natural log).
    """
    import torch

    bsz, heads, seq, d = q.shape
    hr = _head_ratio("attention_forward", q, k, v)
    if variant is None:
        variant = {(128, False): "mha_d128", (64, True): "mha_d64_causal",
                   (128, True): "mha_d128_causal", (64, False): "mha_d64"}.get((d, causal))
        if variant is None:
            raise ValueError(f"attention_forward: no kernel variant for D={d}, causal={causal}")
        if hr > 1:
            variant += "_gqa"
    handle = kernels.handle(variant)
    kv_tile = next(o for o in _loops(handle.kernel)).tile_size
    if seq % kv_tile:
        raise ValueError(f"attention_forward: S={seq} must be a multiple of the KV tile {kv_tile}")
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty(bsz, heads, seq, dtype=torch.float32, device=q.device)
    if any(v_.name == "HR" for v_ in handle.kernel.inputs):
        handle(Q=q, K=k, V=v, N=seq, HR=hr, O=out, L=lse)
    elif hr > 1:
        raise ValueError(f"attention_forward: variant {variant} takes no grouped-query heads")
    else:
        handle(Q=q, K=k, V=v, N=seq, O=out, L=lse)
    return out, lse


def _head_ratio(fn: str, q, k, v) -> int:
    """Query heads per key/value head (grouped-query attention); 1 for plain MHA."""
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape or q.shape[0] != k.shape[0] \
            or q.shape[2:] != k.shape[2:]:
        raise ValueError(f"{fn}: q [B, H, S, D] and k, v [B, H_kv, S, D] shapes do not match")
    if k.shape[1] < 1 or q.shape[1] % k.shape[1]:
        raise ValueError(f"{fn}: {q.shape[1]} query heads are not a multiple of {k.shape[1]} key/value heads")
    return q.shape[1] // k.shape[1]


def attention_backward(q, k, v, o, lse, do, dq=None, dk=None, dv=None, dvec=None, causal: bool = False,
                       workspace=None):
    """Gradients ``(dQ, dK, dV)`` of ``attention_forward`` over ``[B, H, S, D]``
    bf16, from its outputs ``o`` and ``lse`` and the output gradient ``do``
    (``causal`` must match the forward); S must be a multiple of 64.  With
    grouped-query K and V (``[B, H_kv, S, D]``) the key-major kernel writes
    each query head's fp32 dK / dV contribution into ``workspace`` (fp32, at
    least ``2 * B * H * S * D`` elements, allocated if omitted) and a HIP
    reduction sums the ``H / H_kv`` contributions of every key/value head
    into bf16 ``dK`` / ``dV``.  Three WarpIR kernels run
    on the current stream: ``Dv = rowsum(dO * O)`` (into ``dvec``, fp32
    ``[B, H, S]``, allocated if omitted) together with the LSE in log2 units,
    the query-major dQ kernel and the key-major dK/dV kernel (the reference's TK backward,
    ``kernel_examples/attention/mha_h100.cu:253-303,482-642``, computes the
    same gradients with dQ by atomic adds)."""
    import torch

    if q.dim() != 4 or not (q.shape == o.shape == do.shape):
        raise ValueError("attention_backward: q, o, do must share one [B, H, S, D] shape")
    hr = _head_ratio("attention_backward", q, k, v)
    bsz, heads, seq, d = q.shape
    if d not in (64, 128) or seq % 64:
        raise ValueError(f"attention_backward: D must be 64 or 128 and S a multiple of 64 (got D={d}, S={seq})")
    if tuple(lse.shape) != (bsz, heads, seq) or lse.dtype != torch.float32:
        raise ValueError("attention_backward: lse must be fp32 [B, H, S]")
    dq = torch.empty_like(q) if dq is None else dq
    dk = torch.empty_like(k) if dk is None else dk
    dv = torch.empty_like(v) if dv is None else dv
    dvec = torch.empty(bsz, heads, seq, dtype=torch.float32, device=q.device) if dvec is None else dvec
    lse2 = torch.empty_like(lse)   # the LSE in log2 units, for the dK/dV kernel
    kernels.handle(f"mha_bwd_prep_d{d}")(O=o, dO=do, L=lse, Dv=dvec, L2=lse2)
    sfx = "_causal" if causal else ""
    if hr == 1:
        kernels.handle(f"mha_bwd_dq_d{d}{sfx}")(Q=q, K=k, V=v, dO=do, L=lse, Dv=dvec, N=seq, dQ=dq)
        kernels.handle(f"mha_bwd_dkdv_d{d}{sfx}")(Q=q, K=k, V=v, dO=do, L2=lse2, Dv=dvec, N=seq, dK=dk, dV=dv)
        return dq, dk, dv
    numel = q.numel()
    if workspace is None:
        workspace = torch.empty(2 * numel, dtype=torch.float32, device=q.device)
    if workspace.dtype != torch.float32 or workspace.numel() < 2 * numel or not workspace.is_contiguous():
        raise ValueError(f"attention_backward: workspace must be contiguous fp32 with >= {2 * numel} elements")
    dk_part = workspace[:numel].view(q.shape)
    dv_part = workspace[numel:2 * numel].view(q.shape)
    kernels.handle(f"mha_bwd_dq_d{d}{sfx}_gqa")(Q=q, K=k, V=v, dO=do, L=lse, Dv=dvec, N=seq, HR=hr, dQ=dq)
    kernels.handle(f"mha_bwd_dkdv_d{d}{sfx}_gqa")(Q=q, K=k, V=v, dO=do, L2=lse2, Dv=dvec, N=seq, HR=hr,
                                                  dK_part=dk_part, dV_part=dv_part)
    _group_reduce(dk_part, dk, hr)
    _group_reduce(dv_part, dv, hr)
    return dq, dk, dv


_group_reduce_kernel = None


def _group_reduce(partials, out, splits: int) -> None:
    """``out[g] = bf16(sum_r partials[g * splits + r])`` over the key/value head
    groups of a ``[B, H, S, D]`` fp32 contribution tensor (``splitk_reduce.hip``)."""
    import ctypes

    from warpir_amd.runtime import RawKernel

    global _group_reduce_kernel
    if _group_reduce_kernel is None:
        _group_reduce_kernel = RawKernel("splitk_reduce.hsaco", "wir_group_reduce")

    class Args(ctypes.Structure):
        _fields_ = [("partials", ctypes.c_void_p), ("out", ctypes.c_void_p), ("n", ctypes.c_longlong),
                    ("groups", ctypes.c_longlong), ("splits", ctypes.c_int)]

    if not out.is_contiguous() or out.dtype.itemsize != 2:
        raise ValueError("attention_backward: dk / dv must be contiguous bf16")
    if out.numel() == 0:
        return
    n = out.shape[-2] * out.shape[-1]
    groups = out.numel() // n
    if n % 8 or partials.numel() != groups * splits * n:
        raise ValueError("attention_backward: grouped reduction needs S * D % 8 == 0 and matching shapes")
    args = Args(partials.data_ptr(), out.data_ptr(), n, groups, splits)
    _group_reduce_kernel.launch(((groups * n // 8 + 255) // 256, 1, 1), (256, 1, 1), args)


def attention_backward_flops(bsz: int, heads: int, seq: int, d: int, causal: bool = False) -> float:
    """Matmul FLOPs of attention backward counted as the five S x S x D
    products of the standard algorithm (S, dP, dV, dK, dQ): 10*B*H*S^2*D,
    halved when causal.  These kernels run seven (dQ recomputes S and dP
    instead of atomics)."""
    f = 10.0 * bsz * heads * seq * seq * d
    return f / 2 if causal else f


def attention_flops(bsz: int, heads: int, seq: int, d: int, causal: bool = False) -> float:
    """Matmul FLOPs of attention forward: 4*B*H*S^2*D (halved when causal)."""
    f = 4.0 * bsz * heads * seq * seq * d
    return f / 2 if causal else f


def _loops(kernel):
    from warpir_amd.ir.ops import ForOp
    return (op for op in kernel.body if isinstance(op, ForOp))


__all__ = ["gemm", "gemm_split_k", "splitk_count", "gemm_variant", "attention_forward", "attention_backward",
           "attention_flops", "attention_backward_flops"]
