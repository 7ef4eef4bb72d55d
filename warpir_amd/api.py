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


def gemm_variant(m: int, n: int) -> str:
    """Kernel variant for an M x N output on the 256 CUs of one MI355X."""
    if m <= 128:
        return SKINNY_GEMM_VARIANT
    if math.ceil(m / 256) * math.ceil(n / 256) < 256:
        return MID_GEMM_VARIANT
    return GEMM_VARIANT


def gemm(a, b, out=None, variant: Optional[str] = None):
    """``out[M, N] = a[M, K] @ b[K, N]`` in bf16 with fp32 accumulation.

    The default variant is the 256x256 tile; outputs with fewer 256x256
    tiles than CUs take 128x128 tiles and M <= 128 takes 128x32 tiles.
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
        variant = gemm_variant(m, n)
    kernels.handle(variant)(A=a, B=b, N=k, C_global=out)
    return out


def attention_forward(q, k, v, causal: bool = False, out=None, lse=None,
                      variant: Optional[str] = None) -> Tuple[object, object]:
    """FlashAttention forward over ``[B, H, S, D]`` bf16; returns ``(O, LSE)``.

    ``LSE[b, h, s] = logsumexp_j(q_s . k_j / sqrt(D))`` in fp32 (natural log).
    """
    import torch

    if q.dim() != 4 or q.shape != k.shape or k.shape != v.shape:
        raise ValueError("attention_forward: q, k, v must share one [B, H, S, D] shape")
    bsz, heads, seq, d = q.shape
    if variant is None:
        variant = {(128, False): "mha_d128", (64, True): "mha_d64_causal"}.get((d, causal))
        if variant is None:
            raise ValueError(f"attention_forward: no kernel variant for D={d}, causal={causal}")
    handle = kernels.handle(variant)
    kv_tile = next(o for o in _loops(handle.kernel)).tile_size
    if seq % kv_tile:
        raise ValueError(f"attention_forward: S={seq} must be a multiple of the KV tile {kv_tile}")
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty(bsz, heads, seq, dtype=torch.float32, device=q.device)
    handle(Q=q, K=k, V=v, N=seq, O=out, L=lse)
    return out, lse


def attention_flops(bsz: int, heads: int, seq: int, d: int, causal: bool = False) -> float:
    """Matmul FLOPs of attention forward: 4*B*H*S^2*D (halved when causal)."""
    f = 4.0 * bsz * heads * seq * seq * d
    return f / 2 if causal else f


def _loops(kernel):
    from warpir_amd.ir.ops import ForOp
    return (op for op in kernel.body if isinstance(op, ForOp))


__all__ = ["gemm", "gemm_variant", "attention_forward", "attention_flops"]
