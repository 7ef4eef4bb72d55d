"""TEST INFRASTRUCTURE -- numerical oracles (fp32; on the CPU, or on the GPU where a test
evaluates them at full size there with torch's own fp32 matmuls), never used by the product.

Follows the reference's checks:
* GEMM: ``torch.mm(A.float(), B.float())`` (``tests/test_modal_gpu.py:115``).
* attention: ``softmax(q @ k^T / sqrt(d)) @ v`` in fp32
  (``tests/test_modal_attention.py:92-98``), chunked over (batch, head)
  to bound the score matrix, with an optional causal mask
  (``kernel_examples/attention/mha_h100.cu:160-176``) and the natural-log
  log-sum-exp of the scaled scores.
* attention backward: the gradients of that fp32 forward by torch
  autograd (the reference has no backward oracle; its TK backward,
  ``mha_h100.cu:253-303,482-642``, is checked against torch autograd in
  the same way upstream).  Closed forms pinning it are in the tests.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch


def seeded_normal(shape, seed: int, scale: float = 1.0) -> torch.Tensor:
    """``N(0,1) * scale`` from ``torch.Generator().manual_seed(seed)`` on CPU, as bf16."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * scale).to(torch.bfloat16)


def gemm_ref(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """fp32 ``A @ B`` of bf16 inputs (``tests/test_modal_gpu.py:115``)."""
    return torch.matmul(a.float(), b.float())


def attention_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: Optional[float] = None,
                  causal: bool = False, heads: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Naive fp32 attention over ``[..., S, D]`` on the inputs' device; returns ``(O, LSE)``.

    ``LSE[..., s] = logsumexp_j(q_s . k_j * scale)`` (natural log).  With
    ``heads`` set, only the first ``heads`` of the flattened (batch, head)
    rows are computed (a bounded CPU sample).
    """
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    lead = q.shape[:-2]
    qf = q.reshape(-1, q.shape[-2], d)
    kf = k.reshape(-1, k.shape[-2], d)
    vf = v.reshape(-1, v.shape[-2], v.shape[-1])
    n = qf.shape[0] if heads is None else min(heads, qf.shape[0])
    outs, lses = [], []
    for h in range(n):
        s = (qf[h].float() @ kf[h].float().t()) * scale
        if causal:
            sq, sk = s.shape
            mask = torch.ones(sq, sk, dtype=torch.bool, device=s.device).tril_(diagonal=sk - sq)
            s = s.masked_fill(~mask, float("-inf"))
        lses.append(torch.logsumexp(s, dim=-1))
        outs.append(torch.softmax(s, dim=-1) @ vf[h].float())
    o = torch.stack(outs)
    lse = torch.stack(lses)
    if heads is None:
        o = o.reshape(*lead, q.shape[-2], v.shape[-1])
        lse = lse.reshape(*lead, q.shape[-2])
    return o, lse


def attention_bwd_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, do: torch.Tensor,
                      scale: Optional[float] = None, causal: bool = False):
    """``(dQ, dK, dV)`` of ``sum(softmax(q k^T * scale) v * do)`` in fp32 on the inputs'
    device, by autograd over ``[..., S, D]`` inputs (per leading index, to bound memory)."""
    scale = scale if scale is not None else 1.0 / math.sqrt(q.shape[-1])
    lead = q.shape[:-2]
    qf, kf, vf, dof = (t.float().reshape(-1, *t.shape[-2:]) for t in (q, k, v, do))
    outs = ([], [], [])
    for n in range(qf.shape[0]):
        qn, kn, vn = (t[n].clone().requires_grad_(True) for t in (qf, kf, vf))
        s = (qn @ kn.t()) * scale
        if causal:
            rows, cols = s.shape
            s = s.masked_fill(torch.ones(rows, cols, dtype=torch.bool, device=s.device).triu(1), float("-inf"))
        o = torch.softmax(s, dim=-1) @ vn
        o.backward(dof[n])
        for acc, t in zip(outs, (qn, kn, vn)):
            acc.append(t.grad.detach())
    return tuple(torch.stack(a).reshape(*lead, *a[0].shape) for a in outs)


def attention_bwd_ref_bf16(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                           do: torch.Tensor, scale: Optional[float] = None, causal: bool = False,
                           round_operands: bool = True):
    """``(dQ, dK, dV)`` with the reference backward's bf16 MMA operands
    (``kernel_examples/attention/mha_h100.cu:418-448``, dQ ``:132``): P = exp(S - LSE)
    rounded to bf16 for ``dV = P^T dO`` (``:436, :443``); ``dS = P (dP - D)`` times the
    softmax scale, rounded to bf16 for ``dK = dS^T Q`` and ``dQ = dS K`` (``:438-448``);
    ``D = rowsum(dO * O)`` from the given (stored) O.  fp32 elsewhere, on the inputs' device,
    per leading index.  ``round_operands=False`` is the exact gradient (equal to
    ``attention_bwd_ref`` when ``o`` is the exact output)."""
    scale = scale if scale is not None else 1.0 / math.sqrt(q.shape[-1])
    rnd = (lambda t: t.to(torch.bfloat16).float()) if round_operands else (lambda t: t)
    lead = q.shape[:-2]
    qf, kf, vf, of, dof = (t.float().reshape(-1, *t.shape[-2:]) for t in (q, k, v, o, do))
    outs = ([], [], [])
    for n in range(qf.shape[0]):
        s = (qf[n] @ kf[n].t().contiguous()) * scale
        if causal:
            rows, cols = s.shape
            s = s.masked_fill(torch.ones(rows, cols, dtype=torch.bool, device=s.device).triu(1), float("-inf"))
        p = torch.softmax(s, dim=-1)
        dv = rnd(p).t().contiguous() @ dof[n]
        dp = dof[n] @ vf[n].t().contiguous()
        d = (dof[n] * of[n]).sum(-1, keepdim=True)
        ds = rnd(p * (dp - d) * scale)
        outs[0].append(ds @ kf[n])
        outs[1].append(ds.t().contiguous() @ qf[n])
        outs[2].append(dv)
    return tuple(torch.stack(a).reshape(*lead, *a[0].shape) for a in outs)


def rel_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    """``max|out - ref| / max|ref|`` -- the acceptance metric (bar: 1e-2)."""
    out, ref = out.float(), ref.float()
    denom = ref.abs().max().item()
    return (out - ref).abs().max().item() / (denom if denom > 0 else 1.0)
