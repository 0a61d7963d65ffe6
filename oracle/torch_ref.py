"""torch-CPU restatement of braid's reference decode step — TEST
INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg use it: tests pin it
to the scalar C oracle, and bench.py times it on the host's cores as the CPU
baseline of the headline step (the reference's own CPU path is its torch
form). The product path never imports it.

It restates, in torch on the CPU:

* the batched decode recurrence of braid/reference/gdn_ref.py:69-99
  (``gdn_decode_vectorized``): HF-additive l2 norm of q and k, the grouped
  head->group repeat, kv on the undecayed state, delta = (v - alpha kv) beta,
  the in-place state update, and y = (S' q_hat) * 128^-0.5;
* the gates of braid/model/gdn.py:299-300: beta = sigmoid in the activation
  dtype, then widened; alpha = exp(A * softplus(a + dt_bias)) in fp32;
* the slot-indexed pool of braid/kernels/csrc/gdn_decode.cu (rows gathered
  by slot, widened to fp32 for the step and narrowed back to the pool's
  storage type once).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

_L2_EPS = 1e-6


def _l2norm(x: torch.Tensor) -> torch.Tensor:
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + _L2_EPS)


def gates(a_raw: torch.Tensor, b_raw: torch.Tensor, A: torch.Tensor,
          dt_bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(alpha, beta) in fp32 from raw projections in the activation dtype."""
    beta = torch.sigmoid(b_raw).float()
    alpha = torch.exp(A * F.softplus(a_raw.float() + dt_bias))
    return alpha, beta


def decode_rows(state: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                alpha: torch.Tensor, beta: torch.Tensor) -> torch.Tensor:
    """One token on fp32 states [B, H, SS, HD] (updated in place); raw q, k
    [B, G, SS]; v [B, H, HD]; alpha, beta [B, H]. Returns y [B, H, HD]."""
    H, G = state.shape[1], q.shape[1]
    hpg = H // G
    qh = _l2norm(q).repeat_interleave(hpg, dim=1)
    kh = _l2norm(k).repeat_interleave(hpg, dim=1)
    a = alpha[..., None]
    bt = beta[..., None]
    kv = torch.einsum("bhsd,bhs->bhd", state, kh)
    delta = (v - a * kv) * bt
    state.mul_(a[..., None]).add_(kh[..., None] * delta[:, :, None, :])
    return torch.einsum("bhsd,bhs->bhd", state, qh) * (state.shape[-1] ** -0.5)


def decode_step(pool: torch.Tensor, slot_idx: torch.Tensor, q, k, v, a_raw, b_raw, A,
                dt_bias) -> torch.Tensor:
    """gdn_decode_raw's step on a CPU pool [S, H, SS, HD] of any float dtype,
    updated in place at slot_idx rows. Returns y [B, H, HD] fp32."""
    idx = slot_idx.long()
    state = pool.index_select(0, idx).float()
    alpha, beta = gates(a_raw, b_raw, A, dt_bias)
    y = decode_rows(state, q, k, v, alpha, beta)
    pool.index_copy_(0, idx, state.to(pool.dtype))
    return y
