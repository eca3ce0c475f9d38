"""CPU oracle for the RWKV-7 DPLR recurrence (test infrastructure).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s baseline leg; never by the product package.

Recurrence, per (batch, head), head size N, state S [N_v, N_k]::

    S_t = S_{t-1} (diag(w_t) + a_t b_t^T) + v_t k_t^T,    y_t = S_t r_t

(the formula of the benchmark configuration; the reference's own RWKV-7 code
was deleted, ``benchmarks/results/optimizer_wkv_experiments_5090.md:3``, and
its arithmetic lived in the unpinned external ``fla`` package).  PARITY
UNPINNED against the reference: there is no reference implementation, test or
fixture to compare with.  What pins this restatement is mathematics only
(``tests/test_oracle_wkv7.py``):

* with a = b = 0 it must equal causal (decayed) linear attention computed as
  a masked matrix product;
* the low-rank term on hand-computed one-hot states: S = e_i e_j^T,
  a = e_j, b = e_m, w = 0, v = k = 0 gives S' = e_i e_m^T (the order
  (S a) b^T, not (S b) a^T);
* the delta-rule identity: w = 1, a = -kappa, b = kappa, r = kappa with unit
  kappa gives y_t = v_t (k_t . kappa_t) from any state (output on the
  post-update state);
* :func:`wkv7_matrix_form` (numpy, explicit 64x64 transition matrices
  diag(w) + a b^T and a matrix product per step) for a and b drawn
  independently (:func:`make_general_inputs`);
* autograd through it agrees with central finite differences and with the
  explicit reverse recurrence, and the state carried across a split of the
  sequence reproduces the unsplit run;
* planted mistakes ((S b) a^T, output before the update, decay on the value
  index) each fail one of the checks above.
"""

from __future__ import annotations

import torch
from torch import Tensor


def wkv7_loop(
    r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor, state: Tensor | None = None
) -> tuple[Tensor, Tensor]:
    """Sequential recurrence in the inputs' dtype.

    Inputs ``[B, T, H, N]``; ``state`` ``[B, H, N, N]`` (rows: value index,
    columns: key index) or None for zeros.  Returns ``(y [B,T,H,N], S_T)``.
    """
    bsz, steps, heads, n = r.shape
    dt = r.dtype
    s = torch.zeros((bsz, heads, n, n), dtype=dt) if state is None else state.to(dt).clone()
    ys = []
    for t in range(steps):
        rt, wt, kt, vt, at, bt = (x[:, t] for x in (r, w, k, v, a, b))  # [B, H, N]
        sa = torch.einsum("bhij,bhj->bhi", s, at)
        s = s * wt[:, :, None, :] + sa[..., :, None] * bt[:, :, None, :] + vt[..., :, None] * kt[:, :, None, :]
        ys.append(torch.einsum("bhij,bhj->bhi", s, rt))
    y = torch.stack(ys, dim=1) if steps else r.new_empty(r.shape)
    return y, s


def linear_attention(r: Tensor, w: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """Closed form of the a = b = 0 case as a masked matrix product.

    ``y_t[i] = sum_{s<=t} v_s[i] * sum_j k_s[j] r_t[j] prod_{s<u<=t} w_u[j]``,
    evaluated with cumulative log-decays (requires w > 0).
    """
    logw = torch.log(w)
    cum = torch.cumsum(logw, dim=1)  # [B,T,H,N]: sum_{u<=t} log w_u
    # decay from step s (exclusive) to t (inclusive): exp(cum_t - cum_s)
    dec = torch.exp(cum[:, :, None] - cum[:, None, :])  # [B, t, s, H, N]
    steps = r.shape[1]
    mask = torch.tril(torch.ones(steps, steps, dtype=torch.bool))
    scores = torch.einsum("bthj,btshj,bshj->bhts", r, dec, k)
    scores = scores.masked_fill(~mask[None, None], 0.0)
    return torch.einsum("bhts,bshi->bthi", scores, v)


def make_inputs(batch: int, steps: int, heads: int, n: int = 64, *, seed: int, dtype=torch.float32):
    """Seeded inputs with the benchmark distributions, drawn in this order:
    x ~ N(-0.5, 1) -> w = exp(-exp(x)); r, k, v ~ N(0, 1); kappa ~ N(0, 1)
    L2-normalised over each head's N channels; iclr = sigmoid(N(0, 1));
    a = -kappa, b = kappa * iclr.  Returns ``(r, w, k, v, a, b)`` in ``dtype``.
    """
    g = torch.Generator().manual_seed(seed)
    shape = (batch, steps, heads, n)
    x = torch.randn(shape, generator=g) - 0.5
    w = torch.exp(-torch.exp(x))
    r = torch.randn(shape, generator=g)
    k = torch.randn(shape, generator=g)
    v = torch.randn(shape, generator=g)
    kappa = torch.randn(shape, generator=g)
    kappa = kappa / kappa.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    iclr = torch.sigmoid(torch.randn(shape, generator=g))
    a = -kappa
    b = kappa * iclr
    return tuple(t.to(dtype) for t in (r, w, k, v, a, b))


def make_general_inputs(batch: int, steps: int, heads: int, n: int = 64, *, seed: int,
                        dtype=torch.float32):
    """As :func:`make_inputs`, but with a and b along independent directions:
    ``a = -kappa_a``, ``b = kappa_b * iclr`` with ``kappa_a``, ``kappa_b`` two
    independent unit vectors per head.  ``a b^T`` is then not symmetric, so
    ``(S a) b^T`` and ``(S b) a^T`` differ on these inputs (with ``a``
    parallel to ``b`` they coincide).  ``|a| = 1`` and ``|b| <= 1`` keep the
    state bounded over long sequences."""
    g = torch.Generator().manual_seed(seed)
    shape = (batch, steps, heads, n)
    x = torch.randn(shape, generator=g) - 0.5
    w = torch.exp(-torch.exp(x))
    r = torch.randn(shape, generator=g)
    k = torch.randn(shape, generator=g)
    v = torch.randn(shape, generator=g)
    ka = torch.randn(shape, generator=g)
    ka = ka / ka.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    kb = torch.randn(shape, generator=g)
    kb = kb / kb.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    iclr = torch.sigmoid(torch.randn(shape, generator=g))
    return tuple(t.to(dtype) for t in (r, w, k, v, -ka, kb * iclr))


def wkv7_matrix_form(r, w, k, v, a, b, state=None):
    """The recurrence as explicit matrices, in numpy float64: per step the
    transition ``M_t = diag(w_t) + outer(a_t, b_t)`` is built and
    ``S_t = S_{t-1} @ M_t + outer(v_t, k_t)``, ``y_t = S_t @ r_t``.  A second
    formulation, sharing no code with :func:`wkv7_loop`.  Inputs as
    :func:`wkv7_loop` (torch or numpy); returns numpy ``(y, S_T)``."""
    import numpy as np

    r, w, k, v, a, b = (np.asarray(x, dtype=np.float64) for x in (r, w, k, v, a, b))
    bsz, steps, heads, n = r.shape
    y = np.zeros_like(r)
    s_out = np.zeros((bsz, heads, n, n))
    for bi in range(bsz):
        for h in range(heads):
            s = np.zeros((n, n)) if state is None else np.asarray(state, dtype=np.float64)[bi, h].copy()
            for t in range(steps):
                m = np.diag(w[bi, t, h]) + np.outer(a[bi, t, h], b[bi, t, h])
                s = s @ m + np.outer(v[bi, t, h], k[bi, t, h])
                y[bi, t, h] = s @ r[bi, t, h]
            s_out[bi, h] = s
    return y, s_out


def wkv7_autograd_grads(r, w, k, v, a, b, state, gy, gs=None):
    """Gradients of ``sum(y * gy) + sum(S_T * gs)`` by torch autograd through
    :func:`wkv7_loop` (in the inputs' dtype, normally float64).  Returns
    ``(y, S_T, dr, dw, dk, dv, da, db, d_state)``."""
    leaves = [x.detach().clone().requires_grad_(True) for x in (r, w, k, v, a, b)]
    s0 = None if state is None else state.detach().clone().requires_grad_(True)
    y, s = wkv7_loop(*leaves, state=s0)
    loss = (y * gy).sum()
    if gs is not None:
        loss = loss + (s * gs).sum()
    wrt = leaves + ([s0] if s0 is not None else [])
    grads = torch.autograd.grad(loss, wrt, allow_unused=True)
    grads = [torch.zeros_like(x) if g is None else g for g, x in zip(grads, wrt)]
    ds0 = grads[6] if s0 is not None else None
    return (y.detach(), s.detach(), *grads[:6], ds0)


def wkv7_backward_loop(r, w, k, v, a, b, state, gy, gs=None):
    """The explicit reverse recurrence (a second formulation of the gradients,
    the one the HIP backward evaluates), with G = dL/dS_t::

        G += dy_t r_t^T;       dr_t = S_t^T dy_t
        c  = G b_t;            dv_t = G k_t;   dk_t = G^T v_t;  db_t = G^T (S_{t-1} a_t)
        dw_t = colsum(G o S_{t-1});            da_t = S_{t-1}^T c
        G  = G diag(w_t) + c a_t^T             (after t = 0: dL/dS_0)

    Forward states are stored for every step (small inputs only).  Returns
    ``(dr, dw, dk, dv, da, db, d_state)``.
    """
    bsz, steps, heads, n = r.shape
    dt = r.dtype
    s = torch.zeros((bsz, heads, n, n), dtype=dt) if state is None else state.to(dt).clone()
    states = [s]
    sas = []
    for t in range(steps):
        rt, wt, kt, vt, at, bt = (x[:, t] for x in (r, w, k, v, a, b))
        sa = (s * at[:, :, None, :]).sum(-1)
        sas.append(sa)
        s = s * wt[:, :, None, :] + sa[..., :, None] * bt[:, :, None, :] + vt[..., :, None] * kt[:, :, None, :]
        states.append(s)
    g = torch.zeros((bsz, heads, n, n), dtype=dt) if gs is None else gs.to(dt).clone()
    outs = [torch.zeros_like(r) for _ in range(6)]
    dr, dw, dk, dv, da, db = outs
    for t in range(steps - 1, -1, -1):
        rt, wt, kt, vt, at, bt, dyt = (x[:, t] for x in (r, w, k, v, a, b, gy))
        s_t, s_prev = states[t + 1], states[t]
        g = g + dyt[..., :, None] * rt[:, :, None, :]
        dr[:, t] = (s_t * dyt[..., :, None]).sum(-2)
        c = (g * bt[:, :, None, :]).sum(-1)
        dv[:, t] = (g * kt[:, :, None, :]).sum(-1)
        dk[:, t] = (g * vt[..., :, None]).sum(-2)
        db[:, t] = (g * sas[t][..., :, None]).sum(-2)
        dw[:, t] = (g * s_prev).sum(-2)
        da[:, t] = (s_prev * c[..., :, None]).sum(-2)
        g = g * wt[:, :, None, :] + c[..., :, None] * at[:, :, None, :]
    return (*outs, g)
