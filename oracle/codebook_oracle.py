"""torch-CPU restatement of the reference's codebook producers (TEST ORACLE).

Test infrastructure only (see ``oracle/__init__.py``).

The trellis-optimised codebook is data to the decode path: its fp16 values
depend on torch's CPU ``randn`` stream for ``Generator().manual_seed(seed)``,
on ``bucketize``, on ``index_add_`` summation order and on the Viterbi
tie-break, so this restatement uses the same torch calls in the same order.

  * ``lloyd_max_gaussian``      codebooks.py:45-81
  * ``viterbi`` / ``viterbi_full``  trellis.py:111-179
  * ``tcq_optimized_codebook``  trellis.py:206-253  (65536 samples, 8 iters)
  * ``pipeline_tcq_codebook``   pipeline.py:282-301  (8x8192 samples, 6 iters,
                                built from pipeline.py's own Lloyd-Max copy)
  * ``rademacher_signs``        hadamard.py:76-80

Pinning: ``lloyd_max_gaussian`` against the closed forms in
``tests/test_codebooks.py:9-33``; the trellis codebooks and signs against the
golden vectors in ``tests/golden/`` (written by importing the reference in
the build container, see ``tests/golden/make_golden.py``); ``viterbi``
against the window decode (its level codes must equal the decode of its own
path/member bits, ``tests/test_runtime.py:28-42``) and against brute-force
minimum-distortion search on tiny rows.
"""

from __future__ import annotations

import math

import torch

from oracle.tcq_oracle import GENERATORS, N_SUBSETS, subset_table

_SQRT_2PI = math.sqrt(2.0 * math.pi)
_SQRT_2 = math.sqrt(2.0)


def lloyd_max_gaussian(bits: int, max_iters: int = 100_000, tol: float = 1e-12):
    """codebooks.py:45-81: Lloyd iteration to the optimal 2**bits-level
    quantiser of N(0,1), float64; returns (levels, mse)."""
    if not isinstance(bits, int) or not 1 <= bits <= 8:
        raise ValueError(f"bits must be an int in [1, 8], got {bits!r}")
    n = 1 << bits
    p = (torch.arange(n, dtype=torch.float64) + 0.5) / n
    c = _SQRT_2 * torch.erfinv(2.0 * p - 1.0)
    inf = torch.tensor([math.inf], dtype=torch.float64)
    mse = math.inf
    for _ in range(max_iters):
        t = torch.cat([-inf, (c[:-1] + c[1:]) / 2.0, inf])
        big_phi = 0.5 * (1.0 + torch.erf(t / _SQRT_2))
        phi = torch.exp(-0.5 * t * t) / _SQRT_2PI
        mass = big_phi[1:] - big_phi[:-1]
        c_new = (phi[:-1] - phi[1:]) / mass
        mse = 1.0 - float((mass * c_new * c_new).sum())
        moved = float((c_new - c).abs().max())
        c = c_new
        if moved < tol:
            break
    return c, mse


def _pipeline_lloyd_max(bits: int, iters: int = 100_000, tol: float = 1e-12) -> torch.Tensor:
    """pipeline.py:165-181's copy of the Lloyd-Max iteration used by
    ``pipeline.tcq_codebook``: same fixed point, but the cell mass is formed
    as 0.5*(erf(b/sqrt2) - erf(a/sqrt2)) rather than Phi(b) - Phi(a)."""
    n = 1 << bits
    p = (torch.arange(n, dtype=torch.float64) + 0.5) / n
    c = _SQRT_2 * torch.erfinv(2.0 * p - 1.0)
    inf = torch.tensor([math.inf], dtype=torch.float64)
    for _ in range(iters):
        t = torch.cat([-inf, (c[:-1] + c[1:]) / 2, inf])
        mass = 0.5 * (torch.erf(t[1:] / _SQRT_2) - torch.erf(t[:-1] / _SQRT_2))
        phi = torch.exp(-0.5 * t * t) / _SQRT_2PI
        c_new = (phi[:-1] - phi[1:]) / mass
        moved = float((c_new - c).abs().max())
        c = c_new
        if moved < tol:
            break
    return c


class _Tables:
    """trellis.py:64-87: predecessor and branch-subset tables."""

    def __init__(self, n_states: int) -> None:
        self.n_states = n_states
        sub = torch.from_numpy(subset_table(n_states))
        ns = torch.arange(n_states)
        self.prev0 = ns >> 1
        self.prev1 = (ns >> 1) | (n_states >> 1)
        bit = ns & 1
        self.sub0 = sub[self.prev0, bit]
        self.sub1 = sub[self.prev1, bit]


def viterbi(z: torch.Tensor, codebook: torch.Tensor, n_states: int):
    """trellis.py:111-179: minimum-distortion trellis path per row from state 0.
    Returns (level_codes, path_bits, member_codes) as uint8 [n, d]."""
    level, pathb, memb, _ = viterbi_full(z, codebook, n_states)
    return level, pathb, memb


def viterbi_full(z: torch.Tensor, codebook: torch.Tensor, n_states: int,
                 start_state: torch.Tensor | None = None):
    """trellis.py:128-179 with its optional start state and returned end
    state: (level_codes, path_bits, member_codes, end_state)."""
    tr = _Tables(n_states)
    n, d = z.shape
    members = torch.empty(n, d, N_SUBSETS, dtype=torch.int64)
    costs = torch.empty(n, d, N_SUBSETS, dtype=torch.float32)
    for j in range(N_SUBSETS):
        sub_cb = codebook[j::N_SUBSETS]
        if sub_cb.numel() == 1:
            mem = torch.zeros(n, d, dtype=torch.int64)
        else:
            thresholds = (sub_cb[:-1] + sub_cb[1:]) / 2.0
            mem = torch.bucketize(z.contiguous(), thresholds)
        members[:, :, j] = mem
        costs[:, :, j] = (z - sub_cb[mem]).pow(2)
    alpha = torch.full((n, n_states), torch.inf)
    if start_state is None:
        alpha[:, 0] = 0.0
    else:
        alpha[torch.arange(n), start_state.long()] = 0.0
    bp = torch.empty(n, d, n_states, dtype=torch.bool)
    for t in range(d):
        c = costs[:, t, :]
        cand0 = alpha[:, tr.prev0] + c[:, tr.sub0]
        cand1 = alpha[:, tr.prev1] + c[:, tr.sub1]
        take1 = cand1 < cand0
        alpha = torch.where(take1, cand1, cand0)
        bp[:, t, :] = take1
    level = torch.empty(n, d, dtype=torch.uint8)
    pathb = torch.empty(n, d, dtype=torch.uint8)
    memb = torch.empty(n, d, dtype=torch.uint8)
    rows = torch.arange(n)
    state = alpha.argmin(dim=1)
    end_state = state.clone()
    for t in range(d - 1, -1, -1):
        take1 = bp[rows, t, state]
        prev = torch.where(take1, tr.prev1[state], tr.prev0[state])
        sub = torch.where(take1, tr.sub1[state], tr.sub0[state])
        mem = members[rows, t, sub]
        pathb[:, t] = (state & 1).to(torch.uint8)
        memb[:, t] = mem.to(torch.uint8)
        level[:, t] = (mem * N_SUBSETS + sub).to(torch.uint8)
        state = prev
    return level, pathb, memb, end_state


def _lloyd_under_trellis(codebook: torch.Tensor, z: torch.Tensor, n_states: int,
                         iters: int) -> torch.Tensor:
    """Generalised Lloyd with Viterbi assignments (trellis.py:239-250,
    pipeline.py:292-299): move each level to the mean of its samples, then
    re-sort every subset slice."""
    for _ in range(iters):
        level_codes, _, _ = viterbi(z, codebook, n_states)
        flat_codes = level_codes.long().flatten()
        flat_z = z.flatten()
        n_levels = codebook.numel()
        sums = torch.zeros(n_levels).index_add_(0, flat_codes, flat_z)
        counts = torch.zeros(n_levels).index_add_(0, flat_codes, torch.ones_like(flat_z))
        codebook = torch.where(counts > 0, sums / counts.clamp_min(1.0), codebook)
        for j in range(N_SUBSETS):
            codebook[j::N_SUBSETS] = codebook[j::N_SUBSETS].sort().values
    return codebook


def tcq_optimized_codebook(bits: int, n_states: int, n_samples: int = 1 << 16,
                           iters: int = 8, seed: int = 0) -> torch.Tensor:
    """trellis.py:206-253 (the codebook ``pack_linear`` stores): fp32 [2**(bits+1)]."""
    if n_states not in GENERATORS:
        raise ValueError(f"n_states must be one of {sorted(GENERATORS)}")
    codebook = lloyd_max_gaussian(bits + 1)[0].to(torch.float32)
    gen = torch.Generator().manual_seed(seed)
    n_rows = 8
    z = torch.randn(n_rows, n_samples // n_rows, generator=gen)
    return _lloyd_under_trellis(codebook, z, n_states, iters)


def pipeline_tcq_codebook(bits: int, n_states: int, iters: int = 6, seed: int = 0) -> torch.Tensor:
    """pipeline.py:282-301 (the codebook format-v1 artifacts store): fp32."""
    codebook = _pipeline_lloyd_max(bits + 1).to(torch.float32)
    gen = torch.Generator().manual_seed(seed)
    z = torch.randn(8, 8192, generator=gen)
    return _lloyd_under_trellis(codebook, z, n_states, iters)


def rademacher_signs(dim: int, seed: int) -> torch.Tensor:
    """hadamard.py:76-80: int64 0/1 draws from Generator(seed) (+-1 = 2*b-1)."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(0, 2, (dim,), generator=gen, dtype=torch.int64)
