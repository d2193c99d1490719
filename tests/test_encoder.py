"""TCQ Viterbi encoder (trellis.py:111-179): the GPU search against the
oracle restatement, bit for bit, and the quantizer's reference properties
(tests/test_trellis.py:29-89)."""

import math

import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O
from oracle.codebook_oracle import lloyd_max_gaussian, tcq_optimized_codebook, viterbi_full


def _walk(start: int, path_bits: np.ndarray, n_states: int) -> int:
    state = start
    for b in path_bits:
        state = ((state << 1) | int(b)) & (n_states - 1)
    return state


def test_oracle_viterbi_from_a_start_state_is_min_distortion():
    """Brute force over all 2^d paths from a given start state (d=6, S=8);
    the returned end state is where the returned path bits lead."""
    n_states, d = 8, 6
    cb = lloyd_max_gaussian(3)[0].to(torch.float32)
    gen = torch.Generator().manual_seed(11)
    z = torch.randn(4, d, generator=gen)
    start = torch.tensor([0, 3, 5, 7])
    level, path, _, end = viterbi_full(z, cb, n_states, start)
    got = ((cb[level.long()] - z) ** 2).sum(1)
    table = O.subset_table(n_states)
    for r in range(4):
        best = math.inf
        for p in range(1 << d):
            state, cost = int(start[r]), 0.0
            for t in range(d):
                b = (p >> t) & 1
                sub = table[state, b]
                cost += float(((cb[sub::4] - z[r, t]) ** 2).min())
                state = ((state << 1) | b) & (n_states - 1)
            best = min(best, cost)
        assert abs(float(got[r]) - best) < 1e-5
        assert int(end[r]) == _walk(int(start[r]), path[r].numpy(), n_states)


def _tie_rows(cb: torch.Tensor, d: int, gen) -> torch.Tensor:
    """Rows that hit the tie rules: zeros, exact subset midpoints and members,
    repeated values."""
    mids = []
    for j in range(4):
        sub = cb[j::4]
        mids += [float(v) for v in sub]
        mids += [float(v) for v in (sub[:-1] + sub[1:]) / 2.0]
    pool = torch.tensor(mids + [0.0], dtype=torch.float32)
    a = pool[torch.randint(0, pool.numel(), (d,), generator=gen)]
    return torch.stack([torch.zeros(d), a, torch.full((d,), float(pool[1]))])


@pytest.mark.gpu
@pytest.mark.parametrize("n_states", [4, 8, 16, 64])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_viterbi_bit_exact_against_oracle(cuda, n_states, bits):
    from turbopress_amd.encoder import viterbi
    gen = torch.Generator().manual_seed(100 * bits + n_states)
    cb = lloyd_max_gaussian(bits + 1)[0].to(torch.float32)
    d = 37
    z = torch.cat([torch.randn(5, d, generator=gen) * 1.3, _tie_rows(cb, d, gen)])
    start = torch.randint(0, n_states, (z.shape[0],), generator=gen)
    want = viterbi_full(z, cb, n_states, start)
    got = viterbi(z.to(cuda), cb, n_states, start)
    for w, g, name in zip(want, got, ("level", "path", "member", "end")):
        assert torch.equal(g.cpu().to(w.dtype), w), name
    # default start state 0
    want0 = viterbi_full(z, cb, n_states)
    got0 = viterbi(z.to(cuda), cb, n_states)
    assert torch.equal(got0[0].cpu(), want0[0]) and torch.equal(got0[3].cpu(), want0[3])


@pytest.mark.gpu
def test_viterbi_long_rows_and_odd_sizes(cuda):
    """d not a multiple of 16 or 64, a row count not a multiple of the rows per
    workgroup, the stored trellis codebook."""
    from turbopress_amd.encoder import viterbi
    gen = torch.Generator().manual_seed(7)
    cb = tcq_optimized_codebook(3, 64)
    for n, d in ((1, 1), (3, 15), (9, 130), (65, 1000)):
        z = torch.randn(n, d, generator=gen)
        want = viterbi_full(z, cb, 64)
        got = viterbi(z.to(cuda), cb, 64)
        for w, g in zip(want, got):
            assert torch.equal(g.cpu().to(w.dtype), w), (n, d)


@pytest.mark.gpu
def test_gpu_quantizer_round_trip_and_distortion(cuda):
    """tests/test_trellis.py:29-61: the stored bits rebuild the level codes,
    and 8-state TCQ at 2 bits beats the scalar Lloyd-Max optimum on N(0,1)
    without beating the rate-distortion bound."""
    from turbopress_amd.encoder import tcq_quantize_rows
    gen = torch.Generator().manual_seed(0)
    z = torch.randn(4, 8192, generator=gen)
    cb = tcq_optimized_codebook(2, 8)
    q = tcq_quantize_rows(z.to(cuda), bits=2, n_states=8, scale_iters=0, codebook=cb)
    rebuilt = O.decode_levels_sequential(q.path_bits.cpu().numpy(), q.member_codes.cpu().numpy(), 8)
    assert np.array_equal(rebuilt, q.level_codes.cpu().numpy())
    recon = q.codebook[q.level_codes.long()] * q.scales[:, None]
    mse = float((recon.cpu() - z).pow(2).mean())
    assert 0.0625 < mse < 0.96 * lloyd_max_gaussian(2)[1]


@pytest.mark.gpu
def test_gpu_quantizer_scale_refit_and_zero_rows(cuda):
    from turbopress_amd.encoder import tcq_quantize_rows
    gen = torch.Generator().manual_seed(2)
    w = torch.randn(6, 128, generator=gen) * 3.7
    w[3] = 0.0
    q = tcq_quantize_rows(w.to(cuda), bits=2, n_states=64)
    assert float(q.scales[3]) == 0.0
    assert torch.all(q.dequantize()[3] == 0.0)
    rel = float((q.dequantize().cpu() - w).norm() / w.norm())
    assert rel < 0.34
