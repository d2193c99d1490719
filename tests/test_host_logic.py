"""Host-side logic that needs no GPU: the shared-input group's output holds
and the shared split-K workspace bookkeeping (the kernels are replaced by
counting stand-ins)."""

import pytest
import torch

from turbopress_amd import decode_step
from turbopress_amd import hip_kernel as hk


class _FakeGroupLaunch:
    """Stands in for hip_kernel.forward_group: member i's output is
    x * (i + 1) + launch number, so a held output from an earlier launch is
    told apart from a fresh one."""

    def __init__(self):
        self.launches = 0

    def __call__(self, members, x):
        self.launches += 1
        return [x * (i + 1) + self.launches for i in range(len(members))]


@pytest.fixture
def fake_group(monkeypatch):
    fake = _FakeGroupLaunch()
    monkeypatch.setattr(decode_step.hk, "forward_group", fake)
    return fake


def test_shared_input_group_serves_members_in_order(fake_group):
    g = decode_step.SharedInputGroup(["q", "k", "v"])
    x = torch.ones(2, 4)
    outs = [g.run(i, x) for i in range(3)]
    assert fake_group.launches == 1
    for i, o in enumerate(outs):
        assert torch.equal(o, x * (i + 1) + 1)


def test_shared_input_group_skipped_member_gets_no_stale_output(fake_group):
    """Under inference mode a rewritten input buffer has the same storage and
    no version counter.  A member skipped in one pass must not take that
    pass's output in the next."""
    g = decode_step.SharedInputGroup(["q", "k", "v"])
    with torch.inference_mode():
        x = torch.ones(1, 4)
        g.run(0, x)
        g.run(1, x)          # v skipped in this pass
        x.fill_(5.0)         # next step: same buffer, new activations
        q = g.run(0, x)      # a new pass starts at q: the group runs again
        assert fake_group.launches == 2
        v = g.run(2, x)
        assert torch.equal(q, x * 1 + 2) and torch.equal(v, x * 3 + 2)


def test_shared_input_group_reruns_for_out_of_order_member(fake_group):
    g = decode_step.SharedInputGroup(["gate", "up"])
    with torch.inference_mode():
        x = torch.ones(1, 4)
        g.run(1, x)          # up first: nothing after it to hold
        g.run(0, x)          # gate at or before the last served: runs again
    assert fake_group.launches == 2


def test_group_workspace_regions_are_disjoint(monkeypatch):
    """A grouped launch's members get disjoint, 256-byte aligned regions of
    the one shared workspace; a larger need replaces the buffer and keeps the
    old one alive (a captured graph may still name it)."""
    made = []

    def fake_shared(device, nbytes):
        made.append(nbytes)
        return torch.zeros(max(nbytes, 1), dtype=torch.uint8)

    monkeypatch.setattr(hk, "shared_workspace", fake_shared)

    class L:
        def __init__(self, a, b):
            self._ws_bytes = (a, b)
            self.tiled_packed = torch.zeros(1)

    ptrs, sizes = hk.group_workspaces([L(100, 200), L(300, 600), L(5, 9)], batch=24)
    assert sizes == [200, 600, 9]
    assert made == [256 + 768 + 256]
    base = ptrs[0]
    assert [p - base for p in ptrs] == [0, 256, 1024]
    ptrs, sizes = hk.group_workspaces([L(100, 200)], batch=8)
    assert sizes == [100]


def test_shared_workspace_grows_and_retires(monkeypatch):
    """Keyed by (device, stream); growth keeps the retired buffer referenced."""
    monkeypatch.setattr(hk, "_WORKSPACES", {})
    monkeypatch.setattr(hk, "_RETIRED_WORKSPACES", [])

    class S:
        cuda_stream = 1234

    monkeypatch.setattr(hk.torch.cuda, "current_stream", lambda index=None: S())
    monkeypatch.setattr(hk.torch, "zeros", lambda n, dtype, device: torch.empty(n, dtype=dtype))
    a = hk.shared_workspace("cuda:0", 1000)
    assert a.numel() == 1024
    assert hk.shared_workspace("cuda:0", 500) is a
    b = hk.shared_workspace("cuda:0", 5000)
    assert b.numel() == 5120 and hk._RETIRED_WORKSPACES == [a]


def _lin_recip(d: int) -> int:
    """The per-linear kernel's reciprocal for wave-uniform divisions
    (``lin_recip`` in turbopress_amd/csrc/tp_linear.hip): ceil(2^32 / d),
    0 standing for d = 1."""
    return 0 if d <= 1 else -(-(1 << 32) // d)


def test_reciprocal_division_is_exact_below_its_bound():
    """udiv_recip(x, lin_recip(d)) = x // d whenever x * d < 2^32 (its
    stated bound): every x < 2^16 for d <= 1024, and the largest x the bound
    allows for d up to 2^16 (where a reciprocal rounded the other way, or a
    bound one too loose, gives x // d + 1 or - 1)."""
    import numpy as np

    def udiv(x, d):
        m = _lin_recip(d)
        return x if m == 0 else (x.astype(np.uint64) * np.uint64(m)) >> np.uint64(32)

    x = np.arange(1 << 16, dtype=np.uint64)
    for d in range(1, 1025):
        ok = x * np.uint64(d) < np.uint64(1 << 32)
        assert np.array_equal(udiv(x[ok], d), x[ok] // np.uint64(d)), d
    rng = np.random.default_rng(7)
    for d in list(range(1025, 1100)) + [int(v) for v in rng.integers(1100, 1 << 16, 2000)]:
        top = ((1 << 32) - 1) // d
        xs = np.array([top, top - 1, top - d + 1, (top // d) * d, (top // d) * d - 1], dtype=np.uint64)
        xs = xs[xs * np.uint64(d) < np.uint64(1 << 32)]
        assert np.array_equal(udiv(xs, d), xs // np.uint64(d)), d
