"""tp_packed_linear_forward_noalloc (the forward whose split-K workspace is a
fixed device array inside the library) against tp_packed_linear_forward with
a caller workspace, through the C ABI (GPU)."""

import pytest
import torch

from oracle import tcq_oracle as O
from turbopress_amd import hip_kernel as hk
from turbopress_amd.synthetic import make_activation, make_payload, payload_numpy

pytestmark = pytest.mark.gpu

GEMV_TOL = 2e-3


def _call(lib, fn, lin, x, ws=None):
    n, d = lin.out_features, lin.in_features
    y = torch.full((x.shape[0], n), float("nan"), dtype=torch.float16, device=x.device)
    buf, pb = lin.tiled_packed, lin._tiled_geo["path_bytes"]
    args = [x.data_ptr(), d, x.shape[0], lin.rot_scale.data_ptr(), lin.block, buf.data_ptr(), buf.data_ptr() + pb,
            lin.scales.data_ptr(), lin.codebook.data_ptr(), 0 if lin.bias is None else lin.bias.data_ptr(),
            n, d, lin.bits, lin.n_states, y.data_ptr(), n]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    st = getattr(lib, fn)(*args, torch.cuda.current_stream(x.device).cuda_stream)
    assert st == 0, (fn, st)
    return y


def test_noalloc_matches_workspace_entry_point(cuda):
    """Two calls in a row on the shared device array, the second smaller (it
    must not see the first one's sums), then a batch-1 call; each against
    the existing entry point with its own workspace and against the oracle."""
    from turbopress_amd import _lib
    from turbopress_amd.runtime import PackedTCQLinear
    lib = _lib.lib()
    # (n, d, batch, bits): split-K at batch 12, then a smaller batch-6 call;
    # batch 1 (one-pass, no workspace); down_proj at batch 4 (K cut into
    # parts summed through the array); 1024-column Hadamard blocks at batch
    # 4 (the split-K kernel at batch <= 4); 32768 rows at batch 16 (the
    # array's documented limit: the wide kernel's sums fill it exactly)
    cases = [(9728, 2560, 12, 3), (1024, 2560, 6, 4), (2560, 9728, 1, 3), (2560, 9728, 4, 3),
             (512, 4096, 4, 3), (32768, 2560, 16, 3), (2560, 9728, 2, 2)]
    for i, (n, d, batch, bits) in enumerate(cases):
        p = make_payload(n, d, bits, 64, seed=70 + i, bias=(i == 1))
        lin = PackedTCQLinear(p, mode="hip")
        x = make_activation(batch, d, seed=80 + i).to(cuda)
        y_ref = _call(lib, "tp_packed_linear_forward", lin, x, hk.gemv_workspace(n, 32, cuda))
        y = _call(lib, "tp_packed_linear_forward_noalloc", lin, x)
        torch.cuda.synchronize()
        ref = y_ref.float()
        assert float((y.float() - ref).abs().max() / ref.abs().max()) <= GEMV_TOL, (i, n, d, batch)
        oracle = O.tiled_forward(payload_numpy(p), x.cpu().numpy())
        assert O.max_rel(y.float().cpu().numpy(), oracle) <= GEMV_TOL, (i, n, d, batch)
        # the same call again on what this call left in the array
        y2 = _call(lib, "tp_packed_linear_forward_noalloc", lin, x)
        torch.cuda.synchronize()
        assert float((y2.float() - ref).abs().max() / ref.abs().max()) <= GEMV_TOL, (i, "repeat")
