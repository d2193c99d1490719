"""pack_linear / pack_model (nn.Linear -> format-v2 payload) against the
reference's own outputs (tests/golden/pack_linear.json, written by
tests/golden/make_pack_golden.py from turbopress.runtime.pack_linear)."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "pack_linear.json").read_text())


def _f32(bits):
    return torch.tensor(bits, dtype=torch.int64).to(torch.int32).view(torch.float32)


def _case_linear(c):
    from torch import nn
    n, d = c["n"], c["d"]
    lin = nn.Linear(d, n, bias=c["bias_f32"] is not None)
    with torch.no_grad():
        lin.weight.copy_(_f32(c["weight_f32"]).reshape(n, d))
        if c["bias_f32"] is not None:
            lin.bias.copy_(_f32(c["bias_f32"]))
    return lin, _f32(c["act_rms_f32"])


def _f16_bits(t):
    return t.to(torch.float16).contiguous().view(torch.int16).to(torch.int32).bitwise_and(0xFFFF).tolist()


@pytest.mark.parametrize("width", [1, 2, 3, 5, 8])
def test_pack_rows_le_round_trips_through_oracle(width):
    from turbopress_amd.pack import pack_rows_le
    rng = np.random.default_rng(width)
    for n, d in ((3, 1), (4, 7), (2, 77), (5, 256)):
        vals = rng.integers(0, 1 << width, size=(n, d), dtype=np.uint8)
        packed = pack_rows_le(torch.from_numpy(vals), width).numpy()
        assert packed.shape == (n, (d * width + 7) // 8)
        assert np.array_equal(O.unpack_le(packed, d, width), vals)
        assert np.array_equal(packed, O.pack_le(vals, width))


def test_pack_rows_le_known_answer():
    from turbopress_amd.pack import pack_rows_le
    # values 1, 2, 3 at width 2 -> stream bits 10 01 11 -> byte 0b00111001
    assert pack_rows_le(torch.tensor([[1, 2, 3]], dtype=torch.uint8), 2).tolist() == [[0b00111001]]


def test_block_hadamard_rows_matches_oracle_and_dense_matrix():
    from turbopress_amd.pack import block_hadamard_rows
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(5, 96, generator=gen)
    for block in (1, 2, 8, 32):
        got = block_hadamard_rows(x, block).numpy()
        ref = O.block_fwht(x.numpy().astype(np.float32), block)
        assert np.array_equal(got, ref.astype(np.float32))
    # against the dense orthonormal Sylvester matrix (fp64)
    h = np.array([[1.0]])
    while h.shape[0] < 32:
        h = np.block([[h, h], [h, -h]])
    dense = (x.double().numpy().reshape(5, 3, 32) @ (h / np.sqrt(32)).T).reshape(5, 96)
    assert np.allclose(block_hadamard_rows(x, 32).double().numpy(), dense, atol=1e-5)
    with pytest.raises(ValueError):
        block_hadamard_rows(x, 3)


@pytest.mark.parametrize("c", GOLDEN["cases"], ids=lambda c: f"{c['n']}x{c['d']}k{c['bits']}S{c['n_states']}")
def test_equilibration_and_signs_match_reference(c):
    """The CPU half of pack_linear: inv_equil, signs and block bit for bit."""
    from turbopress_amd.pack import equilibration, pack_rows_le, rademacher_signs
    lin, act = _case_linear(c)
    s = equilibration(lin.weight.detach().float(), act)
    assert _f16_bits((1.0 / s)) == c["payload"]["inv_equil_f16"]
    signs = rademacher_signs(c["d"], c["seed"]).to(torch.uint8)[None, :]
    assert pack_rows_le(signs, 1).flatten().tolist() == c["payload"]["signs_packed"]
    assert c["d"] & -c["d"] == c["payload"]["block"]


@pytest.mark.gpu
@pytest.mark.parametrize("c", GOLDEN["cases"], ids=lambda c: f"{c['n']}x{c['d']}k{c['bits']}S{c['n_states']}")
def test_pack_linear_matches_reference_payload(cuda, c):
    """Every payload field equals the reference's pack_linear output bit for
    bit (codes from the GPU Viterbi, statistics with the reference's ops)."""
    from turbopress_amd.pack import pack_linear
    lin, act = _case_linear(c)
    p = pack_linear(lin, act, bits=c["bits"], n_states=c["n_states"], seed=c["seed"])
    g = c["payload"]
    assert p["format"] == 2 and (p["n"], p["d"], p["bits"], p["n_states"]) == (c["n"], c["d"], c["bits"],
                                                                                c["n_states"])
    assert p["block"] == g["block"]
    assert p["path_packed"].flatten().tolist() == g["path_packed"]
    if g["member_packed"] is None:
        assert p["member_packed"] is None
    else:
        assert p["member_packed"].flatten().tolist() == g["member_packed"]
    assert _f16_bits(p["scales"]) == g["scales_f16"]
    assert p["signs_packed"].flatten().tolist() == g["signs_packed"]
    assert _f16_bits(p["inv_equil"]) == g["inv_equil_f16"]
    assert _f16_bits(p["codebook"]) == g["codebook_f16"]
    if g["bias_f16"] is None:
        assert p["bias"] is None
    else:
        assert _f16_bits(p["bias"]) == g["bias_f16"]


def test_pack_linear_rejects_odd_dims_and_bits():
    from torch import nn
    from turbopress_amd.pack import pack_linear
    with pytest.raises(ValueError):
        pack_linear(nn.Linear(77, 8), torch.ones(77), bits=3)
    with pytest.raises(ValueError):
        pack_linear(nn.Linear(64, 8), torch.ones(64), bits=5)


@pytest.mark.gpu
def test_pack_model_replaces_every_decoder_linear(cuda):
    """A small random Qwen3 decoder packed in place at k=3: every decoder
    linear becomes a PackedTCQLinear and the byte accounting matches.  Two
    copies packed in "hip" (fused rotation + decode-GEMV) and "cached"
    (decode once, fold the inverse rotation) mode give the same logits, and
    both stay within 3-bit quantization error of the fp16 model."""
    import copy
    pytest.importorskip("transformers")
    from transformers import AutoModelForCausalLM
    from turbopress_amd.artifact import decoder_layers
    from turbopress_amd.pack import pack_model
    from turbopress_amd.runtime import PackedTCQLinear
    from turbopress_amd.synthetic import tiny_qwen3_config
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(tiny_qwen3_config()).to(cuda, torch.float16).eval()
    ids = torch.randint(0, 1024, (1, 24), generator=torch.Generator().manual_seed(1)).to(cuda)
    # per-channel input RMS of every decoder linear on this prompt
    stats, hooks = {}, []
    for i, block in enumerate(decoder_layers(model)):
        for name, mod in block.named_modules():
            if isinstance(mod, torch.nn.Linear):
                def hook(m, args, out, key=f"{i}.{name}"):
                    stats[key] = args[0].float().pow(2).mean(dim=(0, 1)).sqrt().cpu()
                hooks.append(mod.register_forward_hook(hook))
    with torch.no_grad():
        ref = model(ids).logits.float()
    for h in hooks:
        h.remove()
    n_linear = len(stats)
    twin = copy.deepcopy(model)
    acct = pack_model(model, stats, bits=3, n_states=64, mode="hip")
    pack_model(twin, stats, bits=3, n_states=64, mode="cached")
    packed = [m for blk in decoder_layers(model) for m in blk.modules() if isinstance(m, PackedTCQLinear)]
    assert len(packed) == n_linear and n_linear == 2 * 7
    assert not any(isinstance(m, torch.nn.Linear) for blk in decoder_layers(model) for m in blk.modules())
    assert acct["packed_bytes"] == sum(m.packed_bytes() for m in packed)
    assert acct["fp16_bytes"] == sum(2 * m.in_features * m.out_features for m in packed)
    assert 4.0 < acct["compression"] < 5.4
    with torch.no_grad():
        got = model(ids).logits.float()
        got_cached = twin(ids).logits.float()
    assert torch.isfinite(got).all()
    rel = float((got - got_cached).abs().max() / got_cached.abs().max())
    assert rel < 2e-2, rel
    err = float((got - ref).norm() / ref.norm())
    assert err < 0.5, err
