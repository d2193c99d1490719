"""Format-v1 artifacts: v1 -> v2 conversion (bit-exact against the oracle),
the loader's guards, and (GPU) a synthetic artifact loaded into a packed
Qwen3 model and decoded greedily with and without graph capture
(runtime.py:417-541, tests/test_run.py:20-79, scripts/graph_decode_bench.py)."""

import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O
from turbopress_amd.artifact import load_packed_model, v1_payload_to_packed, v1_stream_to_rows
from turbopress_amd.synthetic import make_v1_payload


def _v1_pack(vals: np.ndarray, width: int) -> np.ndarray:
    """Independent format-v1 packer: value p's bit j at flat stream bit
    p*width + j, stream bits MSB-first within each byte (pipeline.py:106-111)."""
    flat = vals.reshape(-1).astype(np.uint8)
    bits = ((flat[:, None] >> np.arange(width, dtype=np.uint8)) & 1).reshape(-1)
    return np.packbits(bits)


@pytest.mark.parametrize("width", [1, 2, 3])
@pytest.mark.parametrize("n,d", [(7, 100), (5, 64), (3, 9)])
def test_v1_stream_to_rows_regroups_per_row(width, n, d):
    rng = np.random.default_rng(width * 100 + d)
    vals = rng.integers(0, 1 << width, size=(n, d), dtype=np.uint8)
    rows = v1_stream_to_rows(_v1_pack(vals, width), n, d, width)
    assert rows.shape == (n, (d * width + 7) // 8)
    assert np.array_equal(rows, O.pack_le(vals, width))
    assert np.array_equal(O.unpack_le(rows, d, width), vals)
    # the oracle's reading of the v1 stream agrees with the packer above
    assert np.array_equal(O.unpack_bits_v1(_v1_pack(vals, width), n * d, width).reshape(n, d), vals)


def test_v1_stream_too_short_raises():
    with pytest.raises(ValueError):
        v1_stream_to_rows(np.zeros(3, np.uint8), 2, 16, 1)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_v1_payload_to_packed_keeps_every_code(bits):
    """No re-quantization: the v2 payload carries exactly the artifact's codes,
    scales, codebook, signs and 1/equil (runtime.py:437-452)."""
    n, d = 48, 192
    v1 = make_v1_payload(n, d, bits, 64, seed=bits)
    bias = torch.randn(n)
    v2 = v1_payload_to_packed(v1, bias, "cpu")
    assert v2["format"] == 2 and (v2["n"], v2["d"], v2["bits"], v2["n_states"]) == (n, d, bits, 64)
    assert v2["block"] == 64
    path = O.unpack_bits_v1(v1["path_bits"].numpy(), n * d, 1).reshape(n, d)
    assert np.array_equal(O.unpack_le(v2["path_packed"].numpy(), d, 1), path)
    member = O.unpack_bits_v1(v1["member_bits"].numpy(), n * d, bits - 1).reshape(n, d)
    assert np.array_equal(O.unpack_le(v2["member_packed"].numpy(), d, bits - 1), member)
    signs = O.unpack_bits_v1(v1["signs"].numpy(), d, 1)
    assert np.array_equal(O.unpack_le(v2["signs_packed"].numpy(), d, 1)[0], signs)
    want_inv = (1.0 / v1["equil"].float().clamp_min(1e-12)).to(torch.float16)
    assert torch.equal(v2["inv_equil"], want_inv)
    assert torch.equal(v2["scales"], v1["scales"]) and torch.equal(v2["codebook"], v1["codebook"])
    assert torch.equal(v2["bias"], bias.to(torch.float16))
    # and the decoded weights are those of the v1 codes
    lv = O.window_decode_levels(path, member, 64)
    np.testing.assert_array_equal(O.levels_of({k: (v.numpy() if isinstance(v, torch.Tensor) else v)
                                               for k, v in v2.items()}), lv)


def test_load_packed_model_guards(tmp_path):
    with pytest.raises(ValueError):
        load_packed_model("anywhere", device="cpu", mode="nope")
    with pytest.raises(FileNotFoundError):
        load_packed_model(tmp_path, device="cpu", mode="hip")
    torch.save({"meta": {"format_version": 2, "n_states": 64, "generators": [0o133, 0o171]},
                "quantized": {}, "extra_state": {}}, tmp_path / "turbopress_weights.pt")
    with pytest.raises(RuntimeError, match="format_version"):
        load_packed_model(tmp_path, device="cpu", mode="hip")
    torch.save({"meta": {"format_version": 1, "n_states": 64, "generators": [0o23, 0o35]},
                "quantized": {}, "extra_state": {}}, tmp_path / "turbopress_weights.pt")
    with pytest.raises(RuntimeError, match="generator"):
        load_packed_model(tmp_path, device="cpu", mode="hip")
    torch.save({"meta": {"format_version": 1, "n_states": 64, "generators": [0o133, 0o171]},
                "quantized": {}, "extra_state": {}}, tmp_path / "turbopress_weights.pt")
    with pytest.raises(RuntimeError, match="GPU"):
        load_packed_model(tmp_path, device="cpu", mode="hip")


# ---------------------------------------------------------------------------
# GPU: a synthetic artifact end to end
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def tiny_artifact(tmp_path_factory):
    from turbopress_amd.synthetic import tiny_qwen3_config, write_synthetic_artifact
    root = tmp_path_factory.mktemp("artifact")
    write_synthetic_artifact(root, tiny_qwen3_config(), bits=3, n_states=64, seed=0)
    return root


@pytest.mark.gpu
def test_load_packed_model_rejects_an_artifact_missing_a_tensor(cuda, tiny_artifact, tmp_path):
    """The model is built without initialising its parameters, so a tensor
    the artifact does not hold (here a norm weight) is an error, not
    silently uninitialised memory."""
    import shutil
    bad = tmp_path / "bad"
    shutil.copytree(tiny_artifact, bad)
    blob = torch.load(bad / "turbopress_weights.pt", weights_only=True)
    del blob["extra_state"]["model.norm.weight"]
    torch.save(blob, bad / "turbopress_weights.pt")
    with pytest.raises(RuntimeError, match="lacks tensors"):
        load_packed_model(bad, device="cuda", mode="hip")


@pytest.mark.gpu
def test_load_packed_model_replaces_every_decoder_linear(cuda, tiny_artifact):
    from turbopress_amd.artifact import decoder_layers
    from turbopress_amd.runtime import PackedTCQLinear
    model, meta = load_packed_model(tiny_artifact, device="cuda", mode="hip")
    assert meta["format_version"] == 1 and meta["n_states"] == 64
    packed = [m for blk in decoder_layers(model) for m in blk.modules() if isinstance(m, PackedTCQLinear)]
    assert len(packed) == 7 * len(decoder_layers(model))
    assert all(m.mode == "hip" and m.tiled_packed is not None for m in packed)
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()  # still tied


@pytest.mark.gpu
def test_load_packed_model_triton_mode_passes_reference_script_checks(cuda, tiny_artifact):
    """A model loaded with mode="triton" (what the reference's loader script
    passes, scripts/bench_packed.py:261) passes that script's three checks on
    every decoder module (bench_packed.py:286-293): mode is still "triton",
    the packed stream is held, no fp16 weight cache exists -- and it computes
    the same logits as mode="hip"."""
    from turbopress_amd.artifact import decoder_layers
    from turbopress_amd.runtime import PackedTCQLinear
    model, _ = load_packed_model(tiny_artifact, device="cuda", mode="triton")
    count, residual = 0, []
    for i, block in enumerate(decoder_layers(model)):
        for name, module in block.named_modules():
            if isinstance(module, PackedTCQLinear):
                count += 1
                assert module.mode == "triton", f"model.layers.{i}.{name} is not in Triton mode."
                assert module.levels_packed is not None, f"model.layers.{i}.{name} has no packed level stream."
                assert module._w_cache is None, f"model.layers.{i}.{name} contains an FP16 weight cache."
            elif isinstance(module, torch.nn.Linear):
                residual.append(name)
    assert count == 7 * len(decoder_layers(model)) and not residual
    ids = torch.randint(0, 1024, (1, 8), generator=torch.Generator().manual_seed(3)).to(cuda)
    with torch.inference_mode():
        a = model(input_ids=ids).logits.float()
    del model
    hip_model, _ = load_packed_model(tiny_artifact, device="cuda", mode="hip")
    with torch.inference_mode():
        b = hip_model(input_ids=ids).logits.float()
    assert torch.equal(a, b)


@pytest.mark.gpu
def test_packed_model_logits_hip_vs_cached(cuda, tiny_artifact):
    """The bandwidth path (fused rotation + decode-GEMV) and load-time
    decompression (decode + fold + GEMM) give the same model."""
    ids = torch.randint(0, 1024, (1, 12), generator=torch.Generator().manual_seed(0)).to(cuda)
    outs = {}
    for mode in ("hip", "cached"):
        model, _ = load_packed_model(tiny_artifact, device="cuda", mode=mode)
        with torch.inference_mode():
            outs[mode] = model(input_ids=ids).logits.float()
        del model
    a, b = outs["hip"], outs["cached"]
    assert torch.isfinite(a).all()
    rel = ((a - b).abs().max() / b.abs().max()).item()
    assert rel < 2e-2, rel
    assert torch.equal(a[0, -1].argmax(), b[0, -1].argmax()) or rel < 5e-3


@pytest.mark.gpu
def test_graph_decode_matches_eager(cuda, tiny_artifact):
    """One captured decode step replayed per token yields the eager loop's
    greedy tokens (graph_decode_bench.py:135-141)."""
    from turbopress_amd.graph_decode import decode_eager, decode_graph
    model, _ = load_packed_model(tiny_artifact, device="cuda", mode="hip")
    ids = torch.randint(0, 1024, (1, 8), generator=torch.Generator().manual_seed(1)).to(cuda)
    n_new, max_len = 16, 8 + 16 + 8
    toks_e, _ = decode_eager(model, ids, n_new, max_len)
    toks_g, _ = decode_graph(model, ids, n_new, max_len)
    assert len(toks_e) == len(toks_g) == n_new
    assert toks_e == toks_g


@pytest.mark.gpu
def test_graph_decode_from_shared_prefill(cuda, tiny_artifact):
    """A 16-token prompt (its prefill runs the batched split-K GEMV): eager
    and graph loops started from copies of one prefill give the same tokens
    and leave the shared cache and token as they were."""
    from turbopress_amd.graph_decode import decode_eager, decode_graph, prefill
    model, _ = load_packed_model(tiny_artifact, device="cuda", mode="hip")
    ids = torch.randint(0, 1024, (1, 16), generator=torch.Generator().manual_seed(3)).to(cuda)
    n_new, max_len = 12, 16 + 12 + 8
    start = prefill(model, ids, max_len)
    tok0 = start[1].clone()
    keys0 = [lyr.keys.clone() for lyr in start[0].layers]
    toks_e, _ = decode_eager(model, ids, n_new, max_len, start=start)
    toks_g, _ = decode_graph(model, ids, n_new, max_len, start=start)
    assert toks_e == toks_g and toks_e[0] == int(tok0)
    assert torch.equal(start[1], tok0)
    assert all(torch.equal(lyr.keys, k) for lyr, k in zip(start[0].layers, keys0))


@pytest.mark.gpu
def test_fused_shared_input_projections_match(cuda, tiny_artifact):
    """q/k/v and gate/up joined into one launch per group: same logits (to
    the GEMV tolerance) and the same greedy tokens, eager and graph-replayed."""
    from turbopress_amd.decode_step import fuse_shared_input_projections
    from turbopress_amd.graph_decode import decode_eager, decode_graph
    ids = torch.randint(0, 1024, (1, 8), generator=torch.Generator().manual_seed(2)).to(cuda)
    model, _ = load_packed_model(tiny_artifact, device="cuda", mode="hip")
    with torch.inference_mode():
        ref = model(input_ids=ids).logits.float()
    toks_ref, _ = decode_eager(model, ids, 12, 32)
    assert fuse_shared_input_projections(model) == 2 * len(model.model.layers)
    with torch.inference_mode():
        fused = model(input_ids=ids).logits.float()
    rel = ((fused - ref).abs().max() / ref.abs().max()).item()
    assert rel < 5e-3, rel
    toks_e, _ = decode_eager(model, ids, 12, 32)
    toks_g, _ = decode_graph(model, ids, 12, 32)
    assert toks_e == toks_ref and toks_g == toks_ref


@pytest.mark.gpu
def test_qwen3_4b_width_layers_end_to_end(cuda, tmp_path):
    """Two decoder layers at Qwen3-4B's widths -- the headline stack's
    linear shapes (hidden 2560, intermediate 9728, 32 x 128 query and
    8 x 128 key/value heads) -- through the artifact loader: `hip` and
    `cached` give the same logits, so do the fused q/k/v and gate/up groups,
    and greedy decode replayed from a captured step equals the eager loop."""
    from turbopress_amd.decode_step import fuse_shared_input_projections
    from turbopress_amd.graph_decode import decode_eager, decode_graph, prefill
    from turbopress_amd.synthetic import tiny_qwen3_config, write_synthetic_artifact
    cfg = tiny_qwen3_config(layers=2, hidden=2560, intermediate=9728, heads=32, kv_heads=8, head_dim=128,
                            vocab=4096)
    write_synthetic_artifact(tmp_path, cfg, bits=3, n_states=64, seed=1)
    ids = torch.randint(0, 4096, (1, 8), generator=torch.Generator().manual_seed(4)).to(cuda)
    cached, _ = load_packed_model(tmp_path, device="cuda", mode="cached")
    with torch.inference_mode():
        ref = cached(input_ids=ids).logits.float()
    del cached
    model, _ = load_packed_model(tmp_path, device="cuda", mode="hip")
    with torch.inference_mode():
        got = model(input_ids=ids).logits.float()
    assert torch.isfinite(got).all()
    rel = ((got - ref).abs().max() / ref.abs().max()).item()
    assert rel < 2e-2, rel
    assert fuse_shared_input_projections(model) == 2 * 2
    with torch.inference_mode():
        fused = model(input_ids=ids).logits.float()
    rel_f = ((fused - got).abs().max() / got.abs().max()).item()
    assert rel_f < 5e-3, rel_f
    start = prefill(model, ids, 32)
    toks_e, _ = decode_eager(model, ids, 12, 32, start=start)
    toks_g, _ = decode_graph(model, ids, 12, 32, start=start)
    assert toks_e == toks_g
