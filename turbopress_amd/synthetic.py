"""Seeded synthetic packed linears and activations for tests and benchmarks.

Every stream the decode path reads is drawn from a CPU ``torch.Generator``
seeded per linear, in a fixed order:

  1. ``path_packed``   uint8 [n, ceil(d/8)]        uniform bytes
  2. ``member_packed`` uint8 [n, ceil(d(k-1)/8)]   uniform bytes (k > 1)
  3. ``scales``        fp16(|N(0, 0.02)| + 1e-3)    [n]
  4. equilibration     s ~ LogNormal(0, 0.25), ``inv_equil = fp16(1/fp16(s))`` [d]
  5. signs             Rademacher [d], packed little-endian like ``signs_packed``
  6. ``bias``          fp16 N(0, 0.1) [n] (only when requested)

Uniform bytes are legal trellis streams: every path bit sequence is a valid
path of the bitshift trellis and every member code is in range, so they are
what an encoder could have written.  Padding bits past the last weight of a
row are zeroed, as ``pack_le`` leaves them (runtime.py:84-90).  The codebook
is the reference's data-free trellis codebook for (k, S), seed 0.

The result is a format-v2 payload (runtime.py:171-186) that
``PackedTCQLinear`` accepts unchanged.
"""

from __future__ import annotations

import math

import torch

from turbopress_amd.codebooks import available_codebooks, default_codebook

# Qwen3 decoder-layer projection shapes (in_features -> out_features).
QWEN3_0_6B_LAYER = {
    "q_proj": (1024, 2048), "k_proj": (1024, 1024), "v_proj": (1024, 1024),
    "o_proj": (2048, 1024), "gate_proj": (1024, 3072), "up_proj": (1024, 3072),
    "down_proj": (3072, 1024),
}
QWEN3_4B_LAYER = {
    "q_proj": (2560, 4096), "k_proj": (2560, 1024), "v_proj": (2560, 1024),
    "o_proj": (4096, 2560), "gate_proj": (2560, 9728), "up_proj": (2560, 9728),
    "down_proj": (9728, 2560),
}
QWEN3_4B_LAYERS = 36


def _mask_row_padding(packed: torch.Tensor, nbits: int) -> torch.Tensor:
    """Zero the stream bits at positions >= nbits of every row."""
    rem = nbits % 8
    if rem:
        packed[:, -1] &= (1 << rem) - 1
    return packed


def pack_bits_le(bits01: torch.Tensor) -> torch.Tensor:
    """Pack a 1-D 0/1 tensor little-endian into uint8 [1, ceil(len/8)]."""
    n = bits01.numel()
    pad = (-n) % 8
    b = torch.nn.functional.pad(bits01.to(torch.int32).reshape(1, -1), (0, pad))
    w = 1 << torch.arange(8, dtype=torch.int32)
    return (b.reshape(1, -1, 8) * w).sum(-1).to(torch.uint8)


def _synthetic_codebook(bits: int, seed: int) -> torch.Tensor:
    """Seeded fp16 doubled codebook for rates without a stored default: N(0,1)
    draws, each Ungerboeck subset cb[j::4] sorted (trellis.py:249-250)."""
    gen = torch.Generator().manual_seed(10_000 + seed)
    cb = torch.randn(1 << (bits + 1), generator=gen)
    for j in range(4):
        cb[j::4] = cb[j::4].sort().values
    return cb.to(torch.float16)


def unit_gain(payload: dict) -> dict:
    """The payload with its row scales divided by the linear's expected gain
    sqrt(n * mean(scale^2) * mean(codebook^2) * mean(inv_equil^2)), so that
    E||y||^2 = ||x||^2 for uniform codes: chains of such linears keep the
    activations' magnitude (decode-step benchmarks without the model's
    norms).  The codes, codebook and rotation are unchanged."""
    out = dict(payload)
    n = int(payload["n"])
    s = payload["scales"].float()
    cb = payload["codebook"].float()
    ie = payload["inv_equil"].float()
    gain = math.sqrt(n * float(s.pow(2).mean()) * float(cb.pow(2).mean()) * float(ie.pow(2).mean()))
    out["scales"] = (s / gain).to(torch.float16)
    return out


def make_payload(n: int, d: int, bits: int, n_states: int = 64, seed: int = 0,
                 bias: bool = False, codebook: torch.Tensor | None = None) -> dict:
    """A seeded format-v2 payload of an n x d packed linear (CPU tensors)."""
    if bits < 1 or bits > 7:
        raise ValueError(f"bits must be in [1, 7], got {bits}")
    block = d & -d  # hadamard.py:30-34; 1 for odd d (the rotation is then the identity)
    gen = torch.Generator().manual_seed(seed)
    path = torch.randint(0, 256, (n, (d + 7) // 8), generator=gen, dtype=torch.uint8)
    _mask_row_padding(path, d)
    member = None
    if bits > 1:
        mb = d * (bits - 1)
        member = torch.randint(0, 256, (n, (mb + 7) // 8), generator=gen, dtype=torch.uint8)
        _mask_row_padding(member, mb)
    scales = (torch.randn(n, generator=gen).abs() * 0.02 + 1e-3).to(torch.float16)
    s = torch.exp(torch.randn(d, generator=gen) * 0.25)
    inv_equil = (1.0 / s.to(torch.float16).float()).to(torch.float16)
    signs01 = torch.randint(0, 2, (d,), generator=gen, dtype=torch.int64)
    b = (torch.randn(n, generator=gen) * 0.1).to(torch.float16) if bias else None
    if codebook is not None:
        cb = codebook.to(torch.float16)
    elif (bits, n_states) in available_codebooks():
        cb = default_codebook(bits, n_states)
    else:
        cb = _synthetic_codebook(bits, seed)
    return {
        "format": 2, "n": n, "d": d, "bits": bits, "n_states": n_states, "block": block,
        "path_packed": path, "member_packed": member, "scales": scales,
        "signs_packed": pack_bits_le(signs01), "inv_equil": inv_equil,
        "codebook": cb, "bias": b, "seed": seed,
    }


def make_activation(batch: int, d: int, seed: int = 0, outlier_frac: float = 0.01,
                    outlier_scale: float = 20.0) -> torch.Tensor:
    """fp16 N(0,1) [batch, d] with ceil(outlier_frac*d) channels scaled x20."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, d, generator=gen)
    k = math.ceil(outlier_frac * d)
    idx = torch.randperm(d, generator=gen)[:k]
    x[:, idx] *= outlier_scale
    return x.to(torch.float16)


def payload_to(payload: dict, device) -> dict:
    """Copy of a payload with every tensor moved to ``device``."""
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in payload.items()}


def payload_numpy(payload: dict) -> dict:
    """Copy of a payload with every tensor as a CPU numpy array."""
    return {k: (v.detach().cpu().numpy() if isinstance(v, torch.Tensor) else v)
            for k, v in payload.items()}


# ---------------------------------------------------------------------------
# format-v1 matrices and artifacts (the pipeline's on-disk format)
# ---------------------------------------------------------------------------
def make_v1_payload(n: int, d: int, bits: int, n_states: int = 64, seed: int = 0) -> dict:
    """A seeded format-v1 matrix (pipeline.py:445-455): flat MSB-first code
    streams over the whole matrix (uniform bytes are legal codes), fp16 scales,
    packed Rademacher signs, fp16 equilibration and the default codebook."""
    gen = torch.Generator().manual_seed(seed)

    def flat(nbits: int) -> torch.Tensor:
        return torch.randint(0, 256, ((nbits + 7) // 8,), generator=gen, dtype=torch.uint8)

    path = flat(n * d)
    member = flat(n * d * (bits - 1)) if bits > 1 else None
    scales = (torch.randn(n, generator=gen).abs() * 0.02 + 1e-3).to(torch.float16)
    equil = torch.exp(torch.randn(d, generator=gen) * 0.25).to(torch.float16)
    signs = flat(d)
    if (bits, n_states) in available_codebooks():
        cb = default_codebook(bits, n_states)
    else:
        cb = _synthetic_codebook(bits, seed)
    return {"n": n, "d": d, "block": d & -d, "bits": bits, "n_states": n_states,
            "path_bits": path, "member_bits": member, "scales": scales, "signs": signs,
            "equil": equil, "codebook": cb}


def tiny_qwen3_config(layers: int = 2, hidden: int = 256, intermediate: int = 768, heads: int = 4,
                      kv_heads: int = 2, head_dim: int = 64, vocab: int = 1024):
    """A small Qwen3 decoder configuration (random weights only: no checkpoint
    is ever downloaded)."""
    from transformers import Qwen3Config
    return Qwen3Config(vocab_size=vocab, hidden_size=hidden, intermediate_size=intermediate,
                       num_hidden_layers=layers, num_attention_heads=heads, num_key_value_heads=kv_heads,
                       head_dim=head_dim, max_position_embeddings=512, tie_word_embeddings=True,
                       torch_dtype="float16")


def write_synthetic_artifact(root, config, bits: int = 3, n_states: int = 64, seed: int = 0,
                             log=None) -> dict:
    """Write a TurboPress format-v1 artifact directory for a randomly
    initialised model of `config` (pipeline.py:917-931 layout:
    ``turbopress_weights.pt`` = {meta, quantized, extra_state} and
    ``hf_config/``); every decoder linear is a seeded v1 matrix.  Returns the
    metadata.  `log`: optional callable given one progress line per layer."""
    from pathlib import Path

    from torch import nn

    from turbopress_amd.artifact import decoder_layers, empty_causal_lm
    from turbopress_amd.runtime import trellis_generators

    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    model = empty_causal_lm(config)
    quantized = {}
    prefix = None
    for name, _ in model.named_modules():
        if name.endswith(".layers") or name.endswith(".h"):
            prefix = name
            break
    layers = decoder_layers(model)
    for i, block in enumerate(layers):
        for name, mod in block.named_modules():
            if isinstance(mod, nn.Linear):
                key = f"{prefix}.{i}.{name}.weight"
                quantized[key] = make_v1_payload(mod.out_features, mod.in_features, bits, n_states,
                                                 seed=seed * 1000 + len(quantized))
        if log is not None:
            log(f"synthetic artifact: layer {i + 1}/{len(layers)}")
    # The other tensors, seeded: embeddings N(0, initializer_range), biases
    # zero, norm and other 1-D weights one.
    gen = torch.Generator().manual_seed(seed)
    std = float(getattr(config, "initializer_range", 0.02))
    tied = bool(getattr(config, "tie_word_embeddings", False))
    extra = {}
    for k, v in model.state_dict().items():
        if k in quantized or (tied and k == "lm_head.weight"):
            continue
        if v.ndim >= 2:
            extra[k] = (torch.randn(v.shape, generator=gen) * std).to(v.dtype)
        elif k.endswith(".bias"):
            extra[k] = torch.zeros(v.shape, dtype=v.dtype)
        else:
            extra[k] = torch.ones(v.shape, dtype=v.dtype)
    meta = {"format_version": 1, "model_id": "synthetic", "bits": bits, "n_states": n_states,
            "generators": list(trellis_generators(n_states)), "seed": seed}
    torch.save({"meta": meta, "quantized": quantized, "extra_state": extra}, root / "turbopress_weights.pt")
    config.save_pretrained(root / "hf_config")
    return meta
