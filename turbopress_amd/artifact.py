"""TurboPress pipeline artifacts (format v1) -> packed models on MI355X.

The drop-in for ``turbopress/runtime.py:417-541``: ``v1_payload_to_packed``
turns one format-v1 matrix into a format-v2 payload without re-quantizing
(the stored path/member codes, scales, codebook, signs and equilibration are
kept bit for bit), and ``load_packed_model`` builds the artifact's Hugging
Face causal LM with every decoder ``nn.Linear`` replaced by a
:class:`~turbopress_amd.runtime.PackedTCQLinear`.

Bit layouts.  Format v1 (``pipeline.py:106-117``) stores the codes of a
whole matrix as ONE flat stream: value p (row-major over n x d) occupies
stream bits ``p*w .. p*w+w-1`` (value bit j at stream bit p*w+j), and stream
bit i is bit ``7 - i%8`` of byte ``i//8`` (``numpy.packbits`` order,
most-significant first).  Format v2 (``runtime.py:73-100``) restarts the
stream at every row, pads rows to whole bytes and puts stream bit i at bit
``i%8`` of byte ``i//8`` (least-significant first).  Row r's values therefore
sit at v1 stream bits ``r*d*w ..`` in the same order as its v2 row stream; the
conversion regroups the stream per row and re-packs the bytes LSB-first.

The loader reads ``turbopress_weights.pt`` with ``torch.load(...,
weights_only=True)`` (tensors, dicts, lists and scalars only): unlike the
reference it never unpickles code from an artifact.
"""

from __future__ import annotations

from pathlib import Path
from typing import Any

import numpy as np
import torch
from torch import Tensor, nn

from turbopress_amd.runtime import MODES, PackedTCQLinear, trellis_generators

__all__ = ["v1_stream_to_rows", "v1_payload_to_packed", "load_packed_model", "decoder_layers"]


def v1_stream_to_rows(buf, rows: int, cols: int, width: int) -> np.ndarray:
    """Format-v1 flat stream of rows*cols values of `width` bits -> format-v2
    row streams, uint8 [rows, ceil(cols*width/8)] (LSB-first, rows padded
    with zero bits)."""
    a = buf.detach().cpu().contiguous().numpy() if isinstance(buf, Tensor) else np.asarray(buf)
    a = np.ascontiguousarray(a, dtype=np.uint8).reshape(-1)
    nbits = rows * cols * width
    if a.size * 8 < nbits:
        raise ValueError(f"v1 stream holds {a.size * 8} bits, {nbits} needed")
    bits = np.unpackbits(a, bitorder="big")[:nbits].reshape(rows, cols * width)
    pad = (-cols * width) % 8
    if pad:
        bits = np.pad(bits, ((0, 0), (0, pad)))
    return np.packbits(bits, axis=1, bitorder="little")


def v1_payload_to_packed(payload: dict, bias: Tensor | None = None, device: str = "cuda") -> dict[str, Any]:
    """One format-v1 artifact matrix -> format-v2 payload (runtime.py:417-452).

    No re-quantization: a PackedTCQLinear built from the result decodes to the
    weights the artifact's own fp16 loader reconstructs."""
    n, d, bits = int(payload["n"]), int(payload["d"]), int(payload["bits"])
    if n <= 0 or d <= 0 or not 1 <= bits <= 7:
        raise ValueError(f"bad v1 matrix header n={n} d={d} bits={bits}")

    def dev(a: np.ndarray) -> Tensor:
        return torch.from_numpy(a).to(device)

    path = dev(v1_stream_to_rows(payload["path_bits"], n, d, 1))
    member = None
    if bits > 1:
        if payload.get("member_bits") is None:
            raise ValueError("v1 matrix without member_bits at bits > 1")
        member = dev(v1_stream_to_rows(payload["member_bits"], n, d, bits - 1))
    signs = dev(v1_stream_to_rows(payload["signs"], 1, d, 1))
    equil = torch.as_tensor(payload["equil"]).detach().float().clamp_min(1e-12)
    return {
        "format": 2,
        "n": n,
        "d": d,
        "bits": bits,
        "n_states": int(payload["n_states"]),
        "block": int(payload["block"]),
        "path_packed": path,
        "member_packed": member,
        "scales": torch.as_tensor(payload["scales"]).detach().to(device=device, dtype=torch.float16),
        "signs_packed": signs,
        "inv_equil": (1.0 / equil).to(device=device, dtype=torch.float16),
        "codebook": torch.as_tensor(payload["codebook"]).detach().to(device=device, dtype=torch.float16),
        "bias": None if bias is None else bias.detach().to(device=device, dtype=torch.float16),
        "seed": 0,
    }


def decoder_layers(model: nn.Module):
    """The decoder blocks of a Hugging Face causal LM (real_model.py's
    _decoder_layers): ``model.model.layers`` for Llama/Qwen-style models,
    ``transformer.h`` for GPT-2 style ones."""
    for path in ("model.layers", "model.decoder.layers", "transformer.h", "gpt_neox.layers"):
        obj = model
        try:
            for part in path.split("."):
                obj = getattr(obj, part)
        except AttributeError:
            continue
        return obj
    raise RuntimeError(f"cannot locate the decoder layers of {type(model).__name__}")


def empty_causal_lm(config):
    """The causal LM of `config` in fp16 on the CPU with its parameters
    allocated but not filled (transformers' no-init context, as its own
    checkpoint loading uses): the caller loads or replaces every one.  The
    random initialisation skipped here takes minutes on the CPU at 4B
    parameters; buffers computed by the constructors (rotary frequencies,
    norm weights) are set as usual."""
    from transformers import AutoModelForCausalLM
    try:
        from transformers.initialization import no_init_weights
    except ImportError:  # older transformers
        from transformers.modeling_utils import no_init_weights
    prev_dtype = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with no_init_weights():
            model = AutoModelForCausalLM.from_config(config)
    finally:
        torch.set_default_dtype(prev_dtype)
    return model.to(dtype=torch.float16)


@torch.no_grad()
def load_packed_model(artifact_dir, *, device: str = "cuda", mode: str = "cached"):
    """Load a TurboPress artifact directory into a packed causal LM
    (runtime.py:455-541).  Every decoder ``nn.Linear`` becomes a
    PackedTCQLinear in ``mode`` (``"hip"`` keeps the weights trellis-coded,
    ``"triton"`` is its alias, ``"cached"`` decodes once at load).  Returns
    ``(model, meta)``."""
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
    root = Path(artifact_dir)
    weights_path = root / "turbopress_weights.pt"
    if not weights_path.exists():
        raise FileNotFoundError(f"not a TurboPress artifact (missing {weights_path})")
    blob = torch.load(weights_path, map_location="cpu", weights_only=True)
    meta = dict(blob["meta"])
    quantized = blob.pop("quantized")
    extra = blob.pop("extra_state")
    del blob
    if int(meta.get("format_version", -1)) != 1:
        raise RuntimeError("expected a TurboPress format_version=1 artifact")
    n_states = int(meta["n_states"])
    if tuple(meta["generators"]) != tuple(trellis_generators(n_states)):
        raise RuntimeError("trellis generator mismatch (artifact/runtime incompatible)")
    if not str(device).startswith("cuda") or not torch.cuda.is_available():
        raise RuntimeError("turbopress_amd runs on a ROCm GPU: pass a cuda device")

    from transformers import AutoConfig

    config = AutoConfig.from_pretrained(root / "hf_config")
    model = empty_causal_lm(config)

    # Non-quantized tensors; quantized weights and a tied lm_head come back as
    # "missing".  Only a non-".weight" unexpected key is a real mismatch.
    missing, unexpected = model.load_state_dict(extra, strict=False)
    del extra
    unexpected = [k for k in unexpected if not k.endswith(".weight")]
    if unexpected:
        raise RuntimeError(f"unexpected keys in artifact: {unexpected[:8]}")
    model.tie_weights()
    # The parameters were never initialised: every one must come from the
    # artifact, be replaced by a packed linear, or be the tied output head.
    # (Buffers are set by the constructors as usual.)
    out_emb, in_emb = model.get_output_embeddings(), model.get_input_embeddings()
    tied = out_emb is not None and in_emb is not None and out_emb.weight is in_emb.weight
    params = {name for name, _ in model.named_parameters(remove_duplicate=False)}
    absent = [k for k in missing
              if k in params and k not in quantized and not (tied and k == "lm_head.weight")]
    if absent:
        raise RuntimeError(f"artifact lacks tensors of the model: {absent[:8]}")

    for key in list(quantized):
        payload = quantized.pop(key)
        if not key.endswith(".weight"):
            raise RuntimeError(f"invalid quantized key: {key}")
        module_path = key[: -len(".weight")]
        linear = model.get_submodule(module_path)
        if not isinstance(linear, nn.Linear):
            raise RuntimeError(f"{module_path} is not nn.Linear")
        bias = None if linear.bias is None else linear.bias.detach().clone()
        packed = PackedTCQLinear(v1_payload_to_packed(payload, bias, device), mode=mode)
        parent_path, leaf = module_path.rsplit(".", 1)
        setattr(model.get_submodule(parent_path), leaf, packed)

    model = model.to(device=device, dtype=torch.float16).eval()
    model.config.use_cache = True
    model.tie_weights()

    leftover = [f"layers.{i}.{name}" for i, block in enumerate(decoder_layers(model))
                for name, mod in block.named_modules() if isinstance(mod, nn.Linear)]
    if leftover:
        raise RuntimeError(f"unconverted decoder linears remain: {leftover[:8]}")
    return model, meta
