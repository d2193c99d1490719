"""Graph-captured greedy decoding of a packed causal LM (the full-model decode
step; the reference's ``scripts/graph_decode_bench.py:39-118``).

Prefill once, then capture ONE decode step -- static input token, static KV
cache (``transformers.StaticCache``), device-side cache position -- in a HIP
graph and replay it per token, so no Python runs between kernels.
``decode_eager`` is the same loop without capture; the two must produce the
same greedy tokens.  Every PackedTCQLinear forward is capture-safe (no host
synchronisation, no allocation outside torch's graph pool).
"""

from __future__ import annotations

import time

import torch

__all__ = ["build_static_cache", "decode_eager", "decode_graph"]


def build_static_cache(model, max_len: int):
    """A batch-1 StaticCache of `max_len` positions for `model`."""
    from transformers import StaticCache

    for kwargs in (dict(max_cache_len=max_len, max_batch_size=1, device=model.device, dtype=model.dtype),
                   dict(max_cache_len=max_len, batch_size=1, device=model.device, dtype=model.dtype),
                   dict(max_cache_len=max_len)):
        try:
            return StaticCache(config=model.config, **kwargs)
        except TypeError:
            continue
    raise RuntimeError("this transformers version has no usable StaticCache signature")


def _prefill(model, cache, prompt_ids):
    n = prompt_ids.shape[1]
    logits = model(input_ids=prompt_ids, past_key_values=cache, use_cache=True,
                   cache_position=torch.arange(n, device=model.device)).logits
    return logits[:, -1:].argmax(-1)


@torch.inference_mode()
def decode_eager(model, prompt_ids, n_new: int, max_len: int):
    """Greedy tokens (n_new of them) and tokens/s of the uncaptured loop."""
    cache = build_static_cache(model, max_len)
    n = prompt_ids.shape[1]
    tok = _prefill(model, cache, prompt_ids)
    out = [int(tok)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for step in range(1, n_new):
        logits = model(input_ids=tok, past_key_values=cache, use_cache=True,
                       cache_position=torch.tensor([n + step - 1], device=model.device)).logits
        tok = logits[:, -1:].argmax(-1)
        out.append(int(tok))
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return out, (n_new - 1) / dt if dt > 0 else float("inf")


@torch.inference_mode()
def decode_graph(model, prompt_ids, n_new: int, max_len: int, warmup: int = 3):
    """Greedy tokens and tokens/s with one captured decode step replayed per
    token.  The first `warmup` steps run uncaptured on a side stream."""
    cache = build_static_cache(model, max_len)
    dev = model.device
    n = prompt_ids.shape[1]
    static_tok = _prefill(model, cache, prompt_ids).clone()
    static_pos = torch.tensor([n], device=dev)
    out = [int(static_tok)]

    def step():
        return model(input_ids=static_tok, past_key_values=cache, use_cache=True,
                     cache_position=static_pos).logits

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(min(warmup, n_new - 1)):
            logits = step()
            static_tok.copy_(logits[:, -1:].argmax(-1))
            static_pos += 1
            out.append(int(static_tok))
    torch.cuda.current_stream().wait_stream(s)

    # Capture records the step without running it: the static state is not
    # advanced here and no token is taken from the capture itself.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_logits = step()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    timed = 0
    while len(out) < n_new:
        graph.replay()
        static_tok.copy_(g_logits[:, -1:].argmax(-1))
        static_pos += 1
        timed += 1
        out.append(int(static_tok))
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return out, timed / dt if dt > 0 and timed else float("inf")
