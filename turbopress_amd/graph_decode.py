"""Graph-captured greedy decoding of a packed causal LM (the full-model decode
step; the reference's ``scripts/graph_decode_bench.py:39-118``).

Prefill once, then capture ONE decode step -- static input token, static KV
cache (``transformers.StaticCache``), device-side cache position -- in a HIP
graph and replay it per token, so no Python runs between kernels.
``decode_eager`` is the same loop without capture; from the same prefilled
cache the two produce the same greedy tokens.  Every PackedTCQLinear forward
is capture-safe (no host synchronisation, no allocation outside torch's
graph pool).

The prefill runs the prompt as one batch.  Above 8 rows the batched
decode-GEMV splits K over workgroups and adds their fp32 partial sums with
atomics in arrival order (as the reference's split-D configurations do,
``turbopress/triton_kernel.py:126-129``), so two prefills of one prompt can
differ in the last bits of the cache -- enough to flip a greedy token where
the top two logits nearly tie.  ``prefill`` therefore runs once and both
loops start from copies of its cache.  The batch-1 decode steps add in a
fixed order: their tokens are reproducible.
"""

from __future__ import annotations

import copy
import time

import torch

__all__ = ["build_static_cache", "prefill", "decode_eager", "decode_graph"]


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
def prefill(model, prompt_ids, max_len: int):
    """The prompt run into a fresh StaticCache of `max_len` positions:
    (cache, first greedy token [1, 1])."""
    cache = build_static_cache(model, max_len)
    return cache, _prefill(model, cache, prompt_ids)


def _start(model, prompt_ids, max_len, start):
    # a private copy of a shared prefill, or a prefill of our own
    if start is None:
        return prefill(model, prompt_ids, max_len)
    cache, tok = start
    return copy.deepcopy(cache), tok.clone()


@torch.inference_mode()
def decode_eager(model, prompt_ids, n_new: int, max_len: int, start=None):
    """Greedy tokens (n_new of them) and tokens/s of the uncaptured loop.
    `start`: a (cache, token) pair from ``prefill`` of this prompt to begin
    from (copied; the pair is left as it was) instead of prefilling here."""
    n = prompt_ids.shape[1]
    cache, tok = _start(model, prompt_ids, max_len, start)
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
def decode_graph(model, prompt_ids, n_new: int, max_len: int, warmup: int = 3, start=None):
    """Greedy tokens and tokens/s with one captured decode step replayed per
    token.  The first `warmup` steps run uncaptured on a side stream.
    `start` as for ``decode_eager``."""
    dev = model.device
    n = prompt_ids.shape[1]
    cache, static_tok = _start(model, prompt_ids, max_len, start)
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


# ---------------------------------------------------------------------------
# command line: the reference's scripts/graph_decode_bench.py for this build
# ---------------------------------------------------------------------------
# Decoder shapes of the models the reference benchmarks and configures
# (random weights only: nothing is downloaded).
SYNTHETIC = {
    "smollm2-135m": ("llama", dict(vocab_size=49152, hidden_size=576, intermediate_size=1536,
                                   num_hidden_layers=30, num_attention_heads=9, num_key_value_heads=3,
                                   tie_word_embeddings=True, max_position_embeddings=2048)),
    "qwen3-0.6b": ("qwen3", dict(vocab_size=151936, hidden_size=1024, intermediate_size=3072,
                                 num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8,
                                 head_dim=128, tie_word_embeddings=True, max_position_embeddings=2048)),
    # the decoder whose 36 x 7 linears are the headline stack's (config c2)
    "qwen3-4b": ("qwen3", dict(vocab_size=151936, hidden_size=2560, intermediate_size=9728,
                               num_hidden_layers=36, num_attention_heads=32, num_key_value_heads=8,
                               head_dim=128, tie_word_embeddings=True, max_position_embeddings=2048)),
}


def synthetic_config(name: str):
    """A transformers config of one of the SYNTHETIC decoder shapes."""
    from transformers import LlamaConfig, Qwen3Config
    kind, kw = SYNTHETIC[name]
    cls = LlamaConfig if kind == "llama" else Qwen3Config
    return cls(torch_dtype="float16", **kw)


def main(argv=None) -> int:
    """Greedy decode tokens/s of a packed model, eager and with one captured
    decode step replayed per token (graph_decode_bench.py:121-158), optionally
    beside the dense fp16 model of the same shape.  Prints one JSON line."""
    import argparse
    import json
    import sys
    import tempfile

    from turbopress_amd.artifact import load_packed_model
    from turbopress_amd.synthetic import write_synthetic_artifact

    ap = argparse.ArgumentParser(description=main.__doc__.splitlines()[0])
    src = ap.add_mutually_exclusive_group(required=True)
    src.add_argument("--artifact", help="format-v1 artifact directory")
    src.add_argument("--synthetic", choices=sorted(SYNTHETIC), help="seeded synthetic model of this shape")
    ap.add_argument("--bits", type=int, default=3)
    ap.add_argument("--n-states", type=int, default=64)
    ap.add_argument("--mode", default="hip", choices=("hip", "triton", "cached"))
    ap.add_argument("--prompt-len", type=int, default=16)
    ap.add_argument("--new-tokens", type=int, default=128)
    ap.add_argument("--fp16-baseline", action="store_true", help="also time the dense fp16 model")
    ap.add_argument("--fuse", action="store_true",
                    help="one launch per shared-input group (q/k/v, gate/up) instead of per projection")
    args = ap.parse_args(argv)

    def progress(msg: str) -> None:
        # (stderr: stdout carries the one JSON line)
        print(f"[graph_decode] {msg}", file=sys.stderr, flush=True)

    with tempfile.TemporaryDirectory() as tmp:
        root = args.artifact
        if args.synthetic:
            root = tmp
            write_synthetic_artifact(root, synthetic_config(args.synthetic), bits=args.bits,
                                     n_states=args.n_states, seed=0, log=progress)
        progress("loading the packed model")
        model, meta = load_packed_model(root, device="cuda", mode=args.mode)
    if args.fuse:
        from turbopress_amd.decode_step import fuse_shared_input_projections
        fuse_shared_input_projections(model)
    vocab = model.config.vocab_size
    prompt = torch.randint(0, vocab, (1, args.prompt_len), generator=torch.Generator().manual_seed(0)).cuda()
    max_len = args.prompt_len + args.new_tokens + 8
    start = prefill(model, prompt, max_len)
    toks_e, tps_e = decode_eager(model, prompt, args.new_tokens, max_len, start=start)
    toks_g, tps_g = decode_graph(model, prompt, args.new_tokens, max_len, start=start)
    del start
    out = {"model": args.synthetic or str(args.artifact), "mode": args.mode, "fused_groups": args.fuse, "bits": int(meta.get("bits", args.bits)),
           "n_states": int(meta["n_states"]), "prompt_len": args.prompt_len, "new_tokens": args.new_tokens,
           "eager_tok_s": round(tps_e, 1), "graph_tok_s": round(tps_g, 1), "greedy_tokens_match": toks_e == toks_g}
    if args.fp16_baseline:
        from transformers import AutoConfig, AutoModelForCausalLM
        del model
        torch.cuda.empty_cache()
        progress("building the dense fp16 model")
        torch.manual_seed(0)
        config = (synthetic_config(args.synthetic) if args.synthetic
                  else AutoConfig.from_pretrained(f"{args.artifact}/hf_config"))
        # (random weights initialised on the GPU: a CPU initialisation of a
        # 4B model takes minutes)
        prev_dtype = torch.get_default_dtype()
        torch.set_default_dtype(torch.float16)
        try:
            with torch.device("cuda"):
                dense = AutoModelForCausalLM.from_config(config)
        finally:
            torch.set_default_dtype(prev_dtype)
        dense = dense.to(device="cuda", dtype=torch.float16).eval()
        progress("timing the dense fp16 model")
        out["fp16_eager_tok_s"] = round(decode_eager(dense, prompt, args.new_tokens, max_len)[1], 1)
        out["fp16_graph_tok_s"] = round(decode_graph(dense, prompt, args.new_tokens, max_len)[1], 1)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    import sys
    sys.exit(main())
