"""Decode-step executors for stacks of packed linears.

The reference's decode step is an HF decoder replayed from a CUDA graph with
two Triton launches per projection (turbopress/runtime.py:312-316,
scripts/graph_decode_bench.py:70-118).  Two MI355X executors:

  * ``LinearStack`` -- every linear of the step in ONE persistent HIP launch
    (``tp_stack_run``); optional phase ordering makes a linear of phase p
    wait for all linears of phase p-1 (for a decoder layer: q/k/v, then o,
    then gate/up, then down), the order data dependencies impose.  Ordering
    schedules the work but passes no data: every input is rotated before any
    phase runs, so one run cannot feed a phase's outputs to a later phase.
  * ``layer_forward`` -- one fused launch per group of linears sharing an
    input (q/k/v together, o, gate/up together, down): the launch structure a
    model with interleaved attention/norm kernels uses.
  * ``ChainedDecodeStep`` -- the same four launches per layer with the data
    dependencies of a decode step: o reads q's output, gate/up read o's,
    down reads gate's, and the next layer's q/k/v read down's (the order
    scripts/graph_decode_bench.py:86-115 replays through the HF decoder,
    without the attention and norm kernels between the projections).

Inputs are fixed device buffers (write new activations into ``inputs[i]``
before each run), outputs are fixed buffers ``outputs[i]``, so runs can be
captured in a HIP graph and replayed.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from turbopress_amd import _lib
from turbopress_amd import hip_kernel as hk

__all__ = ["LinearStack", "layer_forward", "ChainedDecodeStep", "QWEN_PHASES"]

# Phase of each projection inside one decoder layer (shared-input groups).
QWEN_PHASES = {"q_proj": 0, "k_proj": 0, "v_proj": 0, "o_proj": 1,
               "gate_proj": 2, "up_proj": 2, "down_proj": 3}


class LinearStack:
    """A list of (PackedTCQLinear, input buffer, phase) run by one launch."""

    def __init__(self, entries, ordered: bool = False) -> None:
        if not entries:
            raise ValueError("empty stack")
        lins = [e[0] for e in entries]
        l0 = lins[0]
        for lin in lins:
            if lin.tiled_packed is None:
                raise ValueError("stack linears need mode='hip' with bits in (2, 3, 4)")
            if (lin.bits, lin.n_states) != (l0.bits, l0.n_states) or lin.codebook_key != l0.codebook_key:
                raise ValueError("stack linears must share bits, n_states and codebook")
        self.linears = lins
        self.inputs = [e[1] for e in entries]
        self.phases = [int(e[2]) for e in entries]
        if self.phases[0] != 0 or any(not a <= b <= a + 1 for a, b in zip(self.phases, self.phases[1:])):
            raise ValueError("phases must start at 0 and rise by at most 1 along the stack")
        self.batch = int(self.inputs[0].shape[0])
        if not 1 <= self.batch <= 32:
            raise ValueError("stack batch must be in [1, 32]")
        dev = self.inputs[0].device
        self.ordered = bool(ordered)
        self.outputs = [torch.empty(self.batch, lin.out_features, dtype=torch.float16, device=dev)
                        for lin in lins]
        arr = (_lib.StackLinear * len(lins))()
        for i, (lin, x, ph) in enumerate(zip(lins, self.inputs, self.phases)):
            if x.dtype != torch.float16 or not x.is_contiguous() or x.shape != (self.batch, lin.in_features):
                raise ValueError(f"input {i} must be contiguous fp16 [{self.batch}, {lin.in_features}]")
            pb = lin._tiled_geo["path_bytes"]
            arr[i] = _lib.StackLinear(
                lin.tiled_packed.data_ptr(), lin.tiled_packed.data_ptr() + pb,
                x.data_ptr(), lin.in_features, lin.rot_scale.data_ptr(), lin.block,
                lin.scales.data_ptr(), 0 if lin.bias is None else lin.bias.data_ptr(),
                self.outputs[i].data_ptr(), lin.out_features, lin.out_features, lin.in_features, ph, 0)
        self.n_phases = max(self.phases) + 1
        lib = _lib.lib()
        nbytes = int(lib.tp_stack_plan_bytes(arr, len(lins), l0.bits, self.batch))
        if nbytes <= 0:
            raise ValueError("invalid stack size")
        self.plan = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        torch.cuda.synchronize(dev)
        _lib.check(lib.tp_stack_plan_init(arr, len(lins), l0.bits, self.batch, self.plan.data_ptr(),
                                          nbytes), "stack_plan_init")
        ns = (ctypes.c_int64 * len(lins))(*[lin.out_features for lin in lins])
        self.total_blocks = int(lib.tp_stack_plan_blocks(ns, len(lins)))
        # (a copy of its own: the GEMV reads the codebook as 4-byte words, and a
        # fresh allocation is aligned whatever view the linear holds)
        self.codebook = l0.codebook.detach().clone()
        self.bits, self.n_states = l0.bits, l0.n_states
        self._entries = arr  # keep the host array alive with the plan

    def run(self) -> list:
        """Launch the stack on the current stream; returns the output buffers."""
        st = _lib.lib().tp_stack_run(self.plan.data_ptr(), self.batch, self.codebook.data_ptr(),
                                     self.bits, self.n_states, int(self.ordered), self.total_blocks,
                                     hk.current_stream_ptr(self.plan.device))
        _lib.check(st, "stack_run")
        return self.outputs

    def rotate(self) -> None:
        """First launch of run(): rotate every input into the plan's z buffer."""
        _lib.check(_lib.lib().tp_stack_rotate(self.plan.data_ptr(), self.batch,
                                              hk.current_stream_ptr(self.plan.device)), "stack_rotate")

    def gemv(self) -> list:
        """Second launch of run(): every GEMV, from the z buffer the last
        rotate() filled."""
        st = _lib.lib().tp_stack_gemv(self.plan.data_ptr(), self.batch, self.codebook.data_ptr(),
                                      self.bits, self.n_states, int(self.ordered), self.total_blocks,
                                      hk.current_stream_ptr(self.plan.device))
        _lib.check(st, "stack_gemv")
        return self.outputs

    def error(self) -> int:
        """1 when a phase wait timed out in any run so far (blocking query)."""
        out = ctypes.c_int()
        _lib.check(_lib.lib().tp_stack_error(self.plan.data_ptr(), ctypes.byref(out)), "stack_error")
        return int(out.value)

    def algorithmic_bytes(self) -> int:
        b = self.batch
        return sum(l.out_features * l.in_features * l.bits // 8 + 2 * l.out_features
                   + 2 * (1 << (l.bits + 1)) + 2 * l.in_features + 2 * b * l.in_features
                   + 2 * b * l.out_features for l in self.linears)


def layer_forward(mods: dict, xs: dict) -> dict:
    """One decoder layer's projections with one launch per shared-input group:
    q/k/v (input xs["attn"]), o (xs["o"]), gate/up (xs["mlp"]), down (xs["down"])."""
    out = {}
    q, k, v = hk.forward_group([mods["q_proj"], mods["k_proj"], mods["v_proj"]], xs["attn"])
    out.update(q_proj=q, k_proj=k, v_proj=v)
    out["o_proj"] = hk.forward_tiled(mods["o_proj"], xs["o"])
    g, u = hk.forward_group([mods["gate_proj"], mods["up_proj"]], xs["mlp"])
    out.update(gate_proj=g, up_proj=u)
    out["down_proj"] = hk.forward_tiled(mods["down_proj"], xs["down"])
    return out


class ChainedDecodeStep:
    """Decoder layers of packed linears run as a data-dependent chain.

    ``layers`` is a list of dicts with the seven Qwen-style projections.  In
    each layer ONE group launch runs q/k/v on the layer input, o runs on q's
    output, ONE group launch runs gate/up on o's output, down runs on gate's
    output, and down's output is the next layer's input: the Qwen3 shapes
    chain exactly (2560 -> 4096 -> 2560 -> 9728 -> 2560 for Qwen3-4B).  k, v
    and up are computed beside the chain, as in a decode step.  Four
    launches per layer, each on the previous one's output, all on the
    current stream with no host synchronisation, so a step can be captured
    in a HIP graph: write the step's activations into ``input`` and replay;
    ``outputs[i]`` holds layer i's seven projections of the last run (after
    capture, tensors of the graph's memory pool that each replay rewrites).
    """

    def __init__(self, layers, input_buffer: Tensor) -> None:
        if not layers:
            raise ValueError("no layers")
        for li, mods in enumerate(layers):
            for a, b in (("q_proj", "o_proj"), ("o_proj", "gate_proj"), ("gate_proj", "down_proj")):
                if mods[a].out_features != mods[b].in_features:
                    raise ValueError(f"layer {li}: {a} output does not feed {b}")
            if li + 1 < len(layers) and mods["down_proj"].out_features != layers[li + 1]["q_proj"].in_features:
                raise ValueError(f"layer {li}: down_proj output does not feed the next layer")
        if input_buffer.shape[-1] != layers[0]["q_proj"].in_features:
            raise ValueError("input buffer does not match the first layer")
        self.layers = layers
        self.input = input_buffer
        self.outputs: list = []

    def run(self) -> Tensor:
        """One decode step; returns the last layer's down_proj output."""
        h = self.input
        outs = []
        for mods in self.layers:
            q, k, v = hk.forward_group([mods["q_proj"], mods["k_proj"], mods["v_proj"]], h)
            o = hk.forward_tiled(mods["o_proj"], q)
            g, u = hk.forward_group([mods["gate_proj"], mods["up_proj"]], o)
            h = hk.forward_tiled(mods["down_proj"], g)
            outs.append({"q_proj": q, "k_proj": k, "v_proj": v, "o_proj": o, "gate_proj": g, "up_proj": u,
                         "down_proj": h})
        self.outputs = outs
        return h

    def layer_inputs(self, li: int) -> dict:
        """The input each projection of layer li read in the last run."""
        prev = self.input if li == 0 else self.outputs[li - 1]["down_proj"]
        out = self.outputs[li]
        return {"q_proj": prev, "k_proj": prev, "v_proj": prev, "o_proj": out["q_proj"],
                "gate_proj": out["o_proj"], "up_proj": out["o_proj"], "down_proj": out["gate_proj"]}


class SharedInputGroup:
    """Packed projections of one decoder layer that read the same input
    (q/k/v, gate/up).  A member call runs ONE launch for all of them
    (tp_packed_linear_forward_group) and holds the outputs of the members
    after it in group order; a later member called on that same input (same
    tensor storage, version and shape) takes its held output, once.  A call
    of a member at or before the last one served starts a new pass and runs
    the group again, dropping every held output, so a member skipped in one
    step cannot hand its old output to the next step even when the input
    buffer is rewritten in place under ``torch.inference_mode()`` (whose
    tensors carry no version counter).  Decoders call the members in group
    order each step (q, k, v; gate, up).  Outputs are those of the members'
    own forwards (x's dtype)."""

    def __init__(self, members) -> None:
        self.members = list(members)
        self._key = None
        self._last = -1
        self._pending = {}

    def run(self, index: int, x):
        version = None if x.is_inference() else x._version
        key = (x.data_ptr(), version, tuple(x.shape), tuple(x.stride()), x.dtype)
        if key == self._key and index > self._last and index in self._pending:
            self._last = index
            return self._pending.pop(index)
        outs = [o.to(x.dtype) for o in hk.forward_group(self.members, x)]
        self._key = key
        self._last = index
        self._pending = {i: o for i, o in enumerate(outs) if i > index}
        return outs[index]


GROUPS = (("self_attn", ("q_proj", "k_proj", "v_proj")), ("mlp", ("gate_proj", "up_proj")))


def fuse_shared_input_projections(model) -> int:
    """Join the q/k/v and gate/up projections of every decoder layer of a
    packed model (device layout, one codebook per group) into
    SharedInputGroups, so a decode step makes 4 projection launches per
    layer instead of 7.  Returns the number of groups formed."""
    from turbopress_amd.artifact import decoder_layers
    from turbopress_amd.runtime import PackedTCQLinear
    count = 0
    for block in decoder_layers(model):
        for parent_name, names in GROUPS:
            parent = getattr(block, parent_name, None)
            mods = [getattr(parent, n, None) for n in names] if parent is not None else []
            if len(mods) != len(names) or not all(isinstance(m, PackedTCQLinear) for m in mods):
                continue
            m0 = mods[0]
            if any(m.tiled_packed is None or m.in_features != m0.in_features or m.bits != m0.bits
                   or m.n_states != m0.n_states or m.codebook_key != m0.codebook_key for m in mods):
                continue
            group = SharedInputGroup(mods)
            for i, m in enumerate(mods):
                m._group, m._group_index = group, i
            count += 1
    return count
