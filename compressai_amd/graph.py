"""HIP-graph capture of a decode step on this library's kernels.

The reference captures its whole model step into a CUDA graph and replays it
per token with the input copied into a static tensor (``FastGenerator``,
vq2/generate.py:49-71: warm-up on a side stream, capture, then
``static_tok.copy_(...); g.replay()``).  ``DecodeStepGraph`` is that pattern
for any step built from this library: every C entry takes device pointers,
enqueues work only (no allocation, no host synchronisation), so a step made
of ``PackedLinear``, ``MoELayer`` / ``ResidentMoEExperts``, the RHT, the
small-M GEMM and the LM-head argmax captures as it is.  ``PagedMoEExperts``
captures with ``device_tables=True`` (the pager then runs on the device); its
host pager reads the routed ids on the host and does not.
"""
from __future__ import annotations

import torch


class DecodeStepGraph:
    """Capture ``step(*inputs)`` once and replay it for new inputs.

    ``example_inputs`` fixes the shapes / dtypes; they are copied into static
    tensors the graph reads.  ``__call__(*inputs)`` copies the new values in,
    replays, and returns the graph's static outputs (overwritten by the next
    replay: clone what must be kept)."""

    def __init__(self, step, example_inputs, warmup: int = 3):
        self.step = step
        self.static_in = [t.detach().clone() for t in example_inputs]
        dev = self.static_in[0].device
        cur = torch.cuda.current_stream(dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            for _ in range(warmup):
                step(*self.static_in)
        cur.wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.static_out = step(*self.static_in)

    def __call__(self, *inputs):
        if len(inputs) != len(self.static_in):
            raise ValueError(f"expected {len(self.static_in)} inputs, got {len(inputs)}")
        for dst, src in zip(self.static_in, inputs):
            if dst.shape != src.shape or dst.dtype != src.dtype:
                raise ValueError("inputs must match the captured shapes and dtypes")
            dst.copy_(src)
        self.graph.replay()
        return self.static_out
