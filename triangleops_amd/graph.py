"""Replay a fixed-shape call of an op (or a composition of ops) as one HIP graph.

At small sizes the ops are bound by host-side launch overhead: each call goes through Python,
ctypes and several kernel launches while the kernels run for microseconds.  `capture` records
one call on a side stream with `torch.cuda.CUDAGraph` (HIP stream capture on ROCm) and returns a
`Graphed` object whose `replay()` relaunches every kernel of the call with one graph launch.

The graph reads its inputs from the tensors passed to `capture` and writes its outputs into the
tensors that call returned: to run it on new values, copy them into the captured inputs
(`graphed.inputs`) and replay; the result is `graphed.output` (overwritten by each replay).
Shapes, dtypes, masks' presence and weights are fixed at capture time.  No kernel of this
package issues a memset or a host synchronisation, so every op of the package captures.
"""

from __future__ import annotations

import torch


class Graphed:
    """A captured call: `inputs` (the tensors the graph reads), `output` (what it writes)."""

    def __init__(self, graph, inputs, output):
        self.graph = graph
        self.inputs = inputs
        self.output = output

    def replay(self):
        self.graph.replay()
        return self.output


def capture(fn, *args, warmup=2, **kwargs):
    """Record `fn(*args, **kwargs)` as a HIP graph (after `warmup` eager calls on the capture
    stream, which also settle the caching allocator).  Tensor arguments are used in place."""
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            fn(*args, **kwargs)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn(*args, **kwargs)
    inputs = [a for a in args if torch.is_tensor(a)] + [v for v in kwargs.values() if torch.is_tensor(v)]
    return Graphed(graph, inputs, out)
