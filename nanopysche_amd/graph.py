"""One training step captured as a HIP graph and replayed.

A step of the MoE layer is ~20 kernel launches whose host-side work (Python,
autograd, ctypes argument packing, tensor allocation) takes about as long as
the kernels themselves at configs[2]'s shapes, so an eagerly issued step is
bound by the host.  Captured once with ``torch.cuda.graph`` (HIP graphs on
ROCm), the step replays all of its kernels -- expert-weight re-quantisation,
routing, the expert block and its backward, the router's backward on a
second stream -- with no host work between them.

The library's kernels suit capture: no entry point allocates, synchronises,
copies to the host or records a memset (scratch is cleared by kernels), and
every launch goes to the caller's current stream (the router's backward to a
second stream joined by events, which the capture follows).
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch


class GraphedStep:
    """Captures ``step_fn`` -- forward + backward on tensors whose storage does
    not change between calls -- and replays it.

    ``leaves``: the tensors whose ``.grad`` the step produces.  Their gradients
    are cleared before capture, so the captured backward writes (does not
    accumulate) them; after each replay they hold that step's gradients.
    ``warmup`` eager calls run first on a side stream (as capture requires).
    ``outputs`` holds what ``step_fn`` returned during capture: tensors that
    every replay rewrites in place.
    """

    def __init__(self, step_fn: Callable[[], object], leaves: Sequence[torch.Tensor] = (), warmup: int = 3):
        self.leaves = list(leaves)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._clear_grads()
                step_fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self._clear_grads()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            out = step_fn()
        # detached views of the static outputs: holding the captured autograd
        # graph alive would tie later eager backward passes to its streams
        if isinstance(out, torch.Tensor):
            out = out.detach()
        elif isinstance(out, (tuple, list)):
            out = type(out)(o.detach() if isinstance(o, torch.Tensor) else o for o in out)
        self.outputs = out
        self.grads = [p.grad for p in self.leaves]

    def _clear_grads(self):
        for p in self.leaves:
            p.grad = None

    def replay(self):
        """One step: every kernel of the captured step, on the current stream's device."""
        self.graph.replay()

    __call__ = replay
